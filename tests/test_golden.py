"""The golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the CPU oracle): the CPU tests check that the committed files are intact
and that the oracle still reproduces them exactly; the GPU tests run every
path of the C ABI on the fixture inputs.  Bars as elsewhere: dequantized
weights and the W8A8 output bit-exact; matmul outputs within
max|got - want| / max|want| <= 1e-3 (f32 output)."""
import hashlib
from pathlib import Path

import numpy as np
import pytest

from conftest import announce

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = 1e-3


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel_err(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


# ------------------------------------------------------------------- CPU
def test_manifest_hashes():
    lines = (GOLDEN / "MANIFEST.txt").read_text().split("\n")
    entries = [l.split() for l in lines if l.strip()]
    assert len(entries) == 8
    for digest, name in entries:
        assert hashlib.sha256((GOLDEN / name).read_bytes()).hexdigest() == digest, name


@pytest.mark.parametrize("name", ["q8_0", "q4_0", "q4_1"])
def test_oracle_reproduces_gguf(orc, name):
    f = load(name)
    k = f["x"].shape[1]
    assert np.array_equal(orc.dequantize(int(f["scheme"]), f["w"], k).view(np.uint32), f["dequant"].view(np.uint32))
    assert np.array_equal(orc.matmul_f64(int(f["scheme"]), f["x"], f["w"], int(f["n"])), f["y"])


@pytest.mark.parametrize("name", ["mlx4_g32", "mlx8_g64"])
def test_oracle_reproduces_mlx(orc, name):
    f = load(name)
    k, bits, group, n = f["x"].shape[1], int(f["bits"]), int(f["group"]), int(f["n"])
    d = orc.mlx_dequantize(f["w"], f["scales"], f["biases"], k, bits, group)
    assert np.array_equal(d.view(np.uint32), f["dequant"].view(np.uint32))
    assert np.array_equal(orc.mlx_matmul_f64(f["x"], f["w"], f["scales"], f["biases"], n, bits, group), f["y"])


def test_oracle_reproduces_grouped_and_moe(orc):
    g = load("grouped_q4_1")
    y = orc.grouped_matmul_f64(orc.Q4_1, g["x"], g["bank"], g["expert_idx"], int(g["n"]), int(g["num_experts"]))
    assert np.array_equal(y, g["y"])
    m = load("moe_q4_1")
    ids, probs = orc.topk_softmax(m["logits"], m["ids"].shape[1], renorm=True)
    assert np.array_equal(ids, m["ids"]) and np.array_equal(probs, m["probs"])
    assert np.array_equal(orc.moe_f64(orc.Q4_1, m["x"], m["bank"], m["ids"], m["probs"], int(m["n"]),
                                      int(m["num_experts"])), m["y"])


def test_oracle_reproduces_int8(orc):
    f = load("int8")
    qx, sx = orc.quantize_act_int8(f["x"])
    assert np.array_equal(qx, f["qx"]) and np.array_equal(sx.view(np.uint32), f["sx"].view(np.uint32))
    assert np.array_equal(orc.w8a8_matmul(f["qx"], f["sx"], f["qw"], f["sw"]).view(np.uint32),
                          f["y_w8a8"].view(np.uint32))
    assert np.array_equal(orc.int8_block_matmul_f64(f["x"], f["qw"], f["sw"]), f["y_i8b"])
    assert np.array_equal(orc.int8_block_matmul_f64(f["x"], f["qw"], f["sw"], f["zp"]), f["y_i8b_zp"])


# ------------------------------------------------------------------- GPU
def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["q8_0", "q4_0", "q4_1"])
def test_gpu_gguf_golden(ctx, name):
    import torch

    f = load(name)
    scheme, n, k = int(f["scheme"]), int(f["n"]), f["x"].shape[1]
    announce(f"golden {name}")
    d = ctx.dequantize(_t(f["w"]), scheme, n, k)
    y = ctx.dequant_matmul(_t(f["x"]), _t(f["w"]), scheme, n)
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy().view(np.uint32), f["dequant"].view(np.uint32))
    assert rel_err(y.cpu().numpy(), f["y"]) <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["mlx4_g32", "mlx8_g64"])
def test_gpu_mlx_golden(ctx, name):
    import torch
    import rlxq

    f = load(name)
    bits, group, n, k = int(f["bits"]), int(f["group"]), int(f["n"]), f["x"].shape[1]
    scheme = rlxq.MLX_AFFINE4 if bits == 4 else rlxq.MLX_AFFINE8
    announce(f"golden {name}")
    kw = dict(group=group, scales=_t(f["scales"]), biases=_t(f["biases"]))
    d = ctx.dequantize(_t(f["w"].view(np.uint8)), scheme, n, k, **kw)
    y = ctx.dequant_matmul(_t(f["x"]), _t(f["w"].view(np.uint8)), scheme, n, **kw)
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy().view(np.uint32), f["dequant"].view(np.uint32))
    assert rel_err(y.cpu().numpy(), f["y"]) <= TOL


@pytest.mark.gpu
def test_gpu_grouped_and_moe_golden(ctx):
    import torch
    import rlxq

    g = load("grouped_q4_1")
    announce("golden grouped")
    y = ctx.grouped_matmul(_t(g["x"]), _t(g["bank"]), _t(g["expert_idx"]), rlxq.GGUF_Q4_1, int(g["n"]),
                           int(g["num_experts"]))
    m = load("moe_q4_1")
    announce("golden moe")
    ids, probs = ctx.moe_route(_t(m["logits"]), m["ids"].shape[1], True)
    xe = np.repeat(m["x"], m["ids"].shape[1], axis=0)  # one activation row per (token, slot) entry
    ym = ctx.moe_grouped(_t(xe), _t(m["bank"]), ids, probs, rlxq.GGUF_Q4_1, rlxq.MOE_COMBINE, int(m["n"]),
                         int(m["num_experts"]))
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), g["y"]) <= TOL
    assert np.array_equal(ids.cpu().numpy(), m["ids"])
    assert np.allclose(probs.cpu().numpy(), m["probs"], rtol=1e-6, atol=1e-7)
    assert rel_err(ym.cpu().numpy(), m["y"]) <= TOL


@pytest.mark.gpu
def test_gpu_int8_golden(ctx):
    import torch
    import rlxq

    f = load("int8")
    n, k = f["qw"].shape[1], f["x"].shape[1]
    announce("golden int8")
    y8 = ctx.w8a8_gemm(_t(f["x"]), _t(f["qw"]), _t(f["sw"]), n)
    yb = ctx.dequant_matmul(_t(f["x"]), _t(f["qw"]), rlxq.INT8_BLOCK, n, group=k, scales=_t(f["sw"]))
    yz = ctx.dequant_matmul(_t(f["x"]), _t(f["qw"]), rlxq.INT8_BLOCK, n, group=k, scales=_t(f["sw"]),
                            biases=_t(f["zp"]))
    torch.cuda.synchronize()
    assert np.array_equal(y8.cpu().numpy().view(np.uint32), f["y_w8a8"].view(np.uint32))
    assert rel_err(yb.cpu().numpy(), f["y_i8b"]) <= TOL
    assert rel_err(yz.cpu().numpy(), f["y_i8b_zp"]) <= TOL
