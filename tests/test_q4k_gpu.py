"""GGUF Q4_K (the Q4_K_M checkpoints' main format) through the C ABI: the
bit-exact dequantisation and the dense DequantMatMul (register-activation
GEMV at M=1 with bf16 activations; the LDS-record GEMV for f32 activations
and M > 1), against the oracle's restatement of GGML block_q4_K.  Bar:
max|got - want| / max|want| <= 1e-3, want in float64 from the activations
the kernel saw."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _run(ctx, orc, x32, packed, n, xdt="bf16", **kw):
    import torch
    import rlxq

    xt = _t(x32)
    if xdt == "bf16":
        xt = xt.to(torch.bfloat16)
    y = ctx.dequant_matmul(xt, _t(packed), rlxq.GGUF_Q4_K, n, **kw)
    torch.cuda.synchronize()
    k = x32.shape[1]
    want = xt.float().cpu().numpy().astype(np.float64) @ orc.dequantize(orc.Q4_K, packed, k).astype(np.float64).T
    return y.float().cpu().numpy(), want


@pytest.mark.parametrize("nk", [(37, 4096), (5, 256), (64, 12288)], ids=str)
def test_q4k_dequantize_bit_exact(ctx, orc, nk):
    import torch
    import rlxq

    n, k = nk
    announce(f"q4_k dequantize n={n} k={k}")
    packed = orc.synth_q4_k(np.random.default_rng(n + k), n, k)
    want = orc.dequantize(orc.Q4_K, packed, k).view(np.uint32)
    got = ctx.dequantize(_t(packed), rlxq.GGUF_Q4_K, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)
    buf = torch.full((n * k + 1,), float("nan"), device="cuda")
    ctx.dequantize(_t(packed), rlxq.GGUF_Q4_K, n, k, out=buf[1:].view(n, k))
    torch.cuda.synchronize()
    assert np.array_equal(buf[1:].cpu().numpy().view(np.uint32).reshape(n, k), want)


@pytest.mark.parametrize("kn", [(4096, 1031), (12288, 300), (2048, 64), (8192, 517), (256, 17), (4096, 24576)],
                         ids=str)
def test_q4k_gemv_register_path(ctx, orc, kn):
    k, n = kn
    announce(f"q4_k gemv m=1 bf16 k={k} n={n}")
    rng = np.random.default_rng(k + n)
    packed = orc.synth_q4_k(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, want = _run(ctx, orc, x, packed, n)
    assert ctx.last_kernel.startswith("rlxq_gemvxs_q4_k_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL


@pytest.mark.parametrize("cfg,k", [("1,2,8,1", 2048), ("2,2,8,1", 8192), ("2,1,8,1", 4096), ("3,1,8,1", 12288)])
def test_q4k_every_register_variant(ctx, orc, monkeypatch, cfg, k):
    monkeypatch.setenv("RLXQ_GEMV_XR", cfg)
    n = 777
    announce(f"q4_k xs variant {cfg} k={k}")
    rng = np.random.default_rng(k)
    packed = orc.synth_q4_k(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, want = _run(ctx, orc, x, packed, n)
    nu, d = cfg.split(",")[:2]
    assert ctx.last_kernel == f"rlxq_gemvxs_q4_k_U{nu}_D{d}_W8", ctx.last_kernel
    assert rel_err(got, want) <= TOL


@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 64])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_q4k_record_path(ctx, orc, monkeypatch, m, xdt):
    """The LDS-record GEMV: f32 activations, and every M > 1 (bf16 M = 2..4
    take the register kernel by default, bf16 M >= 5 the batched-decode MFMA
    kernels; RLXQ_GEMV_XR=0 and RLXQ_DECODE=gemv keep them here)."""
    if m == 1 and xdt == "bf16":
        pytest.skip("register path")
    monkeypatch.setenv("RLXQ_GEMV_XR", "0")
    monkeypatch.setenv("RLXQ_DECODE", "gemv")
    k, n = 4096, 520
    announce(f"q4_k gemv m={m} x={xdt}")
    rng = np.random.default_rng(m)
    packed = orc.synth_q4_k(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= 300.0
    got, want = _run(ctx, orc, x, packed, n, xdt=xdt)
    assert ctx.last_kernel.startswith("rlxq_gemv_q4_k_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL


def test_q4k_bf16_output(ctx, orc):
    import torch

    k, n = 4096, 300
    rng = np.random.default_rng(3)
    packed = orc.synth_q4_k(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, want = _run(ctx, orc, x, packed, n, y_dtype=torch.bfloat16)
    assert rel_err(got, want) <= 2e-2


def test_q4k_host_checks(ctx):
    import torch
    import rlxq

    assert rlxq.lib().rlxq_row_bytes(rlxq.GGUF_Q4_K, 4096) == 2304
    assert rlxq.lib().rlxq_row_bytes(rlxq.GGUF_Q4_K, 300) == -1
    x = torch.zeros((1, 512), device="cuda", dtype=torch.bfloat16)
    w = torch.zeros((4, 288 + 16), device="cuda", dtype=torch.uint8)
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul(x[:, :288].contiguous(), w, rlxq.GGUF_Q4_K, 4)
    assert e.value.status == rlxq.E_SHAPE
    wf = torch.zeros((4 * 288 + 16,), device="cuda", dtype=torch.uint8)
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul(x, wf[4:4 + 4 * 288], rlxq.GGUF_Q4_K, 4)
    assert e.value.status == rlxq.E_ALIGN
    idx = torch.zeros((1,), device="cuda")
    with pytest.raises(rlxq.RlxqError) as e:   # the grouped op checks the same way
        ctx.grouped_matmul(x[:, :288].contiguous(), wf[:4 * 288], idx, rlxq.GGUF_Q4_K, 4, 1)
    assert e.value.status == rlxq.E_SHAPE
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.grouped_matmul(x, wf[4:4 + 4 * 288], idx, rlxq.GGUF_Q4_K, 4, 1)
    assert e.value.status == rlxq.E_ALIGN


@pytest.mark.parametrize("mkn", [(64, 4096, 520), (300, 1280, 272), (512, 4096, 1024), (129, 12288, 300)], ids=str)
@pytest.mark.parametrize("tile", [None, "128", "256", "256w8"])
def test_q4k_prefill_gemm(ctx, orc, monkeypatch, mkn, tile):
    """bf16 activations and output from 64 rows: the MFMA dequant-GEMM
    (weights rounded to bf16 in LDS), every tiling, split-K where it applies;
    the prefill bar 2e-2."""
    import torch

    if tile:
        monkeypatch.setenv("RLXQ_GEMM_TILE", tile)
    m, k, n = mkn
    announce(f"q4_k gemm {mkn} tile={tile}")
    rng = np.random.default_rng(m + k)
    packed = orc.synth_q4_k(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = _run(ctx, orc, x, packed, n, y_dtype=torch.bfloat16)
    assert ctx.last_kernel.startswith("rlxq_gemm_q4_k_t" + (tile or "256")), ctx.last_kernel
    assert rel_err(got, want) <= 2e-2


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_q4k_f32_output_prefill_on_f16_gemm(ctx, orc, xdt):
    """f32 output past 256 rows takes the exact GEMM (each weight's f32 value
    d*sc*q - dmin*mn as f16 hi + lo), within the 1e-3 bar; f32 activations
    as hi/lo row pairs."""
    m, k, n = 300, 1024, 200
    rng = np.random.default_rng(5)
    packed = orc.synth_q4_k(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = _run(ctx, orc, x, packed, n, xdt=xdt)
    assert ctx.last_kernel == "rlxq_gemm_q4_k_t256w8p2" + ("xs" if xdt == "f32" else "x"), ctx.last_kernel
    assert rel_err(got, want) <= TOL


def test_q4k_device_matmul_session(orc):
    """The reference's DeviceMatmul scheme table carries GgufQ4K
    (crates/rlx-laguna/src/device_matmul.rs:64-76): the session API serves it."""
    import rlxq

    dm = rlxq.DeviceMatmul(0)
    rng = np.random.default_rng(8)
    m, k, n = 3, 1024, 333
    packed = orc.synth_q4_k(rng, n, k).ravel()
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = dm.matmul(x, packed, m, k, n, rlxq.GGUF_Q4_K).reshape(m, n)
    want = x.astype(np.float64) @ orc.dequantize(orc.Q4_K, packed, k).astype(np.float64).T
    assert rel_err(y, want) <= TOL
    dm.close()
