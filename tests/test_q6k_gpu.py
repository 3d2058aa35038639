"""GGUF Q6_K (the Q4_K_M checkpoints' second format) through the C ABI: the
bit-exact dequantisation and the dense DequantMatMul on the LDS-record GEMV
(any M, f32 or bf16 activations), against the oracle's restatement of GGML
block_q6_K.  Rows of an odd number of super-blocks start 2-byte aligned,
which the kernels read through aligned dwords.  Bar: max|got - want| /
max|want| <= 1e-3 against float64 from the activations the kernel saw."""
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
    y = ctx.dequant_matmul(xt, _t(packed), rlxq.GGUF_Q6_K, n, **kw)
    torch.cuda.synchronize()
    k = x32.shape[1]
    want = xt.float().cpu().numpy().astype(np.float64) @ orc.dequantize(orc.Q6_K, packed, k).astype(np.float64).T
    return y.float().cpu().numpy(), want


@pytest.mark.parametrize("nk", [(37, 4096), (5, 256), (9, 768), (64, 12288)], ids=str)
def test_q6k_dequantize_bit_exact(ctx, orc, nk):
    import torch
    import rlxq

    n, k = nk
    announce(f"q6_k dequantize n={n} k={k}")
    packed = orc.synth_q6_k(np.random.default_rng(n + k), n, k)
    want = orc.dequantize(orc.Q6_K, packed, k).view(np.uint32)
    got = ctx.dequantize(_t(packed), rlxq.GGUF_Q6_K, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)
    buf = torch.full((n * k + 1,), float("nan"), device="cuda")
    ctx.dequantize(_t(packed), rlxq.GGUF_Q6_K, n, k, out=buf[1:].view(n, k))
    torch.cuda.synchronize()
    assert np.array_equal(buf[1:].cpu().numpy().view(np.uint32).reshape(n, k), want)


@pytest.mark.parametrize("kn", [(4096, 1031), (768, 37), (12288, 300), (256, 17), (4096, 24576), (1280, 96)],
                         ids=str)
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_q6k_gemv(ctx, orc, kn, xdt):
    k, n = kn
    announce(f"q6_k gemv m=1 x={xdt} k={k} n={n}")
    rng = np.random.default_rng(k + n)
    packed = orc.synth_q6_k(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, want = _run(ctx, orc, x, packed, n, xdt=xdt)
    assert ctx.last_kernel.startswith("rlxq_gemv_q6_k_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL


@pytest.mark.parametrize("m", [2, 3, 4, 7, 64])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_q6k_multi_row(ctx, orc, m, xdt):
    k, n = 2304, 520
    announce(f"q6_k gemv m={m} x={xdt}")
    rng = np.random.default_rng(m)
    packed = orc.synth_q6_k(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= 300.0
    got, want = _run(ctx, orc, x, packed, n, xdt=xdt)
    assert rel_err(got, want) <= TOL


@pytest.mark.parametrize("cfg", ["64,1,2,1,16", "64,1,2,2,16", "64,1,2,2,8", "64,1,1,4,16", "64,2,1,2,8",
                                 "32,2,1,2,8", "16,2,1,2,8", "8,2,1,2,8"])
def test_q6k_every_record_variant(ctx, orc, monkeypatch, cfg):
    monkeypatch.setenv("RLXQ_GEMV_CFG", cfg)
    k, n = 2816, 300          # 11 super-blocks: rows alternate 2- and 4-byte alignment
    announce(f"q6_k variant {cfg}")
    rng = np.random.default_rng(11)
    packed = orc.synth_q6_k(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, want = _run(ctx, orc, x, packed, n, xdt="f32")
    L, P, C, D, W = cfg.split(",")
    assert ctx.last_kernel == f"rlxq_gemv_q6_k_f32_L{L}_P{P}_C{C}_M1_D{D}_W{W}", ctx.last_kernel
    assert rel_err(got, want) <= TOL


def test_q6k_bf16_output_and_prefill_rows(ctx, orc, monkeypatch):
    """bf16 output from 64 rows: the MFMA GEMM by default, the GEMV's
    multi-row path when forced (RLXQ_PREFILL and RLXQ_DECODE: 80 rows would
    otherwise take the batched-decode MFMA kernels)."""
    import torch

    k, n, m = 1024, 300, 80
    rng = np.random.default_rng(4)
    packed = orc.synth_q6_k(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = _run(ctx, orc, x, packed, n, y_dtype=torch.bfloat16)
    assert ctx.last_kernel.startswith("rlxq_gemm_q6_k_t256"), ctx.last_kernel
    assert rel_err(got, want) <= 2e-2
    monkeypatch.setenv("RLXQ_PREFILL", "gemv")
    monkeypatch.setenv("RLXQ_DECODE", "gemv")
    got, want = _run(ctx, orc, x, packed, n, y_dtype=torch.bfloat16)
    assert ctx.last_kernel.startswith("rlxq_gemv_q6_k_"), ctx.last_kernel
    assert rel_err(got, want) <= 2e-2


def test_q6k_host_checks_and_session(ctx, orc):
    import torch
    import rlxq

    assert rlxq.lib().rlxq_row_bytes(rlxq.GGUF_Q6_K, 768) == 630
    assert rlxq.lib().rlxq_row_bytes(rlxq.GGUF_Q6_K, 300) == -1
    x = torch.zeros((1, 512), device="cuda", dtype=torch.bfloat16)
    wf = torch.zeros((4 * 420 + 16,), device="cuda", dtype=torch.uint8)
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul(x[:, :288].contiguous(), wf[:4 * 420], rlxq.GGUF_Q6_K, 4)
    assert e.value.status == rlxq.E_SHAPE
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul(x, wf[2:2 + 4 * 420], rlxq.GGUF_Q6_K, 4)
    assert e.value.status == rlxq.E_ALIGN
    idx = torch.zeros((1,), device="cuda")
    with pytest.raises(rlxq.RlxqError) as e:   # the grouped op checks the same way
        ctx.grouped_matmul(x, wf[2:2 + 4 * 420], idx, rlxq.GGUF_Q6_K, 4, 1)
    assert e.value.status == rlxq.E_ALIGN
    dm = rlxq.DeviceMatmul(0)
    rng = np.random.default_rng(9)
    m, k, n = 2, 768, 129
    packed = orc.synth_q6_k(rng, n, k).ravel()
    xs = rng.standard_normal((m, k)).astype(np.float32)
    y = dm.matmul(xs, packed, m, k, n, rlxq.GGUF_Q6_K).reshape(m, n)
    want = xs.astype(np.float64) @ orc.dequantize(orc.Q6_K, packed, k).astype(np.float64).T
    assert rel_err(y, want) <= TOL
    dm.close()
