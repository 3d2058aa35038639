"""Prefill dequant-GEMM (bf16 MFMA, weights rounded to bf16 in LDS) for the
GGUF K-quant super-blocks Q6_K, Q5_K, Q3_K, Q2_K and Q8_K and MLX MXFP4
codes, through the C ABI, against the float64 oracle on the activations the
kernel saw.  Q6_K's 210-byte and Q3_K's 110-byte super-blocks start 2-byte
aligned every other time (and whole rows do when K / 256 is odd); the kernel
reads them through aligned dwords.  Bar:
the prefill bar 2e-2 (bf16 output); every tiling agrees with the 128 x 128
one to ~1e-6 on f32 output."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, rel_err

pytestmark = pytest.mark.gpu

TOL_PREFILL = 2e-2
Q6_K, Q8_K, MXFP4, Q5_K, Q3_K, Q2_K = 8, 13, 9, 10, 11, 12
NAMES = {Q6_K: "q6_k", Q8_K: "q8_k", MXFP4: "mxfp4", Q5_K: "q5_k", Q3_K: "q3_k", Q2_K: "q2_k"}
ALL = [Q6_K, Q5_K, Q3_K, Q2_K, Q8_K, MXFP4]


def _weights(orc, scheme, rng, n, k, mx_scales="u8"):
    """(packed weights, kwargs for dequant_matmul, float64 dequantized rows)."""
    import torch

    if scheme == MXFP4:
        codes, eb = orc.synth_mxfp4(rng, n, k)
        if mx_scales == "bf16":
            s = (eb.astype(np.uint16) << 7)
            st = _t(s.view(np.int16)).view(torch.bfloat16)
        else:
            s, st = eb, _t(eb)
        return codes, dict(scales=st), orc.mxfp4_dequantize(codes, s, n, k).astype(np.float64)
    packed = orc.synth(scheme, rng, n, k)
    return packed, {}, orc.dequantize(scheme, packed, k).astype(np.float64)


def _run(ctx, scheme, x32, packed, kw, n, ydt):
    import torch

    xt = _t(x32).to(torch.bfloat16)
    y = ctx.dequant_matmul(xt, _t(packed), scheme, n, y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32,
                           **kw)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), xt.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("scheme", ALL, ids=lambda s: NAMES[s])
@pytest.mark.parametrize("mkn", [(64, 4096, 520), (300, 1280, 272), (512, 4096, 1024), (129, 12288, 300)], ids=str)
def test_prefill_default_kernel(ctx, orc, scheme, mkn):
    """bf16 activations and output from 64 rows take the 256 x 256 GEMM
    (split-K where the tiles do not cover the CUs)."""
    m, k, n = mkn
    announce(f"gemm {NAMES[scheme]} {mkn}")
    rng = np.random.default_rng(m + k + scheme)
    packed, kw, wd = _weights(orc, scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, xv = _run(ctx, scheme, x, packed, kw, n, "bf16")
    assert ctx.last_kernel.startswith(f"rlxq_gemm_{NAMES[scheme]}_t256"), ctx.last_kernel
    assert rel_err(got, xv @ wd.T) <= TOL_PREFILL


@pytest.mark.parametrize("scheme", ALL, ids=lambda s: NAMES[s])
def test_every_tiling_agrees(ctx, orc, monkeypatch, scheme):
    """Every tiling on a ragged shape with an odd super-block count (Q6_K rows
    and Q3_K rows alternate 4- and 2-byte alignment), f32 output forced onto
    the GEMM: each
    within the bar, all within ~1e-6 of the 128 x 128 tiling."""
    m, k, n = 300, 1280, 272
    rng = np.random.default_rng(17 + scheme)
    packed, kw, wd = _weights(orc, scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    monkeypatch.setenv("RLXQ_PREFILL", "gemm")
    outs = {}
    for tile in ("128", "256", "256w8", "256w8l", "256w8p2", "256n128", "256n128w8"):
        if tile == "256w8p2" and scheme in (Q6_K, Q3_K):
            continue   # (its two register stages do not fit these raw blocks)
        monkeypatch.setenv("RLXQ_GEMM_TILE", tile)
        announce(f"gemm tiling {NAMES[scheme]} t{tile}")
        got, xv = _run(ctx, scheme, x, packed, kw, n, "f32")
        assert ctx.last_kernel == f"rlxq_gemm_{NAMES[scheme]}_t{tile}", ctx.last_kernel
        assert rel_err(got, xv @ wd.T) <= TOL_PREFILL
        outs[tile] = got
    for t, o in outs.items():
        assert np.allclose(outs["128"], o, rtol=1e-6, atol=1e-6 * np.abs(outs["128"]).max()), t


def test_mxfp4_bf16_scales_and_split_k(ctx, orc, monkeypatch):
    """MXFP4 with the decoded bf16 scale slab, and K cut into slices."""
    m, k, n = 256, 64 * 13, 300
    rng = np.random.default_rng(5)
    packed, kw, wd = _weights(orc, MXFP4, rng, n, k, mx_scales="bf16")
    x = rng.standard_normal((m, k)).astype(np.float32)
    for sp in ("1", "3"):
        monkeypatch.setenv("RLXQ_GEMM_SPLITS", sp)
        got, xv = _run(ctx, MXFP4, x, packed, kw, n, "bf16")
        assert ctx.last_kernel.startswith("rlxq_gemm_mxfp4_t256"), ctx.last_kernel
        assert rel_err(got, xv @ wd.T) <= TOL_PREFILL, sp


@pytest.mark.parametrize("scheme", ALL, ids=lambda s: NAMES[s])
def test_f32_output_prefill_route(ctx, orc, scheme):
    """f32 output is not routed to the bf16-weight GEMM: the K-quants take the
    exact variant (each weight's f32 value as f16 hi + lo rows), MXFP4 with
    E8M0 scales the bf16 GEMM (its weights are exact in bf16, as are bf16
    activations); both keep the 1e-3 bar."""
    m, k, n = 300, 1024, 200
    rng = np.random.default_rng(3 + scheme)
    packed, kw, wd = _weights(orc, scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, xv = _run(ctx, scheme, x, packed, kw, n, "f32")
    if scheme == MXFP4:
        # (the bf16 GEMM; 256 x 128 tiles where 256 x 256 ones would split K)
        assert ctx.last_kernel in ("rlxq_gemm_mxfp4_t256w8p2", "rlxq_gemm_mxfp4_t256n128w8"), ctx.last_kernel
    else:
        assert ctx.last_kernel.startswith(f"rlxq_gemm_{NAMES[scheme]}_t256w8") and ctx.last_kernel.endswith("x"), \
            ctx.last_kernel
    assert rel_err(got, xv @ wd.T) <= 1e-3
