"""MXFP4 (QuantScheme::MlxMxfp4) through the C ABI against the oracle's
restatement of crates/rlx-models-core/src/mxfp4_pack.rs (itself pinned in
tests/test_oracle.py on the reference's own tests).  Bars: dequantize
bit-exact; products max|got - want| / max|want| <= 1e-3 (f32 accumulate),
2e-2 for bf16 output.  Dense calls take the E8M0 bytes (the reference's
dense operand, U8 [N, K/32]) or the decoded bf16 scales; grouped calls take
the decoded bf16 [E, N, K/32] the reference's grouped op holds."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, _x_as, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3
MX = 9


def _weights(orc, rng, n, k, scale_kind="u8"):
    codes, eb = orc.synth_mxfp4(rng, n, k)
    if scale_kind == "bf16":
        return codes, (eb.astype(np.uint16) << 7)   # 2^(b-127) as bf16 bits, exact
    return codes, eb


def _scales_t(s):
    import torch

    if s.dtype == np.uint16:
        return _t(s.view(np.int16)).view(torch.bfloat16)
    return _t(s)


def test_dequantize_every_code_bit_exact(ctx, orc):
    """All 256 code bytes in every position class, and scale bytes across the
    E8M0 range including 0 (reads as 0) and 255 (2^127)."""
    import torch

    announce("mxfp4 dequantize")
    rows, k = 24, 512
    rng = np.random.default_rng(40)
    codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
    codes[0] = np.arange(256, dtype=np.uint8)
    eb = rng.integers(100, 150, (rows, k // 32), dtype=np.uint8)
    eb[1, :6] = [0, 1, 127, 200, 254, 255]
    for kind in ("u8", "bf16"):
        s = eb if kind == "u8" else np.where(eb == 255, 254, eb).astype(np.uint16) << 7
        out = ctx.dequantize(_t(codes), MX, rows, k, scales=_scales_t(s))
        torch.cuda.synchronize()
        with np.errstate(over="ignore"):   # 6 * 2^127 is inf in f32, as on the device
            want = orc.mxfp4_dequantize(codes, s, rows, k).astype(np.float32)
        got = out.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), kind


@pytest.mark.parametrize("shape", [(1, 2048, 1024), (1, 4096, 4096), (1, 12288, 512), (1, 768, 256),
                                   (3, 4096, 640), (16, 1024, 512), (64, 2048, 256)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_dense_matmul(ctx, orc, shape, xdt):
    import torch

    m, k, n = shape
    announce(f"mxfp4 dense m={m} k={k} n={n} x={xdt}")
    rng = np.random.default_rng(41 + m + k)
    codes, eb = _weights(orc, rng, n, k)
    x32 = rng.standard_normal((m, k)).astype(np.float32)
    xt, xv = _x_as(x32, xdt)
    y = ctx.dequant_matmul(xt, _t(codes), MX, n, scales=_scales_t(eb))
    torch.cuda.synchronize()
    assert "mxfp4" in ctx.last_kernel
    assert rel_err(y.cpu().numpy(), orc.mxfp4_matmul_f64(xv, codes, eb, n)) <= TOL


def test_dense_bf16_scales_and_bf16_out(ctx, orc):
    import torch

    m, k, n = 64, 2048, 384
    announce("mxfp4 dense bf16 scales, bf16 out")
    rng = np.random.default_rng(42)
    codes, s = _weights(orc, rng, n, k, "bf16")
    x32 = rng.standard_normal((m, k)).astype(np.float32)
    xt, xv = _x_as(x32, "bf16")
    y = ctx.dequant_matmul(xt, _t(codes), MX, n, scales=_scales_t(s), y_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert rel_err(y.float().cpu().numpy(), orc.mxfp4_matmul_f64(xv, codes, s, n)) <= 2e-2
    y1 = ctx.dequant_matmul(xt[:1].contiguous(), _t(codes), MX, n, scales=_scales_t(s))
    torch.cuda.synchronize()
    assert rel_err(y1.cpu().numpy(), orc.mxfp4_matmul_f64(xv[:1], codes, s, n)) <= TOL


@pytest.mark.parametrize("shape", [(16, 2048, 768, 8), (10, 768, 1024, 5), (40, 512, 256, 3)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_grouped_matmul(ctx, orc, shape, xdt):
    """Op::DequantGroupedMatMulMlx with MXFP4 experts: codes [E, N, K/2], the
    decoded scales as bf16 [E, N, K/32] (standard_decoder.rs:935-1000)."""
    import torch

    rows, k, n, E = shape
    announce(f"mxfp4 grouped rows={rows} k={k} n={n} E={E} x={xdt}")
    rng = np.random.default_rng(43 + rows)
    codes, s = _weights(orc, rng, E * n, k, "bf16")
    x32 = rng.standard_normal((rows, k)).astype(np.float32)
    xt, xv = _x_as(x32, xdt)
    idx = ((np.arange(rows) * 7 + 2) % E).astype(np.float32)
    y = ctx.grouped_matmul(xt, _t(codes), _t(idx), MX, n, E, scales=_scales_t(s))
    torch.cuda.synchronize()
    assert "mxfp4" in ctx.last_kernel
    W = orc.mxfp4_dequantize(codes, s, E * n, k).reshape(E, n, k)
    want = np.stack([xv[r].astype(np.float64) @ W[int(idx[r])].T for r in range(rows)])
    assert rel_err(y.cpu().numpy(), want) <= TOL


def test_host_checks(ctx, orc):
    import rlxq
    import torch

    announce("mxfp4 host checks")
    rng = np.random.default_rng(44)
    codes, eb = _weights(orc, rng, 64, 256)
    x = _t(rng.standard_normal((1, 256)).astype(np.float32))
    for kw, status in ((dict(group=64, scales=_t(eb)), rlxq.E_SHAPE),
                       (dict(scales=_t(eb.astype(np.float32))), rlxq.E_DTYPE),
                       (dict(scales=None), rlxq.E_NULL)):
        with pytest.raises(rlxq.RlxqError) as e:
            ctx.dequant_matmul(x, _t(codes), MX, 64, **kw)
        assert e.value.status == status
    torch.cuda.synchronize()
