"""CPU checks of the bars the f32-activation GPU tests use
(tests/test_f32_contract_gpu.py): with weights exact in f16 (Q4_1 with d a
power of two and m = 0), the hi + lo split of the activations the kernels
use (f16 pairs on a power-of-two row scale, bf16 pairs on the single-row
GEMV) stays far inside 2e-5 of the float64 product, while the hi row alone
(activations rounded once to f16 or bf16) misses it by an order of magnitude
or more.  So a kernel that dropped or misplaced the lo row fails that bar.
On the reference's structured parity inputs, weights rounded once to f16
miss the 1e-3 bar itself: the reason the MFMA kernels carry exact weights."""
import numpy as np
import pytest

from test_golden import rel_err

TOL_EXACT_W = 2e-5


def _exact_q4_1(orc, rng, n, k):
    packed = orc.synth_q4_1(rng, n, k)
    blk = packed.reshape(-1, 20)
    blk[:, 0:2] = np.frombuffer(np.float16(2.0 ** -6).tobytes(), np.uint8)
    blk[:, 2:4] = 0
    return orc.dequantize(3, packed, k).astype(np.float64)


def _bf16(a):
    """Round-to-nearest-even f32 -> bf16, back to f32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("mkn", [(64, 4096, 256), (1, 8192, 300), (7, 4096, 128)], ids=str)
def test_lo_row_carries_the_bits(orc, mkn):
    m, k, n = mkn
    rng = np.random.default_rng(m + k + n)
    w = _exact_q4_1(orc, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    want = x.astype(np.float64) @ w.T
    # f16 pairs on the row scale that puts the row maximum in [2^13, 2^14)
    amax = np.abs(x).max(axis=1, keepdims=True)
    s = np.ldexp(np.float32(1.0), (13 - np.floor(np.log2(amax))).astype(np.int32)).astype(np.float32)
    xs = x * s
    hi = xs.astype(np.float16).astype(np.float32)
    lo = (xs - hi).astype(np.float16).astype(np.float32)
    assert rel_err((hi.astype(np.float64) + lo) / s @ w.T, want) <= TOL_EXACT_W / 100
    assert rel_err(hi.astype(np.float64) / s @ w.T, want) >= 5 * TOL_EXACT_W
    # bf16 pairs (no scale)
    hb = _bf16(x)
    lb = _bf16(x - hb)
    assert rel_err((hb.astype(np.float64) + lb) @ w.T, want) <= TOL_EXACT_W / 4
    assert rel_err(hb.astype(np.float64) @ w.T, want) >= 20 * TOL_EXACT_W


@pytest.mark.parametrize("scheme", [2, 3], ids=["q4_0", "q4_1"])
def test_reference_inputs_need_exact_weights(orc, scheme):
    """On the reference's own parity data (quant_parity_backends.rs:61-71,
    K = 1792), weights rounded once to f16 already miss the 1e-3 f32-output
    bar, and activations rounded once to f16 (after the power-of-two row
    scale) stay under it but miss the 5e-5 bar of the GPU test
    test_reference_structured_inputs_every_path: that bar catches either
    rounding, so the MFMA kernels carry weights and f32 activations exactly
    (hi + lo)."""
    k, n, m = 1792, 1280, 7
    x = (np.sin(np.arange(m * k, dtype=np.float32) * np.float32(0.031)) * np.float32(0.8)).reshape(m, k)
    wf = (np.cos(np.arange(n * k, dtype=np.float32) * np.float32(0.017) + np.float32(0.3))
          * np.float32(0.35)).reshape(n, k)
    w = orc.dequantize(scheme, orc.quantize(scheme, wf), k).astype(np.float64)
    want = x.astype(np.float64) @ w.T
    w16 = w.astype(np.float16).astype(np.float64)
    assert rel_err(x.astype(np.float64) @ w16.T, want) > 1e-3
    e = (13 - np.floor(np.log2(np.abs(x).max(axis=1, keepdims=True)))).astype(np.int32)
    s = np.ldexp(np.float32(1.0), e)
    x16 = (x * s).astype(np.float16).astype(np.float64) / s
    assert 5e-5 < rel_err(x16 @ w.T, want) < 1e-3
