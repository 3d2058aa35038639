"""CPU check of the bar the f32-activation GPU tests use
(tests/test_f32_contract_gpu.py): with weights exact in f16 (Q4_1 with d a
power of two and m = 0), the hi + lo split of the activations the kernels
use (f16 pairs on a power-of-two row scale, bf16 pairs on the single-row
GEMV) stays far inside 2e-5 of the float64 product, while the hi row alone
(activations rounded once to f16 or bf16) misses it by an order of magnitude
or more.  So a kernel that dropped or misplaced the lo row fails that bar."""
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
