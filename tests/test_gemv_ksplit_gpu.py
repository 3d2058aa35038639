"""The K-split register GEMV (rlxq_gemvxs_q4_1_*_K<KS>: KS waves of a
workgroup take the same Q4_1 weight row, each a contiguous KS-th of its
units, and their row sums are added in LDS in part order), one activation
row, bf16 or f32 (hi + lo bf16 rows), against the oracle in float64.  Bars:
1e-3 for bf16 activations (the GEMV family's f32-output bar), 2e-5 for f32
ones on weights exact in bf16 (test_f32_split.py pins what that bar
catches); the result must not depend on timing (two calls bit-identical).
Shapes cover the Qwen3-8B down projection (K = 12288, N = 4096), rows that
do not fill a workgroup (N = 3), ragged N, and K shorter than the parts
(parts with no units)."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import TOL_F32, _t, _x_as, rel_err, want_f64

pytestmark = pytest.mark.gpu

TOL_EXACT_W = 2e-5
BF16 = ["1,2,8,2", "1,3,8,2", "1,2,16,2", "3,1,8,2", "3,2,8,2", "3,1,16,2", "2,1,8,4", "2,2,8,4", "2,1,16,4"]
F32 = ["3,1,8,2", "2,1,8,2", "1,2,8,2"]


def _exact_q4_1(orc, rng, n, k):
    """Q4_1 rows whose weights are exact in bf16: d a power of two, m = 0."""
    packed = orc.synth_q4_1(rng, n, k)
    blk = packed.reshape(-1, 20)
    blk[:, 0:2] = np.frombuffer(np.float16(2.0 ** -6).tobytes(), np.uint8)
    blk[:, 2:4] = 0
    return packed


def _call(ctx, xt, packed, n):
    import torch
    import rlxq

    y = ctx.dequant_matmul(xt, _t(packed), rlxq.GGUF_Q4_1, n)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("f32", [False, True], ids=["bf16", "f32"])
def test_gemv_k_split_variants(ctx, orc, monkeypatch, f32):
    for cfg in (F32 if f32 else BF16):
        nu, d, w, ks = (int(v) for v in cfg.split(","))
        monkeypatch.setenv("RLXQ_GEMV_XSFK" if f32 else "RLXQ_GEMV_XSK", cfg)
        kmax = 32 * 64 * nu * ks   # K that fits NU * KS unit chunks
        for k, n in sorted({(min(kmax, 12288), 4096), (min(kmax, 4096), 1031), (256, 3), (min(kmax, 2048), 77)}):
            announce(f"gemv k-split {cfg} f32={f32} k={k} n={n}")
            rng = np.random.default_rng(k + n + ks + nu)
            packed = _exact_q4_1(orc, rng, n, k) if f32 else orc.synth_q4_1(rng, n, k)
            x = rng.standard_normal((1, k)).astype(np.float32)
            x[0, : k // 3] *= 50.0
            xt, xv = _x_as(x, "f32" if f32 else "bf16")
            got = _call(ctx, xt, packed, n)
            assert ctx.last_kernel == f"rlxq_gemvxs_q4_1_U{nu}_D{d}_W{w}{'_F' if f32 else ''}_K{ks}", ctx.last_kernel
            want = want_f64(orc, 3, xv, packed, k)
            assert rel_err(got, want) <= (TOL_EXACT_W if f32 else TOL_F32), (cfg, k, n)
            assert np.array_equal(got, _call(ctx, xt, packed, n)), (cfg, k, n)
