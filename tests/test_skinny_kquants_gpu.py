"""Batched decode (5-256 activation rows) for the other GGUF K-quants of the
reference's DeviceMatmul table (Q5_K, Q3_K, Q2_K, Q8_K;
crates/rlx-laguna/src/device_matmul.rs:64-76) on the f16-MFMA register
kernels, through the C ABI, against the oracle's restatements of GGML's
block_q5_K / q3_K / q2_K / q8_K.

The weights reach the MFMA exactly (Q5_K, Q3_K and Q8_K: code times an f16
scale split in two f16 operands, Q5_K's min on the block sums; Q2_K: the f32
weight the CPU decoder computes, fma(d sc, code, -dmin mn), as f16 hi + lo),
and bf16 activations are exact in f16 once row-scaled, f32 ones hi + lo
pairs: so the bar is 2e-5 of max|want| (float64 from the activations the
kernel saw), fifty times inside the 1e-3 f32-output bar.  A kernel that
rounded the weights to f16 once misses it (1.8e-4 to 2.1e-4 on these inputs
in float64); one that dropped Q5_K's min or a Q3_K / Q2_K half scale misses
it by orders of magnitude."""
import numpy as np
import pytest

from conftest import announce, skinny_xl_default
from test_gemv_gpu import TOL_BF16, rel_err, run_dense

pytestmark = pytest.mark.gpu

TOL_EXACT = 2e-5
SCHEMES = {"q5_k": 10, "q3_k": 11, "q2_k": 12, "q8_k": 13}
# compiled register variants "MT,NT,D" (the ring depth follows the raw block
# size: Q5_K 21 dwords, Q3_K 24, Q2_K 11, Q8_K 9)
XR = {
    "q5_k": ["1,2,2", "2,2,2", "4,2,1"],
    "q3_k": ["1,2,2", "2,2,2", "4,2,1"],
    "q2_k": ["1,2,3", "2,2,2", "4,2,2"],
    "q8_k": ["1,2,4", "2,2,3", "4,2,2"],
}


@pytest.fixture(autouse=True)
def _force_skinny(monkeypatch):
    monkeypatch.setenv("RLXQ_DECODE", "skinny")


def _case(orc, scheme, m, k, n, seed, x_row0=300.0):
    rng = np.random.default_rng(seed)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= x_row0
    return packed, x


@pytest.mark.parametrize("name", list(SCHEMES))
@pytest.mark.parametrize("mkn", [(5, 256, 7), (16, 4096, 512), (17, 1280, 300), (33, 2304, 129),
                                 (64, 4096, 256), (100, 768, 200), (256, 512, 40)], ids=str)
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_skinny_kquant_default(ctx, orc, name, mkn, xdt):
    m, k, n = mkn
    scheme = SCHEMES[name]
    announce(f"skinny {name} default {mkn} x={xdt}")
    packed, x = _case(orc, scheme, m, k, n, m * 7 + k + n + scheme)
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt=xdt)
    kind = "xl" if skinny_xl_default(scheme, m, k, xdt) else "xr"
    assert ctx.last_kernel.startswith(f"rlxq_skinny{kind}_{name}_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL_EXACT, (name, mkn, xdt)


@pytest.mark.parametrize("cfg", [(nm, c) for nm, cs in XR.items() for c in cs], ids=str)
def test_skinny_kquant_every_variant(ctx, orc, monkeypatch, cfg):
    name, rest = cfg
    scheme = SCHEMES[name]
    monkeypatch.setenv("RLXQ_SKINNY_XR", rest)
    mt, nt, d = (int(v) for v in rest.split(","))
    for (m, k, n) in [(5, 256, 7), (16 * mt + 3, 2304, 64 * nt * 3 + 5), (9, 12288, 200), (64, 1536, 96),
                      (3, 768, 64 * nt)]:
        announce(f"skinny {name} xr {rest} {(m, k, n)}")
        packed, x = _case(orc, scheme, m, k, n, m + k + n + mt + scheme, x_row0=1.0)
        got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16")
        assert ctx.last_kernel == f"rlxq_skinnyxr_{name}_mt{mt}_nt{nt}_d{d}", ctx.last_kernel
        assert rel_err(got, want) <= TOL_EXACT, (cfg, m, k, n)


@pytest.mark.parametrize("name", list(SCHEMES))
def test_skinny_kquant_split_k_bf16_out_and_activation_range(ctx, orc, name):
    """Few weight rows (the K split and its reduction), bf16 output, and rows
    scaled from 1e-30 to 1e30 (each row's power-of-two factor)."""
    scheme = SCHEMES[name]
    m, k, n = 24, 12288, 64
    announce(f"skinny {name} split-K / bf16 out / range")
    packed, x = _case(orc, scheme, m, k, n, 11 + scheme, x_row0=1.0)
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16", ydt="bf16")
    kind = "xl" if skinny_xl_default(scheme, m, k) else "xr"
    assert ctx.last_kernel.startswith(f"rlxq_skinny{kind}_{name}_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL_BF16
    x = x * np.logspace(-30, 30, m, dtype=np.float64)[:, None].astype(np.float32)
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="f32")
    for r in range(m):
        assert rel_err(got[r], want[r]) <= TOL_EXACT, (name, r)


def test_kquants_take_the_skinny_kernels_by_default(ctx, orc, monkeypatch):
    """Without the test override, 5..63 rows of every K-quant run on the
    batched-decode kernels (not the GEMV family), f32 and bf16 activations."""
    monkeypatch.delenv("RLXQ_DECODE", raising=False)
    for name, scheme in SCHEMES.items():
        for m, xdt in ((5, "f32"), (63, "bf16")):
            packed, x = _case(orc, scheme, m, 1024, 96, m + scheme)
            got, want = run_dense(ctx, orc, scheme, x, packed, 96, xdt=xdt)
            kind = "xl" if skinny_xl_default(scheme, m, 1024, xdt) else "xr"
            assert ctx.last_kernel.startswith(f"rlxq_skinny{kind}_{name}_"), (name, m, ctx.last_kernel)
            assert rel_err(got, want) <= TOL_EXACT
