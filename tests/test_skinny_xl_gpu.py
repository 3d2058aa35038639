"""The LDS-staged batched-decode kernels (rlxq_skinnyxl_*): the weights of a
step reach each wave as row-contiguous 16-byte pieces, go through the
wave's own LDS region, and are read back as the register-streamed kernel's
per-lane blocks.  Every compiled variant "MT,NT,SC,D" is forced through
RLXQ_SKINNY_XL on shapes with a column tail (N no multiple of the tile),
partial row chunks, several K splits and both activation types, against the
float64 oracle: bar 1e-3 (f32 output), 1e-2 (bf16 output); 2e-5 where the
weights are exact in f16 (Q4_1 with d = 2^-6, m = 0), which a block read
from the wrong row, block or step of the LDS region fails."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import TOL_BF16, TOL_F32, rel_err, run_dense

pytestmark = pytest.mark.gpu

Q4_1 = 3
XL_Q4_1 = ["1,2,2,1", "1,2,1,2", "1,2,1,3", "1,1,2,2", "1,4,1,2", "2,1,2,1"]
OTHER = {"q4_0": 2, "q8_0": 1, "q4_k": 7, "q5_k": 10}


@pytest.fixture(autouse=True)
def _force_skinny(monkeypatch):
    monkeypatch.setenv("RLXQ_DECODE", "skinny")


def _exact_q4_1(orc, rng, n, k):
    packed = orc.synth_q4_1(rng, n, k)
    blk = packed.reshape(-1, 20)
    blk[:, 0:2] = np.frombuffer(np.float16(2.0 ** -6).tobytes(), np.uint8)
    blk[:, 2:4] = 0
    return packed


def _name(cfg, sname="q4_1"):
    mt, nt, sc, d = cfg.split(",")
    return f"rlxq_skinnyxl_{sname}_mt{mt}_nt{nt}_s{sc}_d{d}"


@pytest.mark.parametrize("cfg", XL_Q4_1)
@pytest.mark.parametrize("mkn", [(5, 512, 77), (16, 4096, 520), (17, 1024, 300), (33, 2048, 129),
                                 (64, 1024, 200)], ids=str)
def test_xl_q4_1_every_variant(ctx, orc, monkeypatch, cfg, mkn):
    monkeypatch.setenv("RLXQ_SKINNY_XL", cfg)
    m, k, n = mkn
    announce(f"skinny xl q4_1 {cfg} {mkn}")
    rng = np.random.default_rng(m * 131 + k + n)
    packed = orc.synth_q4_1(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, Q4_1, x, packed, n, xdt="bf16")
    assert ctx.last_kernel == _name(cfg), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("cfg", XL_Q4_1)
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_xl_q4_1_exact_weights(ctx, orc, monkeypatch, cfg, xdt):
    """Weights exact in f16: the only error left is the activations' own
    representation (f32: hi + lo rows) and the f32 accumulation."""
    monkeypatch.setenv("RLXQ_SKINNY_XL", cfg)
    m, k, n = 24, 3072, 136
    announce(f"skinny xl q4_1 exact {cfg} {xdt}")
    rng = np.random.default_rng(len(cfg) + len(xdt))
    packed = _exact_q4_1(orc, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, Q4_1, x, packed, n, xdt=xdt)
    assert ctx.last_kernel == _name(cfg), ctx.last_kernel
    assert rel_err(got, want) <= 2e-5


@pytest.mark.parametrize("cfg", ["1,2,2,1", "2,1,2,1"])
def test_xl_split_k_bf16_out_and_long_k(ctx, orc, monkeypatch, cfg):
    """Small N over a long K (several K splits of whole steps) with bf16 and
    f32 output, and the config-3 down shape's K."""
    monkeypatch.setenv("RLXQ_SKINNY_XL", cfg)
    m, k, n = 16, 12288, 136
    announce(f"skinny xl split-k {cfg}")
    rng = np.random.default_rng(9)
    packed = orc.synth_q4_1(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, Q4_1, x, packed, n, xdt="bf16")
    assert ctx.last_kernel == _name(cfg), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32
    got, want = run_dense(ctx, orc, Q4_1, x, packed, n, xdt="bf16", ydt="bf16")
    assert rel_err(got, want) <= TOL_BF16


def test_xl_odd_step_count_falls_back(ctx, orc, monkeypatch):
    """K of an odd number of chunks cannot be whole 2-chunk steps: the
    request for an SC = 2 kernel is not taken and the register-streamed
    kernel serves the call."""
    monkeypatch.setenv("RLXQ_SKINNY_XL", "1,2,2,1")
    m, k, n = 16, 384, 64
    rng = np.random.default_rng(3)
    packed = orc.synth_q4_1(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, Q4_1, x, packed, n, xdt="bf16")
    assert ctx.last_kernel.startswith("rlxq_skinnyxr_q4_1_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("sname", list(OTHER))
@pytest.mark.parametrize("mkn", [(5, 512, 77), (16, 4096, 520), (33, 2048, 129), (64, 1024, 200)], ids=str)
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_xl_other_formats(ctx, orc, monkeypatch, sname, mkn, xdt):
    """Q4_0 (18-byte blocks, 2-byte aligned), Q8_0 (34-byte blocks), Q4_K and
    Q5_K (whole super-blocks per step) through their LDS-staged kernels."""
    monkeypatch.setenv("RLXQ_SKINNY_XL", "1,2,2,1")
    scheme = OTHER[sname]
    m, k, n = mkn
    announce(f"skinny xl {sname} {mkn} {xdt}")
    rng = np.random.default_rng(m + k * 3 + n + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt=xdt)
    assert ctx.last_kernel == _name("1,2,2,1", sname), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32
