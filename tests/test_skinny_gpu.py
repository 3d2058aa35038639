"""Parity of the batched-decode (small M) dequant-GEMM against the CPU oracle,
through the C ABI: exact weights (f16 hi + lo operands, the min / bias term
on block sums) and bf16 activations (exact in f16 after power-of-two row
scaling) on f16 MFMA with fp32 accumulation.  f32 activations run as hi + lo f16 row pairs (see
test_f32_activations_take_the_skinny_kernels and tests/test_f32_contract_gpu.py).  Bar: max|got - want| / max|want| <= 1e-3 (f32 output), 1e-2
(bf16 output), `want` the oracle's dequantized weights contracted in float64."""
import numpy as np
import pytest

from conftest import announce, skinny_xl_default
from test_gemv_gpu import TOL_BF16, TOL_F32, rel_err, run_dense

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _force_skinny(monkeypatch):
    monkeypatch.setenv("RLXQ_DECODE", "skinny")


@pytest.mark.parametrize("scheme", [1, 2, 3])
@pytest.mark.parametrize("mkn", [(5, 128, 7), (16, 640, 128), (17, 1024, 300), (33, 512, 129),
                                 (64, 4096, 256), (65, 256, 64), (100, 384, 200), (256, 128, 40)], ids=str)
@pytest.mark.parametrize("xdt", ["bf16"])
def test_skinny_matches_oracle(ctx, orc, scheme, mkn, xdt):
    m, k, n = mkn
    announce(f"skinny scheme={scheme} x={xdt} {mkn}")
    rng = np.random.default_rng(m * 7 + k + n)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt=xdt)
    assert ctx.last_kernel.startswith("rlxq_skinny"), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("scheme", [1, 3])
def test_skinny_split_k_and_bf16_out(ctx, orc, scheme):
    """Small N with long K takes the split-K path; bf16 output."""
    m, k, n = 16, 12288, 136
    announce(f"skinny split-k scheme={scheme}")
    rng = np.random.default_rng(scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16")
    assert rel_err(got, want) <= TOL_F32
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16", ydt="bf16")
    assert rel_err(got, want) <= TOL_BF16


@pytest.mark.parametrize("scheme", [1, 3])
def test_skinny_activation_range(ctx, orc, scheme):
    """Rows far outside the f16 range and rows of tiny values: the per-row
    power-of-two scale keeps each row's products accurate."""
    m, k, n = 8, 512, 96
    announce(f"skinny activation range scheme={scheme}")
    rng = np.random.default_rng(20 + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= 1e6
    x[1] *= 1e-6
    x[2, 7] = 3e5
    x[3] = 0.0
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16")
    for r in range(m):
        if r == 3:
            assert np.all(got[r] == 0.0)
            continue
        assert rel_err(got[r:r + 1], want[r:r + 1]) <= TOL_F32, r


STAGINGS = {"default": {}, "register": {"RLXQ_SKINNY_NS": "0"}}
KERNEL_PREFIX = {"register": "rlxq_skinnyxr_"}


@pytest.mark.parametrize("staging", list(STAGINGS))
@pytest.mark.parametrize("mkn", [(5, 256, 136), (16, 4096, 512), (33, 768, 200), (64, 1024, 128)], ids=str)
def test_skinny_q4_1_every_staging(ctx, orc, monkeypatch, staging, mkn):
    """Q4_1 through the default choice (LDS-staged up to 32 rows, N-split
    above) and the register-streamed kernel."""
    for key, val in STAGINGS[staging].items():
        monkeypatch.setenv(key, val)
    m, k, n = mkn
    announce(f"skinny q4_1 staging={staging} {mkn}")
    rng = np.random.default_rng(k + n + m)
    packed = orc.synth_q4_1(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, 3, x, packed, n, xdt="bf16")
    prefix = KERNEL_PREFIX.get(staging, "rlxq_skinnyxl_q4_1_" if m <= 32 else "rlxq_skinnyns_q4_1_")
    assert ctx.last_kernel.startswith(prefix), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32


# every compiled register-streamed variant "MT,NT,D"; shapes with partial
# row chunks, partial row tiles, several K splits and a single chunk of K
XR_VARIANTS = ["1,2,4", "1,4,2", "1,4,3", "2,2,3", "2,4,2", "4,2,2", "4,4,1"]


@pytest.mark.parametrize("cfg", XR_VARIANTS)
def test_skinny_every_register_variant(ctx, orc, monkeypatch, cfg):
    monkeypatch.setenv("RLXQ_SKINNY_XR", cfg)
    mt, nt, d = (int(v) for v in cfg.split(","))
    for (m, k, n) in [(5, 128, 7), (16 * mt + 3, 2048, 16 * nt * 3 + 5), (9, 12288, 200), (64, 1536, 96)]:
        announce(f"skinny register {cfg} {(m, k, n)}")
        rng = np.random.default_rng(m + k + n + mt)
        packed = orc.synth_q4_1(rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        got, want = run_dense(ctx, orc, 3, x, packed, n, xdt="bf16")
        assert ctx.last_kernel == f"rlxq_skinnyxr_q4_1_mt{mt}_nt{nt}_d{d}", ctx.last_kernel
        assert rel_err(got, want) <= TOL_F32, (cfg, m, k, n)


def test_f32_activations_take_the_skinny_kernels(ctx, orc, monkeypatch):
    """f32 activations (the reference's operand type) run on the f16 kernels
    as hi and lo row pairs by default; RLXQ_DECODE=gemv keeps them on the
    GEMV, whose products are exact."""
    monkeypatch.delenv("RLXQ_DECODE", raising=False)
    rng = np.random.default_rng(3)
    packed = orc.synth_q4_1(rng, 256, 1024)
    x = rng.standard_normal((32, 1024)).astype(np.float32)
    got, want = run_dense(ctx, orc, 3, x, packed, 256)
    assert ctx.last_kernel.startswith("rlxq_skinnyns_q4_1_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32
    monkeypatch.setenv("RLXQ_DECODE", "gemv")
    got, want = run_dense(ctx, orc, 3, x, packed, 256)
    assert ctx.last_kernel.startswith("rlxq_gemv"), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("scheme", [1, 2])
def test_skinny_q8_0_q4_0_register_kernel(ctx, orc, scheme):
    """Q8_0 (34-byte blocks) and Q4_0 (18-byte blocks) through the default
    kernels: LDS-staged at few rows, register-streamed above."""
    for (m, k, n) in [(6, 256, 40), (16, 2048, 300), (40, 640, 96), (64, 4096, 130)]:
        announce(f"skinny scheme={scheme} {(m, k, n)}")
        rng = np.random.default_rng(scheme * 100 + m + k)
        packed = orc.synth(scheme, rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16")
        kind = "xl" if skinny_xl_default(scheme, m, k) else "xr"
        assert ctx.last_kernel.startswith(f"rlxq_skinny{kind}_"), ctx.last_kernel
        assert rel_err(got, want) <= TOL_F32, (m, k, n)


# every compiled N-split variant "scheme:MT,NT,D" (activations shared through
# LDS, the four waves on different weight rows); shapes with partial row
# chunks and tiles, several K splits, one K chunk, and a long K
NS_VARIANTS = ["3:1,1,3", "3:2,1,3", "3:2,2,3", "3:4,1,3", "3:4,2,2", "1:4,2,2", "2:4,1,3"]


@pytest.mark.parametrize("cfg", NS_VARIANTS)
def test_skinny_every_nsplit_variant(ctx, orc, monkeypatch, cfg):
    scheme, rest = int(cfg.split(":")[0]), cfg.split(":")[1]
    monkeypatch.setenv("RLXQ_SKINNY_NS", rest)
    mt, nt, d = (int(v) for v in rest.split(","))
    name = {1: "q8_0", 2: "q4_0", 3: "q4_1"}[scheme]
    for (m, k, n) in [(5, 128, 7), (16 * mt + 3, 2048, 64 * nt * 3 + 5), (9, 12288, 200), (64, 1536, 96),
                      (3, 640, 64 * nt)]:
        announce(f"skinny n-split {cfg} {(m, k, n)}")
        rng = np.random.default_rng(m + k + n + mt + scheme)
        packed = orc.synth(scheme, rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16")
        assert ctx.last_kernel == f"rlxq_skinnyns_{name}_mt{mt}_nt{nt}_d{d}", ctx.last_kernel
        assert rel_err(got, want) <= TOL_F32, (cfg, m, k, n)



# Q4_K (GGML block_q4_K, 144-byte super-blocks of 256): the same f16-MFMA
# kernels after each 32-value sub-block's 6-bit scale and min are folded into
# one f16 d*sc and m*mn (the Q4_1 form)
Q4K_XR = ["1,2,3", "2,2,2", "4,2,2"]
Q4K_NS = ["1,1,3", "2,1,3", "4,1,3"]


@pytest.mark.parametrize("mkn", [(5, 256, 7), (16, 4096, 512), (17, 1024, 300), (33, 512, 129),
                                 (64, 4096, 256), (100, 768, 200), (256, 256, 40)], ids=str)
def test_skinny_q4_k_default(ctx, orc, mkn):
    m, k, n = mkn
    announce(f"skinny q4_k default {mkn}")
    rng = np.random.default_rng(m * 3 + k + n)
    packed = orc.synth(7, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= 300.0
    got, want = run_dense(ctx, orc, 7, x, packed, n, xdt="bf16")
    prefix = ("rlxq_skinnyxl_q4_k_" if skinny_xl_default(7, m, k) else "rlxq_skinnyxr_q4_k_") if m <= 16 \
        else "rlxq_skinnyns_q4_k_"
    assert ctx.last_kernel.startswith(prefix), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32
    got, want = run_dense(ctx, orc, 7, x, packed, n, xdt="bf16", ydt="bf16")
    assert rel_err(got, want) <= TOL_BF16


@pytest.mark.parametrize("cfg", [("xr", c) for c in Q4K_XR] + [("ns", c) for c in Q4K_NS], ids=str)
def test_skinny_q4_k_every_variant(ctx, orc, monkeypatch, cfg):
    kind, rest = cfg
    monkeypatch.setenv("RLXQ_SKINNY_XR" if kind == "xr" else "RLXQ_SKINNY_NS", rest)
    mt, nt, d = (int(v) for v in rest.split(","))
    for (m, k, n) in [(5, 256, 7), (16 * mt + 3, 2048, 64 * nt * 3 + 5), (9, 12288, 200), (64, 1536, 96),
                      (3, 768, 64 * nt)]:
        announce(f"skinny q4_k {kind} {rest} {(m, k, n)}")
        rng = np.random.default_rng(m + k + n + mt)
        packed = orc.synth(7, rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        got, want = run_dense(ctx, orc, 7, x, packed, n, xdt="bf16")
        assert ctx.last_kernel == f"rlxq_skinny{kind}_q4_k_mt{mt}_nt{nt}_d{d}", ctx.last_kernel
        assert rel_err(got, want) <= TOL_F32, (cfg, m, k, n)


def test_skinny_q4_k_activation_range_and_no_staged_kernel(ctx, orc, monkeypatch):
    """Rows far outside the f16 range; RLXQ_SKINNY_XR=0 (no configuration)
    keeps Q4_K on the register-streamed kernel's default tiling."""
    monkeypatch.setenv("RLXQ_SKINNY_XR", "0")
    m, k, n = 8, 512, 96
    rng = np.random.default_rng(27)
    packed = orc.synth(7, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= 1e6
    x[1] *= 1e-6
    x[3] = 0.0
    got, want = run_dense(ctx, orc, 7, x, packed, n, xdt="bf16")
    assert ctx.last_kernel.startswith("rlxq_skinnyxr_q4_k_"), ctx.last_kernel
    for r in range(m):
        if r == 3:
            assert np.all(got[r] == 0.0)
            continue
        assert rel_err(got[r:r + 1], want[r:r + 1]) <= TOL_F32, r


# Q6_K (GGML block_q6_K, 210-byte super-blocks, 2-byte aligned every other
# time): the int8 form of Q8_0 with one f16 scale d * sc per 16 weights
Q6K_XR = ["1,2,2", "2,2,2", "4,2,1"]
Q6K_NS = ["1,1,3", "2,1,3", "4,1,2"]


@pytest.mark.parametrize("mkn", [(5, 256, 7), (16, 4096, 512), (17, 1280, 300), (33, 2304, 129),
                                 (64, 4096, 256), (100, 768, 200)], ids=str)
def test_skinny_q6_k_default(ctx, orc, mkn):
    m, k, n = mkn
    announce(f"skinny q6_k default {mkn}")
    rng = np.random.default_rng(m * 5 + k + n)
    packed = orc.synth(8, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= 300.0
    got, want = run_dense(ctx, orc, 8, x, packed, n, xdt="bf16")
    prefix = "rlxq_skinnyxr_q6_k_" if m <= 16 else "rlxq_skinnyns_q6_k_"
    assert ctx.last_kernel.startswith(prefix), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("cfg", [("xr", c) for c in Q6K_XR] + [("ns", c) for c in Q6K_NS], ids=str)
def test_skinny_q6_k_every_variant(ctx, orc, monkeypatch, cfg):
    kind, rest = cfg
    monkeypatch.setenv("RLXQ_SKINNY_XR" if kind == "xr" else "RLXQ_SKINNY_NS", rest)
    mt, nt, d = (int(v) for v in rest.split(","))
    for (m, k, n) in [(5, 256, 7), (16 * mt + 3, 2304, 64 * nt * 3 + 5), (9, 12288, 200), (64, 1536, 96),
                      (3, 768, 64 * nt)]:
        announce(f"skinny q6_k {kind} {rest} {(m, k, n)}")
        rng = np.random.default_rng(m + k + n + mt + 1)
        packed = orc.synth(8, rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        got, want = run_dense(ctx, orc, 8, x, packed, n, xdt="bf16")
        assert ctx.last_kernel == f"rlxq_skinny{kind}_q6_k_mt{mt}_nt{nt}_d{d}", ctx.last_kernel
        assert rel_err(got, want) <= TOL_F32, (cfg, m, k, n)


# MLX affine 4-bit (eight codes per little-endian word, per-group f32 or
# bf16 scale and bias): the Q4_1 form with the group's scale and bias rounded
# to f16, activations in MLX's unpacking order
MLX_XR = ["1,2,4", "2,2,3", "4,2,2"]
MLX_NS = ["1,1,3", "2,1,3", "4,1,3"]


def _mlx_case(ctx, orc, rng, m, k, n, group, sb, ydt="f32", x_scale=None, bits=4):
    import torch
    import rlxq
    from test_gemv_gpu import _t, _x_as

    codes = rng.integers(0, 2 ** 32, (n, k * bits // 32), dtype=np.uint32)
    sc = rng.uniform(0.01, 0.1, (n, k // group)).astype(np.float32)
    bi = rng.uniform(-0.5, 0.1, (n, k // group)).astype(np.float32)
    if sb == "bf16":
        sc = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(sc))
        bi = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(bi))
        st, bt = _t(sc).to(torch.bfloat16), _t(bi).to(torch.bfloat16)
    else:
        st, bt = _t(sc), _t(bi)
    x32 = rng.standard_normal((m, k)).astype(np.float32)
    if x_scale is not None:
        x32 *= x_scale[:, None]
    xt, xv = _x_as(x32, "bf16")
    scheme = rlxq.MLX_AFFINE4 if bits == 4 else rlxq.MLX_AFFINE8
    y = ctx.dequant_matmul(xt, _t(codes.view(np.uint8)), scheme, n, group=group, scales=st, biases=bt,
                           y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), orc.mlx_matmul_f64(xv, codes, sc, bi, n, bits, group)


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("sb", ["f32", "bf16"])
@pytest.mark.parametrize("mkn", [(5, 256, 7), (16, 4096, 512), (17, 1024, 300), (33, 768, 129),
                                 (64, 4096, 256), (100, 768, 200), (256, 384, 40)], ids=str)
def test_skinny_mlx4_default(ctx, orc, mkn, group, sb):
    m, k, n = mkn
    if k % group:
        pytest.skip("K not a multiple of the group")
    announce(f"skinny mlx4 default {mkn} group={group} sb={sb}")
    rng = np.random.default_rng(m * 11 + k + n + group)
    got, want = _mlx_case(ctx, orc, rng, m, k, n, group, sb)
    prefix = "rlxq_skinnyxr_mlx4_" if m <= 16 else "rlxq_skinnyns_mlx4_"
    assert ctx.last_kernel.startswith(prefix), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32
    got, want = _mlx_case(ctx, orc, np.random.default_rng(m * 11 + k + n + group), m, k, n, group, sb, ydt="bf16")
    assert rel_err(got, want) <= TOL_BF16


@pytest.mark.parametrize("cfg", [("xr", c) for c in MLX_XR] + [("ns", c) for c in MLX_NS], ids=str)
def test_skinny_mlx4_every_variant(ctx, orc, monkeypatch, cfg):
    kind, rest = cfg
    monkeypatch.setenv("RLXQ_SKINNY_XR" if kind == "xr" else "RLXQ_SKINNY_NS", rest)
    mt, nt, d = (int(v) for v in rest.split(","))
    for (m, k, n, group) in [(5, 256, 7, 32), (16 * mt + 3, 2048, 64 * nt * 3 + 5, 64), (9, 12288, 200, 64),
                             (64, 1536, 96, 128), (3, 768, 64 * nt, 32)]:
        announce(f"skinny mlx4 {kind} {rest} {(m, k, n, group)}")
        rng = np.random.default_rng(m + k + n + mt + 2)
        got, want = _mlx_case(ctx, orc, rng, m, k, n, group, "bf16")
        assert ctx.last_kernel == f"rlxq_skinny{kind}_mlx4_mt{mt}_nt{nt}_d{d}", ctx.last_kernel
        assert rel_err(got, want) <= TOL_F32, (cfg, m, k, n)


def test_skinny_mlx4_activation_range_and_no_staged_kernel(ctx, orc, monkeypatch):
    """Rows far outside the f16 range and a zero row; RLXQ_SKINNY_XR=0 keeps
    MLX4 (no LDS-staged kernel) on the register-streamed kernel."""
    monkeypatch.setenv("RLXQ_SKINNY_XR", "0")
    m, k, n = 8, 512, 96
    xs = np.ones(m, dtype=np.float32)
    xs[0], xs[1], xs[3] = 1e6, 1e-6, 0.0
    got, want = _mlx_case(ctx, orc, np.random.default_rng(31), m, k, n, 64, "f32", x_scale=xs)
    assert ctx.last_kernel.startswith("rlxq_skinnyxr_mlx4_"), ctx.last_kernel
    for r in range(m):
        if r == 3:
            assert np.all(got[r] == 0.0)
            continue
        assert rel_err(got[r:r + 1], want[r:r + 1]) <= TOL_F32, r


# MLX affine 8-bit: four codes per word, natural order, the group's scale
# and bias rounded to f16 as for MLX4
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("mkn", [(5, 256, 7), (16, 4096, 512), (33, 768, 129), (64, 4096, 256), (256, 384, 40)],
                         ids=str)
def test_skinny_mlx8_default(ctx, orc, mkn, group):
    m, k, n = mkn
    if k % group:
        pytest.skip("K not a multiple of the group")
    announce(f"skinny mlx8 default {mkn} group={group}")
    for sb in ("f32", "bf16"):
        got, want = _mlx_case(ctx, orc, np.random.default_rng(m * 17 + k + n + group), m, k, n, group, sb, bits=8)
        assert ctx.last_kernel.startswith("rlxq_skinny") and "_mlx8_" in ctx.last_kernel, ctx.last_kernel
        assert rel_err(got, want) <= TOL_F32, sb
    got, want = _mlx_case(ctx, orc, np.random.default_rng(m + group), m, k, n, group, "bf16", ydt="bf16", bits=8)
    assert rel_err(got, want) <= TOL_BF16


@pytest.mark.parametrize("cfg", [("xr", c) for c in MLX_XR] + [("ns", c) for c in MLX_NS], ids=str)
def test_skinny_mlx8_every_variant(ctx, orc, monkeypatch, cfg):
    kind, rest = cfg
    monkeypatch.setenv("RLXQ_SKINNY_XR" if kind == "xr" else "RLXQ_SKINNY_NS", rest)
    mt, nt, d = (int(v) for v in rest.split(","))
    for (m, k, n, group) in [(5, 256, 7, 32), (16 * mt + 3, 2048, 64 * nt * 3 + 5, 64), (9, 12288, 200, 64),
                             (64, 1536, 96, 128), (3, 768, 64 * nt, 32)]:
        announce(f"skinny mlx8 {kind} {rest} {(m, k, n, group)}")
        rng = np.random.default_rng(m + k + n + mt + 4)
        xs = np.ones(m, dtype=np.float32)
        xs[0] = 1e5
        got, want = _mlx_case(ctx, orc, rng, m, k, n, group, "bf16", x_scale=xs, bits=8)
        assert ctx.last_kernel == f"rlxq_skinny{kind}_mlx8_mt{mt}_nt{nt}_d{d}", ctx.last_kernel
        for r in range(m):
            assert rel_err(got[r:r + 1], want[r:r + 1]) <= TOL_F32, (cfg, m, k, n, r)


# MXFP4 with E8M0 scale bytes: E2M1 codes times a power of two are exact in
# bf16, as are the power-of-two-scaled bf16 activations, so the bf16 MFMA
# products are exact and only the f32 accumulation order differs from the
# float64 oracle: bar 1e-5
MXFP4_TOL = 1e-5
MXFP4_XR = ["1,2,4", "2,2,3", "4,2,2"]
MXFP4_NS = ["1,1,3", "2,1,3", "4,1,3"]


def _mxfp4_case(ctx, orc, rng, m, k, n, ydt="f32", x_scale=None):
    import torch
    from test_gemv_gpu import _t, _x_as

    codes, eb = orc.synth_mxfp4(rng, n, k)
    x32 = rng.standard_normal((m, k)).astype(np.float32)
    if x_scale is not None:
        x32 *= x_scale[:, None]
    xt, xv = _x_as(x32, "bf16")
    y = ctx.dequant_matmul(xt, _t(codes), 9, n, scales=_t(eb),
                           y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), orc.mxfp4_matmul_f64(xv, codes, eb, n)


@pytest.mark.parametrize("mkn", [(5, 256, 7), (16, 4096, 512), (17, 1024, 300), (33, 768, 129),
                                 (64, 4096, 256), (100, 768, 200), (256, 384, 40)], ids=str)
def test_skinny_mxfp4_default(ctx, orc, mkn):
    m, k, n = mkn
    announce(f"skinny mxfp4 default {mkn}")
    got, want = _mxfp4_case(ctx, orc, np.random.default_rng(m * 13 + k + n), m, k, n)
    prefix = "rlxq_skinnyxr_mxfp4_" if m <= 16 else "rlxq_skinnyns_mxfp4_"
    assert ctx.last_kernel.startswith(prefix), ctx.last_kernel
    assert rel_err(got, want) <= MXFP4_TOL
    got, want = _mxfp4_case(ctx, orc, np.random.default_rng(m * 13 + k + n), m, k, n, ydt="bf16")
    assert rel_err(got, want) <= TOL_BF16


@pytest.mark.parametrize("cfg", [("xr", c) for c in MXFP4_XR] + [("ns", c) for c in MXFP4_NS], ids=str)
def test_skinny_mxfp4_every_variant(ctx, orc, monkeypatch, cfg):
    kind, rest = cfg
    monkeypatch.setenv("RLXQ_SKINNY_XR" if kind == "xr" else "RLXQ_SKINNY_NS", rest)
    mt, nt, d = (int(v) for v in rest.split(","))
    for (m, k, n) in [(5, 256, 7), (16 * mt + 3, 2048, 64 * nt * 3 + 5), (9, 12288, 200), (64, 1536, 96),
                      (3, 768, 64 * nt)]:
        announce(f"skinny mxfp4 {kind} {rest} {(m, k, n)}")
        got, want = _mxfp4_case(ctx, orc, np.random.default_rng(m + k + n + mt + 3), m, k, n)
        assert ctx.last_kernel == f"rlxq_skinny{kind}_mxfp4_mt{mt}_nt{nt}_d{d}", ctx.last_kernel
        assert rel_err(got, want) <= MXFP4_TOL, (cfg, m, k, n)


def test_skinny_mxfp4_activation_range_and_bf16_scales_stay_on_gemv(ctx, orc, monkeypatch):
    """Rows far apart in magnitude and a zero row; decoded bf16 scales (a
    general bf16 scale times a code is not exact in bf16) keep the GEMV."""
    import torch
    from test_gemv_gpu import _t, _x_as

    m, k, n = 8, 512, 96
    xs = np.ones(m, dtype=np.float32)
    xs[0], xs[1], xs[3] = 1e6, 1e-6, 0.0
    got, want = _mxfp4_case(ctx, orc, np.random.default_rng(37), m, k, n, x_scale=xs)
    assert ctx.last_kernel.startswith("rlxq_skinnyxr_mxfp4_"), ctx.last_kernel
    for r in range(m):
        if r == 3:
            assert np.all(got[r] == 0.0)
            continue
        assert rel_err(got[r:r + 1], want[r:r + 1]) <= MXFP4_TOL, r
    rng = np.random.default_rng(38)
    codes, eb = orc.synth_mxfp4(rng, n, k)
    sb = (eb.astype(np.uint16) << 7).view(np.int16)
    xt, xv = _x_as(rng.standard_normal((m, k)).astype(np.float32), "bf16")
    y = ctx.dequant_matmul(xt, _t(codes), 9, n, scales=_t(sb).view(torch.bfloat16))
    torch.cuda.synchronize()
    assert not ctx.last_kernel.startswith("rlxq_skinny"), ctx.last_kernel
    assert rel_err(y.cpu().numpy(), orc.mxfp4_matmul_f64(xv, codes, eb, n)) <= TOL_F32
