"""The reference operator's own operand types on the MFMA kernels: F32
activations in, F32 output (Op::DequantMatMul, crates/rlx-laguna/src/
device_matmul.rs:358-377, crates/rlx-qwen3/src/precision.rs:98-112), exactly
as rlxq_dm_matmul passes them.

f32 activations run on the prefill GEMM and the batched-decode kernels as a
hi and a lo f16 row per activation row (hi = f16(s*x), lo = f16(s*x - hi),
~22 significant bits), whose sums the epilogue adds; the single-row register
GEMV holds them as a hi and a lo bf16 row (~16 bits).  Bars: max|got - want|
/ max|want| <= 1e-3 against the float64 oracle on the f32 activations
themselves.  Where the weights are exact in f16 (Q4_1 with d a power of two
and m = 0) the only error left is the activations' representation and the
f32 accumulation, and the bar is 2e-5: rounding the activations to f16 or
bf16 alone (no lo row) misses it by an order of magnitude or more, which
tests/test_f32_split.py checks on the CPU."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_EXACT_W = 2e-5
Q8_0, Q4_0, Q4_1, Q4_K, Q6_K = 1, 2, 3, 7, 8
MLX4, MXFP4 = 4, 9
NAMES = {Q8_0: "q8_0", Q4_0: "q4_0", Q4_1: "q4_1", Q4_K: "q4_k", Q6_K: "q6_k", MLX4: "mlx4", MXFP4: "mxfp4"}


def _f32_run(ctx, scheme, x32, w, n, **kw):
    import torch

    y = ctx.dequant_matmul(_t(x32), w, scheme, n, y_dtype=torch.float32, **kw)
    kern = ctx.last_kernel
    torch.cuda.synchronize()
    return y.cpu().numpy(), kern


def _exact_f16_q4_1(orc, rng, n, k):
    """Q4_1 rows whose weights d*q + m are exact in f16: d = 2^-6, m = 0."""
    packed = orc.synth_q4_1(rng, n, k)
    blk = packed.reshape(-1, 20)
    blk[:, 0:2] = np.frombuffer(np.float16(2.0 ** -6).tobytes(), np.uint8)
    blk[:, 2:4] = 0
    return packed


def _want(orc, scheme, x32, packed, k):
    return x32.astype(np.float64) @ orc.dequantize(scheme, packed, k).astype(np.float64).T


@pytest.mark.parametrize("scheme", [Q4_1, Q4_K, Q8_0, Q6_K, Q4_0], ids=lambda s: NAMES[s])
@pytest.mark.parametrize("mkn", [(5, 1024, 96), (16, 4096, 384), (33, 768, 200), (64, 4096, 256),
                                 (256, 2048, 160)], ids=str)
def test_batched_decode_f32_activations(ctx, orc, scheme, mkn):
    """5..256 rows of f32 activations on the batched-decode MFMA kernels."""
    m, k, n = mkn
    announce(f"f32 contract skinny {NAMES[scheme]} {mkn}")
    rng = np.random.default_rng(m + k + n + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, kern = _f32_run(ctx, scheme, x, _t(packed), n)
    assert kern.startswith("rlxq_skinny"), kern
    assert rel_err(got, _want(orc, scheme, x, packed, k)) <= TOL, kern


@pytest.mark.parametrize("mkn", [(7, 4096, 128), (64, 12288, 136), (200, 1024, 64)], ids=str)
def test_batched_decode_f32_exact_weights(ctx, orc, mkn):
    """Weights exact in f16: the hi + lo rows keep the f32 activations."""
    m, k, n = mkn
    announce(f"f32 contract skinny exact weights {mkn}")
    rng = np.random.default_rng(m * 3 + n)
    packed = _exact_f16_q4_1(orc, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, kern = _f32_run(ctx, Q4_1, x, _t(packed), n)
    assert kern.startswith("rlxq_skinny"), kern
    assert rel_err(got, _want(orc, Q4_1, x, packed, k)) <= TOL_EXACT_W, kern


@pytest.mark.parametrize("cfg", ["1,2,4", "2,4,2", "4,2,2"])
def test_batched_decode_f32_register_variants(ctx, orc, monkeypatch, cfg):
    """Register-streamed variants with the split-K path and partial row chunks."""
    monkeypatch.setenv("RLXQ_SKINNY_XR", cfg)
    mt, nt, d = (int(v) for v in cfg.split(","))
    for (m, k, n) in [(5, 128, 7), (8 * mt + 3, 2048, 16 * nt * 3 + 5), (9, 12288, 200)]:
        announce(f"f32 contract skinny register {cfg} {(m, k, n)}")
        rng = np.random.default_rng(m + k + n + mt)
        packed = orc.synth_q4_1(rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        got, kern = _f32_run(ctx, Q4_1, x, _t(packed), n)
        assert kern == f"rlxq_skinnyxr_q4_1_mt{mt}_nt{nt}_d{d}", kern
        assert rel_err(got, _want(orc, Q4_1, x, packed, k)) <= TOL, (cfg, m, k, n)


def test_batched_decode_f32_mlx4_and_mxfp4(ctx, orc):
    import torch

    m, k, n = 24, 2048, 192
    announce("f32 contract skinny mlx4 / mxfp4")
    rng = np.random.default_rng(77)
    x = rng.standard_normal((m, k)).astype(np.float32)
    codes = rng.integers(0, 16, (n, k)).astype(np.uint32)
    wq = orc.mlx_pack(codes, 4)
    sc = rng.uniform(0.01, 0.1, (n, k // 64)).astype(np.float32)
    bi = rng.uniform(-0.5, 0.1, (n, k // 64)).astype(np.float32)
    got, kern = _f32_run(ctx, MLX4, x, _t(wq.view(np.uint8)), n, group=64, scales=_t(sc), biases=_t(bi))
    assert kern.startswith("rlxq_skinny"), kern
    assert rel_err(got, orc.mlx_matmul_f64(x, wq, sc, bi, n, 4, 64)) <= TOL
    mc, eb = orc.synth_mxfp4(rng, n, k)
    got, kern = _f32_run(ctx, MXFP4, x, _t(mc), n, scales=_t(eb))
    assert kern.startswith("rlxq_skinny"), kern
    assert rel_err(got, orc.mxfp4_matmul_f64(x, mc, eb, n)) <= TOL
    torch.cuda.synchronize()


@pytest.mark.parametrize("scheme", [Q4_1, Q4_K, Q8_0, Q6_K, Q4_0], ids=lambda s: NAMES[s])
@pytest.mark.parametrize("mkn", [(300, 1280, 272), (512, 4096, 1024), (257, 12288, 300)], ids=str)
def test_prefill_f32_activations(ctx, orc, scheme, mkn):
    """More than 256 rows of f32 activations with f32 output: the exact GEMM
    (f16 hi + lo weight rows) on hi/lo activation row pairs (split-K on the
    small grids)."""
    m, k, n = mkn
    announce(f"f32 contract gemm {NAMES[scheme]} {mkn}")
    rng = np.random.default_rng(m + k + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, kern = _f32_run(ctx, scheme, x, _t(packed), n)
    assert kern.startswith(f"rlxq_gemm_{NAMES[scheme]}_t256w8") and kern.endswith("xs"), kern
    assert rel_err(got, _want(orc, scheme, x, packed, k)) <= TOL, kern


def test_prefill_f32_exact_weights_and_bf16_out(ctx, orc):
    import torch

    m, k, n = 320, 4096, 512
    announce("f32 contract gemm exact weights")
    rng = np.random.default_rng(31)
    packed = _exact_f16_q4_1(orc, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, kern = _f32_run(ctx, Q4_1, x, _t(packed), n)
    assert kern == "rlxq_gemm_q4_1_t256w8p2xs", kern
    want = _want(orc, Q4_1, x, packed, k)
    assert rel_err(got, want) <= TOL_EXACT_W
    # bf16 output from f32 activations: the same kernel, rounded at the store
    y = ctx.dequant_matmul(_t(x), _t(packed), Q4_1, n, y_dtype=torch.bfloat16)
    assert ctx.last_kernel == "rlxq_gemm_q4_1_t256w8p2xs", ctx.last_kernel
    torch.cuda.synchronize()
    assert rel_err(y.float().cpu().numpy(), want) <= 8e-3


@pytest.mark.parametrize("scheme", [Q4_1, Q4_K], ids=lambda s: NAMES[s])
@pytest.mark.parametrize("kn", [(4096, 24576), (12288, 4096)], ids=lambda s: f"{s[0]}to{s[1]}")
def test_prefill_f32_config4_full_size_sampled(ctx, orc, scheme, kn):
    """Qwen3-8B gate|up and down at M=4096 with F32 activations and output,
    48 rows x 384 columns against the float64 oracle on the f32 rows."""
    import torch
    import rlxq
    from bench import synth_q4_1_gpu, synth_q4_k_gpu

    k, n = kn
    m = 4096
    announce(f"f32 contract gemm full size {NAMES[scheme]} m={m} k={k} n={n}")
    g = torch.Generator(device="cuda").manual_seed(m + k + n + scheme)
    w = (synth_q4_1_gpu if scheme == Q4_1 else synth_q4_k_gpu)(n, k, g)
    x = torch.randn((m, k), generator=g, device="cuda", dtype=torch.float32)
    y = ctx.dequant_matmul(x, w, scheme, n, y_dtype=torch.float32)
    kern = ctx.last_kernel
    torch.cuda.synchronize()
    assert kern == f"rlxq_gemm_{NAMES[scheme]}_t256w8p2xs", kern
    rs = np.random.default_rng(m + n)
    rows = np.sort(rs.choice(m, 48, replace=False))
    cols = np.sort(rs.choice(n, 384, replace=False))
    wsub = w.view(n, -1)[torch.from_numpy(cols).cuda()].cpu().numpy()
    wd = orc.dequantize(scheme, wsub, k).astype(np.float64)
    want = x[torch.from_numpy(rows).cuda()].cpu().numpy().astype(np.float64) @ wd.T
    got = y.cpu().numpy()[np.ix_(rows, cols)]
    assert rel_err(got, want) <= TOL, kern
    del rlxq


@pytest.mark.parametrize("scheme", [Q4_1, Q4_K, MLX4, MXFP4], ids=lambda s: NAMES[s])
@pytest.mark.parametrize("kn", [(4096, 4096), (2048, 1031), (8192, 517), (256, 17)], ids=str)
def test_single_row_f32_register_path(ctx, orc, scheme, kn):
    """M=1 with f32 activations on the register GEMV (hi and lo bf16 rows)."""
    k, n = kn
    announce(f"f32 contract gemv m=1 {NAMES[scheme]} k={k} n={n}")
    rng = np.random.default_rng(k + n + scheme)
    x = rng.standard_normal((1, k)).astype(np.float32)
    if scheme == MLX4:
        codes = rng.integers(0, 16, (n, k)).astype(np.uint32)
        wq = orc.mlx_pack(codes, 4)
        sc = rng.uniform(0.01, 0.1, (n, k // 64)).astype(np.float32)
        bi = rng.uniform(-0.5, 0.1, (n, k // 64)).astype(np.float32)
        got, kern = _f32_run(ctx, MLX4, x, _t(wq.view(np.uint8)), n, group=64, scales=_t(sc), biases=_t(bi))
        want = orc.mlx_matmul_f64(x, wq, sc, bi, n, 4, 64)
    elif scheme == MXFP4:
        mc, eb = orc.synth_mxfp4(rng, n, k)
        got, kern = _f32_run(ctx, MXFP4, x, _t(mc), n, scales=_t(eb))
        want = orc.mxfp4_matmul_f64(x, mc, eb, n)
    else:
        packed = orc.synth(scheme, rng, n, k)
        got, kern = _f32_run(ctx, scheme, x, _t(packed), n)
        want = _want(orc, scheme, x, packed, k)
    assert kern.startswith(f"rlxq_gemvxs_{NAMES[scheme]}_") and kern.endswith("_F"), kern
    assert rel_err(got, want) <= TOL, kern


# every compiled single-row f32 variant "NU:D,W" (NU unit chunks of 64: K
# up to 2048 NU)
F_VARIANTS = ["1:2,8", "2:2,4", "2:1,4", "2:1,8", "2:2,8", "2:1,16", "3:1,8", "4:1,8"]


@pytest.mark.parametrize("cfg", F_VARIANTS)
def test_single_row_f32_every_variant(ctx, orc, monkeypatch, cfg):
    nu, dw = cfg.split(":")
    monkeypatch.setenv("RLXQ_GEMV_XSF", dw)
    d, w = dw.split(",")
    k = 2048 * int(nu)
    for n in (4096, 77, 3):
        announce(f"f32 contract gemv m=1 variant {cfg} k={k} n={n}")
        rng = np.random.default_rng(k + n + int(w))
        packed = _exact_f16_q4_1(orc, rng, n, k)
        x = rng.standard_normal((1, k)).astype(np.float32)
        got, kern = _f32_run(ctx, Q4_1, x, _t(packed), n)
        assert kern == f"rlxq_gemvxs_q4_1_U{nu}_D{d}_W{w}_F", kern
        assert rel_err(got, _want(orc, Q4_1, x, packed, k)) <= TOL_EXACT_W


@pytest.mark.parametrize("kn", [(4096, 16384), (12288, 520), (10240, 33)], ids=str)
def test_single_row_f32_q4_1_k_split_defaults(ctx, orc, kn):
    """Q4_1 rows at gate_up's width and K past four unit chunks (down) take
    the two-wave K-split register kernel by default."""
    k, n = kn
    announce(f"f32 contract gemv m=1 k-split k={k} n={n}")
    rng = np.random.default_rng(k + n)
    packed = orc.synth(Q4_1, rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, kern = _f32_run(ctx, Q4_1, x, _t(packed), n)
    assert kern.startswith("rlxq_gemvxs_q4_1_") and kern.endswith("_F_K2"), kern
    assert rel_err(got, _want(orc, Q4_1, x, packed, k)) <= TOL
    packed = _exact_f16_q4_1(orc, rng, n, k)
    got, kern = _f32_run(ctx, Q4_1, x, _t(packed), n)
    assert rel_err(got, _want(orc, Q4_1, x, packed, k)) <= TOL_EXACT_W


@pytest.mark.parametrize("kn", [(4096, 4096), (8192, 300)], ids=str)
def test_single_row_f32_exact_weights(ctx, orc, kn):
    k, n = kn
    announce(f"f32 contract gemv m=1 exact weights k={k} n={n}")
    rng = np.random.default_rng(k + 5)
    packed = _exact_f16_q4_1(orc, rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, kern = _f32_run(ctx, Q4_1, x, _t(packed), n)
    assert kern.endswith("_F"), kern
    assert rel_err(got, _want(orc, Q4_1, x, packed, k)) <= TOL_EXACT_W


def test_f32_activation_range(ctx, orc):
    """Rows far outside the f16 range, rows of tiny values and a zero row,
    on the batched-decode and prefill kernels: the row scale is taken before
    the split, so every row keeps its relative accuracy."""
    for m in (8, 300):
        k, n = 512, 96
        announce(f"f32 contract activation range m={m}")
        rng = np.random.default_rng(20 + m)
        packed = orc.synth_q4_1(rng, n, k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        x[0] *= 1e6
        x[1] *= 1e-6
        x[2, 7] = 3e5
        x[3] = 0.0
        got, kern = _f32_run(ctx, Q4_1, x, _t(packed), n)
        assert kern.startswith("rlxq_skinny" if m == 8 else "rlxq_gemm_q4_1"), kern
        want = _want(orc, Q4_1, x, packed, k)
        for r in range(m):
            if r == 3:
                assert np.all(got[r] == 0.0)
                continue
            assert rel_err(got[r:r + 1], want[r:r + 1]) <= TOL, (m, r)


def test_device_matmul_session_f32_on_mfma(orc):
    """The session mirror (rlxq_dm_matmul: F32 x, F32 y, as the Rust shim
    passes them) at decode, batched-decode and prefill sizes."""
    import torch
    import rlxq

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dm = rlxq.DeviceMatmul(0)
    rng = np.random.default_rng(9)
    k, n = 2048, 512
    packed = orc.synth_q4_1(rng, n, k).ravel()
    for m in (1, 16, 300):
        announce(f"DeviceMatmul f32 m={m}")
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = dm.matmul(x, packed, m, k, n, rlxq.GGUF_Q4_1).reshape(m, n)
        assert rel_err(y, _want(orc, Q4_1, x, packed.reshape(n, -1), k)) <= TOL, m
    assert dm.uploads == 1
    dm.close()


@pytest.mark.parametrize("scheme", [Q8_0, Q4_0, Q4_1], ids=lambda s: NAMES[s])
@pytest.mark.parametrize("m", [1, 7, 16, 128, 300])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_reference_structured_inputs_every_path(ctx, orc, scheme, m, xdt):
    """The reference's own parity data (quant_parity_backends.rs:61-71: x =
    0.8 sin(0.031 i), W = 0.35 cos(0.017 i + 0.3), quantized) at K = 1792,
    where rounding each weight once to f16 already costs 1.4e-3 and
    rounding the activations alone 7e-4: every f32-output path (the register
    GEMV at M=1, the batched-decode kernels from 5 rows, the exact prefill
    GEMM past 256) stays within 5e-5, far inside the 1e-3 bar."""
    import torch
    from test_gemv_gpu import _ref_input, _ref_weight

    k, n = 1792, 1280
    announce(f"structured inputs {NAMES[scheme]} m={m} x={xdt}")
    x = _ref_input(m, k)
    packed = orc.quantize(scheme, _ref_weight(n, k, 0.3))
    xt = _t(x) if xdt == "f32" else _t(x).to(torch.bfloat16)
    xv = xt.float().cpu().numpy()
    y = ctx.dequant_matmul(xt, _t(packed), scheme, n, y_dtype=torch.float32)
    kern = ctx.last_kernel
    torch.cuda.synchronize()
    if m >= 300:
        assert kern.startswith(f"rlxq_gemm_{NAMES[scheme]}_t256") and kern.endswith("xs" if xdt == "f32" else "x"), kern
    elif m >= 5:
        assert kern.startswith("rlxq_skinny"), kern
    assert rel_err(y.cpu().numpy(), _want(orc, scheme, xv, packed, k)) <= 5e-5, kern
