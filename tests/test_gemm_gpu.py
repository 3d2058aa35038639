"""Parity of the prefill dequant-GEMM against the CPU oracle, through the C
ABI: the bf16 kernels (weights rounded to bf16 in LDS, bf16 MFMA) and, for
the GGUF schemes, their f16 variant (weights d*q + m rounded once to f16 in
LDS, activations scaled by a power of two into f16, f16 MFMA); fp32
accumulation throughout.  Bar: max|got - want| / max|want| <= 8e-3 with bf16 output
(tighter than the 2e-2 prefill contract: bf16 weights and the bf16 output
rounding account for about 4e-3), 1e-3 for the f16 kernel with f32 output; `want` is the
oracle's dequantized weights contracted in float64 with the bf16 activations
the kernel saw."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, rel_err

pytestmark = pytest.mark.gpu

TOL_PREFILL = 8e-3


def run_gemm(ctx, orc, scheme, x32, packed, n, ydt="bf16", **kw):
    import torch

    k = x32.shape[1]
    xt = _t(x32).to(torch.bfloat16)
    y = ctx.dequant_matmul(xt, _t(packed), scheme, n, y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32, **kw)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), xt.float().cpu().numpy()


@pytest.mark.parametrize("scheme", [1, 2, 3])
@pytest.mark.parametrize("mkn", [(128, 256, 128), (512, 4096, 1024), (300, 1280, 200), (64, 768, 96),
                                 (129, 192, 130)], ids=str)
def test_gemm_matches_oracle(ctx, orc, scheme, mkn):
    m, k, n = mkn
    announce(f"gemm scheme={scheme} {mkn}")
    rng = np.random.default_rng(m + k + n)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, xv = run_gemm(ctx, orc, scheme, x, packed, n)
    assert ctx.last_kernel.startswith("rlxq_gemm")
    w = orc.dequantize(scheme, packed, k).astype(np.float64)
    assert rel_err(got, xv.astype(np.float64) @ w.T) <= TOL_PREFILL


@pytest.mark.parametrize("kn", [(4096, 24576), (12288, 4096)], ids=lambda s: f"{s[0]}to{s[1]}")
def test_gemm_config4_shapes_m512(ctx, orc, kn):
    """Config 4 shapes at M=512 (the larger M use the same tiles); f64 truth."""
    k, n = kn
    m = 512
    announce(f"gemm config4 {k}->{n} m={m}")
    rng = np.random.default_rng(4)
    packed = orc.synth_q4_1(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, xv = run_gemm(ctx, orc, 3, x, packed, n)
    w = orc.dequantize(3, packed, k).astype(np.float64)
    assert rel_err(got, xv.astype(np.float64) @ w.T) <= TOL_PREFILL


def test_gemm_linearity_full_size(ctx, orc):
    """Size-independent check at M=4096, 4096->24576: y(x1 + x2) = y(x1) + y(x2)
    within bf16 rounding, on a sampled set of outputs checked against f64."""
    import torch
    import rlxq

    m, k, n = 4096, 4096, 24576
    announce("gemm linearity full size")
    g = torch.Generator(device="cuda").manual_seed(7)
    from bench import synth_q4_1_gpu

    w = synth_q4_1_gpu(n, k, g)
    x1 = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    y1 = ctx.dequant_matmul(x1, w, rlxq.GGUF_Q4_1, n, y_dtype=torch.float32)
    rows = torch.tensor([0, 1, 777, 2048, 4095], device="cuda")
    torch.cuda.synchronize()
    packed = w.cpu().numpy()
    wd = orc.dequantize(3, packed.reshape(n, -1), k).astype(np.float64)
    want = x1[rows].float().cpu().numpy().astype(np.float64) @ wd.T
    got = y1[rows].cpu().numpy()
    assert rel_err(got, want) <= TOL_PREFILL


@pytest.mark.parametrize("bits", [4, 8])
def test_gemm_mlx(ctx, orc, bits):
    import torch
    import rlxq

    m, k, n, group = 192, 512, 160, 64
    announce(f"gemm mlx bits={bits}")
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint32)
    wq = orc.mlx_pack(codes, bits)
    sc = rng.uniform(0.01, 0.1, (n, k // group)).astype(np.float32)
    bi = rng.uniform(-0.5, 0.1, (n, k // group)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    scheme = rlxq.MLX_AFFINE4 if bits == 4 else rlxq.MLX_AFFINE8
    got, xv = run_gemm(ctx, orc, scheme, x, wq.view(np.uint8), n, group=group, scales=_t(sc), biases=_t(bi))
    assert ctx.last_kernel.startswith("rlxq_gemm_")
    want = xv.astype(np.float64) @ orc.mlx_dequantize(wq, sc, bi, k, bits, group).astype(np.float64).T
    assert rel_err(got, want) <= TOL_PREFILL


def test_gemm_forced_for_small_m_and_f32_output(ctx, orc, monkeypatch):
    """The dispatcher override runs the GEMM for M=1..63 and f32 output too."""
    monkeypatch.setenv("RLXQ_PREFILL", "gemm")
    rng = np.random.default_rng(9)
    for m in (1, 7, 63):
        packed = orc.synth_q4_1(rng, 200, 256)
        x = rng.standard_normal((m, 256)).astype(np.float32)
        got, xv = run_gemm(ctx, orc, 3, x, packed, 200, ydt="f32")
        assert ctx.last_kernel.startswith("rlxq_gemm")
        w = orc.dequantize(3, packed, 256).astype(np.float64)
        assert rel_err(got, xv.astype(np.float64) @ w.T) <= TOL_PREFILL


@pytest.mark.parametrize("scheme", [1, 2, 3, 4, 5])
def test_every_gemm_tiling(ctx, orc, scheme, monkeypatch):
    """Every tiling (128 x 128; 256 x 256 with 4 or 8 waves; 256 x 128 with 4
    or 8 waves) on a ragged shape, every scheme:
    each within the prefill bar, and the two agree to ~1e-6 (f32 output; both
    accumulate K in the same order)."""
    import torch
    import rlxq

    m, k, n = 300, 640, 272
    rng = np.random.default_rng(scheme)
    x = rng.standard_normal((m, k)).astype(np.float32)
    kw = {}
    if scheme in (rlxq.MLX_AFFINE4, rlxq.MLX_AFFINE8):
        bits, group = (4, 32) if scheme == rlxq.MLX_AFFINE4 else (8, 128)
        codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint32)
        wq = orc.mlx_pack(codes, bits)
        sc = rng.uniform(0.01, 0.1, (n, k // group)).astype(np.float32)
        bi = rng.uniform(-0.5, 0.1, (n, k // group)).astype(np.float32)
        packed = wq.view(np.uint8)
        kw = dict(group=group, scales=_t(sc), biases=_t(bi))
        wd = orc.mlx_dequantize(wq, sc, bi, k, bits, group).astype(np.float64)
    else:
        packed = orc.synth(scheme, rng, n, k)
        wd = orc.dequantize(scheme, packed, k).astype(np.float64)
    outs = {}
    monkeypatch.setenv("RLXQ_PREFILL", "gemm")
    for tile in ("128", "256", "256w8", "256w8l", "256w8p2", "256n128", "256n128w8"):
        monkeypatch.setenv("RLXQ_GEMM_TILE", tile)
        announce(f"gemm tiling t{tile} scheme={scheme} m={m} k={k} n={n}")
        got, xv = run_gemm(ctx, orc, scheme, x, packed, n, ydt="f32", **kw)
        assert ctx.last_kernel.endswith(f"_t{tile}")
        assert rel_err(got, xv.astype(np.float64) @ wd.T) <= TOL_PREFILL
        outs[tile] = got
    for t in ("256", "256w8", "256w8l", "256w8p2", "256n128", "256n128w8"):
        assert np.allclose(outs["128"], outs[t], rtol=1e-6, atol=1e-6 * np.abs(outs["128"]).max())


@pytest.mark.parametrize("scheme", [1, 2, 3])
def test_f32_output_prefill_takes_the_exact_kernel(ctx, orc, scheme):
    """GGUF, bf16 activations, f32 output, past the batched-decode sizes: the
    dispatcher picks the exact GEMM (f16 hi + lo weights), and the output
    meets the 1e-3 bar."""
    m, k, n = 384, 1024, 520
    rng = np.random.default_rng(11 + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, xv = run_gemm(ctx, orc, scheme, x, packed, n, ydt="f32")
    assert ctx.last_kernel.endswith("x"), ctx.last_kernel
    wd = orc.dequantize(scheme, packed, k).astype(np.float64)
    assert rel_err(got, xv.astype(np.float64) @ wd.T) <= 1e-3


@pytest.mark.parametrize("scheme", [1, 2, 3])
@pytest.mark.parametrize("mkn", [(256, 64, 256), (300, 640, 272), (513, 1280, 300), (1000, 4096, 520)], ids=str)
def test_gemm_exact_shared_conversion(ctx, orc, monkeypatch, scheme, mkn):
    """The exact variant: weights converted once per workgroup to f16 hi +
    lo rows (128 output columns per tile), f16 MFMA on the prepared
    activations: f32 output within 1e-3."""
    monkeypatch.setenv("RLXQ_PREFILL", "gemm")
    tile = "256w8x" if scheme in (1, 3) else "256w8p2x"   # Q8_0, Q4_1: one register stage
    monkeypatch.setenv("RLXQ_GEMM_TILE", tile)
    m, k, n = mkn
    announce(f"gemm exact shared conversion t{tile} scheme={scheme} {mkn}")
    rng = np.random.default_rng(scheme * 7 + m + k + n)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= 500.0
    got, xv = run_gemm(ctx, orc, scheme, x, packed, n, ydt="f32")
    assert ctx.last_kernel.endswith(f"_t{tile}"), ctx.last_kernel
    wd = orc.dequantize(scheme, packed, k).astype(np.float64)
    assert rel_err(got, xv.astype(np.float64) @ wd.T) <= 1e-3


@pytest.mark.parametrize("scheme", [1, 2, 3, 4])
@pytest.mark.parametrize("tile_ydt", [("256w8p2", "bf16"), ("256w8", "f32"), ("256w8p2x", "f32"), ("256w8x", "f32"),
                                      ("256n128", "bf16"), ("256n128w8", "f32")],
                         ids=lambda t: f"{t[0]}-{t[1]}")
@pytest.mark.parametrize("splits", [2, 3, 8])
def test_gemm_split_k(ctx, orc, monkeypatch, scheme, tile_ydt, splits):
    """K cut into slices (the last one shorter when the steps do not divide),
    slice partial sums added in slice order: within the bar against the
    oracle, and within 1e-5 of the unsplit kernel (f32 output)."""
    import rlxq

    tile, ydt = tile_ydt
    one_stage = scheme in (1, 3, 4)   # Q8_0, Q4_1, MLX 4-bit: the one-stage exact variant (bf16 x)
    if tile == "256w8x" and not one_stage or tile == "256w8p2x" and one_stage:
        pytest.skip("one exact tiling per scheme")
    m, k, n = 300, 64 * 13, 520
    rng = np.random.default_rng(31 * scheme + splits)
    x = rng.standard_normal((m, k)).astype(np.float32)
    kw = {}
    if scheme == rlxq.MLX_AFFINE4:
        codes = rng.integers(0, 16, (n, k)).astype(np.uint32)
        wq = orc.mlx_pack(codes, 4)
        sc = rng.uniform(0.01, 0.1, (n, k // 64)).astype(np.float32)
        bi = rng.uniform(-0.5, 0.1, (n, k // 64)).astype(np.float32)
        packed = wq.view(np.uint8)
        kw = dict(group=64, scales=_t(sc), biases=_t(bi))
        wd = orc.mlx_dequantize(wq, sc, bi, k, 4, 64).astype(np.float64)
    else:
        packed = orc.synth(scheme, rng, n, k)
        wd = orc.dequantize(scheme, packed, k).astype(np.float64)
    monkeypatch.setenv("RLXQ_PREFILL", "gemm")
    monkeypatch.setenv("RLXQ_GEMM_TILE", tile)
    outs = {}
    for sp in (1, splits):
        monkeypatch.setenv("RLXQ_GEMM_SPLITS", str(sp))
        announce(f"gemm split-k t{tile} scheme={scheme} splits={sp} ydt={ydt}")
        got, xv = run_gemm(ctx, orc, scheme, x, packed, n, ydt=ydt, **kw)
        assert ctx.last_kernel.endswith(f"_t{tile}"), ctx.last_kernel
        tol = 1e-3 if tile.endswith("x") else TOL_PREFILL
        assert rel_err(got, xv.astype(np.float64) @ wd.T) <= tol
        outs[sp] = got
    if ydt == "f32":
        assert rel_err(outs[splits], outs[1]) <= 1e-5


@pytest.mark.parametrize("case", ["f32_x", "n_odd", "bf16_x_f32_y"])
@pytest.mark.parametrize("splits", [2, 3])
def test_gemm_split_k_reduction_layouts(ctx, orc, monkeypatch, case, splits):
    """The split-K partial sums of each layout: F32 activations on the exact
    variant (hi / lo x16 rows, m_out output rows), an N that is no multiple
    of 4 (one output per reduction thread), bf16 x with f32 y (the exact
    variant's 128 output columns), all with row and column tails: within the
    bar against the oracle and within 1e-5 of the unsplit kernel."""
    import torch

    m, k, n = 300, 64 * 13, 301 if case == "n_odd" else 392
    rng = np.random.default_rng(5 * splits + len(case))
    packed = orc.synth_q4_1(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wd = orc.dequantize(3, packed, k).astype(np.float64)
    monkeypatch.setenv("RLXQ_PREFILL", "gemm")
    outs = {}
    for sp in (1, splits):
        monkeypatch.setenv("RLXQ_GEMM_SPLITS", str(sp))
        announce(f"gemm split-k reduction {case} splits={sp}")
        if case == "f32_x":
            xt = _t(x)
            y = ctx.dequant_matmul(xt, _t(packed), 3, n, y_dtype=torch.float32)
            assert ctx.last_kernel.endswith("xs"), ctx.last_kernel
        else:
            xt = _t(x).to(torch.bfloat16)
            y = ctx.dequant_matmul(xt, _t(packed), 3, n, y_dtype=torch.float32)
        torch.cuda.synchronize()
        got = y.float().cpu().numpy()
        want = xt.float().cpu().numpy().astype(np.float64) @ wd.T
        assert rel_err(got, want) <= (1e-3 if case != "n_odd" or ctx.last_kernel.endswith("x") else TOL_PREFILL)
        outs[sp] = got
    assert rel_err(outs[splits], outs[1]) <= 1e-5


@pytest.mark.parametrize("mkn", [(512, 12288, 4096), (2048, 12288, 4096), (256, 4096, 24576)], ids=str)
def test_gemm_default_split_on_small_grids(ctx, orc, mkn):
    """Prefill shapes whose 256 x 256 tiles do not cover the CUs: the
    dispatcher takes the 256 x 128 tiles and splits K by itself where those
    do not cover them either; the output stays within the bar."""
    m, k, n = mkn
    announce(f"gemm default split {mkn}")
    rng = np.random.default_rng(m + n)
    packed = orc.synth_q4_1(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, xv = run_gemm(ctx, orc, 3, x, packed, n)
    # (256 x 256 tiles would split K on all three: the 256 x 128 tiles serve)
    assert ctx.last_kernel == "rlxq_gemm_q4_1_t256n128w8", ctx.last_kernel
    w = orc.dequantize(3, packed, k).astype(np.float32)
    want = (xv @ w.T).astype(np.float64)
    assert rel_err(got, want) <= TOL_PREFILL


@pytest.mark.parametrize("mkn,want", [((4096, 4096, 24576), "t256w8p2"), ((2048, 4096, 24576), "t256w8p2"),
                                      ((512, 4096, 24576), "t256w8p2"), ((1024, 4096, 24576), "t256n128w8"),
                                      ((4096, 12288, 4096), "t256w8p2"), ((1024, 4096, 4096), "t256n128w8")], ids=str)
def test_gemm_default_tiling_rule(ctx, orc, mkn, want):
    """The dispatcher's tiling for bf16 in and out on 256 CUs: 256 x 256
    tiles where they fill whole rounds of workgroups without a K split,
    256 x 128 tiles where the 256 x 256 ones would split K or leave a partly
    filled last round (4096->24576 at M=1024: 384 tiles, 768 of 256 x 128).
    A sampled block of the output is checked against the oracle."""
    import torch

    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the rule's cases assume 256 CUs")
    m, k, n = mkn
    announce(f"gemm default tiling {mkn}")
    g = torch.Generator(device="cuda").manual_seed(m + n)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    rng = np.random.default_rng(m + k)
    cols = 256
    packed = orc.synth_q4_1(rng, cols, k)
    wfull = torch.zeros((n * k * 5 // 8,), dtype=torch.uint8, device="cuda")
    wfull[: cols * k * 5 // 8] = _t(packed.ravel())
    y = ctx.dequant_matmul(x, wfull, 3, n, y_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert ctx.last_kernel == f"rlxq_gemm_q4_1_{want}", ctx.last_kernel
    rows = np.arange(0, m, max(1, m // 64))
    xv = x.float().cpu().numpy()[rows].astype(np.float64)
    want_y = xv @ orc.dequantize(3, packed, k).astype(np.float64).T
    assert rel_err(y.float().cpu().numpy()[rows, :cols], want_y) <= TOL_PREFILL


@pytest.mark.parametrize("m,k,n", [(2048, 4096, 24576), (4096, 4096, 24576), (2048, 12288, 4096),
                                   (4096, 12288, 4096)], ids=str)
@pytest.mark.parametrize("ydt", ["bf16", "f32"])
def test_gemm_config4_full_size_sampled(ctx, orc, m, k, n, ydt):
    """The bench's prefill cells at full size (Q4_1, Qwen3-8B gate|up and
    down, M = 2048 and 4096; 12288->4096 at M=4096 is the unsplit path), with
    the output dtype the bench reports (bf16) and the f32-output f16 kernel:
    48 rows x 384 columns of the output against the float64 oracle."""
    import torch
    import rlxq
    from bench import synth_q4_1_gpu

    announce(f"gemm config4 full size m={m} k={k} n={n} y={ydt}")
    g = torch.Generator(device="cuda").manual_seed(m + k + n)
    w = synth_q4_1_gpu(n, k, g)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    y = ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n, y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    kern = ctx.last_kernel
    torch.cuda.synchronize()
    assert kern.startswith("rlxq_gemm_q4_1_t256"), kern
    rs = np.random.default_rng(m + n)
    rows = np.sort(rs.choice(m, 48, replace=False))
    cols = np.sort(rs.choice(n, 384, replace=False))
    wsub = w.view(n, -1)[torch.from_numpy(cols).cuda()].cpu().numpy()
    wd = orc.dequantize(3, wsub, k).astype(np.float64)
    want = x[torch.from_numpy(rows).cuda()].float().cpu().numpy().astype(np.float64) @ wd.T
    got = y.float().cpu().numpy()[np.ix_(rows, cols)]
    # the sampled block's own max is the scale (a subset of the full output's)
    assert rel_err(got, want) <= (TOL_PREFILL if ydt == "bf16" else 1e-3), kern

