"""Parity of the dense DequantMatMul path (GEMV kernels) against the CPU oracle,
called through the C ABI.  Bar: dequantized weights bit-exact; outputs within
max|got - want| / max|want| <= 1e-3 for f32 outputs (fp32 accumulate), 1e-2 for
bf16 outputs.  `want` is the oracle's dequantized weights contracted in
float64."""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_BF16 = 1e-2


def _t(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def want_f64(orc, scheme, x, packed, k):
    w = orc.dequantize(scheme, packed, k).astype(np.float64)
    return x.astype(np.float64) @ w.T


def rel_err(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


def _x_as(x32, xdt):
    """The activations as the kernel will see them, and the same values as f32."""
    import torch

    if xdt == "bf16":
        xt = _t(x32).to(torch.bfloat16)
        return xt, xt.float().cpu().numpy()
    return _t(x32), x32


def run_dense(ctx, orc, scheme, x32, packed, n, xdt="f32", ydt="f32"):
    import torch
    import rlxq

    k = x32.shape[1]
    xt, xv = _x_as(x32, xdt)
    wt = _t(packed)
    y = ctx.dequant_matmul(xt, wt, scheme, n, y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    return got, want_f64(orc, scheme, xv, packed, k)


# ----------------------------------------------------------------------------
def _ref_input(rows, k):
    """crates/rlx-unlimited-ocr/tests/quant_parity_backends.rs:61-71."""
    return (np.sin(np.arange(rows * k, dtype=np.float32) * np.float32(0.031)) * np.float32(0.8)).reshape(rows, k)


def _ref_weight(n, k, seed):
    return (np.cos(np.arange(n * k, dtype=np.float32) * np.float32(0.017) + np.float32(seed))
            * np.float32(0.35)).reshape(n, k)


MATMUL_SHAPES = [(4, 256, 128), (1, 1280, 1280), (128, 1280, 1280), (128, 1280, 1792), (128, 1792, 1280),
                 (1, 1280, 129280)]


@pytest.mark.parametrize("scheme", [1, 2, 3])
@pytest.mark.parametrize("shape", MATMUL_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_reference_matmul_shapes(ctx, orc, scheme, shape):
    """check_matmul (quant_parity_backends.rs:227-253) with its shapes and fills;
    the reference's bar is 1e-2, this build's is 1e-3."""
    rows, k, n = shape
    announce(f"reference shape scheme={scheme} {shape}")
    x = _ref_input(rows, k)
    packed = orc.quantize(scheme, _ref_weight(n, k, 0.3))
    got, want = run_dense(ctx, orc, scheme, x, packed, n)
    assert rel_err(got, want) <= TOL_F32


QWEN3_8B = [(4096, 4096), (4096, 6144), (4096, 24576), (12288, 4096)]


@pytest.mark.parametrize("kn", QWEN3_8B, ids=lambda s: f"{s[0]}to{s[1]}")
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_q4_1_gemv_qwen3_8b_shapes(ctx, orc, kn, xdt):
    """Config 2: Q4_1 group-32 GEMV at M=1, seeded synthetic weights."""
    k, n = kn
    announce(f"q4_1 gemv {k}->{n} x={xdt}")
    rng = np.random.default_rng(0)
    packed = orc.synth_q4_1(rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, 3, x, packed, n, xdt=xdt)
    assert rel_err(got, want) <= TOL_F32


def test_q8_0_gemv_config1(ctx, orc):
    """Config 1: Q8_0 2048->2048, x fp32 N(0,1), q ~U{-127..127}, d ~U(0.002, 0.02)."""
    announce("q8_0 gemv 2048->2048")
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 2048)).astype(np.float32)
    packed = orc.synth_q8_0(rng, 2048, 2048)
    got, want = run_dense(ctx, orc, 1, x, packed, 2048)
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("scheme", [1, 3])
@pytest.mark.parametrize("m", [1, 4, 16, 64])
@pytest.mark.parametrize("kn", [(4096, 24576), (12288, 4096)], ids=lambda s: f"{s[0]}to{s[1]}")
def test_batched_decode(ctx, orc, scheme, m, kn):
    """Config 3: Q4_1 and Q8_0 at M in {1, 4, 16, 64}, bf16 activations, independent rows."""
    k, n = kn
    announce(f"batched scheme={scheme} m={m} {k}->{n}")
    rng = np.random.default_rng(m)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16")
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("scheme", [1, 2, 3])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
@pytest.mark.parametrize("mkn", [(1, 64, 1), (2, 64, 17), (3, 128, 33), (5, 320, 7), (1, 768, 2048),
                                 (7, 2048, 1536), (1, 1792, 100), (9, 192, 300)], ids=str)
def test_ragged_shapes(ctx, orc, scheme, xdt, mkn):
    m, k, n = mkn
    announce(f"ragged scheme={scheme} x={xdt} {mkn}")
    rng = np.random.default_rng(k + n)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt=xdt)
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("k", [32, 96, 160])
def test_q4_1_odd_block_counts(ctx, orc, k):
    announce(f"q4_1 odd blocks k={k}")
    rng = np.random.default_rng(k)
    packed = orc.synth_q4_1(rng, 70, k)
    x = rng.standard_normal((2, k)).astype(np.float32)
    got, want = run_dense(ctx, orc, 3, x, packed, 70)
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("scheme", [1, 3])
def test_bf16_output(ctx, orc, scheme):
    announce(f"bf16 output scheme={scheme}")
    rng = np.random.default_rng(5)
    packed = orc.synth(scheme, rng, 512, 1024)
    x = rng.standard_normal((3, 1024)).astype(np.float32)
    got, want = run_dense(ctx, orc, scheme, x, packed, 512, xdt="bf16", ydt="bf16")
    assert rel_err(got, want) <= TOL_BF16


def test_large_activation_values_q8_0(ctx, orc):
    """f16 pairs carry x scaled per block by a power of two: outliers beyond the
    f16 range and tiny blocks must not overflow or lose the block."""
    announce("q8_0 large activations")
    rng = np.random.default_rng(11)
    k, n = 256, 64
    packed = orc.synth_q8_0(rng, n, k)
    x = rng.standard_normal((2, k)).astype(np.float32)
    x[0, :32] *= 1e6
    x[0, 32:64] *= 1e-6
    x[1, 100] = 3e5
    got, want = run_dense(ctx, orc, 1, x, packed, n)
    assert rel_err(got, want) <= TOL_F32


# ------------------------------------------------------------------ MLX affine
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("sb", ["f32", "bf16"])
def test_mlx_affine(ctx, orc, bits, group, sb):
    import torch
    import rlxq

    m, k, n = 3, 512, 96
    announce(f"mlx bits={bits} group={group} sb={sb}")
    rng = np.random.default_rng(bits * group)
    codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint32)
    wq = orc.mlx_pack(codes, bits)
    scales = rng.uniform(0.01, 0.1, (n, k // group)).astype(np.float32)
    biases = rng.uniform(-0.5, 0.1, (n, k // group)).astype(np.float32)
    if sb == "bf16":
        scales = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(scales))
        biases = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(biases))
        st, bt = _t(scales).to(torch.bfloat16), _t(biases).to(torch.bfloat16)
    else:
        st, bt = _t(scales), _t(biases)
    x = rng.standard_normal((m, k)).astype(np.float32)
    scheme = rlxq.MLX_AFFINE4 if bits == 4 else rlxq.MLX_AFFINE8
    y = ctx.dequant_matmul(_t(x), _t(wq.view(np.uint8)), scheme, n, group=group, scales=st, biases=bt)
    deq = ctx.dequantize(_t(wq.view(np.uint8)), scheme, n, k, group=group, scales=st, biases=bt)
    torch.cuda.synchronize()
    want_w = orc.mlx_dequantize(wq, scales, biases, k, bits, group)
    assert np.array_equal(deq.cpu().numpy(), want_w)
    want = orc.mlx_matmul_f64(x, wq, scales, biases, n, bits, group)
    assert rel_err(y.cpu().numpy(), want) <= TOL_F32


# ------------------------------------------------------------- dequantize exact
@pytest.mark.parametrize("scheme", [1, 2, 3])
def test_dequantize_bit_exact(ctx, orc, scheme):
    import torch

    announce(f"dequantize scheme={scheme}")
    rng = np.random.default_rng(scheme)
    k, n = 4096, 64
    packed = orc.synth(scheme, rng, n, k)
    got = ctx.dequantize(_t(packed), scheme, n, k)
    torch.cuda.synchronize()
    want = orc.dequantize(scheme, packed, k).view(np.uint32)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)
    # an output that is only 4-byte aligned takes the scalar stores
    buf = torch.full((n * k + 1,), float("nan"), device="cuda")
    ctx.dequantize(_t(packed), scheme, n, k, out=buf[1:].view(n, k))
    torch.cuda.synchronize()
    assert np.array_equal(buf[1:].cpu().numpy().view(np.uint32).reshape(n, k), want)


# ------------------------------------------------------------------ error paths
def test_host_checks_reject_bad_arguments(ctx):
    import torch
    import rlxq

    L = rlxq.lib()
    x = torch.zeros((1, 128), device="cuda")
    y = torch.zeros((1, 8), device="cuda")
    w = torch.zeros(8 * 128, dtype=torch.uint8, device="cuda")

    def call(scheme, k, wp=None, group=32, sc=None, bi=None, xp=None):
        return L.rlxq_dequant_matmul(ctx.h, scheme, group, xp or x.data_ptr(), 0, wp or w.data_ptr(), sc, bi, 0,
                                     1, k, 8, y.data_ptr(), 0, None)

    assert call(3, 40) == rlxq.E_SHAPE
    assert call(1, 96) == rlxq.E_ALIGN
    assert call(3, 128, wp=w.data_ptr() + 2) == rlxq.E_ALIGN
    assert call(3, 128, xp=x.data_ptr() + 4) == rlxq.E_ALIGN
    assert call(99, 128) == rlxq.E_SCHEME
    assert call(4, 128, group=16, sc=x.data_ptr(), bi=x.data_ptr()) == rlxq.E_SHAPE
    assert call(4, 128) == rlxq.E_NULL
    assert L.rlxq_dequant_matmul(ctx.h, 3, 32, x.data_ptr(), 7, w.data_ptr(), None, None, 0, 1, 128, 8,
                                 y.data_ptr(), 0, None) == rlxq.E_DTYPE
    assert b"x_dtype" in L.rlxq_last_error(ctx.h)
    # zero-sized calls succeed without launching anything
    assert L.rlxq_dequant_matmul(ctx.h, 3, 32, x.data_ptr(), 0, w.data_ptr(), None, None, 0, 0, 128, 8,
                                 y.data_ptr(), 0, None) == rlxq.OK


# --------------------------------------------------------- host session mirror
def test_device_matmul_session(orc):
    import torch
    import rlxq

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    announce("DeviceMatmul session")
    dm = rlxq.DeviceMatmul(0)
    rng = np.random.default_rng(3)
    m, k, n = 2, 1280, 896
    packed = orc.synth_q4_1(rng, n, k).ravel()
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = dm.matmul(x, packed, m, k, n, rlxq.GGUF_Q4_1).reshape(m, n)
    assert rel_err(y, want_f64(orc, 3, x, packed, k)) <= TOL_F32
    assert dm.uploads == 1
    y2 = dm.matmul(x * 2, packed, m, k, n, rlxq.GGUF_Q4_1).reshape(m, n)
    assert dm.uploads == 1  # same weight pointer: not uploaded again
    assert rel_err(y2, 2 * want_f64(orc, 3, x, packed, k)) <= TOL_F32
    with pytest.raises(rlxq.RlxqError) as e:
        dm.matmul(x[:, :100], packed, m, k, n, rlxq.GGUF_Q4_1)
    assert e.value.status == rlxq.E_SHAPE and "x len" in str(e.value)
    with pytest.raises(rlxq.RlxqError) as e:
        dm.matmul(x, packed, m, k, n, rlxq.MLX_AFFINE4)
    assert e.value.status == rlxq.E_SCHEME
    dm.close()


# Every compiled single-row GEMV variant (lanes per row, rows and unit chunks
# per step, prefetch depth, waves per workgroup), forced through the dispatcher's override, on shapes that
# leave ragged tiles, partial chunks and odd unit counts.
GEMV_VARIANTS = ["64,1,2,1,16", "64,1,2,2,16", "64,1,2,3,16", "64,1,2,2,8", "64,1,1,4,16", "64,2,1,2,8", "32,2,1,2,8",
                 "16,2,1,2,8", "8,2,1,2,8"]


@pytest.mark.parametrize("cfg", GEMV_VARIANTS)
@pytest.mark.parametrize("scheme", [1, 2, 3, 4])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_every_gemv_variant(ctx, orc, monkeypatch, cfg, scheme, xdt):
    import torch
    import rlxq

    monkeypatch.setenv("RLXQ_GEMV_CFG", cfg)
    for (m, k, n) in [(1, 4096, 300), (1, 768, 37), (3, 1280, 129), (1, 12288, 65)]:
        announce(f"variant {cfg} scheme={scheme} x={xdt} {m}x{k}x{n}")
        rng = np.random.default_rng(k + n + scheme)
        x = rng.standard_normal((m, k)).astype(np.float32)
        if scheme == 4:
            codes = rng.integers(0, 16, (n, k)).astype(np.uint32)
            wq = orc.mlx_pack(codes, 4)
            sc = rng.uniform(0.01, 0.1, (n, k // 64)).astype(np.float32)
            bi = rng.uniform(-0.5, 0.1, (n, k // 64)).astype(np.float32)
            xt, xv = _x_as(x, xdt)
            y = ctx.dequant_matmul(xt, _t(wq.view(np.uint8)), rlxq.MLX_AFFINE4, n, group=64, scales=_t(sc),
                                   biases=_t(bi))
            torch.cuda.synchronize()
            got, want = y.cpu().numpy(), orc.mlx_matmul_f64(xv, wq, sc, bi, n, 4, 64)
        else:
            packed = orc.synth(scheme, rng, n, k)
            got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt=xdt)
        assert rel_err(got, want) <= TOL_F32, (cfg, m, k, n)


# The register-activation path (M = 1, bf16 activations, 4-bit codes): every
# compiled variant, including units per lane above what the shape needs
# (masked chunks) and row counts that leave waves idle.  "NU,D,W" reads the
# activations from global memory, "NU,D,W,1" through LDS.
XR_VARIANTS = ["1,2,4", "2,2,4", "2,1,4", "2,3,4", "2,2,2", "3,2,4", "4,1,4", "4,2,4", "6,1,4", "6,2,4",
               "1,2,8,1", "2,2,8,1", "2,2,16,1", "2,2,4,1", "2,1,4,1", "3,2,8,1", "4,1,8,1", "4,2,8,1", "6,1,8,1",
               "6,2,8,1"]


@pytest.mark.parametrize("cfg", XR_VARIANTS)
@pytest.mark.parametrize("scheme", [2, 3, 4])
def test_every_xr_variant(ctx, orc, monkeypatch, cfg, scheme):
    import torch
    import rlxq

    monkeypatch.setenv("RLXQ_GEMV_XR", cfg)
    nu = int(cfg.split(",")[0])
    if scheme == 2 and nu > 4:
        pytest.skip("six-chunk variants exist for the one-block units (Q4_1, MLX4) only")
    for (k, n) in [(2048, 300), (4096, 1031), (768, 37), (64 * 32 * nu, 5000)]:
        if scheme == 2 and (k // 64 + 63) // 64 > nu or scheme != 2 and (k // 32 + 63) // 64 > nu:
            continue
        announce(f"xr {cfg} scheme={scheme} k={k} n={n}")
        rng = np.random.default_rng(k + n + scheme)
        x = rng.standard_normal((1, k)).astype(np.float32)
        if scheme == 4:
            codes = rng.integers(0, 16, (n, k)).astype(np.uint32)
            wq = orc.mlx_pack(codes, 4)
            sc = rng.uniform(0.01, 0.1, (n, k // 32)).astype(np.float32)
            bi = rng.uniform(-0.5, 0.1, (n, k // 32)).astype(np.float32)
            xt, xv = _x_as(x, "bf16")
            y = ctx.dequant_matmul(xt, _t(wq.view(np.uint8)), rlxq.MLX_AFFINE4, n, group=32, scales=_t(sc),
                                   biases=_t(bi))
            torch.cuda.synchronize()
            got, want = y.cpu().numpy(), orc.mlx_matmul_f64(xv, wq, sc, bi, n, 4, 32)
        else:
            packed = orc.synth(scheme, rng, n, k)
            got, want = run_dense(ctx, orc, scheme, x, packed, n, xdt="bf16")
        assert rel_err(got, want) <= TOL_F32, (cfg, k, n)


def test_bound_call_matches_plain_call(ctx, orc):
    """The pre-bound launch (arguments converted once) writes the same output
    as the plain call, on repeated calls."""
    import torch
    import rlxq

    k, n = 4096, 1000
    rng = np.random.default_rng(77)
    packed = orc.synth_q4_1(rng, n, k)
    x = _t(rng.standard_normal((1, k)).astype(np.float32)).to(torch.bfloat16)
    w = _t(packed)
    want = ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n)
    y = torch.full((1, n), float("nan"), device="cuda")
    call = ctx.bind_dequant_matmul(x, w, rlxq.GGUF_Q4_1, n, y=y, stream=torch.cuda.current_stream().cuda_stream)
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    assert torch.equal(y, want)


@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("k,n", [(2048, 1000), (4096, 4096), (4096, 777), (8192, 640), (1536, 320)], ids=str)
def test_multi_row_register_path(ctx, orc, monkeypatch, m, k, n):
    """Q4_1, bf16 activations, M = 2..4: the register-activation kernel with
    the rows side by side (MT = 2 or 4) where it applies, against the oracle
    and against the LDS-record kernel (RLXQ_GEMV_XR=0)."""
    import torch

    announce(f"multi-row register gemv m={m} k={k} n={n}")
    rng = np.random.default_rng(m * 7 + k + n)
    packed = orc.synth_q4_1(rng, n, k)
    x32 = rng.standard_normal((m, k)).astype(np.float32)
    xt, xv = _x_as(x32, "bf16")
    y = ctx.dequant_matmul(xt, _t(packed), 3, n)
    torch.cuda.synchronize()
    mt = 2 if m <= 2 else 4
    chunks = (k // 32 + 63) // 64
    if chunks <= (4 if mt == 2 else 2):
        assert ctx.last_kernel.endswith(f"_M{mt}"), ctx.last_kernel
    got = y.cpu().numpy()
    assert rel_err(got, want_f64(orc, 3, xv, packed, k)) <= 1e-3
    yb = ctx.dequant_matmul(xt, _t(packed), 3, n, y_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert rel_err(yb.float().cpu().numpy(), want_f64(orc, 3, xv, packed, k)) <= 1e-2
    monkeypatch.setenv("RLXQ_GEMV_XR", "0")
    y2 = ctx.dequant_matmul(xt, _t(packed), 3, n)
    torch.cuda.synchronize()
    assert "gemvxs" not in ctx.last_kernel
    assert rel_err(got, y2.cpu().numpy().astype(np.float64)) <= 1e-3


def test_plain_c_caller_on_the_gpu():
    """examples/decode_gemv.c run as its own process: a Q4_1 decode GEMV
    called from C, checked against its double-precision loop (1e-3)."""
    import subprocess

    import rlxq

    announce("plain C caller")
    exe = rlxq.PKG / "lib" / "examples" / "decode_gemv"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=100)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "rlxq_gemv" in r.stdout


@pytest.mark.parametrize("scheme", ["mlx4", "mxfp4", "q4_k"])
@pytest.mark.parametrize("m", [2, 4])
def test_multi_row_register_path_mlx_mxfp4(ctx, orc, m, scheme):
    """M = 2..4 on the register kernel for the other 4-bit formats: MLX
    affine 4-bit (group 64, bf16 slabs), MXFP4 (E8M0 scales) and Q4_K."""
    import torch
    import rlxq

    k, n = 4096, 1000
    announce(f"multi-row register gemv {scheme} m={m}")
    rng = np.random.default_rng(90 + m)
    x32 = rng.standard_normal((m, k)).astype(np.float32)
    xt, xv = _x_as(x32, "bf16")
    if scheme == "mlx4":
        codes = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint32)
        sc = (rng.uniform(0.01, 0.1, (n, k // 64))).astype(np.float32)
        bi = (rng.uniform(-0.5, 0.1, (n, k // 64))).astype(np.float32)
        sct, bit = _t(sc).to(torch.bfloat16), _t(bi).to(torch.bfloat16)
        y = ctx.dequant_matmul(xt, _t(codes.view(np.uint8)), rlxq.MLX_AFFINE4, n, group=64, scales=sct, biases=bit)
        want = orc.mlx_matmul_f64(xv, codes, sct.float().cpu().numpy(), bit.float().cpu().numpy(), n, 4, 64)
    elif scheme == "mxfp4":
        codes, eb = orc.synth_mxfp4(rng, n, k)
        y = ctx.dequant_matmul(xt, _t(codes), rlxq.MLX_MXFP4, n, scales=_t(eb))
        want = orc.mxfp4_matmul_f64(xv, codes, eb, n)
    else:
        packed = orc.synth_q4_k(rng, n, k)
        y = ctx.dequant_matmul(xt, _t(packed), rlxq.GGUF_Q4_K, n)
        want = want_f64(orc, rlxq.GGUF_Q4_K, xv, packed, k)
    torch.cuda.synchronize()
    assert ctx.last_kernel.endswith(f"_M{m}"), ctx.last_kernel
    assert rel_err(y.cpu().numpy(), want) <= 1e-3
