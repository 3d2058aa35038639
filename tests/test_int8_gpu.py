"""Parity of the int8 paths against the CPU oracle, through the C ABI.

W8A8 (per-row int8 activations, crates/rlx-quant-calib/src/bitnet.rs:76-93,
times per-channel int8 weights, crates/rlx-kimi-k3/src/common.rs:466-482):
the activation quantiser is bit-exact, and so is the GEMM output, since int32
accumulation is exact and the epilogue rounds (float(acc) * sx) * sw in the
same order as the oracle.

Int8Block (crates/rlx-kimi-k3/examples/int8_kernel.rs:59-89, y = x . ((Wq - zp) * s)
with f32 activations): within max|got - want| / max|want| <= 1e-3 of the
float64 contraction (1e-2 for bf16 outputs)."""
import os

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_BF16 = 1e-2


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rel_err(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


def _x(rng, m, k, xdt):
    """Activations ~N(0,1) as the kernel sees them, and the same values in f32."""
    import torch

    x32 = rng.standard_normal((m, k)).astype(np.float32)
    if xdt == "bf16":
        xt = _t(x32).to(torch.bfloat16)
        return xt, xt.float().cpu().numpy()
    return _t(x32), x32


def _w8(rng, k, n):
    w = rng.standard_normal((k, n)).astype(np.float32) * np.float32(0.05)
    return w


# ---------------------------------------------------------------- quantiser
@pytest.mark.parametrize("m,k", [(1, 64), (3, 1000), (17, 4096), (64, 12288), (2, 12800), (5, 4104)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_quantize_act_int8_bit_exact(ctx, orc, rng, m, k, xdt):
    import torch

    announce(f"quantize_act_int8 m={m} k={k} x={xdt}")
    xt, xv = _x(rng, m, k, xdt)
    q, s = ctx.quantize_act_int8(xt)
    torch.cuda.synchronize()
    qw, sw = orc.quantize_act_int8(xv)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sw.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), qw)


def test_quantize_act_int8_special_rows(ctx, orc):
    """An all-zero row (scale 1), exact ties at .5 (half away from zero), one
    dominant element, negative extremes."""
    import torch

    k = 256
    x = np.zeros((4, k), np.float32)
    x[1, :] = np.linspace(-127.0, 127.0, k, dtype=np.float32)      # amax 127 -> s = 1, exact ties
    x[1, :8] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]
    x[2, 0] = 1e30
    x[2, 1:] = 1e-3
    x[3, :] = -np.arange(k, dtype=np.float32)
    announce("quantize_act_int8 special rows")
    q, s = ctx.quantize_act_int8(_t(x))
    torch.cuda.synchronize()
    qw, sw = orc.quantize_act_int8(x)
    assert sw[0] == 1.0 and np.all(qw[0] == 0)
    assert list(qw[1, :6]) == [1, -1, 2, -2, 3, -3]
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sw.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), qw)


# ---------------------------------------------------------------- W8A8 GEMM
def _w8a8_case(ctx, orc, rng, m, k, n, xdt="f32", ydt="f32"):
    import torch

    xt, xv = _x(rng, m, k, xdt)
    qw, sw = orc.quantize_int8_col(_w8(rng, k, n))
    y = ctx.w8a8_gemm(xt, _t(qw), _t(sw), n, y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    qx, sx = orc.quantize_act_int8(xv)
    want = orc.w8a8_matmul(qx, sx, qw, sw)
    if ydt == "bf16":
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        want = orc.f32_to_bf16_bits(want)
    else:
        got = y.cpu().numpy()
    return got, want


@pytest.mark.parametrize("m,k,n", [(1, 64, 16), (5, 256, 128), (64, 512, 272), (128, 1024, 256),
                                   (300, 4096, 1024), (129, 80, 144)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_w8a8_bit_exact(ctx, orc, rng, m, k, n, xdt):
    announce(f"w8a8 m={m} k={k} n={n} x={xdt}")
    got, want = _w8a8_case(ctx, orc, rng, m, k, n, xdt)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{np.count_nonzero(got != want)} of {got.size} differ"


def test_w8a8_bf16_output_bit_exact(ctx, orc, rng):
    announce("w8a8 bf16 out m=200 k=768 n=512")
    got, want = _w8a8_case(ctx, orc, rng, 200, 768, 512, "bf16", "bf16")
    assert np.array_equal(got, want)


W8A8_CFGS = ["m128n128k64w22", "m128n128k128w22", "m256n128k64w22", "m128n256k64w22", "m256n256k64w24",
             "m128n128k128w22_p2", "m256n256k128w24", "m256n256k64w24_kf", "m256n256k128w24_kf"]


@pytest.mark.parametrize("cfg", W8A8_CFGS)
def test_every_w8a8_tiling(ctx, orc, rng, cfg, monkeypatch):
    """Every compiled tiling, on a ragged shape (M, N, K not multiples of the
    tile; the _kf tilings, which need K to be a multiple of their K step, on
    K = 640 or 768 with M and N ragged)."""
    monkeypatch.setenv("RLXQ_W8A8_CFG", cfg)
    k = (768 if "k128" in cfg else 640) if cfg.endswith("_kf") else 592
    announce(f"w8a8 tiling {cfg} m=333 k={k} n=400")
    got, want = _w8a8_case(ctx, orc, rng, 333, k, 400)
    assert ctx.last_kernel == f"rlxq_w8a8_{cfg}"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_w8a8_whole_step_tiling_refuses_other_k(ctx, monkeypatch):
    """A _kf tiling forced on a K that is not a multiple of its K step is
    refused before any launch."""
    import torch
    import rlxq

    monkeypatch.setenv("RLXQ_W8A8_CFG", "m256n256k128w24_kf")
    x = torch.zeros((4, 576), device="cuda")
    wq = torch.zeros((576, 32), dtype=torch.int8, device="cuda")
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.w8a8_gemm(x, wq, torch.ones((32,), device="cuda"), 32)
    assert e.value.status == rlxq.E_SHAPE


@pytest.mark.parametrize("k,n", [(4096, 24576), (12288, 4096)], ids=lambda s: str(s))
def test_w8a8_prefill_config_sampled(ctx, orc, k, n):
    """The prefill W8A8 shapes at full size (M=4096; Qwen3-8B gate|up
    4096 -> 24576 and down 12288 -> 4096): the oracle checks a sample of 64
    rows x 256 columns bit for bit, plus the activation quantiser on every
    row."""
    import torch

    m = 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    announce(f"w8a8 prefill m={m} k={k} n={n}")
    x = torch.randn((m, k), device="cuda", generator=g, dtype=torch.float32).to(torch.bfloat16)
    wq = torch.randint(-127, 128, (k, n), device="cuda", generator=g, dtype=torch.int8)
    sw = torch.rand((n,), device="cuda", generator=g) * 0.01 + 1e-4
    y = ctx.w8a8_gemm(x, wq, sw, n, y_dtype=torch.bfloat16)
    q, s = ctx.quantize_act_int8(x)
    torch.cuda.synchronize()
    xv = x.float().cpu().numpy()
    qx, sx = orc.quantize_act_int8(xv)
    assert np.array_equal(q.cpu().numpy(), qx)
    rs = np.random.default_rng(1)
    rows = np.sort(rs.choice(m, 64, replace=False))
    cols = np.sort(rs.choice(n, 256, replace=False))
    wsub = wq[:, torch.from_numpy(cols).cuda()].contiguous().cpu().numpy()
    want = orc.w8a8_matmul(qx[rows], sx[rows], wsub, sw.cpu().numpy()[cols])
    got = y.view(torch.int16).cpu().numpy().view(np.uint16)[np.ix_(rows, cols)]
    assert np.array_equal(got, orc.f32_to_bf16_bits(want))


def test_w8a8_host_checks(ctx):
    import torch
    import rlxq

    x = torch.zeros((4, 64), device="cuda")
    wq = torch.zeros((64, 32), dtype=torch.int8, device="cuda")
    sw = torch.ones((32,), device="cuda")
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.w8a8_gemm(x[:, :40].contiguous(), wq[:40], sw, 32)
    assert e.value.status == rlxq.E_ALIGN
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.w8a8_gemm(x, wq[:, :24].contiguous(), sw[:24], 24)
    assert e.value.status == rlxq.E_ALIGN
    y = ctx.w8a8_gemm(x[:0], wq, sw, 32)
    assert y.shape == (0, 32)


# -------------------------------------------------------------- Int8Block
def _i8b_case(ctx, orc, rng, m, k, n, xdt="f32", ydt="f32", zp=False):
    import torch
    import rlxq

    xt, xv = _x(rng, m, k, xdt)
    qw, sw = orc.quantize_int8_col(_w8(rng, k, n))
    zpv = (rng.standard_normal(n) * 3).astype(np.float32) if zp else None
    y = ctx.dequant_matmul(xt, _t(qw), rlxq.INT8_BLOCK, n, group=k, scales=_t(sw),
                           biases=_t(zpv) if zp else None,
                           y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), orc.int8_block_matmul_f64(xv, qw, sw, zpv)


@pytest.mark.parametrize("m,k,n", [(1, 128, 16), (1, 4096, 4096), (3, 1000, 272), (16, 2048, 1024),
                                   (17, 512, 256), (33, 300, 528), (64, 4096, 1536), (100, 640, 320)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_int8_block(ctx, orc, rng, m, k, n, xdt):
    announce(f"int8_block m={m} k={k} n={n} x={xdt}")
    got, want = _i8b_case(ctx, orc, rng, m, k, n, xdt)
    assert rel_err(got, want) <= TOL_F32


@pytest.mark.parametrize("m,k,n", [(1, 4096, 512), (8, 256, 96), (64, 4096, 256)])
def test_int8_block_zero_point(ctx, orc, rng, m, k, n):
    announce(f"int8_block zp m={m} k={k} n={n}")
    got, want = _i8b_case(ctx, orc, rng, m, k, n, zp=True)
    assert rel_err(got, want) <= TOL_F32


def test_int8_block_bf16_output(ctx, orc, rng):
    announce("int8_block bf16 out m=8 k=2048 n=512")
    got, want = _i8b_case(ctx, orc, rng, 8, 2048, 512, ydt="bf16")
    assert rel_err(got, want) <= TOL_BF16


def test_int8_block_kimi_sweep_shape(ctx, orc, rng):
    """The reference's int8_kernel sweep, M in {1, 4, 16, 64}, on a q_proj-sized
    weight (K=7168, N=12288 here), checked on a column sample."""
    import torch
    import rlxq

    k, n = 7168, 12288
    g = torch.Generator(device="cuda").manual_seed(0)
    wq = torch.randint(-127, 128, (k, n), device="cuda", generator=g, dtype=torch.int8)
    sw = torch.rand((n,), device="cuda", generator=g) * 0.01 + 1e-4
    cols = np.sort(np.random.default_rng(2).choice(n, 192, replace=False))
    wsub = wq[:, torch.from_numpy(cols).cuda()].contiguous().cpu().numpy()
    for m in (1, 4, 16, 64):
        announce(f"int8_block kimi m={m}")
        x = torch.randn((m, k), device="cuda", generator=g)
        y = ctx.dequant_matmul(x, wq, rlxq.INT8_BLOCK, n, group=k, scales=sw)
        torch.cuda.synchronize()
        want = orc.int8_block_matmul_f64(x.cpu().numpy(), wsub, sw.cpu().numpy()[cols])
        assert rel_err(y.cpu().numpy()[:, cols], want) <= TOL_F32, m


def test_int8_block_host_checks(ctx):
    import torch
    import rlxq

    x = torch.zeros((2, 64), device="cuda")
    wq = torch.zeros((64, 32), dtype=torch.int8, device="cuda")
    sw = torch.ones((32,), device="cuda")
    for kw, code in [(dict(scales=None), rlxq.E_NULL), (dict(scales=sw, group=32), rlxq.E_SCHEME),
                     (dict(scales=sw.to(torch.bfloat16)), rlxq.E_DTYPE)]:
        kw.setdefault("group", 64)
        with pytest.raises(rlxq.RlxqError) as e:
            ctx.dequant_matmul(x, wq, rlxq.INT8_BLOCK, 32, **kw)
        assert e.value.status == code, kw
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul(x, wq[:, :24].contiguous(), rlxq.INT8_BLOCK, 24, group=64, scales=sw[:24])
    assert e.value.status == rlxq.E_ALIGN


@pytest.mark.parametrize("m,k,n", [(1, 12288, 4096), (2, 1001, 1040), (3, 3000, 2064), (4, 4096, 24576 // 8),
                                   (1, 5, 16)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
@pytest.mark.parametrize("zp", [False, True])
def test_int8_block_decode_gemv(ctx, orc, rng, monkeypatch, m, k, n, xdt, zp):
    """The streaming GEMV (M = 1 by default, M <= 4 when forced; K slices of
    at most 1024 rows, ragged column groups) and the MFMA kernel both meet
    the f32 bar."""
    announce(f"int8_block gemv m={m} k={k} n={n} x={xdt} zp={zp}")
    monkeypatch.setenv("RLXQ_I8B_GEMV", "1")
    seed = rng.integers(1 << 30)
    got, want = _i8b_case(ctx, orc, np.random.default_rng(seed), m, k, n, xdt, zp=zp)
    assert ctx.last_kernel.startswith("rlxq_i8bv_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL_F32
    monkeypatch.setenv("RLXQ_I8B_MFMA", "1")
    got2, want2 = _i8b_case(ctx, orc, np.random.default_rng(seed), m, k, n, xdt, zp=zp)
    assert ctx.last_kernel.startswith("rlxq_i8b_"), ctx.last_kernel
    assert rel_err(got2, want2) <= TOL_F32
