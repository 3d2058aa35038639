"""The grouped f16-MFMA path of the expert ops for prefill-sized calls
(GGUF Q4_1, Q4_0, Q8_0, Q4_K, Q6_K codes, bf16 activations, at least 8 entries per
fired expert): the device table, the gathered-row layout (each expert's
entries padded to whole chunks), the prepared f16 rows and the grouped
kernel, through the C ABI.  Against the float64 oracle on the activations
the kernel saw; bar max|got - want| / max|want| <= 1e-3 (f32 output), as the
other grouped tests."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, _x_as, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3
SCHEMES = {"q4_1": 3, "q4_0": 2, "q8_0": 1, "q4_k": 7, "q6_k": 8}


@pytest.mark.parametrize("name", list(SCHEMES))
@pytest.mark.parametrize("shape", [(512, 1024, 200, 16), (300, 2048, 96, 4), (2000, 768, 130, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_grouped_matmul_mfma(ctx, orc, name, shape):
    """dequant_grouped_matmul with many rows per expert, a crowded expert and
    invalid indices (zero rows)."""
    import torch

    scheme = SCHEMES[name]
    rows, k, n, E = shape
    announce(f"grouped mfma {name} {shape}")
    rng = np.random.default_rng(rows + k + scheme)
    packed = orc.synth(scheme, rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[3] *= 300.0
    xt = _t(x).to(torch.bfloat16)
    idx = rng.integers(0, E, rows).astype(np.float32)
    idx[::5] = 1                                   # a crowded expert: several chunks
    bad = [7, 12, rows - 1]
    idx[bad[0]], idx[bad[1]], idx[bad[2]] = -1, 0.5, E
    y = ctx.grouped_matmul(xt, _t(packed), _t(idx), scheme, n, E)
    torch.cuda.synchronize()
    assert ctx.last_kernel.startswith(f"rlxq_moesk_{name}_"), ctx.last_kernel
    got = y.cpu().numpy()
    for r in bad:
        assert np.all(got[r] == 0.0), r
    ok = np.ones(rows, bool)
    ok[bad] = False
    want = orc.grouped_matmul_f64(scheme, xt.float().cpu().numpy()[ok], packed, idx[ok], n, E)
    assert rel_err(got[ok], want) <= TOL


@pytest.mark.parametrize("name", list(SCHEMES))
@pytest.mark.parametrize("tokens", [128, 256, 1024])
def test_moe_ffn_prefill_mfma(ctx, orc, name, tokens):
    """A MoE FFN at prefill sizes (64 experts, hidden 1024, intermediate 256,
    top-8 of softmax(N(0,1)) logits; 16, 32 and 128 entries per expert take
    chunks of 16, 32 and 64 rows): EXPAND_SWIGLU then COMBINE on the grouped
    MFMA kernels, against the float64 chain on the same bf16 intermediate."""
    import torch
    import rlxq

    scheme = SCHEMES[name]
    H, I, E, TOPK = 1024, 256, 64, 8
    announce(f"moe ffn prefill mfma {name} tokens={tokens}")
    rng = np.random.default_rng(tokens + scheme)
    gate_up = orc.synth(scheme, rng, E * 2 * I, H)
    down = orc.synth(scheme, rng, E * H, I)
    x = rng.standard_normal((tokens, H)).astype(np.float32)
    logits = rng.standard_normal((tokens, E)).astype(np.float32)
    xt = _t(x).to(torch.bfloat16)
    xv = xt.float().cpu().numpy()
    ids, probs = ctx.moe_route(_t(logits), TOPK, True)
    act = ctx.moe_grouped(xt, _t(gate_up), ids, probs, scheme, rlxq.MOE_EXPAND_SWIGLU, 2 * I, E,
                          y_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    mt = {128: 1, 256: 2, 1024: 4}[tokens]
    assert ctx.last_kernel.startswith(f"rlxq_moesk_{name}_mt{mt}_") and ctx.last_kernel.endswith("_sw"), ctx.last_kernel
    y = ctx.moe_grouped(act, _t(down), ids, probs, scheme, rlxq.MOE_COMBINE, H, E)
    torch.cuda.synchronize()
    flat = ids.cpu().numpy().ravel().astype(np.float32)
    sel = np.arange(0, tokens * TOPK, 7)           # a sample of the entries (the f64 chain is slow)
    gu = orc.grouped_matmul_f64(scheme, np.repeat(xv, TOPK, axis=0)[sel], gate_up, flat[sel], 2 * I, E)
    g, u = gu[:, :I], gu[:, I:]
    assert rel_err(act.float().cpu().numpy()[sel], g / (1.0 + np.exp(-g)) * u) <= 1e-2   # bf16 output
    rows = np.arange(0, tokens, 9)
    av = act.float().cpu().numpy()
    ent = (rows[:, None] * TOPK + np.arange(TOPK)[None, :]).ravel()
    dn = orc.grouped_matmul_f64(scheme, av[ent], down, flat[ent], H, E).reshape(len(rows), TOPK, H)
    want = np.einsum("rk,rkh->rh", probs.cpu().numpy()[rows].astype(np.float64), dn)
    assert rel_err(y.cpu().numpy()[rows], want) <= TOL


@pytest.mark.parametrize("route_kernel", ["sk", "lds"])
def test_mfma_path_matches_gemv_path(ctx, orc, monkeypatch, route_kernel):
    """The same call through the grouped MFMA kernel and through the
    LDS-record GEMV (RLXQ_MOE_KERNEL): both within the bar, and within 2e-3
    of each other; a skewed routing (one expert takes most entries)."""
    import torch

    monkeypatch.setenv("RLXQ_MOE_KERNEL", route_kernel)
    rows, k, n, E = 640, 1536, 320, 8
    rng = np.random.default_rng(99)
    packed = orc.synth_q4_1(rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    xt = _t(x).to(torch.bfloat16)
    idx = np.where(rng.uniform(size=rows) < 0.7, 5, rng.integers(0, E, rows)).astype(np.float32)
    y = ctx.grouped_matmul(xt, _t(packed), _t(idx), 3, n, E)
    torch.cuda.synchronize()
    assert ctx.last_kernel.startswith("rlxq_moesk_" if route_kernel == "sk" else "rlxq_moe_gemv_"), ctx.last_kernel
    want = orc.grouped_matmul_f64(3, xt.float().cpu().numpy(), packed, idx, n, E)
    assert rel_err(y.cpu().numpy(), want) <= TOL


def test_mfma_path_forced_small_and_repeated(ctx, orc, monkeypatch):
    """Forced onto the MFMA path at a decode-like size (fewer than 8 entries
    per expert, partial chunks everywhere), twice in a row on one stream with
    different routings (the gathered layout is rebuilt per call)."""
    import torch

    monkeypatch.setenv("RLXQ_MOE_KERNEL", "sk")
    rows, k, n, E = 37, 1024, 72, 16
    rng = np.random.default_rng(5)
    packed = orc.synth_q4_1(rng, E * n, k)
    bt = _t(packed)
    for call in range(2):
        x = rng.standard_normal((rows, k)).astype(np.float32)
        xt = _t(x).to(torch.bfloat16)
        idx = rng.integers(0, E, rows).astype(np.float32)
        y = ctx.grouped_matmul(xt, bt, _t(idx), 3, n, E)
        torch.cuda.synchronize()
        assert ctx.last_kernel.startswith("rlxq_moesk_q4_1_mt1_"), ctx.last_kernel
        want = orc.grouped_matmul_f64(3, xt.float().cpu().numpy(), packed, idx, n, E)
        assert rel_err(y.cpu().numpy(), want) <= TOL, call


@pytest.mark.parametrize("cfg", ["1,2,4", "1,4,2", "1,8,2", "2,2,3", "2,4,2", "2,8,1", "4,2,2", "4,4,1"])
@pytest.mark.parametrize("sw", [False, True])
def test_every_grouped_mfma_variant(ctx, orc, monkeypatch, cfg, sw):
    """Every compiled chunk/tile/ring variant "MT,NT,D" of the grouped MFMA
    kernel (RLXQ_MOE_SK), plain and SwiGLU, on Q4_1 with partial chunks and
    a column count that is no multiple of the tile width."""
    import torch
    import rlxq

    monkeypatch.setenv("RLXQ_MOE_KERNEL", "sk")
    monkeypatch.setenv("RLXQ_MOE_SK", cfg)
    mt, nt, d = (int(v) for v in cfg.split(","))
    T, H, n, E, TOPK = 40, 512, 2 * 72, 6, 3
    announce(f"grouped mfma variant {cfg} sw={sw}")
    rng = np.random.default_rng(mt * 10 + nt + int(sw))
    bank = orc.synth_q4_1(rng, E * n, H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = _t(x).to(torch.bfloat16)
    ids = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(T)]).astype(np.int32)
    probs = rng.uniform(0.1, 0.5, (T, TOPK)).astype(np.float32)
    mode = rlxq.MOE_EXPAND_SWIGLU if sw else rlxq.MOE_EXPAND
    y = ctx.moe_grouped(xt, _t(bank), _t(ids), _t(probs), 3, mode, n, E)
    torch.cuda.synchronize()
    assert ctx.last_kernel == f"rlxq_moesk_q4_1_mt{mt}_nt{nt}_d{d}" + ("_sw" if sw else ""), ctx.last_kernel
    gu = orc.grouped_matmul_f64(3, np.repeat(xt.float().cpu().numpy(), TOPK, axis=0), bank,
                                ids.ravel().astype(np.float32), n, E)
    want = gu[:, :n // 2] / (1.0 + np.exp(-gu[:, :n // 2])) * gu[:, n // 2:] if sw else gu
    assert rel_err(y.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("fmt", ["mlx4_f32", "mlx4_bf16", "mlx8_bf16", "mxfp4"])
@pytest.mark.parametrize("forced", [False, True])
def test_grouped_mfma_mlx_and_mxfp4(ctx, orc, monkeypatch, fmt, forced):
    """Op::DequantGroupedMatMulMlx at prefill sizes on the grouped MFMA
    kernel: MLX affine 4/8-bit banks with [E, N, K / group] scale and bias
    slabs (group 64) and MXFP4 banks with E8M0 bytes [E, N, K / 32], every
    row's expert slab picked per chunk; against the oracle row by row."""
    import torch
    import rlxq

    if forced:
        monkeypatch.setenv("RLXQ_MOE_KERNEL", "sk")
    rows, k, n, E, group = (37, 512, 200, 3, 64) if forced else (160, 1024, 136, 4, 64)
    announce(f"grouped mfma {fmt} forced={forced} rows={rows}")
    rng = np.random.default_rng(71 + rows + len(fmt))
    x = rng.standard_normal((rows, k)).astype(np.float32)
    xt, xv = _x_as(x, "bf16")
    idx = rng.integers(0, E, rows).astype(np.float32)
    want = np.zeros((rows, n))
    if fmt == "mxfp4":
        codes, eb = orc.synth_mxfp4(rng, E * n, k)
        y = ctx.grouped_matmul(xt, _t(codes), _t(idx), rlxq.MLX_MXFP4, n, E, scales=_t(eb))
        for r in range(rows):
            sl = slice(int(idx[r]) * n, (int(idx[r]) + 1) * n)
            want[r] = orc.mxfp4_matmul_f64(xv[r:r + 1], codes[sl], eb[sl], n)[0]
        name, tol = "mxfp4", 1e-5
    else:
        bits = 4 if fmt.startswith("mlx4") else 8
        codes = rng.integers(0, 2 ** 32, (E * n, k * bits // 32), dtype=np.uint32)
        sc = rng.uniform(0.01, 0.1, (E * n, k // group)).astype(np.float32)
        bi = rng.uniform(-0.5, 0.1, (E * n, k // group)).astype(np.float32)
        if fmt.endswith("bf16"):
            sc = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(sc))
            bi = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(bi))
            st, bt = _t(sc).to(torch.bfloat16), _t(bi).to(torch.bfloat16)
        else:
            st, bt = _t(sc), _t(bi)
        scheme = rlxq.MLX_AFFINE4 if bits == 4 else rlxq.MLX_AFFINE8
        y = ctx.grouped_matmul(xt, _t(codes.view(np.uint8)), _t(idx), scheme, n, E, group=group, scales=st,
                               biases=bt)
        for r in range(rows):
            sl = slice(int(idx[r]) * n, (int(idx[r]) + 1) * n)
            want[r] = orc.mlx_matmul_f64(xv[r:r + 1], codes[sl], sc[sl], bi[sl], n, bits, group)[0]
        name, tol = f"mlx{bits}", TOL
    torch.cuda.synchronize()
    assert ctx.last_kernel.startswith(f"rlxq_moesk_{name}_"), ctx.last_kernel
    got = y.cpu().numpy()
    for r in range(rows):
        assert rel_err(got[r:r + 1], want[r:r + 1]) <= tol, (fmt, r)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("slab", ["f32", "bf16"])
def test_grouped_mfma_mlx_every_group_and_slab(ctx, orc, monkeypatch, bits, group, slab):
    """The per-expert slab offset e * N * (K / group) and the slab element
    size on every group size and slab dtype of both bit widths: nine experts,
    one of them crowded (half the rows), so several chunks of the grouped MFMA
    kernel read the slabs of different experts."""
    import torch
    import rlxq

    monkeypatch.setenv("RLXQ_MOE_KERNEL", "sk")
    rows, k, n, E = 96, 768, 72, 9
    announce(f"grouped mfma mlx{bits} group={group} slab={slab}")
    rng = np.random.default_rng(bits * 1000 + group + len(slab))
    x = rng.standard_normal((rows, k)).astype(np.float32)
    xt, xv = _x_as(x, "bf16")
    idx = rng.integers(0, E, rows)
    idx[::2] = 5
    idx = idx.astype(np.float32)
    codes = rng.integers(0, 2 ** 32, (E * n, k * bits // 32), dtype=np.uint32)
    sc = rng.uniform(0.01, 0.1, (E * n, k // group)).astype(np.float32)
    bi = rng.uniform(-0.5, 0.1, (E * n, k // group)).astype(np.float32)
    if slab == "bf16":
        sc = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(sc))
        bi = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(bi))
        st, bt = _t(sc).to(torch.bfloat16), _t(bi).to(torch.bfloat16)
    else:
        st, bt = _t(sc), _t(bi)
    scheme = rlxq.MLX_AFFINE4 if bits == 4 else rlxq.MLX_AFFINE8
    y = ctx.grouped_matmul(xt, _t(codes.view(np.uint8)), _t(idx), scheme, n, E, group=group, scales=st, biases=bt)
    torch.cuda.synchronize()
    assert ctx.last_kernel.startswith(f"rlxq_moesk_mlx{bits}_"), ctx.last_kernel
    got = y.cpu().numpy()
    for r in range(rows):
        sl = slice(int(idx[r]) * n, (int(idx[r]) + 1) * n)
        want = orc.mlx_matmul_f64(xv[r:r + 1], codes[sl], sc[sl], bi[sl], n, bits, group)
        assert rel_err(got[r:r + 1], want) <= TOL, (r, int(idx[r]))


@pytest.mark.parametrize("path", ["grouped", "dense"])
def test_mlx8_small_scales_on_f16_kernels(ctx, orc, monkeypatch, path):
    """MLX 8-bit group scales near 1e-5 (a group of small weights: f16
    subnormals if rounded unscaled) on the f16 MFMA kernels, which hold the
    scales and biases times 2^8: within the 1e-3 bar, grouped and dense."""
    import torch
    import rlxq

    rows, k, n, E, group = 48, 1024, 96, 3, 64
    announce(f"mlx8 small scales {path}")
    rng = np.random.default_rng(404)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    xt, xv = _x_as(x, "bf16")
    codes = rng.integers(0, 2 ** 32, (E * n, k // 4), dtype=np.uint32)
    sc = rng.uniform(5e-6, 2e-5, (E * n, k // group)).astype(np.float32)
    bi = rng.uniform(-2e-3, 0.0, (E * n, k // group)).astype(np.float32)
    if path == "grouped":
        monkeypatch.setenv("RLXQ_MOE_KERNEL", "sk")
        idx = (np.arange(rows) % E).astype(np.float32)
        y = ctx.grouped_matmul(xt, _t(codes.view(np.uint8)), _t(idx), rlxq.MLX_AFFINE8, n, E, group=group,
                               scales=_t(sc), biases=_t(bi))
        torch.cuda.synchronize()
        assert ctx.last_kernel.startswith("rlxq_moesk_mlx8_"), ctx.last_kernel
        got = y.cpu().numpy()
        for r in range(rows):
            sl = slice(int(idx[r]) * n, (int(idx[r]) + 1) * n)
            want = orc.mlx_matmul_f64(xv[r:r + 1], codes[sl], sc[sl], bi[sl], n, 8, group)
            assert rel_err(got[r:r + 1], want) <= TOL, r
    else:
        sl = slice(0, n)
        y = ctx.dequant_matmul(xt, _t(codes[sl].view(np.uint8)), rlxq.MLX_AFFINE8, n, group=group,
                               scales=_t(sc[sl]), biases=_t(bi[sl]))
        torch.cuda.synchronize()
        assert ctx.last_kernel.startswith("rlxq_skinny"), ctx.last_kernel
        want = orc.mlx_matmul_f64(xv, codes[sl], sc[sl], bi[sl], n, 8, group)
        assert rel_err(y.cpu().numpy(), want) <= TOL
