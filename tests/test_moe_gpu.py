"""Parity of the grouped-expert path (device routing table + grouped GEMV),
the router and SwiGLU, against the CPU oracle, through the C ABI.  Bar:
max|got - want| / max|want| <= 1e-3 with f32 output (the reference's own
bars are 1e-2 grouped and 2e-2 MoE accumulate,
crates/rlx-unlimited-ocr/tests/quant_parity_backends.rs:301,424)."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _ref_input, _ref_weight, _t, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3

# (rows, k, n, experts), quant_parity_backends.rs:260-266
GROUPED_SHAPES = [(4, 256, 128, 3), (1, 1280, 896, 8), (128, 1280, 896, 64), (128, 896, 1280, 64)]


def _bank(orc, scheme, n, k, e_count, seed0=0.3, step=1.0):
    bank = np.concatenate([_ref_weight(n, k, seed0 + e * step) for e in range(e_count)])
    return orc.quantize(scheme, bank)


@pytest.mark.parametrize("scheme", [1, 2, 3])
@pytest.mark.parametrize("shape", GROUPED_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_grouped_reference_shapes(ctx, orc, scheme, shape):
    """check_grouped: bank [E, N, K], row r uses expert (7r + 1) % E."""
    import torch

    rows, k, n, E = shape
    announce(f"grouped scheme={scheme} {shape}")
    x = _ref_input(rows, k)
    packed = _bank(orc, scheme, n, k, E)
    idx = np.array([(r * 7 + 1) % E for r in range(rows)], np.float32)
    y = ctx.grouped_matmul(_t(x), _t(packed), _t(idx), scheme, n, E)
    torch.cuda.synchronize()
    want = orc.grouped_matmul_f64(scheme, x, packed, idx, n, E)
    assert rel_err(y.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_grouped_many_rows_per_expert(ctx, orc, xdt):
    """Skewed routing: one expert takes most rows (several MT chunks)."""
    import torch

    rows, k, n, E = 37, 512, 300, 5
    announce(f"grouped skewed x={xdt}")
    rng = np.random.default_rng(1)
    packed = orc.synth_q4_1(rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    idx = np.where(np.arange(rows) % 5 == 0, 4, 2).astype(np.float32)
    xt = _t(x) if xdt == "f32" else _t(x).to(torch.bfloat16)
    y = ctx.grouped_matmul(xt, _t(packed), _t(idx), 3, n, E)
    torch.cuda.synchronize()
    xv = xt.float().cpu().numpy()
    assert rel_err(y.cpu().numpy(), orc.grouped_matmul_f64(3, xv, packed, idx, n, E)) <= TOL


def test_grouped_invalid_index_gives_zero_row(ctx, orc):
    import torch

    rows, k, n, E = 6, 256, 64, 4
    announce("grouped invalid index")
    rng = np.random.default_rng(2)
    packed = orc.synth_q8_0(rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    idx = np.array([0, 1.5, 3, 4, -1, 2], np.float32)
    y = ctx.grouped_matmul(_t(x), _t(packed), _t(idx), 1, n, E)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for r in (1, 3, 4):
        assert np.all(got[r] == 0.0)
    for r in (0, 2, 5):
        want = orc.matmul_f64(1, x[r:r + 1], packed[int(idx[r]) * n:(int(idx[r]) + 1) * n], n)
        assert rel_err(got[r:r + 1], want) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
def test_grouped_mlx_bf16_slabs(ctx, orc, bits):
    """Op::DequantGroupedMatMulMlx: bf16 scale/bias slabs [E, N, K/group]."""
    import torch
    import rlxq

    rows, k, n, E, group = 9, 256, 96, 3, 64
    announce(f"grouped mlx bits={bits}")
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (E * n, k)).astype(np.uint32)
    wq = orc.mlx_pack(codes, bits)
    sc = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(rng.uniform(0.01, 0.1, (E * n, k // group))))
    bi = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(rng.uniform(-0.5, 0.1, (E * n, k // group))))
    x = rng.standard_normal((rows, k)).astype(np.float32)
    idx = (np.arange(rows) % E).astype(np.float32)
    scheme = rlxq.MLX_AFFINE4 if bits == 4 else rlxq.MLX_AFFINE8
    y = ctx.grouped_matmul(_t(x), _t(wq.view(np.uint8)), _t(idx), scheme, n, E, group=group,
                           scales=_t(sc).to(torch.bfloat16), biases=_t(bi).to(torch.bfloat16))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = np.zeros((rows, n))
    for r in range(rows):
        e = int(idx[r])
        sl = slice(e * n, (e + 1) * n)
        want[r] = orc.mlx_matmul_f64(x[r:r + 1], wq[sl], sc[sl], bi[sl], n, bits, group)[0]
    assert rel_err(got, want) <= TOL


def _moe_logits(rows, ne):
    """quant_parity_backends.rs:350-352."""
    i = np.arange(rows * ne, dtype=np.float32)
    return ((np.sin(i * np.float32(0.29)) * np.float32(2.0)) + (i // ne).astype(np.float32) * np.float32(0.05)).reshape(rows, ne)


@pytest.mark.parametrize("scheme", [1, 2])
@pytest.mark.parametrize("top_k", [1, 6])
def test_moe_accumulate_reference(ctx, orc, scheme, top_k):
    """check_moe_accumulate: softmax -> top-k -> per-slot grouped matmul ->
    probability-weighted sum (64 rows, K=1280, N=896, E=64), through the
    device router and the COMBINE mode."""
    import torch
    import rlxq

    ROWS, K, N, NE = 64, 1280, 896, 64
    announce(f"moe accumulate scheme={scheme} k={top_k}")
    x = _ref_input(ROWS, K)
    packed = _bank(orc, scheme, N, K, NE, 0.3, 0.11)
    logits = _moe_logits(ROWS, NE)
    ids, probs = ctx.moe_route(_t(logits), top_k, False)
    torch.cuda.synchronize()
    oids, oprobs = orc.topk_softmax(logits, top_k)
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert np.allclose(probs.cpu().numpy(), oprobs, rtol=1e-5, atol=1e-7)
    x_exp = np.repeat(x, top_k, axis=0)
    y = ctx.moe_grouped(_t(x_exp), _t(packed), ids, probs, scheme, rlxq.MOE_COMBINE, N, NE)
    torch.cuda.synchronize()
    want = orc.moe_f64(scheme, x, packed, oids, probs.cpu().numpy(), N, NE)
    assert rel_err(y.cpu().numpy(), want) <= TOL
    y_exp = ctx.moe_grouped(_t(x), _t(packed), ids, probs, scheme, rlxq.MOE_EXPAND, N, NE)
    torch.cuda.synchronize()
    want_exp = orc.grouped_matmul_f64(scheme, x_exp, packed, oids.ravel().astype(np.float32), N, NE)
    assert rel_err(y_exp.cpu().numpy(), want_exp) <= TOL


def test_moe_ffn_config5(ctx, orc):
    """Config 5: 128 experts, hidden 2048, expert intermediate 768 (gate|up
    2048->1536 fused, down 768->2048), top-8 of softmax(N(0,1)) logits, 16
    tokens, Q4_1; renormalised top-k (norm_topk_prob)."""
    import torch
    import rlxq

    T, H, I, E, TOPK = 16, 2048, 768, 128, 8
    announce("moe ffn config 5")
    rng = np.random.default_rng(0)
    gate_up = orc.synth_q4_1(rng, E * 2 * I, H)
    down = orc.synth_q4_1(rng, E * H, I)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    xt = _t(x).to(torch.bfloat16)
    xv = xt.float().cpu().numpy()
    ids, probs = ctx.moe_route(_t(logits), TOPK, True)
    gu = ctx.moe_grouped(xt, _t(gate_up), ids, probs, rlxq.GGUF_Q4_1, rlxq.MOE_EXPAND, 2 * I, E)
    act = ctx.swiglu(gu, I, out_dtype=torch.bfloat16)
    y = ctx.moe_grouped(act, _t(down), ids, probs, rlxq.GGUF_Q4_1, rlxq.MOE_COMBINE, H, E)
    torch.cuda.synchronize()
    oids, oprobs = orc.topk_softmax(logits, TOPK, renorm=True)
    assert np.array_equal(ids.cpu().numpy(), oids)
    # oracle chain in float64 on the same intermediate rounding points
    gu_w = orc.grouped_matmul_f64(3, np.repeat(xv, TOPK, axis=0), gate_up, oids.ravel().astype(np.float32), 2 * I, E)
    assert rel_err(gu.cpu().numpy(), gu_w) <= TOL
    g, u = gu.cpu().numpy()[:, :I].astype(np.float64), gu.cpu().numpy()[:, I:].astype(np.float64)
    act_w = g / (1.0 + np.exp(-g)) * u
    assert rel_err(act.float().cpu().numpy(), act_w) <= 1e-2  # bf16 output
    act_v = act.float().cpu().numpy()
    want = np.zeros((T, H))
    dn = orc.grouped_matmul_f64(3, act_v, down, oids.ravel().astype(np.float32), H, E)
    pv = probs.cpu().numpy()
    for r in range(T):
        for j in range(TOPK):
            want[r] += pv[r, j] * dn[r * TOPK + j]
    assert rel_err(y.cpu().numpy(), want) <= TOL


def test_route_matches_oracle(ctx, orc):
    import torch

    rng = np.random.default_rng(5)
    for (rows, E, k, renorm) in [(16, 128, 8, True), (3, 7, 7, False), (33, 1024, 2, False), (1, 64, 1, True)]:
        announce(f"route rows={rows} E={E} k={k}")
        logits = rng.standard_normal((rows, E)).astype(np.float32) * 3
        ids, probs = ctx.moe_route(_t(logits), k, renorm)
        torch.cuda.synchronize()
        oids, oprobs = orc.topk_softmax(logits, k, renorm)
        assert np.array_equal(ids.cpu().numpy(), oids)
        assert np.allclose(probs.cpu().numpy(), oprobs, rtol=1e-5, atol=1e-7)


def test_swiglu(ctx):
    import torch

    rng = np.random.default_rng(6)
    gu = rng.standard_normal((5, 2 * 300)).astype(np.float32) * 4
    out = ctx.swiglu(_t(gu), 300)
    torch.cuda.synchronize()
    g, u = gu[:, :300].astype(np.float64), gu[:, 300:].astype(np.float64)
    assert np.allclose(out.cpu().numpy(), g / (1 + np.exp(-g)) * u, rtol=1e-5, atol=1e-6)


def test_device_matmul_grouped_session(orc):
    import torch
    import rlxq

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    announce("DeviceMatmul grouped session")
    dm = rlxq.DeviceMatmul(0)
    rng = np.random.default_rng(8)
    m, k, n, E = 12, 1280, 896, 8
    packed = orc.synth_q8_0(rng, E * n, k).ravel()
    x = rng.standard_normal((m, k)).astype(np.float32)
    idx = (np.arange(m) * 3 % E).astype(np.float32)
    y = dm.grouped_matmul(x, packed, idx, m, k, n, E, rlxq.GGUF_Q8_0).reshape(m, n)
    assert rel_err(y, orc.grouped_matmul_f64(1, x, packed, idx, n, E)) <= TOL
    bad = idx.copy()
    bad[3] = E
    with pytest.raises(rlxq.RlxqError) as e:
        dm.grouped_matmul(x, packed, bad, m, k, n, E, rlxq.GGUF_Q8_0)
    assert e.value.status == rlxq.E_INDEX
    with pytest.raises(rlxq.RlxqError) as e:
        dm.grouped_matmul(x, packed, idx[:5], m, k, n, E, rlxq.GGUF_Q8_0)
    assert e.value.status == rlxq.E_SHAPE and "expert_idx len" in str(e.value)
    dm.close()


def _swiglu_f64(orc, x, idx, wg, gs, wu, us, wd, ds, h, inter, E):
    g = orc.grouped_matmul_f64(gs, x, wg, idx, inter, E)
    u = orc.grouped_matmul_f64(us, x, wu, idx, inter, E)
    return orc.grouped_matmul_f64(ds, g / (1 + np.exp(-g)) * u, wd, idx, h, E)


@pytest.mark.parametrize("schemes", [(3, 3, 3), (1, 1, 2), (2, 1, 3)], ids=lambda s: "-".join(map(str, s)))
def test_device_matmul_grouped_swiglu(orc, schemes):
    """DeviceMatmul::grouped_swiglu: down(silu(gate(x)) * up(x)) with the
    expert of each row for all three projections (device_matmul.rs:221-296,
    graph :383-426); gate and up of one scheme run as one gate|up launch."""
    import torch
    import rlxq

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    gs, us, ds = schemes
    announce(f"DeviceMatmul grouped_swiglu schemes={schemes}")
    dm = rlxq.DeviceMatmul(0)
    rng = np.random.default_rng(21)
    m, h, inter, E = 11, 512, 384, 6
    wg = _bank(orc, gs, inter, h, E, 0.2, 0.7)
    wu = _bank(orc, us, inter, h, E, 0.45, 0.9)
    wd = _bank(orc, ds, h, inter, E, 0.65, 1.1)
    x = rng.standard_normal((m, h)).astype(np.float32)
    idx = (np.arange(m) * 5 % E).astype(np.float32)
    y = dm.grouped_swiglu(x, idx, wg, gs, wu, us, wd, ds, m, h, inter, E).reshape(m, h)
    assert rel_err(y, _swiglu_f64(orc, x, idx, wg, gs, wu, us, wd, ds, h, inter, E)) <= TOL
    assert dm.uploads == (2 if gs == us else 3)
    y2 = dm.grouped_swiglu(x[:4] * 0.5, idx[:4], wg, gs, wu, us, wd, ds, 4, h, inter, E).reshape(4, h)
    assert dm.uploads == (2 if gs == us else 3)   # same host stacks: resident
    assert rel_err(y2, _swiglu_f64(orc, x[:4] * 0.5, idx[:4], wg, gs, wu, us, wd, ds, h, inter, E)) <= TOL
    bad = idx.copy()
    bad[2] = -1
    with pytest.raises(rlxq.RlxqError) as e:
        dm.grouped_swiglu(x, bad, wg, gs, wu, us, wd, ds, m, h, inter, E)
    assert e.value.status == rlxq.E_INDEX
    with pytest.raises(rlxq.RlxqError) as e:
        dm.grouped_swiglu(x, idx, wg, gs, wu, us, wd[:-1], ds, m, h, inter, E)
    assert e.value.status == rlxq.E_SHAPE and "down weight bytes" in str(e.value)
    with pytest.raises(rlxq.RlxqError) as e:
        dm.grouped_swiglu(x[:, :9], idx, wg, gs, wu, us, wd, ds, m, h, inter, E)
    assert e.value.status == rlxq.E_SHAPE and "x len" in str(e.value)
    dm.close()


def test_device_matmul_grouped_swiglu_bank_layout(ctx, orc):
    """The session's gate|up bank (per expert: gate rows, then up rows) gives
    exactly what the fused EXPAND_SWIGLU call gives on a bank built that way
    on the host, followed by the grouped down projection."""
    import torch
    import rlxq

    m, h, inter, E = 9, 256, 160, 5
    announce("DeviceMatmul grouped_swiglu bank layout")
    rng = np.random.default_rng(22)
    wg = orc.synth_q4_1(rng, E * inter, h)
    wu = orc.synth_q4_1(rng, E * inter, h)
    wd = orc.synth_q4_1(rng, E * h, inter)
    x = rng.standard_normal((m, h)).astype(np.float32)
    idx = (np.arange(m) * 3 % E).astype(np.float32)
    dm = rlxq.DeviceMatmul(0)
    y = dm.grouped_swiglu(x, idx, wg, 3, wu, 3, wd, 3, m, h, inter, E).reshape(m, h)
    dm.close()
    gu = np.concatenate([wg.reshape(E, inter, -1), wu.reshape(E, inter, -1)], axis=1).reshape(-1)
    ids = _t(idx.astype(np.int32).reshape(m, 1))
    mid = ctx.moe_grouped(_t(x), _t(gu), ids, None, 3, rlxq.MOE_EXPAND_SWIGLU, 2 * inter, E)
    want = ctx.grouped_matmul(mid, _t(wd), _t(idx), 3, h, E)
    torch.cuda.synchronize()
    assert np.array_equal(y, want.cpu().numpy())


# ------------------------------------------------- routing variants and SwiGLU
@pytest.mark.parametrize("route", ["table", "fused"])
@pytest.mark.parametrize("scheme", [1, 3])
def test_grouped_both_routings(ctx, orc, monkeypatch, route, scheme):
    """The device routing table and the in-workgroup routing give the same
    rows, including skewed experts and invalid indices (zero rows)."""
    import torch

    monkeypatch.setenv("RLXQ_MOE_ROUTE", route)
    rows, k, n, E = 45, 640, 200, 9
    announce(f"grouped routing={route} scheme={scheme}")
    rng = np.random.default_rng(30 + scheme)
    packed = orc.synth(scheme, rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    idx = rng.integers(0, E, rows).astype(np.float32)
    idx[::7] = 3            # a crowded expert
    idx[5], idx[11], idx[20] = -1, 2.5, E   # invalid indices
    y = ctx.grouped_matmul(_t(x), _t(packed), _t(idx), scheme, n, E)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for r in (5, 11, 20):
        assert np.all(got[r] == 0.0)
    ok = np.array([r not in (5, 11, 20) for r in range(rows)])
    want = orc.grouped_matmul_f64(scheme, x[ok], packed, idx[ok], n, E)
    assert rel_err(got[ok], want) <= TOL


@pytest.mark.parametrize("route", ["table", "fused"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_moe_expand_swiglu(ctx, orc, monkeypatch, route, xdt):
    """EXPAND_SWIGLU: y = silu(x.Wg) * (x.Wu) per (token, slot), against the
    float64 chain (grouped products, then g / (1 + e^-g) * u)."""
    import torch
    import rlxq

    monkeypatch.setenv("RLXQ_MOE_ROUTE", route)
    T, H, I, E, TOPK = 7, 512, 96, 12, 3
    announce(f"moe expand swiglu route={route} x={xdt}")
    rng = np.random.default_rng(41)
    gate_up = orc.synth_q4_1(rng, E * 2 * I, H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    xt = _t(x) if xdt == "f32" else _t(x).to(torch.bfloat16)
    xv = xt.float().cpu().numpy()
    ids, probs = ctx.moe_route(_t(logits), TOPK, True)
    act = ctx.moe_grouped(xt, _t(gate_up), ids, probs, rlxq.GGUF_Q4_1, rlxq.MOE_EXPAND_SWIGLU, 2 * I, E)
    torch.cuda.synchronize()
    assert act.shape == (T * TOPK, I)
    flat = ids.cpu().numpy().ravel().astype(np.float32)
    gu = orc.grouped_matmul_f64(3, np.repeat(xv, TOPK, axis=0), gate_up, flat, 2 * I, E)
    g, u = gu[:, :I], gu[:, I:]
    assert rel_err(act.cpu().numpy(), g / (1.0 + np.exp(-g)) * u) <= TOL


def test_moe_ffn_config5_fused_swiglu(ctx, orc):
    """Config 5 with the fused gate|up + SwiGLU launch: route, EXPAND_SWIGLU,
    COMBINE (three launches) against the float64 chain."""
    import torch
    import rlxq

    T, H, I, E, TOPK = 16, 2048, 768, 128, 8
    announce("moe ffn config 5 fused swiglu")
    rng = np.random.default_rng(0)
    gate_up = orc.synth_q4_1(rng, E * 2 * I, H)
    down = orc.synth_q4_1(rng, E * H, I)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    xt = _t(x).to(torch.bfloat16)
    xv = xt.float().cpu().numpy()
    ids, probs = ctx.moe_route(_t(logits), TOPK, True)
    act = ctx.moe_grouped(xt, _t(gate_up), ids, probs, rlxq.GGUF_Q4_1, rlxq.MOE_EXPAND_SWIGLU, 2 * I, E,
                          y_dtype=torch.bfloat16)
    y = ctx.moe_grouped(act, _t(down), ids, probs, rlxq.GGUF_Q4_1, rlxq.MOE_COMBINE, H, E)
    torch.cuda.synchronize()
    oids = ids.cpu().numpy().ravel().astype(np.float32)
    gu = orc.grouped_matmul_f64(3, np.repeat(xv, TOPK, axis=0), gate_up, oids, 2 * I, E)
    g, u = gu[:, :I], gu[:, I:]
    assert rel_err(act.float().cpu().numpy(), g / (1.0 + np.exp(-g)) * u) <= 1e-2   # bf16 output
    act_v = act.float().cpu().numpy()
    dn = orc.grouped_matmul_f64(3, act_v, down, oids, H, E)
    pv = probs.cpu().numpy()
    want = np.zeros((T, H))
    for r in range(T):
        for j in range(TOPK):
            want[r] += pv[r, j] * dn[r * TOPK + j]
    assert rel_err(y.cpu().numpy(), want) <= TOL


# (k, lane-group shape the register path picks for Q4_1: L lanes x NU units)
XR_SHAPES = [(96, "L8_U1"), (512, "L8_U2"), (768, "L8_U3"), (1024, "L8_U4"), (2048, "L32_U2"),
             (2560, "L64_U2"), (8192, "L64_U4")]


@pytest.mark.parametrize("mt", ["1", "2", "4"])
@pytest.mark.parametrize("route", ["table", "fused"])
@pytest.mark.parametrize("k,shape", XR_SHAPES, ids=[str(k) for k, _ in XR_SHAPES])
def test_grouped_register_path(ctx, orc, monkeypatch, k, shape, route, mt):
    """Register-activation kernels (Q4_1, bf16 activations): every lane-group
    shape, both routings, 1/2/4 entries per weight pass, a crowded expert
    (several passes) and invalid indices (zero rows)."""
    import torch

    monkeypatch.setenv("RLXQ_MOE_ROUTE", route)
    monkeypatch.setenv("RLXQ_MOE_MT", mt)
    rows, n, E = 23, 136, 6
    announce(f"grouped register path k={k} route={route} mt={mt}")
    rng = np.random.default_rng(k + int(mt))
    packed = orc.synth_q4_1(rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    idx = rng.integers(0, E, rows).astype(np.float32)
    idx[::4] = 2
    idx[3], idx[9] = -1, E
    xt = _t(x).to(torch.bfloat16)
    y = ctx.grouped_matmul(xt, _t(packed), _t(idx), 3, n, E)
    torch.cuda.synchronize()
    assert shape in ctx.last_kernel and "moexr" in ctx.last_kernel
    got = y.cpu().numpy()
    assert np.all(got[3] == 0.0) and np.all(got[9] == 0.0)
    ok = np.array([r not in (3, 9) for r in range(rows)])
    want = orc.grouped_matmul_f64(3, xt.float().cpu().numpy()[ok], packed, idx[ok], n, E)
    assert rel_err(got[ok], want) <= TOL


@pytest.mark.parametrize("route", ["table", "fused"])
def test_register_path_matches_lds_path(ctx, orc, monkeypatch, route):
    """EXPAND_SWIGLU over config-5-like shapes: the register-activation and
    the LDS-record kernels agree within the bar."""
    import torch
    import rlxq

    monkeypatch.setenv("RLXQ_MOE_ROUTE", route)
    T, H, I, E, TOPK = 16, 2048, 768, 64, 8
    announce(f"register vs lds route={route}")
    rng = np.random.default_rng(5)
    gate_up = _t(orc.synth_q4_1(rng, E * 2 * I, H))
    xt = _t(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16)
    ids, probs = ctx.moe_route(_t(rng.standard_normal((T, E)).astype(np.float32)), TOPK, True)
    out = {}
    for kern in ("xr", "lds"):
        monkeypatch.setenv("RLXQ_MOE_KERNEL", kern)
        out[kern] = ctx.moe_grouped(xt, gate_up, ids, probs, rlxq.GGUF_Q4_1, rlxq.MOE_EXPAND_SWIGLU, 2 * I, E)
        torch.cuda.synchronize()
        assert ("moexr" in ctx.last_kernel) == (kern == "xr")
    a, b = out["xr"].cpu().numpy(), out["lds"].cpu().numpy().astype(np.float64)
    assert rel_err(a, b) <= TOL


@pytest.mark.parametrize("route", ["table", "fused"])
@pytest.mark.parametrize("k", [768, 2048, 4096])
def test_grouped_register_path_q4_0(ctx, orc, monkeypatch, k, route):
    """Register-activation kernels on Q4_0 (two blocks per unit)."""
    import torch

    monkeypatch.setenv("RLXQ_MOE_ROUTE", route)
    rows, n, E = 19, 72, 5
    announce(f"grouped register path q4_0 k={k} route={route}")
    rng = np.random.default_rng(k + 7)
    packed = orc.synth(2, rng, E * n, k)
    xt = _t(rng.standard_normal((rows, k)).astype(np.float32)).to(torch.bfloat16)
    idx = rng.integers(0, E, rows).astype(np.float32)
    y = ctx.grouped_matmul(xt, _t(packed), _t(idx), 2, n, E)
    torch.cuda.synchronize()
    assert "moexr" in ctx.last_kernel
    want = orc.grouped_matmul_f64(2, xt.float().cpu().numpy(), packed, idx, n, E)
    assert rel_err(y.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("sb", ["f32", "bf16"])
@pytest.mark.parametrize("k,group", [(768, 32), (2048, 64), (4096, 128)])
def test_grouped_register_path_mlx4(ctx, orc, k, group, sb):
    """Register-activation kernels on MLX affine 4-bit codes with f32 or bf16
    scale/bias slabs."""
    import torch
    import rlxq

    rows, n, E = 11, 80, 4
    announce(f"grouped register path mlx4 k={k} group={group} sb={sb}")
    rng = np.random.default_rng(k + group)
    codes = rng.integers(0, 16, (E * n, k)).astype(np.uint32)
    wq = orc.mlx_pack(codes, 4)
    sc = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(rng.uniform(0.01, 0.1, (E * n, k // group))))
    bi = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(rng.uniform(-0.5, 0.1, (E * n, k // group))))
    xt = _t(rng.standard_normal((rows, k)).astype(np.float32)).to(torch.bfloat16)
    idx = (np.arange(rows) * 3 % E).astype(np.float32)
    cast = (lambda a: _t(a).to(torch.bfloat16)) if sb == "bf16" else _t
    y = ctx.grouped_matmul(xt, _t(wq.view(np.uint8)), _t(idx), rlxq.MLX_AFFINE4, n, E, group=group,
                           scales=cast(sc), biases=cast(bi))
    torch.cuda.synchronize()
    assert "moexr" in ctx.last_kernel
    xv = xt.float().cpu().numpy()
    want = np.zeros((rows, n))
    for r in range(rows):
        e = int(idx[r])
        sl = slice(e * n, (e + 1) * n)
        want[r] = orc.mlx_matmul_f64(xv[r:r + 1], wq[sl], sc[sl], bi[sl], n, 4, group)[0]
    assert rel_err(y.cpu().numpy(), want) <= TOL


# ----------------------------------------- K-quant experts (Q4_K_M MoE files)
KQ_NAMES = {7: "q4_k", 8: "q6_k", 10: "q5_k", 11: "q3_k", 12: "q2_k", 13: "q8_k"}


@pytest.mark.parametrize("scheme", list(KQ_NAMES), ids=list(KQ_NAMES.values()))
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_grouped_k_quants(ctx, orc, scheme, xdt):
    """GGUF K-quant expert stacks through the grouped op (Q4_K / Q6_K: the
    formats of Q4_K_M MoE checkpoints; Q5_K, Q3_K, Q2_K, Q8_K: the rest of
    the reference's DeviceMatmul table), on the LDS-record kernels."""
    import torch

    rows, k, n, E = 20, 1024, 320, 6
    announce(f"grouped k-quant scheme={scheme} x={xdt}")
    rng = np.random.default_rng(50 + scheme)
    bank = orc.synth(scheme, rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    xt = _t(x) if xdt == "f32" else _t(x).to(torch.bfloat16)
    xv = xt.float().cpu().numpy()
    idx = ((np.arange(rows) * 5 + 1) % E).astype(np.float32)
    y = ctx.grouped_matmul(xt, _t(bank), _t(idx), scheme, n, E)
    torch.cuda.synchronize()
    assert KQ_NAMES[scheme] in ctx.last_kernel, ctx.last_kernel
    assert rel_err(y.cpu().numpy(), orc.grouped_matmul_f64(scheme, xv, bank, idx, n, E)) <= TOL


@pytest.mark.parametrize("scheme", list(KQ_NAMES), ids=list(KQ_NAMES.values()))
def test_moe_ffn_k_quants(ctx, orc, scheme):
    """Route, EXPAND_SWIGLU and COMBINE over K-quant banks (Qwen3-30B-A3B's
    expert shapes, 32 experts) against the float64 chain."""
    import torch
    import rlxq

    T, H, I, E, TOPK = 6, 2048, 768, 32, 8
    announce(f"moe ffn k-quant scheme={scheme}")
    rng = np.random.default_rng(60 + scheme)
    gate_up = orc.synth(scheme, rng, E * 2 * I, H)
    down = orc.synth(scheme, rng, E * H, I)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = _t(x).to(torch.bfloat16)
    xv = xt.float().cpu().numpy()
    ids, probs = ctx.moe_route(_t(rng.standard_normal((T, E)).astype(np.float32)), TOPK, True)
    act = ctx.moe_grouped(xt, _t(gate_up), ids, probs, scheme, rlxq.MOE_EXPAND_SWIGLU, 2 * I, E)
    y = ctx.moe_grouped(act, _t(down), ids, probs, scheme, rlxq.MOE_COMBINE, H, E)
    torch.cuda.synchronize()
    flat = ids.cpu().numpy().ravel().astype(np.float32)
    gu = orc.grouped_matmul_f64(scheme, np.repeat(xv, TOPK, axis=0), gate_up, flat, 2 * I, E)
    g, u = gu[:, :I], gu[:, I:]
    a64 = g / (1.0 + np.exp(-g)) * u
    assert rel_err(act.cpu().numpy(), a64) <= TOL
    dn = orc.grouped_matmul_f64(scheme, act.cpu().numpy(), down, flat, H, E)
    pv = probs.cpu().numpy()
    want = np.stack([sum(pv[r, j] * dn[r * TOPK + j] for j in range(TOPK)) for r in range(T)])
    assert rel_err(y.cpu().numpy(), want) <= TOL


# (k, lane-group shape the register path picks for Q4_K's 64-weight units)
XR_Q4K_SHAPES = [(256, "L8_U1"), (768, "L8_U2"), (1024, "L8_U2"), (2048, "L32_U1"), (4096, "L64_U1"),
                 (8192, "L64_U2")]


@pytest.mark.parametrize("mt", ["1", "2"])
@pytest.mark.parametrize("route", ["table", "fused"])
@pytest.mark.parametrize("k,shape", XR_Q4K_SHAPES, ids=[str(k) for k, _ in XR_Q4K_SHAPES])
def test_grouped_register_path_q4_k(ctx, orc, monkeypatch, k, shape, route, mt):
    """Register-activation kernels over Q4_K expert banks (bf16 activations):
    every lane-group shape, both routings, 1/2 entries per weight pass, a
    crowded expert and invalid indices (zero rows)."""
    import torch

    monkeypatch.setenv("RLXQ_MOE_ROUTE", route)
    monkeypatch.setenv("RLXQ_MOE_MT", mt)
    monkeypatch.setenv("RLXQ_MOE_KERNEL", "xr")   # also where the host would pick the LDS kernel
    rows, n, E = 19, 72, 5
    announce(f"grouped register path q4_k k={k} route={route} mt={mt}")
    rng = np.random.default_rng(k + 7 * int(mt))
    packed = orc.synth_q4_k(rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    idx = rng.integers(0, E, rows).astype(np.float32)
    idx[::4] = 1
    idx[2], idx[7] = -1, E
    xt = _t(x).to(torch.bfloat16)
    y = ctx.grouped_matmul(xt, _t(packed), _t(idx), 7, n, E)
    torch.cuda.synchronize()
    assert shape in ctx.last_kernel and "moexr" in ctx.last_kernel and "q4_k" in ctx.last_kernel
    got = y.cpu().numpy()
    assert np.all(got[2] == 0.0) and np.all(got[7] == 0.0)
    ok = np.array([r not in (2, 7) for r in range(rows)])
    want = orc.grouped_matmul_f64(7, xt.float().cpu().numpy()[ok], packed, idx[ok], n, E)
    assert rel_err(got[ok], want) <= TOL


def test_two_streams_use_their_own_workspace(ctx, orc):
    """Calls that use the library's scratch (the routing table and per-entry
    rows here) on two streams at once: each stream has its own workspace, so
    both results stay right."""
    import torch

    announce("two streams, grouped op with device tables")
    rng = np.random.default_rng(77)
    rows, k, n, E = 300, 1024, 512, 16
    bank = orc.synth_q4_1(rng, E * n, k)
    xs = [rng.standard_normal((rows, k)).astype(np.float32) for _ in range(2)]
    idxs = [rng.integers(0, E, rows).astype(np.float32) for _ in range(2)]
    bt = _t(bank)
    xt = [_t(x) for x in xs]
    it = [_t(i) for i in idxs]
    ys = [torch.empty((rows, n), device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for _ in range(4):
        for j in range(2):
            with torch.cuda.stream(streams[j]):
                ctx.grouped_matmul(xt[j], bt, it[j], 3, n, E, y=ys[j], stream=streams[j].cuda_stream)
    torch.cuda.synchronize()
    for j in range(2):
        assert rel_err(ys[j].cpu().numpy(), orc.grouped_matmul_f64(3, xs[j], bank, idxs[j], n, E)) <= TOL


@pytest.mark.parametrize("tokens", [16, 64, 128])
@pytest.mark.parametrize("ydt", ["f32", "bf16"])
def test_combine_in_down_launch_matches_combine_kernel(ctx, orc, monkeypatch, tokens, ydt):
    """COMBINE on the register kernels with the routing in the workgroups
    can sum each token's top-k rows in the down launch itself
    (RLXQ_MOE_COMBINE=fused: the workgroup that completes a (token, tile)
    does it).  It must equal the separate
    combine kernel bit for bit, with invalid expert ids in some rows (they
    contribute nothing), over consecutive calls (the counters reset), and
    against the float64 oracle."""
    import torch
    import rlxq

    H, I, E, TOPK = 2048, 768, 128, 8
    announce(f"moe fused combine tokens={tokens} y={ydt}")
    monkeypatch.setenv("RLXQ_MOE_KERNEL", "xr")   # (128 tokens would take the grouped MFMA path)
    rng = np.random.default_rng(tokens)
    down = orc.synth_q4_1(rng, E * H, I)
    dt = _t(down)
    ydtype = torch.bfloat16 if ydt == "bf16" else torch.float32
    for call in range(6):
        act = rng.standard_normal((tokens * TOPK, I)).astype(np.float32)
        at = _t(act).to(torch.bfloat16)
        ids = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(tokens)]).astype(np.int32)
        ids[1, 3] = -1
        ids[tokens - 1, 0] = E + 5
        probs = rng.uniform(0.01, 0.3, (tokens, TOPK)).astype(np.float32)
        it, pt = _t(ids), _t(probs)
        monkeypatch.setenv("RLXQ_MOE_COMBINE", "fused")
        y = ctx.moe_grouped(at, dt, it, pt, rlxq.GGUF_Q4_1, rlxq.MOE_COMBINE, H, E, y_dtype=ydtype)
        torch.cuda.synchronize()
        assert ctx.last_kernel.startswith("rlxq_moexrf_q4_1_"), ctx.last_kernel
        monkeypatch.setenv("RLXQ_MOE_COMBINE", "launch")
        y2 = ctx.moe_grouped(at, dt, it, pt, rlxq.GGUF_Q4_1, rlxq.MOE_COMBINE, H, E, y_dtype=ydtype)
        torch.cuda.synchronize()
        assert ctx.last_kernel == "rlxq_moe_combine_k", ctx.last_kernel
        assert torch.equal(y, y2), call
        valid = (ids >= 0) & (ids < E)
        av = at.float().cpu().numpy()
        dn = orc.grouped_matmul_f64(3, av, down, np.where(valid, ids, 0).ravel().astype(np.float32), H, E)
        want = np.einsum("tk,tkh->th", np.where(valid, probs, 0.0).astype(np.float64), dn.reshape(tokens, TOPK, H))
        assert rel_err(y.float().cpu().numpy(), want) <= (1e-2 if ydt == "bf16" else TOL), call


# (scheme, K, tokens, top_k): config 5's down (Q4_1 K=768: 8-lane groups of
# three units; Q4_K: 8-lane groups of two), K=2048 (32-lane groups), Q4_0,
# one token, top-1 and top-2, 64 tokens
XC_CASES = [(3, 768, 16, 8), (7, 768, 16, 8), (3, 2048, 16, 8), (2, 512, 7, 4), (3, 768, 1, 8), (3, 256, 5, 1),
            (7, 1024, 3, 2), (3, 768, 64, 8)]


@pytest.mark.parametrize("ydt", ["f32", "bf16"])
@pytest.mark.parametrize("case", XC_CASES, ids=lambda c: "_".join(map(str, c)))
def test_token_major_down_matches_two_launches(ctx, orc, monkeypatch, case, ydt):
    """COMBINE at decode sizes runs down and combine in one token-major launch
    (rlxq_moexc_*: a workgroup per token and column tile, a wave per slot,
    the slots summed in slot order in the workgroup).  It must equal the
    expert-major kernel plus rlxq_moe_combine_k bit for bit, with invalid
    expert ids contributing nothing, and match the float64 oracle."""
    import torch
    import rlxq

    scheme, K, tokens, topk = case
    H, E = 1000 if scheme == 2 else 2048, 40
    announce(f"moe token-major down {case} y={ydt}")
    rng = np.random.default_rng(K + tokens + topk)
    down = orc.synth(scheme, rng, E * H, K)
    dt = _t(down)
    ydtype = torch.bfloat16 if ydt == "bf16" else torch.float32
    act = rng.standard_normal((tokens * topk, K)).astype(np.float32)
    at = _t(act).to(torch.bfloat16)
    ids = np.stack([rng.choice(E, topk, replace=False) for _ in range(tokens)]).astype(np.int32)
    if tokens > 2:
        ids[1, topk - 1] = -1
        ids[tokens - 1, 0] = E + 5
    probs = rng.uniform(0.01, 0.3, (tokens, topk)).astype(np.float32)
    it, pt = _t(ids), _t(probs)
    monkeypatch.setenv("RLXQ_MOE_KERNEL", "xr")   # (64 tokens of 40 experts would take the grouped MFMA path)
    monkeypatch.delenv("RLXQ_MOE_COMBINE", raising=False)
    y = ctx.moe_grouped(at, dt, it, pt, scheme, rlxq.MOE_COMBINE, H, E, y_dtype=ydtype)
    torch.cuda.synchronize()
    assert ctx.last_kernel.startswith("rlxq_moexc_"), ctx.last_kernel
    monkeypatch.setenv("RLXQ_MOE_COMBINE", "launch")
    y2 = ctx.moe_grouped(at, dt, it, pt, scheme, rlxq.MOE_COMBINE, H, E, y_dtype=ydtype)
    torch.cuda.synchronize()
    assert ctx.last_kernel == "rlxq_moe_combine_k", ctx.last_kernel
    assert torch.equal(y, y2)
    valid = (ids >= 0) & (ids < E)
    av = at.float().cpu().numpy()
    dn = orc.grouped_matmul_f64(scheme, av, down, np.where(valid, ids, 0).ravel().astype(np.float32), H, E)
    want = np.einsum("tk,tkh->th", np.where(valid, probs, 0.0).astype(np.float64), dn.reshape(tokens, topk, H))
    assert rel_err(y.float().cpu().numpy(), want) <= (1e-2 if ydt == "bf16" else TOL)
