"""The grouped f16-MFMA path of the expert ops with the reference's own
operand types (F32 activations, F32 output: Op::DequantGroupedMatMul, crates/
rlx-models-core/src/standard_decoder.rs:12634-12760) and on every GGUF
K-quant (Q5_K, Q3_K, Q2_K, Q8_K beside Q4_K and Q6_K).

F32 activations run as a hi and a lo f16 row per gathered row (hi = f16(s*x),
lo = f16(s*x - hi), ~22 significant bits): a chunk of 16 MT x16 rows holds
8 MT entries, and the epilogue adds each pair's sums (a lane's registers 0 + 1
and 2 + 3) before the row scale, the SwiGLU and the store.  Bars: max|got -
want| / max|want| <= 1e-3 against the float64 oracle on the f32 activations
themselves; 2e-5 where the weights are exact in f16 (Q4_1 with d = 2^-6,
m = 0), which bf16 or f16 activations alone miss by an order of magnitude,
so a dropped or misplaced lo row fails it."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_EXACT_W = 2e-5
SCHEMES = {"q8_0": 1, "q4_0": 2, "q4_1": 3, "q4_k": 7, "q6_k": 8, "q5_k": 10, "q3_k": 11, "q2_k": 12, "q8_k": 13}
NEW_KQ = ["q5_k", "q3_k", "q2_k", "q8_k"]
# compiled (MT, NT, D) of each K-quant's grouped kernel
SHALLOW = ["1,2,2", "1,4,1", "2,2,2", "2,4,1", "4,2,1"]
VARIANTS = {
    "q5_k": SHALLOW,
    "q3_k": SHALLOW,
    "q2_k": ["1,2,3", "1,4,2", "1,8,2", "2,2,3", "2,4,2", "2,8,1", "4,2,2", "4,4,1"],
    "q8_k": ["1,2,4", "1,4,2", "1,8,2", "2,2,3", "2,4,2", "2,8,1", "4,2,2", "4,4,1"],
}


def _exact_q4_1(orc, rng, rows, k):
    """Q4_1 rows whose weights d*q + m are exact in f16: d = 2^-6, m = 0."""
    packed = orc.synth_q4_1(rng, rows, k)
    blk = packed.reshape(-1, 20)
    blk[:, 0:2] = np.frombuffer(np.float16(2.0 ** -6).tobytes(), np.uint8)
    blk[:, 2:4] = 0
    return packed


@pytest.mark.parametrize("name", list(SCHEMES))
@pytest.mark.parametrize("shape", [(512, 1024, 136, 16), (300, 2048, 96, 4)], ids=lambda s: "x".join(map(str, s)))
def test_grouped_f32_activations(ctx, orc, name, shape):
    """dequant_grouped_matmul with f32 activations at prefill sizes on every
    GGUF format: a crowded expert, a row of large values and invalid indices
    (zero rows)."""
    import torch

    scheme = SCHEMES[name]
    rows, k, n, E = shape
    announce(f"grouped mfma f32 {name} {shape}")
    rng = np.random.default_rng(rows + k + 17 * scheme)
    packed = orc.synth(scheme, rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[3] *= 300.0
    idx = rng.integers(0, E, rows).astype(np.float32)
    idx[::5] = 1
    bad = [7, 12, rows - 1]
    idx[bad[0]], idx[bad[1]], idx[bad[2]] = -1, 0.5, E
    y = ctx.grouped_matmul(_t(x), _t(packed), _t(idx), scheme, n, E)
    torch.cuda.synchronize()
    assert ctx.last_kernel.startswith(f"rlxq_moesk_{name}_"), ctx.last_kernel
    got = y.cpu().numpy()
    for r in bad:
        assert np.all(got[r] == 0.0), r
    ok = np.ones(rows, bool)
    ok[bad] = False
    want = orc.grouped_matmul_f64(scheme, x[ok], packed, idx[ok], n, E)
    assert rel_err(got[ok], want) <= TOL


@pytest.mark.parametrize("name", NEW_KQ)
@pytest.mark.parametrize("shape", [(512, 1024, 200, 16), (2000, 768, 130, 64)], ids=lambda s: "x".join(map(str, s)))
def test_grouped_k_quants_bf16(ctx, orc, name, shape):
    """Q5_K, Q3_K, Q2_K and Q8_K banks on the grouped MFMA kernel with bf16
    activations (prefill sizes: 32 entries per expert on average)."""
    import torch

    scheme = SCHEMES[name]
    rows, k, n, E = shape
    announce(f"grouped mfma bf16 {name} {shape}")
    rng = np.random.default_rng(rows + k + scheme)
    packed = orc.synth(scheme, rng, E * n, k)
    xt = _t(rng.standard_normal((rows, k)).astype(np.float32)).to(torch.bfloat16)
    idx = rng.integers(0, E, rows).astype(np.float32)
    y = ctx.grouped_matmul(xt, _t(packed), _t(idx), scheme, n, E)
    torch.cuda.synchronize()
    assert ctx.last_kernel.startswith(f"rlxq_moesk_{name}_"), ctx.last_kernel
    want = orc.grouped_matmul_f64(scheme, xt.float().cpu().numpy(), packed, idx, n, E)
    assert rel_err(y.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("cfg", ["1,2,4", "1,4,2", "1,8,2", "2,2,3", "2,4,2", "2,8,1", "4,2,2", "4,4,1"])
@pytest.mark.parametrize("sw", [False, True])
def test_f32_pairs_every_variant_exact_weights(ctx, orc, monkeypatch, cfg, sw):
    """Every compiled chunk/tile/ring variant of the grouped kernel, plain
    and SwiGLU, with f32 activations on weights exact in f16: the 2e-5 bar
    holds only if each hi row meets its own lo row; partial chunks and a
    column count that is no multiple of the tile width."""
    import torch
    import rlxq

    monkeypatch.setenv("RLXQ_MOE_KERNEL", "sk")
    monkeypatch.setenv("RLXQ_MOE_SK", cfg)
    mt, nt, d = (int(v) for v in cfg.split(","))
    T, H, n, E, TOPK = 40, 512, 2 * 72, 6, 3
    announce(f"grouped mfma f32 pairs {cfg} sw={sw}")
    rng = np.random.default_rng(mt * 10 + nt + int(sw) + 1000)
    bank = _exact_q4_1(orc, rng, E * n, H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(T)]).astype(np.int32)
    probs = rng.uniform(0.1, 0.5, (T, TOPK)).astype(np.float32)
    mode = rlxq.MOE_EXPAND_SWIGLU if sw else rlxq.MOE_EXPAND
    y = ctx.moe_grouped(_t(x), _t(bank), _t(ids), _t(probs), 3, mode, n, E)
    torch.cuda.synchronize()
    assert ctx.last_kernel == f"rlxq_moesk_q4_1_mt{mt}_nt{nt}_d{d}" + ("_sw" if sw else ""), ctx.last_kernel
    gu = orc.grouped_matmul_f64(3, np.repeat(x, TOPK, axis=0), bank, ids.ravel().astype(np.float32), n, E)
    want = gu[:, :n // 2] / (1.0 + np.exp(-gu[:, :n // 2])) * gu[:, n // 2:] if sw else gu
    assert rel_err(y.cpu().numpy(), want) <= TOL_EXACT_W


@pytest.mark.parametrize("name", NEW_KQ)
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_new_k_quants_every_variant(ctx, orc, monkeypatch, name, xdt):
    """Every compiled variant of the Q5_K / Q3_K / Q2_K / Q8_K grouped
    kernels, plain and SwiGLU, with f32 or bf16 activations."""
    import torch
    import rlxq

    scheme = SCHEMES[name]
    monkeypatch.setenv("RLXQ_MOE_KERNEL", "sk")
    T, H, n, E, TOPK = 24, 512, 2 * 40, 5, 2
    rng = np.random.default_rng(scheme * 7 + len(xdt))
    bank = orc.synth(scheme, rng, E * n, H)
    x = rng.standard_normal((T, H)).astype(np.float32)
    xt = _t(x) if xdt == "f32" else _t(x).to(torch.bfloat16)
    xv = xt.float().cpu().numpy()
    ids = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(T)]).astype(np.int32)
    probs = rng.uniform(0.1, 0.5, (T, TOPK)).astype(np.float32)
    gu = orc.grouped_matmul_f64(scheme, np.repeat(xv, TOPK, axis=0), bank, ids.ravel().astype(np.float32), n, E)
    for cfg in VARIANTS[name]:
        monkeypatch.setenv("RLXQ_MOE_SK", cfg)
        mt, nt, d = (int(v) for v in cfg.split(","))
        for sw in (False, True):
            announce(f"grouped mfma {name} {xdt} {cfg} sw={sw}")
            mode = rlxq.MOE_EXPAND_SWIGLU if sw else rlxq.MOE_EXPAND
            y = ctx.moe_grouped(xt, _t(bank), _t(ids), _t(probs), scheme, mode, n, E)
            torch.cuda.synchronize()
            assert ctx.last_kernel == f"rlxq_moesk_{name}_mt{mt}_nt{nt}_d{d}" + ("_sw" if sw else ""), \
                ctx.last_kernel
            want = gu[:, :n // 2] / (1.0 + np.exp(-gu[:, :n // 2])) * gu[:, n // 2:] if sw else gu
            assert rel_err(y.cpu().numpy(), want) <= TOL, (cfg, sw)


@pytest.mark.parametrize("name", ["q4_1", "q4_k", "q6_k", "q2_k"])
def test_moe_ffn_prefill_f32_chain(ctx, orc, name):
    """A MoE FFN at prefill size with the reference's operand types all the
    way: f32 hidden rows, EXPAND_SWIGLU to an f32 intermediate, COMBINE of
    the f32 intermediate (both on the grouped MFMA kernels), against the
    float64 chain on a sample of rows."""
    import torch
    import rlxq

    scheme = SCHEMES[name]
    T, H, I, E, TOPK = 512, 1024, 256, 64, 8
    announce(f"moe ffn prefill f32 chain {name}")
    rng = np.random.default_rng(scheme + 4242)
    gate_up = orc.synth(scheme, rng, E * 2 * I, H)
    down = orc.synth(scheme, rng, E * H, I)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids, probs = ctx.moe_route(_t(rng.standard_normal((T, E)).astype(np.float32)), TOPK, True)
    act = ctx.moe_grouped(_t(x), _t(gate_up), ids, probs, scheme, rlxq.MOE_EXPAND_SWIGLU, 2 * I, E,
                          y_dtype=torch.float32)
    torch.cuda.synchronize()
    assert ctx.last_kernel.startswith(f"rlxq_moesk_{name}_") and ctx.last_kernel.endswith("_sw"), ctx.last_kernel
    y = ctx.moe_grouped(act, _t(down), ids, probs, scheme, rlxq.MOE_COMBINE, H, E)
    torch.cuda.synchronize()
    flat = ids.cpu().numpy().ravel().astype(np.float32)
    av = act.cpu().numpy()
    sel = np.arange(0, T * TOPK, 11)
    gu = orc.grouped_matmul_f64(scheme, np.repeat(x, TOPK, axis=0)[sel], gate_up, flat[sel], 2 * I, E)
    g, u = gu[:, :I], gu[:, I:]
    assert rel_err(av[sel], g / (1.0 + np.exp(-g)) * u) <= TOL
    rows = np.arange(0, T, 13)
    ent = (rows[:, None] * TOPK + np.arange(TOPK)[None, :]).ravel()
    dn = orc.grouped_matmul_f64(scheme, av[ent], down, flat[ent], H, E).reshape(len(rows), TOPK, H)
    want = np.einsum("rk,rkh->rh", probs.cpu().numpy()[rows].astype(np.float64), dn)
    assert rel_err(y.cpu().numpy()[rows], want) <= TOL


def test_f32_and_bf16_paths_agree_on_bf16_values(ctx, orc):
    """Activations that are exact in bf16, passed once as bf16 and once as
    f32: the pair path (lo rows all zero) gives the bf16 path's result to
    the f32 accumulation's rounding."""
    import torch

    rows, k, n, E = 400, 1024, 96, 8
    rng = np.random.default_rng(77)
    packed = orc.synth_q4_1(rng, E * n, k)
    xb = _t(rng.standard_normal((rows, k)).astype(np.float32)).to(torch.bfloat16)
    idx = _t(rng.integers(0, E, rows).astype(np.float32))
    yb = ctx.grouped_matmul(xb, _t(packed), idx, 3, n, E)
    kb = ctx.last_kernel
    yf = ctx.grouped_matmul(xb.float(), _t(packed), idx, 3, n, E)
    kf = ctx.last_kernel
    torch.cuda.synchronize()
    assert kb.startswith("rlxq_moesk_q4_1_") and kf.startswith("rlxq_moesk_q4_1_"), (kb, kf)
    assert rel_err(yf.cpu().numpy(), yb.cpu().numpy().astype(np.float64)) <= 1e-6
