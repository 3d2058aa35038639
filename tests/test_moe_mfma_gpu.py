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
from test_gemv_gpu import _t, rel_err

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
