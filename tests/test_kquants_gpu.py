"""The other GGUF K-quants of the reference's DeviceMatmul table (Q5_K, Q3_K,
Q2_K, Q8_K; crates/rlx-laguna/src/device_matmul.rs:64-76) through the C ABI:
the bit-exact dequantisation, the dense DequantMatMul on the LDS-record GEMV
(any M, f32 or bf16 activations, every compiled record variant) and the
DeviceMatmul session, against the oracle's restatements of GGML's
block_q5_K / q3_K / q2_K / q8_K.  Q3_K's 110-byte super-blocks leave rows
of an odd count 2-byte aligned, which the kernels read through aligned
dwords.  Bar: max|got - want| / max|want| <= 1e-3 against float64 from the
activations the kernel saw."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3
SCHEMES = {"q5_k": 10, "q3_k": 11, "q2_k": 12, "q8_k": 13}
SUPER = {10: 176, 11: 110, 12: 84, 13: 292}


def _run(ctx, orc, scheme, x32, packed, n, xdt="bf16", **kw):
    import torch

    xt = _t(x32)
    if xdt == "bf16":
        xt = xt.to(torch.bfloat16)
    y = ctx.dequant_matmul(xt, _t(packed), scheme, n, **kw)
    torch.cuda.synchronize()
    k = x32.shape[1]
    want = xt.float().cpu().numpy().astype(np.float64) @ orc.dequantize(scheme, packed, k).astype(np.float64).T
    return y.float().cpu().numpy(), want


@pytest.mark.parametrize("name", list(SCHEMES))
@pytest.mark.parametrize("nk", [(37, 4096), (5, 256), (9, 768), (64, 12288)], ids=str)
def test_kquant_dequantize_bit_exact(ctx, orc, name, nk):
    import torch

    scheme = SCHEMES[name]
    n, k = nk
    announce(f"{name} dequantize n={n} k={k}")
    packed = orc.synth(scheme, np.random.default_rng(n + k + scheme), n, k)
    want = orc.dequantize(scheme, packed, k).view(np.uint32)
    got = ctx.dequantize(_t(packed), scheme, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)


@pytest.mark.parametrize("name", list(SCHEMES))
@pytest.mark.parametrize("kn", [(4096, 1031), (768, 37), (12288, 300), (256, 17), (4096, 24576), (1280, 96)],
                         ids=str)
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_kquant_gemv(ctx, orc, name, kn, xdt):
    scheme = SCHEMES[name]
    k, n = kn
    announce(f"{name} gemv m=1 x={xdt} k={k} n={n}")
    rng = np.random.default_rng(k + n + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    got, want = _run(ctx, orc, scheme, x, packed, n, xdt=xdt)
    # (bf16 activations and K up to the register kernel's unit chunks: Q5_K
    # three of 64-weight units, Q2_K four and Q3_K three of 32-weight units)
    xr = xdt == "bf16" and k // XR_UNIT[name] <= 64 * XR_CHUNKS.get(name, 0)
    assert ctx.last_kernel.startswith(f"rlxq_gemvxs_{name}_" if xr else f"rlxq_gemv_{name}_"), ctx.last_kernel
    assert rel_err(got, want) <= TOL


XR_UNIT = {"q5_k": 64, "q3_k": 32, "q2_k": 32, "q8_k": 32}
XR_CHUNKS = {"q5_k": 3, "q3_k": 3, "q2_k": 4}
XR_VARIANTS = [("q5_k", c) for c in ("1,2,8", "1,1,8", "2,1,8", "3,1,8")] + \
              [(nm, c) for nm in ("q2_k", "q3_k") for c in ("1,2,8", "2,1,8", "2,2,8", "3,1,8")] + [("q2_k", "4,1,8")]


@pytest.mark.parametrize("name,cfg", XR_VARIANTS, ids=str)
@pytest.mark.parametrize("kn", [(256, 17), (4096, 1031), (6144, 300), (8192, 520)], ids=str)
def test_kquant_register_gemv_every_variant(ctx, orc, monkeypatch, name, cfg, kn):
    """Every compiled register GEMV of Q5_K (64-weight units: the 32 qh
    bytes and the group's qs bytes in 21 dwords), Q2_K and Q3_K (32-weight
    units with a scale, Q2_K also a min, per 16 weights: two dot chains per
    block on the halves' activation sums): activations of NU unit chunks in
    registers; K a whole number of units or not of chunks."""
    scheme = SCHEMES[name]
    k, n = kn
    nu = int(cfg.split(",")[0])
    if (k // XR_UNIT[name] + 63) // 64 > nu:
        pytest.skip("K needs more unit chunks than the variant holds")
    monkeypatch.setenv("RLXQ_GEMV_XR", cfg + ",1")
    announce(f"{name} register gemv {cfg} {kn}")
    rng = np.random.default_rng(k * 3 + n + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    x[0, :7] *= 300.0
    got, want = _run(ctx, orc, scheme, x, packed, n, xdt="bf16")
    assert ctx.last_kernel == f"rlxq_gemvxs_{name}_U{{}}_D{{}}_W{{}}".format(*cfg.split(",")), ctx.last_kernel
    assert rel_err(got, want) <= TOL


@pytest.mark.parametrize("name", list(SCHEMES))
@pytest.mark.parametrize("m", [2, 3, 4, 7, 64])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_kquant_multi_row(ctx, orc, name, m, xdt):
    scheme = SCHEMES[name]
    k, n = 2304, 520
    announce(f"{name} gemv m={m} x={xdt}")
    rng = np.random.default_rng(m + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] *= 300.0
    got, want = _run(ctx, orc, scheme, x, packed, n, xdt=xdt)
    assert rel_err(got, want) <= TOL


# every compiled single-row record variant "L,P,C,D,W" that stays free of
# scratch for the scheme (the 16-wave two-step variants of Q5_K and Q3_K
# spill and are not selected)
VARIANTS = {
    "q5_k": ["64,1,2,1,16", "64,1,2,2,8", "64,2,1,2,8", "32,2,1,2,8", "16,2,1,2,8", "8,2,1,2,8"],
    "q3_k": ["64,1,2,1,16", "64,1,2,2,8", "64,2,1,2,8", "32,2,1,2,8", "16,2,1,2,8", "8,2,1,2,8"],
    "q2_k": ["64,1,2,1,16", "64,1,2,2,16", "64,1,2,2,8", "64,1,1,4,16", "64,2,1,2,8", "32,2,1,2,8", "8,2,1,2,8"],
    "q8_k": ["64,1,2,1,16", "64,1,2,2,16", "64,1,2,3,16", "64,1,2,2,8", "64,1,1,4,16", "64,2,1,2,8",
             "16,2,1,2,8", "8,2,1,2,8"],
}


@pytest.mark.parametrize("name,cfg", [(nm, c) for nm, cs in VARIANTS.items() for c in cs])
def test_kquant_every_record_variant(ctx, orc, monkeypatch, name, cfg):
    scheme = SCHEMES[name]
    monkeypatch.setenv("RLXQ_GEMV_CFG", cfg)
    monkeypatch.setenv("RLXQ_GEMV_XR", "0")   # (Q5_K's bf16 rows: not the register kernel)
    k, n = 2816, 300          # 11 super-blocks: Q3_K rows alternate 2- and 4-byte alignment
    announce(f"{name} variant {cfg}")
    rng = np.random.default_rng(11 + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    for xdt in ("f32", "bf16"):
        got, want = _run(ctx, orc, scheme, x, packed, n, xdt=xdt)
        L, P, C, D, W = cfg.split(",")
        assert ctx.last_kernel == f"rlxq_gemv_{name}_{xdt}_L{L}_P{P}_C{C}_M1_D{D}_W{W}", ctx.last_kernel
        assert rel_err(got, want) <= TOL, xdt


@pytest.mark.parametrize("name", list(SCHEMES))
def test_kquant_bf16_output_and_prefill_rows(ctx, orc, name):
    import torch

    scheme = SCHEMES[name]
    k, n, m = 1024, 300, 80
    rng = np.random.default_rng(4 + scheme)
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, want = _run(ctx, orc, scheme, x, packed, n, y_dtype=torch.bfloat16)
    # bf16-output prefill runs on the MFMA GEMM (weights rounded to bf16)
    assert ctx.last_kernel.startswith(f"rlxq_gemm_{name}_t256"), ctx.last_kernel
    assert rel_err(got, want) <= 2e-2


@pytest.mark.parametrize("name", list(SCHEMES))
def test_kquant_host_checks_and_session(ctx, orc, name):
    import torch
    import rlxq

    scheme = SCHEMES[name]
    sb = SUPER[scheme]
    assert rlxq.lib().rlxq_row_bytes(scheme, 768) == 3 * sb
    assert rlxq.lib().rlxq_row_bytes(scheme, 300) == -1
    x = torch.zeros((1, 512), device="cuda", dtype=torch.bfloat16)
    wf = torch.zeros((4 * 2 * sb + 32,), device="cuda", dtype=torch.uint8)
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul(x[:, :288].contiguous(), wf[:4 * 2 * sb], scheme, 4)
    assert e.value.status == rlxq.E_SHAPE
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul(x, wf[2:2 + 4 * 2 * sb], scheme, 4)
    assert e.value.status == rlxq.E_ALIGN
    dm = rlxq.DeviceMatmul(0)
    rng = np.random.default_rng(9 + scheme)
    m, k, n = 2, 768, 129
    packed = orc.synth(scheme, rng, n, k).ravel()
    xs = rng.standard_normal((m, k)).astype(np.float32)
    y = dm.matmul(xs, packed, m, k, n, scheme).reshape(m, n)
    want = xs.astype(np.float64) @ orc.dequantize(scheme, packed, k).astype(np.float64).T
    assert rel_err(y, want) <= TOL
    dm.close()
