"""Pins the CPU oracle (oracle/rlxq_oracle.c) before anything is compared with it.

Each check is chosen so that a plausible mistake in the restatement -- a wrong
nibble order, a dropped min term, a sign or rounding-mode slip, a transposed
operand -- fails at least one of them:
  * known-answer tests taken from the reference's own tests (file:line cited),
  * closed forms evaluated independently (exact rationals / numpy / torch),
  * exhaustive or randomised cross-checks of the scalar conversions,
  * round trips of representable blocks through quantize -> dequantize.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch


# ---------------------------------------------------------------- conversions
def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    got = orc.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(orc, rng):
    u = rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x477FE000, 0x477FF000, 0x477FEFFF,
                        0x33000000, 0x33000001, 0x387FC000, 0x38800000, 0x3F800000, 0x3F801000,
                        0x3F803000, 0x3F802000, 0x33800000], dtype=np.uint32)
    f = np.concatenate([u, special]).view(np.float32)
    # scale most samples into the f16 range so every rounding path is exercised
    with np.errstate(invalid="ignore", over="ignore"):
        f = np.where(np.arange(f.size) % 2 == 0, f, (f / np.float32(2.0**100)).astype(np.float32))
    f = f[~np.isnan(f)]
    got = orc.f32_to_f16_bits(f)
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f32_to_bf16_matches_torch_rne(orc, rng):
    u = rng.integers(0, 2**32, 300000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    f = f[~np.isnan(f)]
    got = orc.f32_to_bf16_bits(f)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    back = orc.bf16_bits_to_f32(got)
    assert np.array_equal(back, torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


# -------------------------------------------------------------- GGUF Q4_0 KAT
def _synthetic_q4_0(k, n):
    """crates/rlx-models/tests/gguf_legacy_quant_matmul.rs:53-65."""
    d = np.float16(0.5).view(np.uint16)
    blocks = k * n // 32
    out = bytearray()
    for b in range(blocks):
        out += int(d).to_bytes(2, "little")
        for j in range(16):
            out.append(((b + j) & 0x0F) | (((b + j + 1) & 0x0F) << 4))
    return np.frombuffer(bytes(out), np.uint8)


def test_q4_0_known_answer_fused_matches_reference(orc):
    """fused_q4_0_matches_reference (gguf_legacy_quant_matmul.rs:124-142), m=2 k=32 n=4,
    x = 0.01*(i+1); want computed here in exact rationals from the blob's definition."""
    k, n, m = 32, 4, 2
    packed = _synthetic_q4_0(k, n)
    x = np.array([0.01 * (i + 1) for i in range(m * k)], np.float32).reshape(m, k)
    w = orc.dequantize(orc.Q4_0, packed, k)
    for b in range(n):
        for j in range(16):
            lo = ((b + j) & 15) - 8
            hi = ((b + j + 1) & 15) - 8
            assert w[b, j] == 0.5 * lo and w[b, j + 16] == 0.5 * hi
    exact = [[sum(Fraction(float(x[r, i])) * Fraction(float(w[c, i])) for i in range(k)) for c in range(n)]
             for r in range(m)]
    y64 = orc.matmul_f64(orc.Q4_0, x, packed, n)
    yref = orc.matmul_refl(orc.Q4_0, x, packed, n)
    for r in range(m):
        for c in range(n):
            assert abs(y64[r, c] - float(exact[r][c])) < 1e-12
            assert abs(yref[r, c] - float(exact[r][c])) < 1e-4  # the reference's tolerance


def test_q4_0_representable_block_round_trips(orc):
    """crates/rlx-flint/src/quant.rs:525-536: d=0.25, x_i = d*((i%16)-8); one-hot dots give x_i exactly."""
    d = 0.25
    x = np.array([d * ((i % 16) - 8) for i in range(32)], np.float32)
    q = orc.quantize(orc.Q4_0, x.reshape(1, 32))
    for i in range(32):
        onehot = np.zeros((1, 32), np.float32)
        onehot[0, i] = 1.0
        assert orc.matmul_refl(orc.Q4_0, onehot, q, 1)[0, 0] == x[i]


@pytest.mark.parametrize("scheme,tol", [("Q8_0", 0.15), ("Q4_0", 0.6)])
def test_lm_precision_round_trips(orc, scheme, tol):
    """crates/rlx-unlimited-ocr/src/lm_precision.rs:639-658: v = 0.1*i - 3, i < 64."""
    v = np.array([i * 0.1 - 3.0 for i in range(64)], np.float32).reshape(2, 32)
    s = getattr(orc, scheme)
    back = orc.dequantize(s, orc.quantize(s, v), 32)
    assert np.max(np.abs(back - v)) < tol


def test_q8_0_encoder_rule(orc):
    """quant.rs:86-95: d = amax/127 stored f16, q = round_half_away(v/d) clamped."""
    x = np.zeros((1, 32), np.float32)
    x[0, :4] = [127.0, -63.5, 0.5, -0.5]  # amax 127 -> d = 1; ties round away from zero
    q = orc.quantize(orc.Q8_0, x)
    assert q[0, 0] == 0x00 and q[0, 1] == 0x3C  # f16(1.0) little-endian
    codes = q[0, 2:].view(np.int8)
    assert list(codes[:4]) == [127, -64, 1, -1]
    assert np.all(codes[4:] == 0)
    z = orc.quantize(orc.Q8_0, np.zeros((1, 32), np.float32))
    assert np.all(z == 0)


def test_q8_0_representable_round_trip(orc, rng):
    n = 64
    codes = rng.integers(-127, 128, (n, 32)).astype(np.int8)
    codes[:, 5] = np.where(rng.random(n) < 0.5, 127, -127)
    d = rng.uniform(0.002, 0.02, n).astype(np.float16).astype(np.float32)
    w = (codes.astype(np.float32) * d[:, None]).astype(np.float32)
    q = orc.quantize(orc.Q8_0, w)
    assert np.array_equal(q[:, 2:].view(np.int8), codes)
    assert np.array_equal(orc.dequantize(orc.Q8_0, q, 32), w)


# ----------------------------------------------------------------------- Q4_1
def _q4_1_block(d, m, lo, hi):
    b = bytearray()
    b += np.float16(d).tobytes() + np.float16(m).tobytes()
    for j in range(16):
        b.append((lo[j] & 15) | ((hi[j] & 15) << 4))
    return np.frombuffer(bytes(b), np.uint8)


def test_q4_1_layout_and_closed_form(orc):
    """GGML block_q4_1: f16 d at +0, f16 m at +2, byte j = element j (low nibble) and
    element j+16 (high nibble); w = d*q + m."""
    lo = list(range(16))
    hi = [15 - j for j in range(16)]
    blk = _q4_1_block(0.25, -1.5, lo, hi)
    w = orc.dequantize(orc.Q4_1, blk, 32)[0]
    want = [0.25 * q - 1.5 for q in lo + hi]
    assert list(w) == want


def test_q4_1_representable_round_trip(orc, rng):
    """quantize(min/max rule of real_layer_precision.rs:129-146) recovers codes, d and m."""
    n = 256
    codes = rng.integers(0, 16, (n, 32))
    codes[:, 3] = 0
    codes[:, 7] = 15
    d = rng.uniform(0.005, 0.05, n).astype(np.float16)
    mn = rng.uniform(-0.4, 0.0, n).astype(np.float16)
    w = (codes * d.astype(np.float32)[:, None] + mn.astype(np.float32)[:, None]).astype(np.float32)
    q = orc.quantize(orc.Q4_1, w)
    assert np.array_equal(q[:, 0:2].copy().view(np.float16).ravel(), d)
    assert np.array_equal(q[:, 2:4].copy().view(np.float16).ravel(), mn)
    got_codes = np.concatenate([q[:, 4:] & 15, q[:, 4:] >> 4], axis=1)
    assert np.array_equal(got_codes, codes)
    assert np.array_equal(orc.dequantize(orc.Q4_1, q, 32), w)


def test_q4_1_matmul_min_term(orc):
    """With all codes 0, y = m * sum(x) per block: a dropped or mis-scaled min term fails."""
    blk = np.concatenate([_q4_1_block(0.5, -0.25, [0] * 16, [0] * 16), _q4_1_block(0.5, 2.0, [0] * 16, [0] * 16)])
    x = np.arange(64, dtype=np.float32).reshape(1, 64) * 0.125
    want = -0.25 * x[0, :32].sum() + 2.0 * x[0, 32:].sum()
    assert orc.matmul_f64(orc.Q4_1, x, blk, 1)[0, 0] == pytest.approx(want, abs=1e-9)
    assert orc.matmul_refl(orc.Q4_1, x, blk, 1)[0, 0] == pytest.approx(want, rel=1e-6)


def _np_dequant(scheme, packed, k):
    """An independent vectorised numpy restatement of the three GGUF decoders."""
    bb = {1: 34, 2: 18, 3: 20}[scheme]
    blk = packed.reshape(-1, bb)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
    if scheme == 1:
        return (d * blk[:, 2:].view(np.int8).astype(np.float32)).reshape(-1, k)
    off = 2 if scheme == 2 else 4
    q = np.concatenate([blk[:, off:] & 15, blk[:, off:] >> 4], axis=1).astype(np.float32)
    if scheme == 2:
        return (d * (q - 8)).reshape(-1, k)
    m = blk[:, 2:4].copy().view(np.float16).astype(np.float32)
    return (d * q + m).astype(np.float32).reshape(-1, k)


@pytest.mark.parametrize("scheme", [1, 2, 3])
def test_dequant_matches_independent_numpy(orc, rng, scheme):
    k, n = 256, 48
    packed = orc.synth(scheme, rng, n, k)
    assert np.array_equal(orc.dequantize(scheme, packed, k), _np_dequant(scheme, packed.ravel(), k))


@pytest.mark.parametrize("scheme", [1, 2, 3])
def test_matmul_f64_and_reference_order(orc, rng, scheme):
    m, k, n = 3, 512, 40
    packed = orc.synth(scheme, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = _np_dequant(scheme, packed.ravel(), k)
    want = x.astype(np.float64) @ w.astype(np.float64).T  # y = x . W^T, W [n, k]
    y64 = orc.matmul_f64(scheme, x, packed, n)
    assert np.allclose(y64, want, rtol=1e-12, atol=1e-12)
    yr = orc.matmul_refl(scheme, x, packed, n)
    assert np.max(np.abs(yr - want)) / np.max(np.abs(want)) < 1e-5
    yp = orc.matmul_refl(scheme, x, packed, n, threads=4)
    assert np.array_equal(yp, yr)


def test_matmul_is_not_transposed(orc, rng):
    """A non-square case where using W [k, n] instead of [n, k] cannot match."""
    k, n = 64, 3
    w = rng.standard_normal((n, k)).astype(np.float32)
    packed = orc.quantize(orc.Q8_0, w)
    x = np.zeros((1, k), np.float32)
    x[0, 33] = 1.0
    y = orc.matmul_f64(orc.Q8_0, x, packed, n)
    assert np.allclose(y[0], orc.dequantize(orc.Q8_0, packed, k)[:, 33])


# ------------------------------------------------------------------ MLX affine
def test_mlx_lsb_first_known_answer(orc):
    """crates/rlx-moshi/src/mlx_dequant.rs:100-110: 0x76543210 -> codes 0..7; scale 2, bias -1."""
    wq = np.array([[0x76543210]], np.uint32)
    out = orc.mlx_dequantize(wq, np.array([[2.0]]), np.array([[-1.0]]), 8, 4, 8)
    assert list(out[0]) == [2.0 * c - 1.0 for c in range(8)]


def test_mlx_pack_matches_reference_pack_codes(orc):
    """pack_codes, crates/rlx-laguna/src/mlx_affine.rs:272-288, for 4 and 8 bits."""
    codes4 = np.arange(16, dtype=np.uint32).reshape(1, 16) % 16
    assert list(orc.mlx_pack(codes4, 4)[0]) == [0x76543210, 0xFEDCBA98]
    codes8 = np.array([[1, 2, 3, 250]], np.uint32)
    assert list(orc.mlx_pack(codes8, 8)[0]) == [0xFA030201]


def test_mlx_affine_matmul_matches_reference_test(orc):
    """affine_matmul_matches_reference, crates/rlx-laguna/src/mlx_affine.rs:290-330."""
    out, inn, bits, gs = 3, 64, 4, 64
    ng = inn // gs
    codes = (np.arange(out * inn) % 13).astype(np.uint32).reshape(out, inn)
    wq = orc.mlx_pack(codes, bits)
    scales = np.array([0.1 + 0.05 * i for i in range(out * ng)], np.float32).reshape(out, ng)
    biases = np.array([-0.3 + 0.02 * i for i in range(out * ng)], np.float32).reshape(out, ng)
    seq = 2
    x = np.sin(np.arange(seq * inn, dtype=np.float32) * np.float32(0.01)).astype(np.float32).reshape(seq, inn)
    w_ref = (scales.repeat(gs, axis=1) * codes.astype(np.float32) + biases.repeat(gs, axis=1)).astype(np.float32)
    assert np.array_equal(orc.mlx_dequantize(wq, scales, biases, inn, bits, gs), w_ref)
    y_ref = x.astype(np.float64) @ w_ref.astype(np.float64).T
    y = orc.mlx_matmul_f64(x, wq, scales, biases, out, bits, gs)
    assert np.max(np.abs(y - y_ref)) < 1e-5


# --------------------------------------------------------------- grouped / MoE
def test_grouped_matches_per_row_dense(orc, rng):
    """quant_parity_backends.rs:268-281: bank [E, N, K], row r uses expert (7r+1) % E."""
    rows, k, n, E = 6, 128, 16, 3
    bank = orc.synth(orc.Q4_1, rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    idx = np.array([(7 * r + 1) % E for r in range(rows)], np.float32)
    y = orc.grouped_matmul_f64(orc.Q4_1, x, bank, idx, n, E)
    for r in range(rows):
        e = int(idx[r])
        want = orc.matmul_f64(orc.Q4_1, x[r:r + 1], bank[e * n:(e + 1) * n], n)
        assert np.array_equal(y[r], want[0])
    with pytest.raises(ValueError):
        orc.grouped_matmul_f64(orc.Q4_1, x, bank, np.full(rows, 3.0, np.float32), n, E)


def test_topk_softmax_known_answer(orc):
    """topk_softmax_picks_largest, crates/rlx-unlimited-ocr/src/nn.rs:445-452."""
    ids, probs = orc.topk_softmax(np.array([[0.0, 5.0, 1.0, -2.0]]), 2)
    assert list(ids[0]) == [1, 2] and probs[0, 0] > probs[0, 1]
    e = np.exp(np.array([0.0, 5.0, 1.0, -2.0]) - 5.0)
    assert probs[0, 0] == pytest.approx(e[1] / e.sum(), rel=1e-6)
    ids2, p2 = orc.topk_softmax(np.array([[0.0, 5.0, 1.0, -2.0]]), 2, renorm=True)
    assert p2[0].sum() == pytest.approx(1.0, rel=1e-6) and list(ids2[0]) == [1, 2]


def test_moe_is_prob_weighted_sum_of_grouped(orc, rng):
    rows, k, n, E, topk = 4, 64, 8, 5, 2
    bank = orc.synth(orc.Q8_0, rng, E * n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    ids, probs = orc.topk_softmax(rng.standard_normal((rows, E)).astype(np.float32), topk)
    y = orc.moe_f64(orc.Q8_0, x, bank, ids, probs, n, E)
    want = np.zeros((rows, n))
    for j in range(topk):
        want += probs[:, j:j + 1].astype(np.float64) * orc.grouped_matmul_f64(orc.Q8_0, x, bank,
                                                                               ids[:, j].astype(np.float32), n, E)
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------------ int8
def test_act_int8_known_answers(orc):
    """bitnet.rs:76-93: s = amax/127 (1 for an all-zero row), q = f32::round (half away from zero)."""
    x = np.array([[2.5, -2.5, 127.0, 0.49], [0.0, 0.0, 0.0, 0.0]], np.float32)
    q, s = orc.quantize_act_int8(x)
    assert list(q[0]) == [3, -3, 127, 0] and s[0] == 1.0
    assert list(q[1]) == [0, 0, 0, 0] and s[1] == 1.0


def test_int8_col_is_per_output_channel(orc):
    """common.rs:466-482: w [k, n], one scale per column n."""
    w = np.array([[1.0, 10.0, 0.0], [-2.0, 5.0, 0.0]], np.float32)  # k=2, n=3
    q, s = orc.quantize_int8_col(w)
    assert np.allclose(s, [2.0 / 127, 10.0 / 127, 1.0])
    assert q[1, 0] == -127 and q[0, 1] == 127 and q[1, 1] == 64 and q[0, 2] == 0


def test_w8a8_exact_integer_sum(orc, rng):
    m, k, n = 3, 96, 5
    qx = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (k, n)).astype(np.int8)
    sx = rng.uniform(0.01, 0.1, m).astype(np.float32)
    sw = rng.uniform(0.01, 0.1, n).astype(np.float32)
    acc = qx.astype(np.int64) @ qw.astype(np.int64)
    want = ((acc.astype(np.float32) * sx[:, None]).astype(np.float32) * sw[None, :]).astype(np.float32)
    assert np.array_equal(orc.w8a8_matmul(qx, sx, qw, sw), want)


def test_int8_block_matmul(orc, rng):
    """int8_kernel.rs:59-89: y = x . ((Wq - zp) * s), Wq [k, n]."""
    m, k, n = 2, 64, 7
    x = rng.standard_normal((m, k)).astype(np.float32)
    wq = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(0.01, 0.1, n).astype(np.float32)
    zp = np.zeros(n, np.float32)
    want = x.astype(np.float64) @ ((wq.astype(np.float32) - zp) * s).astype(np.float64)
    assert np.allclose(orc.int8_block_matmul_f64(x, wq, s, zp), want, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------- Q4_K
# GGML block_q4_K (256 weights, 144 B).  The reference decodes it with the
# absent rlx_gguf::dequant_q4_k, so these tests pin the restatement by bit
# probes of the scale packing and closed forms built from scratch here.
def _q4k_block(orc, d, dmin, sc, mn, codes):
    """One packed block from explicit fields; codes [256] in weight order."""
    b = np.zeros(144, np.uint8)
    b[0:2] = orc.f32_to_f16_bits(np.float32([d])).view(np.uint8)
    b[2:4] = orc.f32_to_f16_bits(np.float32([dmin])).view(np.uint8)
    b[4:16] = orc.q4k_pack_scales(np.asarray(sc), np.asarray(mn))
    codes = np.asarray(codes, np.uint8)
    for g in range(4):
        lo, hi = codes[64 * g:64 * g + 32], codes[64 * g + 32:64 * g + 64]
        b[16 + 32 * g:48 + 32 * g] = lo | (hi << 4)
    return b


def test_q4k_scale_packing_round_trip(orc, rng):
    """Every 6-bit (scale, min) value in every one of the eight slots comes
    back from the packed 12 bytes, alone and mixed with random neighbours."""
    for s in range(8):
        for v in range(64):
            sc = rng.integers(0, 64, 8)
            mn = rng.integers(0, 64, 8)
            sc[s], mn[s] = v, 63 - v
            q = orc.q4k_pack_scales(sc, mn)
            for t in range(8):
                assert orc.q4k_scale_min(q, t) == (int(sc[t]), int(mn[t])), (s, v, t)


def test_q4k_scale_bits_reach_the_right_slot(orc):
    """Each of the 96 bits of the packed scales moves exactly one field of one
    sub-block, by the power of two GGML's layout gives it (a transposed byte
    index, a wrong shift or a swapped scale/min fails here)."""
    want = {}
    for byte in range(12):
        for bit in range(8):
            if byte < 4:
                want[(byte, bit)] = ("sc", byte, 1 << bit) if bit < 6 else ("sc", byte + 4, 1 << (bit - 2))
            elif byte < 8:
                want[(byte, bit)] = ("mn", byte - 4, 1 << bit) if bit < 6 else ("mn", byte, 1 << (bit - 2))
            else:
                want[(byte, bit)] = ("sc", byte - 4, 1 << bit) if bit < 4 else ("mn", byte - 4, 1 << (bit - 4))
    for (byte, bit), (field, slot, val) in want.items():
        q = np.zeros(12, np.uint8)
        q[byte] = 1 << bit
        got = [orc.q4k_scale_min(q, s) for s in range(8)]
        for s in range(8):
            exp = (val if field == "sc" and s == slot else 0, val if field == "mn" and s == slot else 0)
            assert got[s] == exp, (byte, bit, s)


def test_q4k_code_layout_and_closed_form(orc, rng):
    """d = 1, dmin = 0, unit scales: the weights are the codes, in GGML's
    order (low nibbles of a 32-byte group = the group's first 32 weights);
    then w = (d*sc)*q - dmin*mn per sub-block."""
    codes = rng.integers(0, 16, 256)
    b = _q4k_block(orc, 1.0, 0.0, [1] * 8, [0] * 8, codes)
    np.testing.assert_array_equal(orc.dequantize(orc.Q4_K, b, 256)[0], codes.astype(np.float32))
    sc, mn = rng.integers(1, 64, 8), rng.integers(0, 64, 8)
    d, dmin = np.float32(0.01171875), np.float32(0.03125)   # exact in f16
    b = _q4k_block(orc, d, dmin, sc, mn, codes)
    got = orc.dequantize(orc.Q4_K, b, 256)[0]
    for s in range(8):
        d1, m1 = np.float32(d * np.float32(sc[s])), np.float32(dmin * np.float32(mn[s]))
        want = (d1 * codes[32 * s:32 * s + 32].astype(np.float32)).astype(np.float32) - m1
        np.testing.assert_array_equal(got[32 * s:32 * s + 32], want.astype(np.float32))


def test_q4k_single_rounding(orc, rng):
    """d and dmin are f16 (11 significant bits), scales and mins 6 bits, codes
    4 bits: (d*sc)*q and dmin*mn are exact in f32, so every weight is the
    exact value d*sc*q - dmin*mn rounded once to f32 (checked against float64
    over random d, dmin and every scale, min and code)."""
    for _ in range(6):
        d = orc.f16_bits_to_f32(orc.f32_to_f16_bits(rng.uniform(1e-4, 0.05, 1).astype(np.float32)))[0]
        dmin = orc.f16_bits_to_f32(orc.f32_to_f16_bits(rng.uniform(1e-4, 0.05, 1).astype(np.float32)))[0]
        for base in range(0, 64, 8):
            sc = np.arange(base, base + 8)
            mn = rng.integers(0, 64, 8)
            codes = rng.integers(0, 16, 256)
            got = orc.dequantize(orc.Q4_K, _q4k_block(orc, d, dmin, sc, mn, codes), 256)[0]
            s = np.repeat(np.arange(8), 32)
            exact = float(d) * sc[s].astype(np.float64) * codes - float(dmin) * mn[s].astype(np.float64)
            np.testing.assert_array_equal(got, exact.astype(np.float32))


def test_q4k_rows_and_matmul(orc, rng):
    """Row stride K/256*144; the f64 matmul is x @ dequant(W)^T."""
    n, k = 7, 512
    w = orc.synth_q4_k(rng, n, k)
    assert w.shape == (n, k // 256 * 144) and orc.row_bytes(orc.Q4_K, k) == 288
    assert orc.row_bytes(orc.Q4_K, 300) == -1
    x = rng.standard_normal((3, k)).astype(np.float32)
    deq = orc.dequantize(orc.Q4_K, w, k).astype(np.float64)
    np.testing.assert_allclose(orc.matmul_f64(orc.Q4_K, x, w, n), x.astype(np.float64) @ deq.T, rtol=1e-12)


# ------------------------------------------------------------------- Q6_K
# GGML block_q6_K (256 weights, 210 B: ql[128], qh[64], int8 scales[16], f16
# d).  The reference decodes it with the absent rlx_gguf::dequant_q6_k.
def _q6k_zero(d=1.0):
    b = np.zeros(210, np.uint8)
    b[192:208] = 1                                   # unit scales
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    return b


def test_q6k_low_bits_reach_the_right_weight(orc):
    """Each of the 1024 ql bits, alone: one weight moves from -32 by 2^bit,
    at 128h + 32j + l with j = (byte % 64) // 32 for the low nibble and
    j + 2 for the high one (GGML's q1..q4 order)."""
    for byte in range(128):
        for bit in range(8):
            b = _q6k_zero()
            b[byte] = 1 << bit
            got = orc.dequantize(orc.Q6_K, b, 256)[0]
            h, r = divmod(byte, 64)
            j = r // 32 + (2 if bit >= 4 else 0)
            e = 128 * h + 32 * j + r % 32
            want = np.full(256, -32.0, np.float32)
            want[e] += 1 << (bit % 4)
            np.testing.assert_array_equal(got, want, err_msg=f"ql byte {byte} bit {bit}")


def test_q6k_high_bits_reach_the_right_weight(orc):
    """Each of the 512 qh bits: bit pair p of byte 32h + l holds code bits 4-5
    of weight 128h + 32p + l."""
    for byte in range(64):
        for bit in range(8):
            b = _q6k_zero()
            b[128 + byte] = 1 << bit
            got = orc.dequantize(orc.Q6_K, b, 256)[0]
            h, l = divmod(byte, 32)
            e = 128 * h + 32 * (bit // 2) + l
            want = np.full(256, -32.0, np.float32)
            want[e] += 16 << (bit % 2)
            np.testing.assert_array_equal(got, want, err_msg=f"qh byte {byte} bit {bit}")


def test_q6k_scales_cover_sixteen_weights_each(orc):
    """scales[t] multiplies exactly weights 16t..16t+15 (signed), and d the
    whole block: w = d * scale * (code - 32), exact in f32."""
    for t in range(16):
        b = _q6k_zero(d=0.5)
        b[192:208] = 0
        b[192 + t] = np.int8(-3).view(np.uint8)
        got = orc.dequantize(orc.Q6_K, b, 256)[0]
        want = np.zeros(256, np.float32)
        want[16 * t:16 * t + 16] = 0.5 * -3 * -32
        np.testing.assert_array_equal(got, want)


def test_q6k_exact_products(orc, rng):
    """d (f16, 11 bits) * scale (int8) * (code - 32) (6 bits) fits 24 bits: every
    weight equals its exact value, over random blocks."""
    w = orc.synth_q6_k(rng, 16, 256)
    got = orc.dequantize(orc.Q6_K, w, 256)
    for r in range(16):
        b = w[r]
        d = float(orc.f16_bits_to_f32(b[208:210].view(np.uint16))[0])
        sc = b[192:208].view(np.int8).astype(np.float64)
        for e in range(256):
            h, rem = divmod(e, 128)
            j, l = divmod(rem, 32)
            lo = (int(b[64 * h + l + 32 * (j & 1)]) >> (4 * (j >> 1))) & 15
            hi = (int(b[128 + 32 * h + l]) >> (2 * j)) & 3
            exact = d * sc[8 * h + 2 * j + l // 16] * ((lo | hi << 4) - 32)
            assert got[r, e] == np.float32(exact)


def test_q6k_rows_and_matmul(orc, rng):
    n, k = 5, 768
    w = orc.synth_q6_k(rng, n, k)
    assert w.shape == (n, 3 * 210) and orc.row_bytes(orc.Q6_K, k) == 630
    x = rng.standard_normal((2, k)).astype(np.float32)
    deq = orc.dequantize(orc.Q6_K, w, k).astype(np.float64)
    np.testing.assert_allclose(orc.matmul_f64(orc.Q6_K, x, w, n), x.astype(np.float64) @ deq.T, rtol=1e-12)


def test_q6k_reference_probe_block(orc):
    """The reference's own Q6_K probe block (crates/rlx-models-core/src/
    weight_loader.rs:573-581: d = 1, scale byte 0 = 0xFF, ql[0] = 0x21,
    qh[0] = 0x08), which it uses to reject decoders that read the scales
    unsigned: with the signed scale -1, weight 0 is -1 * (1 - 32) = 31 and
    weights 1..15 (code 0) are 32; every other scale is 0."""
    b = np.zeros(210, np.uint8)
    b[192] = 0xFF
    b[0] = 0x21
    b[128] = 0x08
    b[208:210] = np.array([1.0], np.float16).view(np.uint8)
    got = orc.dequantize(orc.Q6_K, b, 256)[0]
    want = np.zeros(256, np.float32)
    want[0] = 31.0
    want[1:16] = 32.0
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------------ Q5_K
# GGML block_q5_K (the reference maps GgmlType::Q5K to QuantScheme::GgufQ5K,
# crates/rlx-models-core/src/weight_loader.rs:503, and decodes it with the
# absent rlx_gguf::dequant_q5_k): f16 d, f16 dmin, the 12 Q4_K scale bytes,
# qh[32], qs[128].  Probes: every code bit alone moves one weight by its
# place value, at the weight the layout names.

def _q5k_unit(d=1.0, dmin=0.0):
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    return b


def _set_q4k_scales(b, off, sc, mn, orc):
    b[off:off + 12] = orc.q4k_pack_scales(np.asarray(sc), np.asarray(mn))


def test_q5k_low_bits_reach_the_right_weight(orc):
    """qs byte 32g + l, bit t: weight 64g + 32 (t >= 4) + l moves by
    2^(t % 4), all scales 1."""
    for byte in range(128):
        for bit in range(8):
            b = _q5k_unit()
            _set_q4k_scales(b, 4, [1] * 8, [0] * 8, orc)
            b[48 + byte] = 1 << bit
            got = orc.dequantize(orc.Q5_K, b, 256)[0]
            g, l = divmod(byte, 32)
            want = np.zeros(256, np.float32)
            want[64 * g + 32 * (bit // 4) + l] = 1 << (bit % 4)
            np.testing.assert_array_equal(got, want, err_msg=f"qs byte {byte} bit {bit}")


def test_q5k_high_bits_reach_the_right_weight(orc):
    """qh byte l, bit t: the fifth code bit (16) of weight 32t + l."""
    for byte in range(32):
        for bit in range(8):
            b = _q5k_unit()
            _set_q4k_scales(b, 4, [1] * 8, [0] * 8, orc)
            b[16 + byte] = 1 << bit
            got = orc.dequantize(orc.Q5_K, b, 256)[0]
            want = np.zeros(256, np.float32)
            want[32 * bit + byte] = 16.0
            np.testing.assert_array_equal(got, want, err_msg=f"qh byte {byte} bit {bit}")


def test_q5k_scales_and_mins_per_sub_block(orc, rng):
    """Sub-block s (weights 32s..32s+31) takes scale s and min s of the
    Q4_K packing: w = (d * sc) * code - dmin * mn, products rounded to f32,
    then the subtraction."""
    for _ in range(8):
        b = _q5k_unit(d=0.25, dmin=0.125)
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        _set_q4k_scales(b, 4, sc, mn, orc)
        b[16:176] = rng.integers(0, 256, 160, dtype=np.uint8)
        got = orc.dequantize(orc.Q5_K, b, 256)[0]
        for e in range(256):
            s, l = divmod(e, 32)
            g, h = divmod(s, 2)
            code = ((int(b[48 + 32 * g + l]) >> (4 * h)) & 15) | (((int(b[16 + l]) >> s) & 1) << 4)
            want = np.float32(np.float32(0.25 * sc[s]) * np.float32(code)) - np.float32(0.125 * mn[s])
            assert got[e] == want, (e, got[e], want)


def test_q5k_rows_and_matmul(orc, rng):
    n, k = 5, 768
    w = orc.synth_q5_k(rng, n, k)
    assert w.shape == (n, 3 * 176) and orc.row_bytes(orc.Q5_K, k) == 528
    x = rng.standard_normal((2, k)).astype(np.float32)
    deq = orc.dequantize(orc.Q5_K, w, k).astype(np.float64)
    np.testing.assert_allclose(orc.matmul_f64(orc.Q5_K, x, w, n), x.astype(np.float64) @ deq.T, rtol=1e-12)


# ------------------------------------------------------------------ Q3_K
# GGML block_q3_K (GgmlType::Q3K -> QuantScheme::GgufQ3K,
# weight_loader.rs:500; absent rlx_gguf::dequant_q3_k): hmask[32], qs[64],
# 12 bytes of sixteen 6-bit scales, f16 d; w = d * (scale - 32) * code with
# code = 2 low bits - (4 unless the hmask bit is set).

def _q3k_unit(scales=None, d=1.0):
    from oracle import oracle as o

    b = np.zeros(110, np.uint8)
    b[96:108] = o.q3k_pack_scales(np.full(16, 33) if scales is None else np.asarray(scales))
    b[108:110] = np.array([d], np.float16).view(np.uint8)
    return b


def test_q3k_scale_bits_reach_the_right_scale(orc):
    """Each of the 96 scale bits alone: byte t < 8, bit i sets bit i % 4 of
    scale t + 8 (i // 4); byte 8 + t, bit i sets bit 4 + i % 2 of scale
    t + 4 (i // 2) -- GGML's aux[] unpacking of block_q3_K.scales."""
    for byte in range(12):
        for bit in range(8):
            q = np.zeros(12, np.uint8)
            q[byte] = 1 << bit
            got = [orc.q3k_scale(q, s) for s in range(16)]
            want = [0] * 16
            if byte < 8:
                want[byte + 8 * (bit // 4)] = 1 << (bit % 4)
            else:
                want[(byte - 8) + 4 * (bit // 2)] = 1 << (4 + bit % 2)
            assert got == want, (byte, bit, got)


def test_q3k_scale_packing_round_trip(orc, rng):
    for _ in range(50):
        sc = rng.integers(0, 64, 16)
        q = orc.q3k_pack_scales(sc)
        assert [orc.q3k_scale(q, s) for s in range(16)] == list(sc)


def test_q3k_low_bits_reach_the_right_weight(orc):
    """qs byte 32n + 16i + l, bit pair j: weight 128n + 32j + 16i + l, the
    hmask bits all set (no -4), all scales 33 (scale - 32 = 1)."""
    for byte in range(64):
        for bit in range(8):
            b = _q3k_unit()
            b[0:32] = 0xFF
            b[32 + byte] = 1 << bit
            got = orc.dequantize(orc.Q3_K, b, 256)[0]
            n, r = divmod(byte, 32)
            i, l = divmod(r, 16)
            want = np.zeros(256, np.float32)
            want[128 * n + 32 * (bit // 2) + 16 * i + l] = 1 << (bit % 2)
            np.testing.assert_array_equal(got, want, err_msg=f"qs byte {byte} bit {bit}")


def test_q3k_hmask_bits_reach_the_right_weight(orc):
    """hmask byte 16i + l, bit t (t = 4n + j): only weight 128n + 32j + 16i + l
    escapes the -4 offset (codes 0, scales 33)."""
    for byte in range(32):
        for bit in range(8):
            b = _q3k_unit()
            b[byte] = 1 << bit
            got = orc.dequantize(orc.Q3_K, b, 256)[0]
            n, j = divmod(bit, 4)
            i, l = divmod(byte, 16)
            want = np.full(256, -4.0, np.float32)
            want[128 * n + 32 * j + 16 * i + l] = 0.0
            np.testing.assert_array_equal(got, want, err_msg=f"hmask byte {byte} bit {bit}")


def test_q3k_scales_cover_sixteen_weights_each(orc):
    """Scale s multiplies weights 16s..16s+15, signed (scale - 32)."""
    for s in range(16):
        sc = np.full(16, 32)
        sc[s] = 29                                     # -3
        b = _q3k_unit(scales=sc, d=0.5)
        got = orc.dequantize(orc.Q3_K, b, 256)[0]     # codes 0, hmask 0: code -4
        want = np.zeros(256, np.float32)
        want[16 * s:16 * s + 16] = 0.5 * -3 * -4
        np.testing.assert_array_equal(got, want)


def test_q3k_rows_and_matmul(orc, rng):
    n, k = 4, 512
    w = orc.synth_q3_k(rng, n, k)
    assert w.shape == (n, 2 * 110) and orc.row_bytes(orc.Q3_K, k) == 220
    x = rng.standard_normal((3, k)).astype(np.float32)
    deq = orc.dequantize(orc.Q3_K, w, k).astype(np.float64)
    np.testing.assert_allclose(orc.matmul_f64(orc.Q3_K, x, w, n), x.astype(np.float64) @ deq.T, rtol=1e-12)


# ------------------------------------------------------------------ Q2_K
# GGML block_q2_K (GgmlType::Q2K -> QuantScheme::GgufQ2K,
# weight_loader.rs:499; absent rlx_gguf::dequant_q2_k): scales[16] (scale
# nibble, min nibble), qs[64], f16 d, f16 dmin.

def _q2k_unit(d=1.0, dmin=0.0, sc=0x01):
    b = np.zeros(84, np.uint8)
    b[0:16] = sc
    b[80:82] = np.array([d], np.float16).view(np.uint8)
    b[82:84] = np.array([dmin], np.float16).view(np.uint8)
    return b


def test_q2k_code_bits_reach_the_right_weight(orc):
    """qs byte 32n + 16i + l, bit pair j: weight 128n + 32j + 16i + l."""
    for byte in range(64):
        for bit in range(8):
            b = _q2k_unit()
            b[16 + byte] = 1 << bit
            got = orc.dequantize(orc.Q2_K, b, 256)[0]
            n, r = divmod(byte, 32)
            i, l = divmod(r, 16)
            want = np.zeros(256, np.float32)
            want[128 * n + 32 * (bit // 2) + 16 * i + l] = 1 << (bit % 2)
            np.testing.assert_array_equal(got, want, err_msg=f"qs byte {byte} bit {bit}")


def test_q2k_scale_and_min_per_sixteen(orc):
    """scales[t]: low nibble times d scales weights 16t..16t+15, high nibble
    times dmin is subtracted from them."""
    for t in range(16):
        b = _q2k_unit(d=0.5, dmin=0.25, sc=0)
        b[t] = 0x3 | (0x5 << 4)
        b[16:80] = 0xFF                                # every code 3
        got = orc.dequantize(orc.Q2_K, b, 256)[0]
        want = np.zeros(256, np.float32)
        want[16 * t:16 * t + 16] = 0.5 * 3 * 3 - 0.25 * 5
        np.testing.assert_array_equal(got, want)


def test_q2k_rows_and_matmul(orc, rng):
    n, k = 4, 512
    w = orc.synth_q2_k(rng, n, k)
    assert w.shape == (n, 2 * 84) and orc.row_bytes(orc.Q2_K, k) == 168
    x = rng.standard_normal((3, k)).astype(np.float32)
    deq = orc.dequantize(orc.Q2_K, w, k).astype(np.float64)
    np.testing.assert_allclose(orc.matmul_f64(orc.Q2_K, x, w, n), x.astype(np.float64) @ deq.T, rtol=1e-12)


# ------------------------------------------------------------------ Q8_K
# GGML block_q8_K (GgmlType::Q8K -> QuantScheme::GgufQ8K,
# weight_loader.rs:504): f32 d, int8 qs[256], int16 bsums[16].

def test_q8k_is_f32_scale_times_int8(orc, rng):
    w = orc.synth_q8_k(rng, 3, 512)
    got = orc.dequantize(orc.Q8_K, w, 512)
    for r in range(3):
        for sb in range(2):
            blk = w[r, 292 * sb:292 * (sb + 1)]
            d = blk[0:4].view(np.float32)[0]
            q = blk[4:260].view(np.int8).astype(np.float32)
            np.testing.assert_array_equal(got[r, 256 * sb:256 * (sb + 1)], d * q)
            # the synthetic bsums are the format's own sums of 16 codes
            np.testing.assert_array_equal(blk[260:292].view(np.int16), q.reshape(16, 16).sum(1).astype(np.int16))


def test_q8k_rows_and_matmul(orc, rng):
    n, k = 4, 256
    w = orc.synth_q8_k(rng, n, k)
    assert orc.row_bytes(orc.Q8_K, k) == 292
    x = rng.standard_normal((2, k)).astype(np.float32)
    deq = orc.dequantize(orc.Q8_K, w, k).astype(np.float64)
    np.testing.assert_allclose(orc.matmul_f64(orc.Q8_K, x, w, n), x.astype(np.float64) @ deq.T, rtol=1e-12)


# ------------------------------------------------------------------ MXFP4
# The oracle's MXFP4 codec against the reference's own tests of its encoder
# and decoder (crates/rlx-models-core/src/mxfp4_pack.rs:290-398) and the E8M0
# known answers of crates/rlx-models-core/src/dsv4_quant.rs:184-188.
def test_mxfp4_e8m0_known_answers(orc):
    assert list(orc.e8m0_value([127, 128, 126])) == [1.0, 2.0, 0.5]
    assert orc.e8m0_value(0) == 0.0 and orc.e8m0_value(255) == 2.0 ** 127 and orc.e8m0_value(254) == 2.0 ** 127
    assert orc.e8m0_value(1) == 2.0 ** -126


def test_mxfp4_layout_low_nibble_is_the_even_element(orc):
    """mxfp4_pack.rs:30-31: element c of row r is byte r*k/2 + c/2, low
    nibble when c is even."""
    rows, k = 2, 64
    codes = np.zeros((rows, k // 2), np.uint8)
    scales = np.full((rows, k // 32), 127, np.uint8)
    codes[1, 5] = 0x72        # element 10: code 2 (1.0), element 11: code 7 (6.0)
    d = orc.mxfp4_dequantize(codes, scales, rows, k)
    want = np.zeros((rows, k))
    want[1, 10], want[1, 11] = 1.0, 6.0
    assert np.array_equal(d, want)
    scales[1, 0] = 129        # group 0 of row 1 scaled by 4
    assert orc.mxfp4_dequantize(codes, scales, rows, k)[1, 11] == 24.0


def test_mxfp4_exact_grid_round_trip(orc):
    """mxfp4_pack.rs:294-308: quantization is the identity on its own grid,
    bit for bit (signed zero included)."""
    for e in (-8, -2, 0, 5):
        row = (orc.E2M1[np.arange(32) % 16] * 2.0 ** e).astype(np.float32)[None, :]
        codes, eb = orc.mxfp4_quantize(row)
        back = orc.mxfp4_dequantize(codes, eb, 1, 32).astype(np.float32)
        assert np.array_equal(back.view(np.uint32), row.view(np.uint32)), e


def test_mxfp4_saturation_never_happens(orc):
    """mxfp4_pack.rs:310-335."""
    for amax in (1e-6, 0.017, 1.0, 1.9, 6.0, 7.9, 1e4):
        row = np.zeros((1, 32), np.float32)
        row[0, 7] = amax
        codes, eb = orc.mxfp4_quantize(row)
        scale = orc.e8m0_value(eb[0, 0])
        assert scale * 6.0 >= np.float32(amax)
        assert (codes[0, 3] >> 4) <= 7      # element 7: byte 3, high nibble, positive
        back = orc.mxfp4_dequantize(codes, eb, 1, 32)[0, 7]
        assert abs(back - np.float32(amax)) <= 0.2 * np.float32(amax)


def test_mxfp4_zero_group(orc):
    """mxfp4_pack.rs:337-343."""
    codes, eb = orc.mxfp4_quantize(np.zeros((1, 32), np.float32))
    assert (orc.mxfp4_dequantize(codes, eb, 1, 32) == 0).all() and (eb != 0xFF).all()


def test_mxfp4_ties_to_even(orc):
    """mxfp4_pack.rs:345-361."""
    for v, want in ((0.25, 0.0), (0.75, 1.0), (1.25, 1.0), (1.75, 2.0), (2.5, 2.0), (3.5, 4.0), (5.0, 4.0)):
        assert orc.E2M1[orc.e2m1_code(np.float32(v), np.float32(1.0))] == want, v


def test_mxfp4_gaussian_cosine(orc):
    """mxfp4_pack.rs:363-388: the reference's LCG weights (64 x 256, scaled
    by 0.02) keep cosine > 0.99 through a round trip."""
    rows, k = 64, 256
    s = 0x12345678
    w = np.empty(rows * k, np.float32)
    for i in range(rows * k):
        s = (s * 6364136223846793005 + 1) & 0xFFFFFFFFFFFFFFFF
        u = np.float32(s >> 33) / np.float32(np.float32(0xFFFFFFFF) / np.float32(2.0)) - np.float32(1.0)
        w[i] = u * np.float32(0.02)
    w = w.reshape(rows, k)
    codes, eb = orc.mxfp4_quantize(w)
    back = orc.mxfp4_dequantize(codes, eb, rows, k)
    cos = float((w.astype(np.float64) * back).sum() / np.sqrt((w.astype(np.float64) ** 2).sum() * (back ** 2).sum()))
    assert cos > 0.99


def test_mxfp4_exponent_is_the_smallest(orc):
    """e8m0_exponent's contract (mxfp4_pack.rs:114-128) against brute force:
    the smallest b with 6 * 2^(b-127) >= amax, powers of two included."""
    rng = np.random.default_rng(3)
    amax = np.concatenate([6.0 * 2.0 ** np.arange(-20, 20), rng.uniform(1e-6, 1e3, 200)]).astype(np.float32)
    got = orc.e8m0_exponent(amax)
    for a, b in zip(amax, got):
        want = next(bb for bb in range(1, 255) if 6.0 * 2.0 ** (bb - 127) >= float(a))
        assert b == want, (a, b, want)
