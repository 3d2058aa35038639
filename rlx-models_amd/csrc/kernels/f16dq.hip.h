// f16 dequantisation of packed 4/8-bit codes into MFMA operands, shared by
// the batched-decode (skinny) and f16 prefill GEMM kernels.
//
// A lane's 8 consecutive operand positions 8g .. 8g + 7 of a 32-element
// block hold, for the GGUF nibble formats, elements 4g .. 4g + 3 and
// 16 + 4g .. 16 + 4g + 3, for MLX's 4-bit codes (eight per little-endian
// word, low nibble first) elements 8g, 8g + 2, 8g + 4, 8g + 6, 8g + 1, ..,
// 8g + 7 (the orders in which code dword g unpacks); the activations are
// stored in the same order (perm_k).
#ifndef RLXQ_F16DQ_HIP_H
#define RLXQ_F16DQ_HIP_H
#include "common.hip.h"
#include "gemm_dq.hip.h"

namespace rlxq {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// Element of a 32-block held at position p (see above); order 0 natural,
// 1 GGUF nibbles, 2 MLX nibbles.
RLXQ_DEV int perm_k(int p, int order) {
  if (order == 0) return p;
  const int g = p >> 3, e = p & 7;
  if (order == 2) return 8 * g + (e < 4 ? 2 * e : 2 * (e - 4) + 1);
  return e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4);
}


// Normalised block: scale dwords, then the code dwords (sk_cw<SCH>() of them
// from o[sk_hdr<SCH>()]).  The weights are carried exactly by two f16 MFMA
// operands per 8 codes (sk_b2): b1 = q * dh rounded to f16 and
// b2 = fma(q, dh, -b1) [+ q * dl], with q the code (minus its offset) exact in
// f16.  Since q is an integer of at most 8 bits and dh an f16, q * dh - b1 is
// a multiple of dh's quantum below b1's rounding step, so b2 holds it exactly
// (TwoProduct); dl, where present, is the f16 remainder of a scale that f16
// does not hold (the K-quants' d * sc, MLX's f32 scales), rounded once at
// ~2^-22 of the weight.  The min / bias term m * sum(x) of a block is carried
// by one more MFMA per step on the prepared block sums (sk_mb), with m as
// f16 hi + lo.
//   Q4_1:  o[0] = d | m << 16 (the stored f16s), codes o[1..4]
//   Q4_0:  o[0] = d, codes o[1..4] (q - 8 through the -1032 offset)
//   Q8_0:  o[0] = d, codes o[1..8] (sign-flipped bytes, -1152 offset)
//   Q4_K:  o[0] = dh | dl << 16 of d * sc, o[1] = mh | ml << 16 of
//          -dmin * mn, codes o[2..5] in the Q4_1 nibble arrangement
//   Q6_K:  o[0] = dh0 | dh1 << 16, o[1] = dl0 | dl1 << 16 (d * sc of the two
//          16-weight halves), codes o[2..9] as code + 96 bytes (so that
//          code - 32 = byte - 128, the Q8_0 form)
//   Q5_K:  o[0], o[1] as Q4_K's, codes o[2..9] as the 5-bit code per byte
//   Q3_K:  o[0], o[1] as Q6_K's (d * (scale - 32) of the two halves), codes
//          o[2..9] as code + 128 per byte (code in -4 .. 3)
//   Q8_K:  o[0] = dh | dl << 16 of 2^8 * d, codes o[1..8] (int8, as stored)
//   Q2_K:  o[0], o[1] = 2^8 * d * sc of the two halves, o[2], o[3] = 2^8 *
//          dmin * mn (f32), codes o[4..11] one per byte: each weight
//          fma(d sc, code, -dmin mn) in f32 (the CPU decoder's one rounding)
//          then splits into f16 hi + lo (two mins per block do not fit the
//          one block-sum term)
//   MLX4 / MLX8: o[0] = sh | sl << 16 of 2^8 * scale, o[1] = bh | bl << 16 of
//          2^8 * bias, codes o[2..5] / o[2..9] as stored
//   MXFP4: o[0] = the f32 scale (a power of two), codes o[1..4]; its E2M1
//          codes times the scale are exact in bf16 (one bf16 operand)
// (2^8: sk_wscale, which keeps small scales normal in f16; the activation
// preparation folds 2^-8 into the row factors.)

template <int SCH> constexpr int sk_hdr() {
  return SCH == SCH_Q2_K ? 4
         : (SCH == SCH_Q4_K || SCH == SCH_Q6_K || SCH == SCH_Q5_K || SCH == SCH_Q3_K || SCH == SCH_MLX4 ||
            SCH == SCH_MLX8)
             ? 2
             : 1;
}
// code dwords: one byte per code (8) or one nibble (4)
template <int SCH> constexpr int sk_cw() {
  return (SCH == SCH_Q4_0 || SCH == SCH_Q4_1 || SCH == SCH_Q4_K || SCH == SCH_MLX4 || SCH == SCH_MXFP4) ? 4 : 8;
}
template <int SCH> constexpr int sk_bdw() { return sk_hdr<SCH>() + sk_cw<SCH>(); }
// formats with a min / bias term (m * block sum)
template <int SCH> constexpr bool sk_has_m() {
  return SCH == SCH_Q4_1 || SCH == SCH_Q4_K || SCH == SCH_Q5_K || SCH == SCH_MLX4 || SCH == SCH_MLX8;
}
// formats with a second scale half dl
template <int SCH> constexpr bool sk_has_dl() {
  return SCH == SCH_Q4_K || SCH == SCH_Q6_K || SCH == SCH_Q5_K || SCH == SCH_Q3_K || SCH == SCH_Q8_K ||
         SCH == SCH_MLX4 || SCH == SCH_MLX8;
}
// formats whose block has two 16-weight halves with scales of their own
template <int SCH> constexpr bool sk_halves() { return SCH == SCH_Q6_K || SCH == SCH_Q3_K; }

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt
// 6:4, lgkmcnt 11:8): wait on one counter, leave the others unconstrained.
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (((n >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8); }
constexpr int lgkmcnt0_imm() { return 0xF | (0x3 << 14) | (0x7 << 4); }

RLXQ_DEV f16x2_t as_h2(uint32_t v) { return __builtin_bit_cast(f16x2_t, v); }
RLXQ_DEV uint32_t as_u(f16x2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Two codes of bytes (b0, b1) or (b2, b3) of `u` as f16 1024 + code.
RLXQ_DEV f16x2_t magic_lo(uint32_t u) { return as_h2(perm_b32(0x64646464u, u, 0x04010400u)); }
RLXQ_DEV f16x2_t magic_hi(uint32_t u) { return as_h2(perm_b32(0x64646464u, u, 0x04030402u)); }

// f32 -> f16 hi | f16 lo << 16 with hi + lo ~ v to ~2^-22.
RLXQ_DEV uint32_t f16_split(float v) {
  const uint32_t h = f32_to_f16_bits(v);
  return h | (f32_to_f16_bits(v - f16_bits_to_f32(h)) << 16);
}

// The lane's B operands for positions 8g .. 8g + 7 of a block: the codes as
// exact f16 values q (four pairs), then b1 = q * dh, b2 = fma(q, dh, -b1)
// [+ q * dl].  `bp` points at the normalised block.
template <int SCH>
RLXQ_DEV void sk_b2(const uint32_t* bp, int g, f16x8_t& b1, f16x8_t& b2) {
  constexpr int H = sk_hdr<SCH>();
  if constexpr (SCH == SCH_Q2_K) {
    // f32 weight (half g / 2's scale and min), then hi = f16(w), lo = f16(w - hi)
    const float dl = __uint_as_float(bp[g >> 1]), ml = __uint_as_float(bp[2 + (g >> 1)]);
    const uint32_t u[2] = {bp[H + 2 * g], bp[H + 1 + 2 * g]};
    uint32_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t w = u[e >> 1] >> (16 * (e & 1));
      const float v0 = fmaf(dl, (float)(w & 0xffu), -ml), v1 = fmaf(dl, (float)((w >> 8) & 0xffu), -ml);
      const uint32_t h0 = f32_to_f16_bits(v0), h1 = f32_to_f16_bits(v1);
      h[e] = h0 | (h1 << 16);
      l[e] = f32_to_f16_bits(v0 - f16_bits_to_f32(h0)) | (f32_to_f16_bits(v1 - f16_bits_to_f32(h1)) << 16);
    }
    b1 = __builtin_bit_cast(f16x8_t, u32x4_t{h[0], h[1], h[2], h[3]});
    b2 = __builtin_bit_cast(f16x8_t, u32x4_t{l[0], l[1], l[2], l[3]});
    return;
  }
  f16x2_t q[4];
  if constexpr (sk_cw<SCH>() == 8) {
    // bytes: Q8_0 / Q8_K sign-flipped (byte ^ 0x80 = code + 128), Q6_K
    // code + 96 (= (code - 32) + 128), Q3_K code + 128, MLX8 and Q5_K the
    // unsigned code
    const uint32_t flip = (SCH == SCH_Q8_0 || SCH == SCH_Q8_K) ? 0x80808080u : 0u;
    const uint32_t u0 = bp[H + 2 * g] ^ flip, u1 = bp[H + 1 + 2 * g] ^ flip;
    const _Float16 off = (SCH == SCH_MLX8 || SCH == SCH_Q5_K) ? (_Float16)-1024.f : (_Float16)-1152.f;
    const f16x2_t o2 = {off, off};
    q[0] = magic_lo(u0) + o2;
    q[1] = magic_hi(u0) + o2;
    q[2] = magic_lo(u1) + o2;
    q[3] = magic_hi(u1) + o2;
  } else {
    const uint32_t qs = bp[H + g];
    const uint32_t lo = qs & 0x0F0F0F0Fu, hi = (qs >> 4) & 0x0F0F0F0Fu;
    const _Float16 off = SCH == SCH_Q4_0 ? (_Float16)-1032.f : (_Float16)-1024.f;
    const f16x2_t o2 = {off, off};
    q[0] = magic_lo(lo) + o2;
    q[1] = magic_hi(lo) + o2;
    q[2] = magic_lo(hi) + o2;
    q[3] = magic_hi(hi) + o2;
  }
  // (two halves: positions 8g.. lie in half g / 2 of the block)
  const uint32_t sel = (sk_halves<SCH>() && g >= 2) ? 0x03020302u : 0x01000100u;
  const f16x2_t dh = as_h2(perm_b32(bp[0], bp[0], sk_halves<SCH>() ? sel : 0x01000100u));
  f16x2_t w1[4], w2[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    w1[i] = q[i] * dh;
    w2[i] = __builtin_elementwise_fma(q[i], dh, -w1[i]);
  }
  if constexpr (sk_has_dl<SCH>()) {
    const uint32_t dlw = sk_halves<SCH>() ? bp[1] : bp[0];
    const uint32_t dsel = sk_halves<SCH>() ? sel : 0x03020302u;
    const f16x2_t dl = as_h2(perm_b32(dlw, dlw, dsel));
#pragma unroll
    for (int i = 0; i < 4; i++) w2[i] = __builtin_elementwise_fma(q[i], dl, w2[i]);
  }
  b1 = f16x8_t{w1[0].x, w1[0].y, w1[1].x, w1[1].y, w1[2].x, w1[2].y, w1[3].x, w1[3].y};
  b2 = f16x8_t{w2[0].x, w2[0].y, w2[1].x, w2[1].y, w2[2].x, w2[2].y, w2[3].x, w2[3].y};
}

// The B operand of the block's min / bias term: K slots 0, 1, 2 of the lane
// hold m hi, m hi, m lo (the A operand holds the block sum's hi, lo, hi), so
// one MFMA adds (S hi + S lo) * m hi + S hi * m lo.
template <int SCH>
RLXQ_DEV f16x8_t sk_mb(const uint32_t* bp) {
  uint32_t mw;
  if constexpr (SCH == SCH_Q4_1) mw = bp[0] >> 16;   // the stored f16 m (lo 0)
  else mw = bp[1];
  const _Float16 mh = __builtin_bit_cast(_Float16, (uint16_t)(mw & 0xffffu));
  const _Float16 ml = __builtin_bit_cast(_Float16, (uint16_t)(mw >> 16));
  const _Float16 z = (_Float16)0.f;
  return f16x8_t{mh, mh, ml, z, z, z, z, z};
}

// The A operand of the min / bias term from a block sum (f32).
RLXQ_DEV f16x8_t sk_ma(float s) {
  const uint32_t hs = f32_to_f16_bits(s);
  const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)hs);
  const _Float16 l = (_Float16)(s - f16_bits_to_f32(hs));
  const _Float16 z = (_Float16)0.f;
  return f16x8_t{h, l, h, z, z, z, z, z};
}

// MXFP4's single bf16 operand: E2M1 codes times an E8M0 scale (a power of
// two) are exact in bf16 (v_cvt_scalef32_pk_bf16_fp4, one per code pair), as
// are the bf16 activations scaled by a power of two; natural code order.
RLXQ_DEV bf16x8_t sk_b_mxfp4(const uint32_t* bp, int g) {
  const float sc = __uint_as_float(bp[0]);
  const uint32_t q = bp[1 + g];
  const u32x4_t b = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 0)),
                     __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 1)),
                     __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 2)),
                     __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 3))};
  return __builtin_bit_cast(bf16x8_t, b);
}

// One MFMA step of a normalised block: A (the activation fragment) times the
// block's weights at positions 8g .. 8g + 7 into acc.
template <int SCH>
RLXQ_DEV f32x4_t sk_step(f16x8_t a, const uint32_t* bp, int g, f32x4_t acc) {
  if constexpr (SCH == SCH_MXFP4) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), sk_b_mxfp4(bp, g), acc, 0, 0, 0);
  } else {
    f16x8_t b1, b2;
    sk_b2<SCH>(bp, g, b1, b2);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b1, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b2, acc, 0, 0, 0);
  }
}

// Raw block -> normalised dwords.
template <int SCH>
RLXQ_DEV void normalise(const RawBlk<SCH>& r, uint32_t* o) {
  if constexpr (SCH == SCH_Q6_K) {
    // d * sc is exact in f32 (11 + 8 bits)
    const float d = f16_bits_to_f32(r.d);
    const uint32_t s0 = f16_split(d * (float)(int8_t)(r.sc & 0xffu)), s1 = f16_split(d * (float)(int8_t)(r.sc >> 8));
    o[0] = (s0 & 0xffffu) | (s1 << 16);
    o[1] = (s0 >> 16) | (s1 & 0xffff0000u);
    const uint32_t sh1 = 4u * (r.q >> 1), sh2 = 2u * r.q;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t l = align_bytes(r.ql[i + 1], r.ql[i], r.off), hq = align_bytes(r.qh[i + 1], r.qh[i], r.off);
      // code (0..63) + 96 per byte: no carry between bytes
      o[2 + i] = (((l >> sh1) & 0x0F0F0F0Fu) | (((hq >> sh2) & 0x03030303u) << 4)) + 0x60606060u;
    }
  } else if constexpr (SCH == SCH_Q4_K) {
    // d * sc and dmin * mn are exact in f32 (11 + 6 bits)
    const uint32_t hd[4] = {r.hd.x, r.hd.y, r.hd.z, r.hd.w};
    float sc, mn;
    q4k_scale_min(hd, (int)r.sub, sc, mn);
    o[0] = f16_split(f16_bits_to_f32(hd[0] & 0xffffu) * sc);
    o[1] = f16_split(-(f16_bits_to_f32(hd[0] >> 16) * mn));
    const uint32_t qs[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t sh = 4 * (r.sub & 1u);
#pragma unroll
    for (int g = 0; g < 4; g++) o[2 + g] = ((qs[g] >> sh) & 0x0F0F0F0Fu) | (((qs[4 + g] >> sh) & 0x0F0F0F0Fu) << 4);
  } else if constexpr (SCH == SCH_Q5_K) {
    // d * sc and dmin * mn are exact in f32 (11 + 6 bits); code = low or
    // high nibble | qh bit sub << 4
    const uint32_t hd[4] = {r.hd.x, r.hd.y, r.hd.z, r.hd.w};
    float sc, mn;
    q4k_scale_min(hd, (int)r.sub, sc, mn);
    o[0] = f16_split(f16_bits_to_f32(hd[0] & 0xffffu) * sc);
    o[1] = f16_split(-(f16_bits_to_f32(hd[0] >> 16) * mn));
    const uint32_t qs[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
    const uint32_t sh = 4u * (r.sub & 1u);
#pragma unroll
    for (int i = 0; i < 8; i++) o[2 + i] = ((qs[i] >> sh) & 0x0F0F0F0Fu) | (((qh[i] >> r.sub) & 0x01010101u) << 4);
  } else if constexpr (SCH == SCH_Q3_K) {
    float ds0, ds1;
    q3k_half_scales(r, ds0, ds1);
    const uint32_t s0 = f16_split(ds0), s1 = f16_split(ds1);
    o[0] = (s0 & 0xffffu) | (s1 << 16);
    o[1] = (s0 >> 16) | (s1 & 0xffff0000u);
    const uint32_t n = r.sub >> 2, j = r.sub & 3;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t q = align_bytes(r.qs[i + 1], r.qs[i], r.off), hm = align_bytes(r.hm[i + 1], r.hm[i], r.off);
      // code + 4 = low bits | 4 (mask bit set), per byte; + 124 gives code + 128
      o[2 + i] = (((q >> (2 * j)) & 0x03030303u) | (((hm >> (4 * n + j)) & 0x01010101u) << 2)) + 0x7C7C7C7Cu;
    }
  } else if constexpr (SCH == SCH_Q2_K) {
    // d * sc and dmin * mn (4-bit sc, mn) are exact in f32
    const float d = f16_bits_to_f32(r.dd & 0xffffu), dmin = f16_bits_to_f32(r.dd >> 16);
    const uint32_t c0 = r.sc & 0xffu, c1 = (r.sc >> 8) & 0xffu;
    constexpr float P = sk_wscale<SCH_Q2_K>();
    o[0] = __float_as_uint(d * (float)(c0 & 15u) * P);
    o[1] = __float_as_uint(d * (float)(c1 & 15u) * P);
    o[2] = __float_as_uint(dmin * (float)(c0 >> 4) * P);
    o[3] = __float_as_uint(dmin * (float)(c1 >> 4) * P);
    const uint32_t qs[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t j = r.sub & 3;
#pragma unroll
    for (int i = 0; i < 8; i++) o[4 + i] = (qs[i] >> (2 * j)) & 0x03030303u;
  } else if constexpr (SCH == SCH_Q8_K) {
    o[0] = f16_split(r.d * sk_wscale<SCH_Q8_K>());
    o[1] = r.q0.x; o[2] = r.q0.y; o[3] = r.q0.z; o[4] = r.q0.w;
    o[5] = r.q1.x; o[6] = r.q1.y; o[7] = r.q1.z; o[8] = r.q1.w;
  } else if constexpr (SCH == SCH_MXFP4) {
    o[0] = __float_as_uint(r.s);
    o[1] = r.q.x; o[2] = r.q.y; o[3] = r.q.z; o[4] = r.q.w;
  } else if constexpr (SCH == SCH_MLX4) {
    o[0] = f16_split(r.s * sk_wscale<SCH_MLX4>());
    o[1] = f16_split(r.b * sk_wscale<SCH_MLX4>());
    o[2] = r.q.x; o[3] = r.q.y; o[4] = r.q.z; o[5] = r.q.w;
  } else if constexpr (SCH == SCH_MLX8) {
    o[0] = f16_split(r.s * sk_wscale<SCH_MLX8>());
    o[1] = f16_split(r.b * sk_wscale<SCH_MLX8>());
    o[2] = r.q0.x; o[3] = r.q0.y; o[4] = r.q0.z; o[5] = r.q0.w;
    o[6] = r.q1.x; o[7] = r.q1.y; o[8] = r.q1.z; o[9] = r.q1.w;
  } else if constexpr (SCH == SCH_Q4_1) {
    o[0] = r.h;
    o[1] = r.q.x; o[2] = r.q.y; o[3] = r.q.z; o[4] = r.q.w;
  } else {
    constexpr int NQ = SCH == SCH_Q8_0 ? 8 : 4;
    o[0] = r.off ? (r.w[0] >> 16) : (r.w[0] & 0xffffu);
#pragma unroll
    for (int i = 0; i < NQ; i++) o[1 + i] = r.off ? r.w[i + 1] : align_bytes(r.w[i + 1], r.w[i], 2);
  }
}

}  // namespace rlxq

#endif
