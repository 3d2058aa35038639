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


// Normalised block: scale dword (Q4_1, Q4_K, MLX4: d | m << 16, else d) +
// code dwords.  A Q4_K sub-block normalises to the Q4_1 form: d = d * sc and
// m = -dmin * mn rounded to f16, and code dword g holding elements 4g..4g+3
// (low nibbles) and 16 + 4g.. (high nibbles) of the sub-block.
// An MXFP4 block: its f32 scale (a power of two) and its four code words.
// An MLX4 (MLX8) block: the group's f32 scale and bias rounded to f16 (the
// f16 range covers the scales of real weight slabs; scales below 2^-14 lose
// bits as f16 subnormals) and its four (eight) code words as they are; MLX8's
// codes, four per word LSB first, unpack in natural order.
// A Q6_K block normalises to the int8 form of Q8_0 with one f16 scale per
// 16 weights: scale dword d0 | d1 << 16 (d * sc of the two halves, rounded
// to f16) and code bytes code + 96, so that code - 32 = byte - 128 as for
// Q8_0's sign-flipped bytes; its activations stay in natural order.
template <int SCH> constexpr int sk_bdw() { return (SCH == SCH_Q8_0 || SCH == SCH_Q6_K || SCH == SCH_MLX8) ? 9 : 5; }

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt
// 6:4, lgkmcnt 11:8): wait on one counter, leave the others unconstrained.
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (((n >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8); }
constexpr int lgkmcnt0_imm() { return 0xF | (0x3 << 14) | (0x7 << 4); }

RLXQ_DEV f16x2_t as_h2(uint32_t v) { return __builtin_bit_cast(f16x2_t, v); }
RLXQ_DEV uint32_t as_u(f16x2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Two codes of bytes (b0, b1) or (b2, b3) of `u` as f16 1024 + code.
RLXQ_DEV f16x2_t magic_lo(uint32_t u) { return as_h2(perm_b32(0x64646464u, u, 0x04010400u)); }
RLXQ_DEV f16x2_t magic_hi(uint32_t u) { return as_h2(perm_b32(0x64646464u, u, 0x04030402u)); }

// The lane's B operand: 8 f16 weights of one block of one row, positions
// 8g .. 8g + 7.  `bp` points at the normalised block.
template <int SCH>
RLXQ_DEV f16x8_t dequant_lane(const uint32_t* bp, int g) {
  const uint32_t dm = bp[0];
  const f16x2_t d2 = as_h2(perm_b32(dm, dm, 0x01000100u));
  f16x2_t w[4];
  if constexpr (SCH == SCH_MLX8) {
    // unsigned codes in natural order: d*q + m with one rounding
    const uint32_t u0 = bp[1 + 2 * g], u1 = bp[2 + 2 * g];
    const f16x2_t m2 = as_h2(perm_b32(dm, dm, 0x03020302u));
    const f16x2_t off = {(_Float16)-1024.f, (_Float16)-1024.f};
    w[0] = __builtin_elementwise_fma(magic_lo(u0) + off, d2, m2);
    w[1] = __builtin_elementwise_fma(magic_hi(u0) + off, d2, m2);
    w[2] = __builtin_elementwise_fma(magic_lo(u1) + off, d2, m2);
    w[3] = __builtin_elementwise_fma(magic_hi(u1) + off, d2, m2);
  } else if constexpr (SCH == SCH_Q8_0 || SCH == SCH_Q6_K) {
    const uint32_t flip = SCH == SCH_Q8_0 ? 0x80808080u : 0u;
    const uint32_t u0 = bp[1 + 2 * g] ^ flip, u1 = bp[2 + 2 * g] ^ flip;
    // (Q6_K: positions 8g.. lie in half g / 2 of the block)
    const f16x2_t dd = SCH == SCH_Q6_K ? as_h2(perm_b32(dm, dm, g < 2 ? 0x01000100u : 0x03020302u)) : d2;
    const f16x2_t off = {(_Float16)-1152.f, (_Float16)-1152.f};
    w[0] = (magic_lo(u0) + off) * dd;
    w[1] = (magic_hi(u0) + off) * dd;
    w[2] = (magic_lo(u1) + off) * dd;
    w[3] = (magic_hi(u1) + off) * dd;
  } else {
    const uint32_t qs = bp[1 + g];
    const uint32_t lo = qs & 0x0F0F0F0Fu, hi = (qs >> 4) & 0x0F0F0F0Fu;
    if constexpr (SCH == SCH_Q4_1 || SCH == SCH_Q4_K || SCH == SCH_MLX4) {
      const f16x2_t m2 = as_h2(perm_b32(dm, dm, 0x03020302u));
      const f16x2_t off = {(_Float16)-1024.f, (_Float16)-1024.f};
      w[0] = __builtin_elementwise_fma(magic_lo(lo) + off, d2, m2);
      w[1] = __builtin_elementwise_fma(magic_hi(lo) + off, d2, m2);
      w[2] = __builtin_elementwise_fma(magic_lo(hi) + off, d2, m2);
      w[3] = __builtin_elementwise_fma(magic_hi(hi) + off, d2, m2);
    } else {
      const f16x2_t off = {(_Float16)-1032.f, (_Float16)-1032.f};
      w[0] = (magic_lo(lo) + off) * d2;
      w[1] = (magic_hi(lo) + off) * d2;
      w[2] = (magic_lo(hi) + off) * d2;
      w[3] = (magic_hi(hi) + off) * d2;
    }
  }
  return f16x8_t{w[0].x, w[0].y, w[1].x, w[1].y, w[2].x, w[2].y, w[3].x, w[3].y};
}

// The B operand of one MFMA step and the step itself.  MXFP4 takes bf16
// MFMA: E2M1 codes times an E8M0 scale (a power of two) are exact in bf16
// (v_cvt_scalef32_pk_bf16_fp4, one per code pair), as are the bf16
// activations scaled by a power of two, and its codes unpack in natural
// order.  The other formats take f16 MFMA with dequant_lane's weights.
template <int SCH> struct SkOp { typedef f16x8_t type; };
template <> struct SkOp<SCH_MXFP4> { typedef bf16x8_t type; };

template <int SCH>
RLXQ_DEV typename SkOp<SCH>::type sk_b(const uint32_t* bp, int g) {
  if constexpr (SCH == SCH_MXFP4) {
    const float sc = __uint_as_float(bp[0]);
    const uint32_t q = bp[1 + g];
    const u32x4_t b = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 0)),
                       __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 1)),
                       __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 2)),
                       __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 3))};
    return __builtin_bit_cast(bf16x8_t, b);
  } else {
    return dequant_lane<SCH>(bp, g);
  }
}

template <int SCH>
RLXQ_DEV f32x4_t sk_mfma(f16x8_t a, typename SkOp<SCH>::type b, f32x4_t c) {
  if constexpr (SCH == SCH_MXFP4)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Raw block -> normalised dwords.
template <int SCH>
RLXQ_DEV void normalise(const RawBlk<SCH>& r, uint32_t* o) {
  if constexpr (SCH == SCH_Q6_K) {
    const float d = f16_bits_to_f32(r.d);
    const float ds0 = d * (float)(int8_t)(r.sc & 0xffu), ds1 = d * (float)(int8_t)(r.sc >> 8);
    o[0] = f32_to_f16_bits(ds0) | (f32_to_f16_bits(ds1) << 16);
    const uint32_t s1 = 4u * (r.q >> 1), s2 = 2u * r.q;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t l = align_bytes(r.ql[i + 1], r.ql[i], r.off), hq = align_bytes(r.qh[i + 1], r.qh[i], r.off);
      // code (0..63) + 96 per byte: no carry between bytes
      o[1 + i] = (((l >> s1) & 0x0F0F0F0Fu) | (((hq >> s2) & 0x03030303u) << 4)) + 0x60606060u;
    }
  } else if constexpr (SCH == SCH_Q4_K) {
    const uint32_t hd[4] = {r.hd.x, r.hd.y, r.hd.z, r.hd.w};
    float sc, mn;
    q4k_scale_min(hd, (int)r.sub, sc, mn);
    const uint32_t d1 = f32_to_f16_bits(f16_bits_to_f32(hd[0] & 0xffffu) * sc);
    const uint32_t m1 = f32_to_f16_bits(-(f16_bits_to_f32(hd[0] >> 16) * mn));
    o[0] = d1 | (m1 << 16);
    const uint32_t qs[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t sh = 4 * (r.sub & 1u);
#pragma unroll
    for (int g = 0; g < 4; g++) o[1 + g] = ((qs[g] >> sh) & 0x0F0F0F0Fu) | (((qs[4 + g] >> sh) & 0x0F0F0F0Fu) << 4);
  } else if constexpr (SCH == SCH_MXFP4) {
    o[0] = __float_as_uint(r.s);
    o[1] = r.q.x; o[2] = r.q.y; o[3] = r.q.z; o[4] = r.q.w;
  } else if constexpr (SCH == SCH_MLX4) {
    o[0] = f32_to_f16_bits(r.s) | (f32_to_f16_bits(r.b) << 16);
    o[1] = r.q.x; o[2] = r.q.y; o[3] = r.q.z; o[4] = r.q.w;
  } else if constexpr (SCH == SCH_MLX8) {
    o[0] = f32_to_f16_bits(r.s) | (f32_to_f16_bits(r.b) << 16);
    o[1] = r.q0.x; o[2] = r.q0.y; o[3] = r.q0.z; o[4] = r.q0.w;
    o[5] = r.q1.x; o[6] = r.q1.y; o[7] = r.q1.z; o[8] = r.q1.w;
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
