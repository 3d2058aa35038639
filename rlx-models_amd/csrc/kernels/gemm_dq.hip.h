// Per-block weight loaders shared by the MFMA kernels: raw bytes of one
// 32-weight block (loaded ahead of use) and their conversion to bf16 pairs.
#pragma once
#include "common.hip.h"
#include "gemm_args.h"

namespace rlxq {

// Raw bytes of one 32-weight block, loaded ahead of their conversion so the
// global loads of a K step can be in flight while the previous step computes.
// All-zero raw bytes convert to zero weights (d = 0, or scale = bias = 0).
template <int SCH> struct RawBlk;
template <> struct RawBlk<SCH_Q4_1> { uint32_t h; uint4 q; };
template <> struct RawBlk<SCH_Q4_0> { uint32_t w[5]; uint32_t off; };
template <> struct RawBlk<SCH_Q8_0> { uint32_t w[9]; uint32_t off; };
template <> struct RawBlk<SCH_MLX4> { uint4 q; float s, b; };
template <> struct RawBlk<SCH_MLX8> { uint4 q0, q1; float s, b; };
// Q4_K: block kb is sub-block kb % 8 of super-block kb / 8: the super-block's
// head and the 32 code bytes of its group (low nibbles for even sub-blocks)
template <> struct RawBlk<SCH_Q4_K> { uint4 hd; uint4 q0, q1; uint32_t sub; };
// Q6_K: block kb is quarter (kb & 3) of half (kb >> 2) & 1 of super-block
// kb / 8: 32 ql bytes and the half's 32 qh bytes as 9 aligned dwords each
// (210-byte super-blocks start 2-byte aligned; `off` is 0 or 2), the dword
// holding the two int8 scales and the one holding f16 d.
template <> struct RawBlk<SCH_Q6_K> { uint32_t ql[9], qh[9], sc, d; uint32_t off, q; };
// Q5_K: the super-block's 16-byte head (as Q4_K's), the 32 qs bytes of the
// sub-block's pair and qh[32]; `sub` = kb % 8.
template <> struct RawBlk<SCH_Q5_K> { uint4 hd, q0, q1, h0, h1; uint32_t sub; };
// Q3_K: block kb is quarter j = kb % 4 of half n = (kb / 4) % 2 of super-block
// kb / 8: the half's 32 qs bytes and hmask[32] as 9 aligned dwords each
// (110-byte super-blocks start 2-byte aligned; `off` is 0 or 2) and the 4
// aligned dwords holding the 12 scale bytes and f16 d.
template <> struct RawBlk<SCH_Q3_K> { uint32_t qs[9], hm[9], sd[4]; uint32_t off, sub; };
// Q2_K: the half's 32 qs bytes, the two scale/min bytes of the block and the
// dword of f16 d | f16 dmin; `sub` = kb % 8.
template <> struct RawBlk<SCH_Q2_K> { uint4 q0, q1; uint32_t sc, dd, sub; };
// Q8_K: f32 d and the 32 int8 codes of sub-block kb % 8 of super-block kb / 8.
template <> struct RawBlk<SCH_Q8_K> { uint4 q0, q1; float d; };
// MXFP4: 16 bytes of E2M1 codes and the block's slab scale, raw.
template <> struct RawBlk<SCH_MXFP4> { uint4 q; float s; };

// Loads block `kb` of weight row `row` (a valid row); `ok` = false zeroes it
// with selects, so the caller's loop body stays free of branches.
template <int SCH>
RLXQ_DEV void load_blk(const rlxq_gemm_args& a, int64_t row, int64_t kb, bool ok, RawBlk<SCH>& r) {
  const uint8_t* rp = a.w + row * a.rb;
  if constexpr (SCH == SCH_Q6_K) {
    // GGML block_q6_K: ql[128], qh[64], int8 scales[16], f16 d (offset 208)
    const uint8_t* sb = rp + (kb >> 3) * 210;
    const int h = (int)((kb >> 2) & 1), q = (int)(kb & 3);
    const uint32_t off = (uint32_t)reinterpret_cast<uintptr_t>(sb) & 3u;
    const uint8_t* al = sb - off;   // aligned: every read below stays in the super-block or the one before
    const uint8_t* pl = al + 64 * h + 32 * (q & 1);
    const uint8_t* ph = al + 128 + 32 * h;
#pragma unroll
    for (int i = 0; i < 9; i++) {
      r.ql[i] = ld_u32(pl + 4 * i);
      r.qh[i] = ld_u32(ph + 4 * i);
    }
    // the two scales and d, each read from the aligned dword that holds it
    const uint32_t po = off + 192 + 8 * h + 2 * q;
    r.sc = (ld_u32(al + (po & ~3u)) >> (8 * (po & 3u))) & 0xffffu;
    // (the load is not left to the select: the compiler would move it into a
    // branch and wait for it there)
    uint32_t dw = ld_u32(al + 208);
    asm volatile("" : "+v"(dw));
    r.d = ok ? (dw >> (8 * off)) & 0xffffu : 0u;   // zero d: no weight
    r.off = off;
    r.q = (uint32_t)q;
  } else if constexpr (SCH == SCH_Q5_K) {
    // GGML block_q5_K: f16 d, f16 dmin, scales[12], qh[32] (16), qs[128] (48)
    const uint8_t* sb = rp + (kb >> 3) * 176;
    const uint4 h = ld_u128(sb);
    r.hd = ok ? h : make_uint4(0u, 0u, 0u, 0u);   // zero head: d = dmin = 0
    const uint8_t* q = sb + 48 + 32 * ((kb & 7) >> 1);
    r.q0 = ld_u128(q);
    r.q1 = ld_u128(q + 16);
    r.h0 = ld_u128(sb + 16);
    r.h1 = ld_u128(sb + 32);
    r.sub = (uint32_t)(kb & 7);
  } else if constexpr (SCH == SCH_Q3_K) {
    // GGML block_q3_K: hmask[32], qs[64] (32), scales[12] (96), f16 d (108)
    const uint8_t* sb = rp + (kb >> 3) * 110;
    const int n = (int)((kb >> 2) & 1);
    const uint32_t off = (uint32_t)reinterpret_cast<uintptr_t>(sb) & 3u;
    const uint8_t* al = sb - off;   // aligned: every read below stays in the super-block or the one before
#pragma unroll
    for (int i = 0; i < 9; i++) {
      r.qs[i] = ld_u32(al + 32 + 32 * n + 4 * i);
      r.hm[i] = ld_u32(al + 4 * i);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) r.sd[i] = ld_u32(al + 96 + 4 * i);
    // (d is the last two bytes; a zero d zeroes the block)
    if (!ok) r.sd[3] = 0u;
    r.off = off;
    r.sub = (uint32_t)(kb & 7);
  } else if constexpr (SCH == SCH_Q2_K) {
    // GGML block_q2_K: scales[16], qs[64] (16), f16 d (80), f16 dmin (82)
    const uint8_t* sb = rp + (kb >> 3) * 84;
    const int blk = (int)(kb & 7), n = blk >> 2, j = blk & 3;
    r.q0 = ld_u128(sb + 16 + 32 * n);
    r.q1 = ld_u128(sb + 32 + 32 * n);
    const uint32_t so = 8 * n + 2 * j;   // scale bytes so, so + 1
    r.sc = (ld_u32(sb + (so & ~3u)) >> (8 * (so & 3u))) & 0xffffu;
    uint32_t dd = ld_u32(sb + 80);
    asm volatile("" : "+v"(dd));
    r.dd = ok ? dd : 0u;
    r.sub = (uint32_t)blk;
  } else if constexpr (SCH == SCH_Q8_K) {
    const uint8_t* sb = rp + (kb >> 3) * 292;
    const float d = *reinterpret_cast<const float*>(sb);
    r.d = ok ? d : 0.f;
    r.q0 = ld_u128(sb + 4 + 32 * (kb & 7));
    r.q1 = ld_u128(sb + 20 + 32 * (kb & 7));
  } else if constexpr (SCH == SCH_MXFP4) {
    r.q = ld_u128(rp + kb * 16);
    const int64_t gi = row * (int64_t)(a.K / 32) + kb;
    const uint8_t* sp = reinterpret_cast<const uint8_t*>(a.scales);
    // E8M0 byte (sb_bf16 == 2) or bf16 (1): two byte loads from addresses
    // chosen without a branch, both in bounds either way
    const int64_t i0 = a.sb_bf16 == 2 ? gi : 2 * gi;
    const uint32_t lo = sp[i0], hi = sp[a.sb_bf16 == 2 ? i0 : i0 + 1];
    const float s = a.sb_bf16 == 2 ? e8m0_to_f32(lo) : bf16_bits_to_f32(lo | (hi << 8));
    r.s = ok ? s : 0.f;
  } else if constexpr (SCH == SCH_Q4_K) {
    const uint8_t* sb = rp + (kb >> 3) * 144;
    const uint4 h = ld_u128(sb);
    r.hd = ok ? h : make_uint4(0u, 0u, 0u, 0u);   // zero head: d = dmin = 0
    const uint8_t* q = sb + 16 + 32 * ((kb & 7) >> 1);
    r.q0 = ld_u128(q);
    r.q1 = ld_u128(q + 16);
    r.sub = (uint32_t)(kb & 7);
  } else if constexpr (SCH == SCH_Q4_1) {
    const uint8_t* p = rp + kb * 20;
    r.h = ok ? ld_u32(p) : 0u;
    const uint4 q = ld_u128(p + 4);
    r.q = q;
  } else if constexpr (SCH == SCH_Q4_0 || SCH == SCH_Q8_0) {
    // 18- and 34-byte blocks are 2-byte aligned: read the dwords covering the
    // block without touching a byte beyond it (the tail is a 16-bit load when
    // the block starts dword aligned)
    constexpr int BB = SCH == SCH_Q4_0 ? 18 : 34, NW = SCH == SCH_Q4_0 ? 5 : 9;
    const uint32_t off = (uint32_t)(kb * BB) & 3u;
    const uint8_t* base = rp + kb * BB - off;
#pragma unroll
    for (int i = 0; i < NW - 1; i++) r.w[i] = ld_u32(base + 4 * i);
    r.w[NW - 1] = off ? ld_u32(base + 4 * (NW - 1))
                      : (uint32_t)*reinterpret_cast<const uint16_t*>(base + 4 * (NW - 1));
    r.off = off;
    if (!ok) r.w[0] = 0u, r.w[1] = 0u;  // zero scale (it sits in w[0] or the low half of w[1])
  } else {
    constexpr int BITS = SCH == SCH_MLX4 ? 4 : 8;
    const uint8_t* q = rp + kb * BITS * 4;
    const int64_t gi = row * (int64_t)(a.K / a.group) + (kb * 32) / a.group;
    float s, bi;
    if (a.sb_bf16) {
      s = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.scales)[gi]);
      bi = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.biases)[gi]);
    } else {
      s = reinterpret_cast<const float*>(a.scales)[gi];
      bi = reinterpret_cast<const float*>(a.biases)[gi];
    }
    r.s = ok ? s : 0.f;
    r.b = ok ? bi : 0.f;
    if constexpr (SCH == SCH_MLX4) {
      r.q = ld_u128(q);
    } else {
      r.q0 = ld_u128(q);
      r.q1 = ld_u128(q + 16);
    }
  }
}

template <int SCH>
RLXQ_DEV void blk_f32(const RawBlk<SCH>& r, float* v);

// Power-of-two factor on the f16 weight operands of the exact-weight MFMA
// paths, undone in the activation row factors (post_exp = -8): 2^8 keeps the
// small scales of the f32-scaled formats (MLX affine's f32 scales, Q8_K's f32
// d, Q2_K's per-half d * sc) and their f16 remainders out of the subnormal
// range.  Weights then have to stay below 2^8 in magnitude.
template <int SCH> constexpr float sk_wscale() {
  return (SCH == SCH_MLX4 || SCH == SCH_MLX8 || SCH == SCH_Q8_K || SCH == SCH_Q2_K) ? 256.f : 1.f;
}

// Q3_K block kb's two 16-weight half scales d * (scale - 32), exact in f32:
// scale s = 8n + 2j + half (n = (kb / 4) % 2, j = kb % 4), 6 bits held as
// the low nibble of byte s % 8 (the high nibble past 7) and bits 2 (s / 4)
// .. + 1 of byte 8 + s % 4 of the 12 scale bytes.
RLXQ_DEV void q3k_half_scales(const RawBlk<SCH_Q3_K>& r, float& ds0, float& ds1) {
  const uint32_t w0 = align_bytes(r.sd[1], r.sd[0], r.off), w1 = align_bytes(r.sd[2], r.sd[1], r.off),
                 w2 = align_bytes(r.sd[3], r.sd[2], r.off);
  const float d = f16_bits_to_f32((r.sd[3] >> (8 * r.off)) & 0xffffu);
  // byte i of the 12 scale bytes (selects, not a runtime array index)
  auto byte = [&](uint32_t i) { return ((i < 4 ? w0 : (i < 8 ? w1 : w2)) >> (8 * (i & 3))) & 0xffu; };
  auto scale = [&](uint32_t s6) {
    return (int)(((byte(s6 & 7) >> (4 * (s6 >> 3))) & 15) | (((byte(8 + (s6 & 3)) >> (2 * (s6 >> 2))) & 3) << 4));
  };
  const uint32_t s0 = 8 * (r.sub >> 2) + 2 * (r.sub & 3);
  ds0 = d * (float)(scale(s0) - 32);
  ds1 = d * (float)(scale(s0 + 1) - 32);
}

// Converts a raw block into 16 dwords of bf16 pairs in natural element order:
// f32 d*q + m (the CPU decoder's arithmetic), rounded to bf16 (nearest even).
template <int SCH>
RLXQ_DEV void conv_blk(const RawBlk<SCH>& r, uint32_t* out) {
  if constexpr (SCH == SCH_MXFP4) {
    // E2M1 x scale, one conversion per code pair: exact in bf16 for E8M0
    // scales (powers of two); with a bf16 scale the f32 product is rounded
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      out[4 * i + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q[i], r.s, 0));
      out[4 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q[i], r.s, 1));
      out[4 * i + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q[i], r.s, 2));
      out[4 * i + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q[i], r.s, 3));
    }
  } else {
    float v[32];
    blk_f32<SCH>(r, v);
#pragma unroll
    for (int i = 0; i < 16; i++) out[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
  }
}

// A raw block's 32 weights in f32, natural element order, with the CPU
// decoder's arithmetic (d*q + m, one rounding where it has one).
template <int SCH>
RLXQ_DEV void blk_f32(const RawBlk<SCH>& r, float* v) {
  if constexpr (SCH == SCH_Q6_K) {
    // code = (ql >> 4 (q >> 1) & 15) | (qh >> 2q & 3) << 4 for each byte;
    // w = (d * sc) * (code - 32), computed as fma(d * sc, code, -32 (d * sc))
    // (exact: -32 (d * sc) is)
    const float d = f16_bits_to_f32(r.d);
    const float ds0 = d * (float)(int8_t)(r.sc & 0xffu), ds1 = d * (float)(int8_t)(r.sc >> 8);
    const uint32_t s1 = 4u * (r.q >> 1), s2 = 2u * r.q;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t l = align_bytes(r.ql[i + 1], r.ql[i], r.off), hq = align_bytes(r.qh[i + 1], r.qh[i], r.off);
      uint32_t c = ((l >> s1) & 0x0F0F0F0Fu) | (((hq >> s2) & 0x03030303u) << 4);
      asm volatile("" : "+v"(c));
      const float ds = i < 4 ? ds0 : ds1;
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = fmaf(ds, (float)((c >> (8 * e)) & 0xffu), -32.f * ds);
    }
  } else if constexpr (SCH == SCH_Q5_K) {
    // code = (qs >> 4 (sub & 1) & 15) | (qh >> sub & 1) << 4; w = (d sc) code -
    // dmin mn with the products exact in f32, so one fma
    const uint32_t hd[4] = {r.hd.x, r.hd.y, r.hd.z, r.hd.w};
    float sc, mn;
    q4k_scale_min(hd, (int)r.sub, sc, mn);
    const float d1 = f16_bits_to_f32(hd[0] & 0xffffu) * sc, m1 = f16_bits_to_f32(hd[0] >> 16) * mn;
    const uint32_t qs[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
    const uint32_t sh = 4u * (r.sub & 1u);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t c = ((qs[i] >> sh) & 0x0F0F0F0Fu) | (((qh[i] >> r.sub) & 0x01010101u) << 4);
      asm volatile("" : "+v"(c));
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = fmaf(d1, (float)((c >> (8 * e)) & 0xffu), -m1);
    }
  } else if constexpr (SCH == SCH_Q3_K) {
    // code = (qs >> 2j & 3) - (hmask bit 4n + j ? 0 : 4) with the half's
    // scale d (scale - 32), exact products rounded once
    const uint32_t n = r.sub >> 2, j = r.sub & 3;
    float dl0, dl1;
    q3k_half_scales(r, dl0, dl1);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t q = align_bytes(r.qs[i + 1], r.qs[i], r.off), hm = align_bytes(r.hm[i + 1], r.hm[i], r.off);
      // code + 4 = low bits | 4 (mask bit set)
      uint32_t c = ((q >> (2 * j)) & 0x03030303u) | (((hm >> (4 * n + j)) & 0x01010101u) << 2);
      asm volatile("" : "+v"(c));
      const float dl = i < 4 ? dl0 : dl1;
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = fmaf(dl, (float)((c >> (8 * e)) & 0xffu), -4.f * dl);
    }
  } else if constexpr (SCH == SCH_Q2_K) {
    // code = qs >> 2j & 3; w = (d (c & 15)) code - dmin (c >> 4), the products
    // exact, so one fma
    const float d = f16_bits_to_f32(r.dd & 0xffffu), dmin = f16_bits_to_f32(r.dd >> 16);
    const uint32_t j = r.sub & 3;
    const uint32_t c0 = r.sc & 0xffu, c1 = (r.sc >> 8) & 0xffu;
    const float dl0 = d * (float)(c0 & 15u), ml0 = dmin * (float)(c0 >> 4);
    const float dl1 = d * (float)(c1 & 15u), ml1 = dmin * (float)(c1 >> 4);
    const uint32_t qs[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t c = (qs[i] >> (2 * j)) & 0x03030303u;
      asm volatile("" : "+v"(c));
      const float dl = i < 4 ? dl0 : dl1, ml = i < 4 ? ml0 : ml1;
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = fmaf(dl, (float)((c >> (8 * e)) & 0xffu), -ml);
    }
  } else if constexpr (SCH == SCH_Q8_K) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = r.d * (float)(int8_t)((q[i] >> (8 * e)) & 0xffu);
  } else if constexpr (SCH == SCH_Q4_K) {
    const uint32_t hd[4] = {r.hd.x, r.hd.y, r.hd.z, r.hd.w};
    float sc, mn;
    q4k_scale_min(hd, (int)r.sub, sc, mn);
    const float d1 = f16_bits_to_f32(hd[0] & 0xffffu) * sc, m1 = -(f16_bits_to_f32(hd[0] >> 16) * mn);
    const uint32_t qs[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const int sh = 4 * (int)(r.sub & 1u);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t c = (qs[i] >> sh) & 0x0F0F0F0Fu;
      asm volatile("" : "+v"(c));
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = fmaf(d1, (float)((c >> (8 * e)) & 0xffu), m1);
    }
  } else if constexpr (SCH == SCH_Q4_1 || SCH == SCH_Q4_0) {
    uint32_t qs[4];
    float d, m;
    if constexpr (SCH == SCH_Q4_1) {
      qs[0] = r.q.x; qs[1] = r.q.y; qs[2] = r.q.z; qs[3] = r.q.w;
      d = f16_bits_to_f32(r.h & 0xffffu);
      m = f16_bits_to_f32(r.h >> 16);
    } else {
      const uint32_t hd = r.off ? (r.w[0] >> 16) : (r.w[0] & 0xffffu);
      // qs starts 2 bytes after the block start: byte off + 2 of the span
      // (v_alignbyte takes shifts 0..3, so a 4-byte shift is the next dword)
#pragma unroll
      for (int i = 0; i < 4; i++) qs[i] = r.off ? r.w[i + 1] : align_bytes(r.w[i + 1], r.w[i], 2);
      d = f16_bits_to_f32(hd);
      m = -8.f * d;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t lo = qs[i] & 0x0F0F0F0Fu, hi = (qs[i] >> 4) & 0x0F0F0F0Fu;
      // opaque to the optimiser, so each byte converts with one v_cvt_f32_ubyteN
      asm volatile("" : "+v"(lo), "+v"(hi));
      v[4 * i + 0] = fmaf(d, (float)(lo & 0xffu), m);
      v[4 * i + 1] = fmaf(d, (float)((lo >> 8) & 0xffu), m);
      v[4 * i + 2] = fmaf(d, (float)((lo >> 16) & 0xffu), m);
      v[4 * i + 3] = fmaf(d, (float)(lo >> 24), m);
      v[16 + 4 * i + 0] = fmaf(d, (float)(hi & 0xffu), m);
      v[16 + 4 * i + 1] = fmaf(d, (float)((hi >> 8) & 0xffu), m);
      v[16 + 4 * i + 2] = fmaf(d, (float)((hi >> 16) & 0xffu), m);
      v[16 + 4 * i + 3] = fmaf(d, (float)(hi >> 24), m);
    }
  } else if constexpr (SCH == SCH_Q8_0) {
    const float d = f16_bits_to_f32(r.off ? (r.w[0] >> 16) : (r.w[0] & 0xffffu));
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t q = r.off ? r.w[i + 1] : align_bytes(r.w[i + 1], r.w[i], 2);
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = d * (float)(int8_t)((q >> (8 * e)) & 0xffu);
    }
  } else {
    // MLX affine: codes LSB-first in u32 words, scale * code + bias
    constexpr int BITS = SCH == SCH_MLX4 ? 4 : 8;
    uint32_t wq[BITS];
    if constexpr (SCH == SCH_MLX4) {
      wq[0] = r.q.x; wq[1] = r.q.y; wq[2] = r.q.z; wq[3] = r.q.w;
    } else {
      wq[0] = r.q0.x; wq[1] = r.q0.y; wq[2] = r.q0.z; wq[3] = r.q0.w;
      wq[4] = r.q1.x; wq[5] = r.q1.y; wq[6] = r.q1.z; wq[7] = r.q1.w;
    }
    constexpr int PER = 32 / BITS;
#pragma unroll
    for (int i = 0; i < BITS; i++)
#pragma unroll
      for (int e = 0; e < PER; e++) v[PER * i + e] = fmaf(r.s, (float)((wq[i] >> (BITS * e)) & ((1u << BITS) - 1u)), r.b);
  }
}

// Half h of a raw block's f32 weights (elements 16h .. 16h + 15, natural
// order), h given as a bit mask (all ones for the second half), the same
// arithmetic as blk_f32.  The nibble formats pick their code half before
// converting; the others convert the whole block and pick by the mask
// (bit operations: a select on h became an indexed access into a scratch
// copy of the block's values).
template <int SCH>
RLXQ_DEV void blk_f32_half(const RawBlk<SCH>& r, uint32_t mh, float* v) {
  auto pick4 = [&](uint4 a0, uint4 a1) {
    return make_uint4((a1.x & mh) | (a0.x & ~mh), (a1.y & mh) | (a0.y & ~mh), (a1.z & mh) | (a0.z & ~mh),
                      (a1.w & mh) | (a0.w & ~mh));
  };
  if constexpr (SCH == SCH_Q4_1 || SCH == SCH_Q4_0) {
    uint32_t qs[4];
    float d, m;
    if constexpr (SCH == SCH_Q4_1) {
      qs[0] = r.q.x; qs[1] = r.q.y; qs[2] = r.q.z; qs[3] = r.q.w;
      d = f16_bits_to_f32(r.h & 0xffffu);
      m = f16_bits_to_f32(r.h >> 16);
    } else {
      const uint32_t hd = r.off ? (r.w[0] >> 16) : (r.w[0] & 0xffffu);
#pragma unroll
      for (int i = 0; i < 4; i++) qs[i] = r.off ? r.w[i + 1] : align_bytes(r.w[i + 1], r.w[i], 2);
      d = f16_bits_to_f32(hd);
      m = -8.f * d;
    }
    // elements 0..15: low nibbles, 16..31: high nibbles
    const uint32_t sh = mh & 4u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t c = (qs[i] >> sh) & 0x0F0F0F0Fu;
      asm volatile("" : "+v"(c));
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = fmaf(d, (float)((c >> (8 * e)) & 0xffu), m);
    }
  } else if constexpr (SCH == SCH_Q4_K) {
    const uint32_t hd[4] = {r.hd.x, r.hd.y, r.hd.z, r.hd.w};
    float sc, mn;
    q4k_scale_min(hd, (int)r.sub, sc, mn);
    const float d1 = f16_bits_to_f32(hd[0] & 0xffffu) * sc, m1 = -(f16_bits_to_f32(hd[0] >> 16) * mn);
    const uint4 q = pick4(r.q0, r.q1);
    const uint32_t qs[4] = {q.x, q.y, q.z, q.w};
    const int sh = 4 * (int)(r.sub & 1u);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t c = (qs[i] >> sh) & 0x0F0F0F0Fu;
      asm volatile("" : "+v"(c));
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = fmaf(d1, (float)((c >> (8 * e)) & 0xffu), m1);
    }
  } else {
    float w[32];
    blk_f32<SCH>(r, w);
#pragma unroll
    for (int e = 0; e < 16; e++) v[e] = __uint_as_float((__float_as_uint(w[16 + e]) & mh) | (__float_as_uint(w[e]) & ~mh));
  }
}

// The block's f32 weights times `scale` (a power of two) as f16 hi and lo
// halves, natural order, two per dword: hi = f16(w), lo = f16(w - hi), so
// that hi + lo keeps ~22 significant bits of the f32 weight.
template <int SCH>
RLXQ_DEV void conv_blk_f16_split(const RawBlk<SCH>& r, float scale, uint32_t* hi, uint32_t* lo) {
  float v[32];
  blk_f32<SCH>(r, v);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const float a = v[2 * i] * scale, b = v[2 * i + 1] * scale;
    const uint32_t ha = f32_to_f16_bits(a), hb = f32_to_f16_bits(b);
    hi[i] = ha | (hb << 16);
    lo[i] = f32_to_f16_bits(a - f16_bits_to_f32(ha)) | (f32_to_f16_bits(b - f16_bits_to_f32(hb)) << 16);
  }
}

// Dequantize one 32-weight block of row `row` (K-block `kb`) into 16 dwords of
// bf16 pairs in natural element order.  `ok` = false yields zeros.
template <int SCH>
RLXQ_DEV void dequant_block_bf16(const rlxq_gemm_args& a, int64_t row, int64_t kb, bool ok, uint32_t* out) {
  RawBlk<SCH> r;
  load_blk<SCH>(a, row, kb, ok, r);
  conv_blk<SCH>(r, out);
}

}  // namespace rlxq
