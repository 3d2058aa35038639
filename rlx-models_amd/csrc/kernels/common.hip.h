// Device-side helpers shared by the gfx950 kernels of librlxq.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#define RLXQ_DEV __device__ __forceinline__

// A large kernel file is compiled as several code objects, each holding the
// instantiations of one part (-DRLXQ_PART=i); without RLXQ_PART a file holds
// all of them.
#ifdef RLXQ_PART
#define RLXQ_PART_IS(i) (RLXQ_PART == (i))
#else
#define RLXQ_PART_IS(i) 1
#endif

typedef __bf16 rlxq_bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 rlxq_f16x2_t __attribute__((ext_vector_type(2)));

namespace rlxq {
// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N - 1>{})
template <class F, int... I>
RLXQ_DEV void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
RLXQ_DEV void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
}  // namespace rlxq

// Scheme ids (same numbering as include/rlxq.h).
enum : int {
  SCH_Q8_0 = 1,
  SCH_Q4_0 = 2,
  SCH_Q4_1 = 3,
  SCH_MLX4 = 4,
  SCH_MLX8 = 5,
  SCH_Q4_K = 7,
  SCH_Q6_K = 8,
  SCH_MXFP4 = 9,
  SCH_Q5_K = 10,
  SCH_Q3_K = 11,
  SCH_Q2_K = 12,
  SCH_Q8_K = 13,
};

// MXFP4 (OCP microscaling FP4): E2M1 codes, two per byte (low nibble = even
// element), and one E8M0 exponent byte b per 32 codes, scale 2^(b - 127).
// b = 0 reads as 0 and b = 255 as 2^127, as the reference decoder's clamped
// exponent (crates/rlx-models-core/src/mxfp4_pack.rs:130-135, 263-281).
RLXQ_DEV float e8m0_to_f32(uint32_t b) { return __uint_as_float((b < 254u ? b : 254u) << 23); }

// The two E2M1 codes of byte SEL of w as a bf16 pair (low nibble in the low
// half), exact: v_cvt_scalef32_pk_bf16_fp4 with scale 1.
template <int SEL>
RLXQ_DEV uint32_t fp4x2_to_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, SEL));
}

// GGUF Q4_K: 6-bit scale and min of sub-block s (0..7) from a super-block's
// 16-byte head held as dwords (head[0] = f16 d | f16 dmin << 16, head[1..3] =
// the 12 packed bytes), GGML's packing.
RLXQ_DEV void q4k_scale_min(const uint32_t* head, int s, float& sc, float& mn) {
  // (the dword picked by selects, not by a runtime array index, which would
  // keep the caller's copy of the head in scratch memory)
  const uint32_t h1 = head[1], h2 = head[2], h3 = head[3];
  auto byte = [&](int i) {
    const uint32_t w = i < 4 ? h1 : (i < 8 ? h2 : h3);
    return (w >> (8 * (i & 3))) & 0xffu;
  };
  uint32_t a, b;
  if (s < 4) {
    a = byte(s) & 63u;
    b = byte(s + 4) & 63u;
  } else {
    a = (byte(s + 4) & 15u) | ((byte(s - 4) >> 6) << 4);
    b = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
  }
  sc = (float)a;
  mn = (float)b;
}

// D = a.lo*b.lo + a.hi*b.hi + c with bf16 pairs and an f32 accumulator
// (v_dot2c_f32_bf16).  Products of two bf16 values are exact in f32.
RLXQ_DEV float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(rlxq_bf16x2_t, a),
                                         __builtin_bit_cast(rlxq_bf16x2_t, b), c, false);
}

// Same with f16 pairs (v_dot2c_f32_f16).  Products of two f16 values are
// exact in f32.
RLXQ_DEV float dot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(rlxq_f16x2_t, a),
                                __builtin_bit_cast(rlxq_f16x2_t, b), c, false);
}

RLXQ_DEV float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

// f32 -> bf16 bits with the hardware conversion (v_cvt_pk_bf16_f32: round to
// nearest even, NaN stays NaN).
RLXQ_DEV uint32_t f32_to_bf16_bits(float v) { return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v); }

typedef __bf16 rlxq_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float rlxq_f32x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> one dword of two bf16 (lo in bits 0..15), one v_cvt_pk_bf16_f32.
RLXQ_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((rlxq_f32x2_t){lo, hi}, rlxq_bf16x2_t));
}

RLXQ_DEV float f16_bits_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// f32 -> f16 bits with the hardware conversion (round to nearest even).
RLXQ_DEV uint32_t f32_to_f16_bits(float v) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
}

// 32-bit byte funnel: bytes [s, s+4) of the 8-byte value hi:lo.
RLXQ_DEV uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t s) {
  return __builtin_amdgcn_alignbyte(hi, lo, s);
}

RLXQ_DEV uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Workgroup -> output tile (tm, tn) of a tiles_m x tiles_n grid.  The
// dispatcher deals workgroups to the 8 XCDs round-robin (workgroup b runs on
// XCD b % 8) and every XCD has its own L2, so each XCD is given a contiguous
// range of logical tiles; logical tiles run in bands of GM tile-rows, so the
// workgroups resident on one XCD at a time share activation rows and weight
// columns in that L2.  The grid is launched rounded up to a multiple of 8;
// returns false for the padding workgroups.
RLXQ_DEV bool tile_of(int bid, int tiles_m, int tiles_n, int GM, int& tm, int& tn) {
  const int G = tiles_m * tiles_n;
  const int per = (G + 7) >> 3;
  const int logical = (bid & 7) * per + (bid >> 3);
  if (logical >= G) return false;
  const int band = GM * tiles_n;
  const int first = (logical / band) * GM;
  const int gm = tiles_m - first < GM ? tiles_m - first : GM;
  const int r = logical % band;
  tm = first + r % gm;
  tn = r / gm;
  return true;
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int WIDTH>
RLXQ_DEV float group_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Global loads.  GGUF blocks are 18/20/34 bytes, so a 16-byte load is only
// dword aligned; the vector type says so (global_load_dwordx4 needs 4).
typedef uint32_t rlxq_u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
RLXQ_DEV uint32_t ld_u32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
RLXQ_DEV uint4 ld_u128(const uint8_t* p) {
  rlxq_u32x4_a4 v = *reinterpret_cast<const rlxq_u32x4_a4*>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
