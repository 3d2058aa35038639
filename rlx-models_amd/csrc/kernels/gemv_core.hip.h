// Building blocks of the dequant-GEMV family (dense decode and grouped
// experts): per-scheme unit geometry, activation records, code unpacking and
// block dot products.  See gemv.hip for how they are put together.
#pragma once
#include "common.hip.h"
#include "gemv_args.h"

namespace rlxq {

template <int SCH>
struct Unit;
template <>
struct Unit<SCH_Q4_1> {
  static constexpr int BLOCKS = 1, BYTES = 20, DW = 5;
  static constexpr bool BIT8 = false;
};
template <>
struct Unit<SCH_Q4_0> {
  static constexpr int BLOCKS = 2, BYTES = 36, DW = 9;
  static constexpr bool BIT8 = false;
};
template <>
struct Unit<SCH_Q8_0> {
  static constexpr int BLOCKS = 2, BYTES = 68, DW = 17;
  static constexpr bool BIT8 = true;
};
template <>
struct Unit<SCH_MLX4> {
  static constexpr int BLOCKS = 1, BYTES = 16, DW = 4;
  static constexpr bool BIT8 = false;
};
template <>
struct Unit<SCH_MLX8> {
  static constexpr int BLOCKS = 1, BYTES = 32, DW = 8;
  static constexpr bool BIT8 = true;
};
// MXFP4: 16 code bytes per 32 weights (the MLX 4-bit code layout), the E8M0
// scale in a slab of its own.
template <>
struct Unit<SCH_MXFP4> {
  static constexpr int BLOCKS = 1, BYTES = 16, DW = 4;
  static constexpr bool BIT8 = false;
};

// Schemes whose scales live in a slab of their own (MLX affine: scale and
// bias; MXFP4: scale only).
template <int SCH>
RLXQ_DEV constexpr bool slab_scales() {
  return SCH == SCH_MLX4 || SCH == SCH_MLX8 || SCH == SCH_MXFP4;
}
template <int SCH>
RLXQ_DEV constexpr bool slab_bias() {
  return SCH == SCH_MLX4 || SCH == SCH_MLX8;
}
// GGUF Q4_K: a unit is one 64-weight group of a 256-weight super-block (two
// 32-weight sub-blocks sharing 32 code bytes): the super-block's 16-byte head
// (f16 d, f16 dmin, 12 bytes of 6-bit scales and mins) plus the group's 32
// code bytes.  BYTES is the row stride per unit (144 / 4).
template <>
struct Unit<SCH_Q4_K> {
  static constexpr int BLOCKS = 2, BYTES = 36, DW = 12;
  static constexpr bool BIT8 = false;
};
// GGUF Q6_K: a unit is one 32-weight sub-block (half h, quarter j) of a
// 210-byte super-block, which is only 2-byte aligned: the nine aligned dwords
// covering its 32 ql bytes and the nine covering its 32 qh bytes, its two
// int8 scales, the f16 d, and a word with the alignment and j (computed from
// the address, not loaded).  BYTES is the row stride per unit (210 / 8).
template <>
struct Unit<SCH_Q6_K> {
  static constexpr int BLOCKS = 1, BYTES = 26, DW = 21;
  static constexpr bool BIT8 = true;   // 6-bit codes take the byte path (f16 1024 + code)
};

// GGUF Q5_K: a unit is one 64-weight group (sub-blocks 2g, 2g + 1) of a
// 176-byte super-block: the 16-byte head (f16 d, f16 dmin, the Q4_K scale
// bytes), the 32 qh bytes (the fifth code bit of every weight, bit 2g + h),
// the group's 32 qs bytes, and g (computed).  BYTES is the row stride per
// unit (176 / 4).
template <>
struct Unit<SCH_Q5_K> {
  static constexpr int BLOCKS = 2, BYTES = 44, DW = 21;
  static constexpr bool BIT8 = false;
};
// GGUF Q8_K: a unit is one 32-weight block of a 292-byte super-block: its 32
// int8 codes and the super-block's f32 d (load_unit_at addresses the
// super-block; 292 / 8 is not a whole byte count).
template <>
struct Unit<SCH_Q8_K> {
  static constexpr int BLOCKS = 1, BYTES = 36, DW = 9;
  static constexpr bool BIT8 = true;
};
// GGUF Q2_K: a unit is one 32-weight block (n, j) = (b / 4, b % 4) of an
// 84-byte super-block: the 32 qs bytes of half n (2-bit codes at bit 2j),
// the dword holding its two scale bytes (scale | min << 4 for its two
// 16-weight halves), the f16 d | f16 dmin dword, and j (computed).
template <>
struct Unit<SCH_Q2_K> {
  static constexpr int BLOCKS = 1, BYTES = 10, DW = 11;
  static constexpr bool BIT8 = false;
};
// GGUF Q3_K: a unit is one 32-weight block (n, j) of a 110-byte super-block,
// which is only 2-byte aligned: the nine aligned dwords covering the 32
// hmask bytes (bit 4n + j) and the nine covering its 32 qs bytes (bit 2j),
// its two scales' low-nibble bytes and high-bit bytes (16-bit loads), the f16
// d, and a word with the alignment, j and n (computed).
template <>
struct Unit<SCH_Q3_K> {
  static constexpr int BLOCKS = 1, BYTES = 13, DW = 22;
  static constexpr bool BIT8 = false;
};
// K-quants whose 32-weight blocks carry a scale per 16 weights.
template <int SCH>
RLXQ_DEV constexpr bool half_scales() {
  return SCH == SCH_Q6_K || SCH == SCH_Q2_K || SCH == SCH_Q3_K;
}

// Offset that the code -> float trick adds to each code, and the value the
// dot chain starts from (in units of the block's plane sum) so that the chain
// ends at sum(w_int * x) where w_int is the scheme's integer weight:
//   Q4_1/MLX4: q (bias 128)    Q4_0: q - 8 (bias 136)
//   Q8_0: q (bias 1024 + 128, codes stored as q ^ 0x80)   MLX8: code (1024)
//   Q6_K: code - 32 (bias 1024 + 32)
//   Q8_K: q (bias 1024 + 128, as Q8_0)   Q5_K, Q2_K: code (128)
//   Q3_K: (2 bits + 4 * hmask bit) - 4 (bias 132)
//   MXFP4: none (the pairs carry the signed E2M1 values themselves)
template <int SCH>
RLXQ_DEV constexpr float chain_bias() {
  return SCH == SCH_MXFP4 ? 0.f
         : (SCH == SCH_Q4_0 ? 136.f
            : ((SCH == SCH_Q8_0 || SCH == SCH_Q8_K) ? 1152.f
               : (SCH == SCH_MLX8 ? 1024.f : (SCH == SCH_Q6_K ? 1056.f : (SCH == SCH_Q3_K ? 132.f : 128.f)))));
}
// Start of a block's dot chain: -bias * (sum of the block's x).
template <int SCH>
RLXQ_DEV float chain_start(float s) {
  if constexpr (SCH == SCH_MXFP4) return 0.f;
  return -chain_bias<SCH>() * s;
}

// Element pair (a, b) of a 32-element block that plane dword t carries.
template <int SCH>
RLXQ_DEV void plane_pair(int t, int& a, int& b) {
  if constexpr (SCH == SCH_Q4_0 || SCH == SCH_Q4_1) {
    // qs dword i holds bytes 4i..4i+3; byte j = element j (low nibble) and
    // element j+16 (high nibble).  Extraction e shifts by 4e and masks
    // 0x000F000F: e=0 -> (4i, 4i+2), e=1 -> (4i+16, 4i+18),
    // e=2 -> (4i+1, 4i+3), e=3 -> (4i+17, 4i+19).
    int i = t >> 2, e = t & 3;
    int base = 4 * i + ((e & 1) ? 16 : 0) + ((e & 2) ? 1 : 0);
    a = base;
    b = base + 2;
  } else if constexpr (SCH == SCH_Q4_K || SCH == SCH_Q6_K || SCH == SCH_Q5_K || SCH == SCH_Q2_K || SCH == SCH_Q3_K) {
    // code dword i = bytes 4i..4i+3 of the group: low nibbles are the first
    // sub-block's elements 4i..4i+3 (the high ones the second's); extraction
    // e = 0 -> (4i, 4i+2), e = 1 -> (4i+1, 4i+3).
    int i = t >> 1, e = t & 1;
    a = 4 * i + e;
    b = 4 * i + e + 2;
  } else if constexpr (SCH == SCH_MLX4) {
    // u32 word i holds codes 8i..8i+7 LSB-first; extraction e -> (8i+e, 8i+e+4).
    int i = t >> 2, e = t & 3;
    a = 8 * i + e;
    b = 8 * i + e + 4;
  } else if constexpr (SCH == SCH_MXFP4) {
    // code byte t converts to (2t, 2t+1)
    a = 2 * t;
    b = 2 * t + 1;
  } else {
    // byte codes, dword i = codes 4i..4i+3; e=0 -> (4i, 4i+2), e=1 -> (4i+1, 4i+3).
    int i = t >> 1, e = t & 1;
    a = 4 * i + e;
    b = 4 * i + e + 2;
  }
}

// Record layout (dwords): NPL planes of 16 pair-dwords, then
// [S = sum of the plane values, SX = sum of x, SCL = block x scale, 0].
template <int NPL>
struct Rec {
  static constexpr int STRIDE = NPL * 16 + 4;
};

// Sum / max over aligned groups of 8 lanes (DPP quad butterflies, then the
// half-row mirror); every lane of the group gets the result.
RLXQ_DEV float group8_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  return v;
}
RLXQ_DEV float group4_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  return v;
}
RLXQ_DEV float group8_max(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
  return v;
}
RLXQ_DEV uint32_t swap_lane_pair(uint32_t v) {  // value of lane ^ 1
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}

// Building the x records of MT activation rows into LDS.  Eight lanes share
// a record; lane q converts elements 4q..4q+3 of it and writes the two plane
// dwords they form (and their lo twins), lane 0 of the group the sums and the
// block scale.  Tasks (record, q) of one activation row are numbered
// 8*block + q; a thread handles tasks threadIdx.x + i*blockDim.x in batches of
// XB: stage_fetch issues a batch's activation loads, stage_store converts and
// writes it.  The loop structure is uniform over the workgroup (the group
// reductions use DPP).
template <bool XBF16>
struct XRaw {
  static constexpr int XB = XBF16 ? 8 : 4;
  uint32_t w[XB][XBF16 ? 2 : 4];
};

template <bool XBF16>
RLXQ_DEV void stage_fetch(XRaw<XBF16>& raw, const void* xv, int64_t row, int64_t M, int K, int base) {
  constexpr int XB = XRaw<XBF16>::XB;
  const int ntask = (K >> 5) * 8;
#pragma unroll
  for (int i = 0; i < XB; i++) {
    const int task = base + i * blockDim.x + threadIdx.x;
    const int64_t off = row * (int64_t)K + 4 * task;
    if constexpr (XBF16) {
      uint2 u = make_uint2(0u, 0u);
      if (task < ntask && row < M) u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(xv) + off);
      raw.w[i][0] = u.x;
      raw.w[i][1] = u.y;
    } else {
      uint4 u = make_uint4(0u, 0u, 0u, 0u);
      if (task < ntask && row < M) u = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(xv) + off);
      raw.w[i][0] = u.x; raw.w[i][1] = u.y; raw.w[i][2] = u.z; raw.w[i][3] = u.w;
    }
  }
}

template <int SCH, bool XBF16, int NPL>
RLXQ_DEV void stage_store(uint32_t* lds, const XRaw<XBF16>& raw, int m, int K, int base) {
  constexpr bool BIT8 = Unit<SCH>::BIT8;
  constexpr int RS = Rec<NPL>::STRIDE;
  constexpr int XB = XRaw<XBF16>::XB;
  const int bpr = K >> 5;
  const int ntask = bpr * 8;
#pragma unroll
  for (int i = 0; i < XB; i++) {
    if (base + i * (int)blockDim.x >= ntask) break;  // uniform
    const int task = base + i * blockDim.x + threadIdx.x;
    const bool active = task < ntask;
    const int r = m * bpr + (task >> 3), q = task & 7;
    float v[4];
    if constexpr (XBF16) {
      v[0] = bf16_bits_to_f32(raw.w[i][0] & 0xffffu);
      v[1] = bf16_bits_to_f32(raw.w[i][0] >> 16);
      v[2] = bf16_bits_to_f32(raw.w[i][1] & 0xffffu);
      v[3] = bf16_bits_to_f32(raw.w[i][1] >> 16);
    } else {
#pragma unroll
      for (int k = 0; k < 4; k++) v[k] = __uint_as_float(raw.w[i][k]);
    }
    const float sx = group8_sum((v[0] + v[1]) + (v[2] + v[3]));
    float scl = 1.f;
    if constexpr (BIT8) {
      const float amax = group8_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
      if (amax > 0.f && amax < INFINITY) {
        const int e = ilogbf(amax) - 14;  // scaled max lands in [2^14, 2^15)
        scl = ldexpf(1.f, e);
        const float inv = ldexpf(1.f, -e);
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] *= inv;
      }
    }
    uint32_t hi[4], lo[4];
    float ps = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      if constexpr (BIT8) {
        hi[k] = f32_to_f16_bits(v[k]);
        const float hv = f16_bits_to_f32(hi[k]);
        lo[k] = NPL == 2 ? f32_to_f16_bits(v[k] - hv) : 0u;
        ps += NPL == 2 ? hv + f16_bits_to_f32(lo[k]) : hv;
      } else if constexpr (XBF16) {
        hi[k] = __float_as_uint(v[k]) >> 16;  // exact: the input is bf16
        lo[k] = 0u;
      } else {
        hi[k] = f32_to_bf16_bits(v[k]);
        const float hv = bf16_bits_to_f32(hi[k]);
        lo[k] = f32_to_bf16_bits(v[k] - hv);
        ps += hv + bf16_bits_to_f32(lo[k]);
      }
    }
    const float S = (!BIT8 && XBF16) ? sx : group8_sum(ps);
    // sum of the record's first 16 elements (lanes q < 4; the per-half
    // scales of Q6_K, Q2_K, Q3_K)
    float S_lo = 0.f;
    if constexpr (half_scales<SCH>()) S_lo = group4_sum((!BIT8 && XBF16) ? (v[0] + v[1]) + (v[2] + v[3]) : ps);
    // the two plane dwords of this lane and their positions t0, t1
    uint32_t h0, h1, l0 = 0u, l1 = 0u;
    int t0, t1;
    if constexpr (SCH == SCH_MXFP4) {
      // pairs (4q, 4q+1) and (4q+2, 4q+3)
      h0 = hi[0] | (hi[1] << 16);
      h1 = hi[2] | (hi[3] << 16);
      l0 = lo[0] | (lo[1] << 16);
      l1 = lo[2] | (lo[3] << 16);
      t0 = 2 * q;
      t1 = 2 * q + 1;
    } else if constexpr (SCH == SCH_MLX4) {
      // pairs (8j+e, 8j+e+4): even lanes hold 8j..8j+3, odd lanes 8j+4..8j+7
      const uint32_t hp01 = swap_lane_pair(hi[0] | (hi[1] << 16)), hp23 = swap_lane_pair(hi[2] | (hi[3] << 16));
      const uint32_t lp01 = swap_lane_pair(lo[0] | (lo[1] << 16)), lp23 = swap_lane_pair(lo[2] | (lo[3] << 16));
      const int j = q >> 1;
      if ((q & 1) == 0) {
        h0 = hi[0] | (hp01 << 16);
        h1 = hi[1] | (hp01 & 0xffff0000u);
        l0 = lo[0] | (lp01 << 16);
        l1 = lo[1] | (lp01 & 0xffff0000u);
        t0 = 4 * j;
        t1 = 4 * j + 1;
      } else {
        h0 = (hp23 & 0xffffu) | (hi[2] << 16);
        h1 = (hp23 >> 16) | (hi[3] << 16);
        l0 = (lp23 & 0xffffu) | (lo[2] << 16);
        l1 = (lp23 >> 16) | (lo[3] << 16);
        t0 = 4 * j + 2;
        t1 = 4 * j + 3;
      }
    } else {
      // pairs (4q, 4q+2) and (4q+1, 4q+3)
      h0 = hi[0] | (hi[2] << 16);
      h1 = hi[1] | (hi[3] << 16);
      l0 = lo[0] | (lo[2] << 16);
      l1 = lo[1] | (lo[3] << 16);
      if constexpr (BIT8 || SCH == SCH_Q4_K || SCH == SCH_Q6_K || SCH == SCH_Q5_K || SCH == SCH_Q2_K ||
                    SCH == SCH_Q3_K) {
        t0 = 2 * q;
        t1 = 2 * q + 1;
      } else {
        // GGUF nibble order: elements 4i.. -> e = 0/2, elements 16+4i.. -> e = 1/3
        t0 = q < 4 ? 4 * q : 4 * (q - 4) + 1;
        t1 = t0 + 2;
      }
    }
    if (active) {
      uint32_t* rec = lds + (size_t)r * RS;
      rec[t0] = h0;
      rec[t1] = h1;
      if constexpr (NPL == 2) {
        rec[16 + t0] = l0;
        rec[16 + t1] = l1;
      }
      if (q == 0) {
        rec[NPL * 16 + 0] = __float_as_uint(S);
        rec[NPL * 16 + 1] = __float_as_uint(sx);
        rec[NPL * 16 + 2] = __float_as_uint(scl);
        rec[NPL * 16 + 3] = __float_as_uint(S_lo);
      }
    }
  }
}

// Constants of the code -> float tricks, held in VGPRs so that the unpack
// compiles to one v_and_or_b32 per pair (a VOP3 instruction on gfx950 cannot
// take two literal operands).
struct UnpackK {
  uint32_t mask, magic;
};
RLXQ_DEV UnpackK unpack_consts() {
  UnpackK k{0x000F000Fu, 0x43004300u};
  asm volatile("" : "+v"(k.mask), "+v"(k.magic));
  return k;
}

// 4-bit: four bf16 (128 + q) pairs per dword of nibbles.
RLXQ_DEV void nib_pairs(uint32_t w, uint32_t* out, const UnpackK& k) {
  out[0] = (w & k.mask) | k.magic;
  out[1] = ((w >> 4) & k.mask) | k.magic;
  out[2] = ((w >> 8) & k.mask) | k.magic;
  out[3] = ((w >> 12) & k.mask) | k.magic;
}

// 8-bit: two f16 (1024 + u) pairs per dword of unsigned byte codes.
RLXQ_DEV void byte_pairs(uint32_t u, uint32_t* out) {
  out[0] = perm_b32(0x64646464u, u, 0x04020400u);
  out[1] = perm_b32(0x64646464u, u, 0x04030401u);
}

// Fetch one unit at p (always a valid address; out-of-range units are
// clamped by the caller and their scales zeroed).
template <int SCH>
RLXQ_DEV void load_unit(uint32_t* dw, const uint8_t* p) {
  if constexpr (SCH == SCH_Q4_1) {
    dw[0] = ld_u32(p);
    uint4 q = ld_u128(p + 4);
    dw[1] = q.x; dw[2] = q.y; dw[3] = q.z; dw[4] = q.w;
  } else if constexpr (SCH == SCH_Q4_0) {
    uint4 a = ld_u128(p), b = ld_u128(p + 16);
    dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
    dw[4] = b.x; dw[5] = b.y; dw[6] = b.z; dw[7] = b.w;
    dw[8] = ld_u32(p + 32);
  } else if constexpr (SCH == SCH_Q8_0) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint4 a = ld_u128(p + 16 * q);
      dw[4 * q] = a.x; dw[4 * q + 1] = a.y; dw[4 * q + 2] = a.z; dw[4 * q + 3] = a.w;
    }
    dw[16] = ld_u32(p + 64);
  } else if constexpr (SCH == SCH_MLX4 || SCH == SCH_MXFP4) {
    uint4 a = ld_u128(p);
    dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
  } else if constexpr (SCH == SCH_Q4_K) {
    static_assert(SCH != SCH_Q4_K, "Q4_K units are fetched with load_unit_at");
  } else {
    uint4 a = ld_u128(p), b = ld_u128(p + 16);
    dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
    dw[4] = b.x; dw[5] = b.y; dw[6] = b.z; dw[7] = b.w;
  }
}

// Unit u of the packed row at rp.  Q4_K: super-block u / 4 (16-byte head)
// and its 32 code bytes of group u % 4, all 16-byte aligned loads.
template <int SCH>
RLXQ_DEV void load_unit_at(uint32_t* dw, const uint8_t* rp, int u) {
  if constexpr (SCH == SCH_Q5_K) {
    const uint8_t* sb = rp + (int64_t)(u >> 2) * 176;
    const int g = u & 3;
    const uint4 h = ld_u128(sb), qh0 = ld_u128(sb + 16), qh1 = ld_u128(sb + 32);
    const uint4 q0 = ld_u128(sb + 48 + 32 * g), q1 = ld_u128(sb + 64 + 32 * g);
    dw[0] = h.x; dw[1] = h.y; dw[2] = h.z; dw[3] = h.w;
    dw[4] = qh0.x; dw[5] = qh0.y; dw[6] = qh0.z; dw[7] = qh0.w;
    dw[8] = qh1.x; dw[9] = qh1.y; dw[10] = qh1.z; dw[11] = qh1.w;
    dw[12] = q0.x; dw[13] = q0.y; dw[14] = q0.z; dw[15] = q0.w;
    dw[16] = q1.x; dw[17] = q1.y; dw[18] = q1.z; dw[19] = q1.w;
    dw[20] = (uint32_t)g;
  } else if constexpr (SCH == SCH_Q8_K) {
    const uint8_t* sb = rp + (int64_t)(u >> 3) * 292;
    const uint8_t* c = sb + 4 + 32 * (u & 7);
    const uint4 a = ld_u128(c), b = ld_u128(c + 16);
    dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
    dw[4] = b.x; dw[5] = b.y; dw[6] = b.z; dw[7] = b.w;
    dw[8] = ld_u32(sb);
  } else if constexpr (SCH == SCH_Q2_K) {
    const uint8_t* sb = rp + (int64_t)(u >> 3) * 84;
    const int n = (u >> 2) & 1, j = u & 3;
    const uint4 a = ld_u128(sb + 16 + 32 * n), b = ld_u128(sb + 32 + 32 * n);
    dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
    dw[4] = b.x; dw[5] = b.y; dw[6] = b.z; dw[7] = b.w;
    dw[8] = ld_u32(sb + 8 * n + 4 * (j >> 1));   // scale bytes 8n + 2j, 8n + 2j + 1
    dw[9] = ld_u32(sb + 80);                      // f16 d | f16 dmin
    dw[10] = (uint32_t)j;
  } else if constexpr (SCH == SCH_Q3_K) {
    const uint8_t* sb = rp + (int64_t)(u >> 3) * 110;
    const int n = (u >> 2) & 1, j = u & 3;
    const uint32_t off = (uint32_t)reinterpret_cast<uintptr_t>(sb) & 3u;   // 0 or 2
    const uint8_t* hm = sb - off;
    const uint8_t* qs = sb + 32 + 32 * n - off;
    const uint4 h0 = ld_u128(hm), h1 = ld_u128(hm + 16), q0 = ld_u128(qs), q1 = ld_u128(qs + 16);
    dw[0] = h0.x; dw[1] = h0.y; dw[2] = h0.z; dw[3] = h0.w;
    dw[4] = h1.x; dw[5] = h1.y; dw[6] = h1.z; dw[7] = h1.w;
    dw[8] = ld_u32(hm + 32);
    dw[9] = q0.x; dw[10] = q0.y; dw[11] = q0.z; dw[12] = q0.w;
    dw[13] = q1.x; dw[14] = q1.y; dw[15] = q1.z; dw[16] = q1.w;
    dw[17] = ld_u32(qs + 32);
    // scales 8n + 2j and 8n + 2j + 1: low nibbles in bytes 2j, 2j + 1 (the
    // high nibbles for n = 1), bits 4..5 in bytes 8 + 2 (j & 1), + 1
    dw[18] = *reinterpret_cast<const uint16_t*>(sb + 96 + 2 * j);
    dw[19] = *reinterpret_cast<const uint16_t*>(sb + 104 + 2 * (j & 1));
    dw[20] = *reinterpret_cast<const uint16_t*>(sb + 108);
    dw[21] = off | ((uint32_t)j << 8) | ((uint32_t)n << 16);
  } else if constexpr (SCH == SCH_Q6_K) {
    const uint8_t* sb = rp + (int64_t)(u >> 3) * 210;
    const int h = (u >> 2) & 1, j = u & 3;
    const uint32_t off = (uint32_t)reinterpret_cast<uintptr_t>(sb) & 3u;   // 0 or 2
    const uint8_t* ql = sb + 64 * h + 32 * (j & 1) - off;
    const uint8_t* qh = sb + 128 + 32 * h - off;
    // 4-byte aligned: two 16-byte loads and a dword each
    const uint4 l0 = ld_u128(ql), l1 = ld_u128(ql + 16), h0 = ld_u128(qh), h1 = ld_u128(qh + 16);
    dw[0] = l0.x; dw[1] = l0.y; dw[2] = l0.z; dw[3] = l0.w;
    dw[4] = l1.x; dw[5] = l1.y; dw[6] = l1.z; dw[7] = l1.w;
    dw[8] = ld_u32(ql + 32);
    dw[9] = h0.x; dw[10] = h0.y; dw[11] = h0.z; dw[12] = h0.w;
    dw[13] = h1.x; dw[14] = h1.y; dw[15] = h1.z; dw[16] = h1.w;
    dw[17] = ld_u32(qh + 32);
    dw[18] = *reinterpret_cast<const uint16_t*>(sb + 192 + 8 * h + 2 * j);
    dw[19] = *reinterpret_cast<const uint16_t*>(sb + 208);
    dw[20] = off | ((uint32_t)j << 8);
  } else if constexpr (SCH == SCH_Q4_K) {
    const uint8_t* sb = rp + (int64_t)(u >> 2) * 144;
    const uint4 h = ld_u128(sb), a = ld_u128(sb + 16 + 32 * (u & 3)), b = ld_u128(sb + 32 + 32 * (u & 3));
    dw[0] = h.x; dw[1] = h.y; dw[2] = h.z; dw[3] = h.w;
    dw[4] = a.x; dw[5] = a.y; dw[6] = a.z; dw[7] = a.w;
    dw[8] = b.x; dw[9] = b.y; dw[10] = b.z; dw[11] = b.w;
  } else {
    load_unit<SCH>(dw, rp + (int64_t)u * Unit<SCH>::BYTES);
  }
}

// Q2_K / Q3_K: the two 16-weight halves' multipliers of the code chains (d,
// d2) and of the halves' x sums (m, m2; Q2_K: minus dmin * min, Q3_K: 0).
template <int SCH>
RLXQ_DEV void block_scales_half(const uint32_t* dw, float& d, float& d2, float& m, float& m2) {
  if constexpr (SCH == SCH_Q2_K) {
    const uint32_t c = (dw[8] >> (16 * (dw[10] & 1))) & 0xffffu;   // bytes 8n + 2j, + 1
    const float dd = f16_bits_to_f32(dw[9] & 0xffffu), dm = f16_bits_to_f32(dw[9] >> 16);
    d = dd * (float)(c & 15u);
    m = -(dm * (float)((c >> 4) & 15u));
    d2 = dd * (float)((c >> 8) & 15u);
    m2 = -(dm * (float)(c >> 12));
  } else {
    const uint32_t j = (dw[21] >> 8) & 3u, n = dw[21] >> 16;
    const uint32_t ls = 4 * n, hs = 2 * (2 * n + (j >> 1));
    const int s0 = (int)(((dw[18] >> ls) & 15u) | (((dw[19] >> hs) & 3u) << 4));
    const int s1 = (int)(((dw[18] >> (8 + ls)) & 15u) | (((dw[19] >> (8 + hs)) & 3u) << 4));
    const float dd = f16_bits_to_f32(dw[20] & 0xffffu);
    d = dd * (float)(s0 - 32);
    d2 = dd * (float)(s1 - 32);
    m = 0.f;
    m2 = 0.f;
  }
}

// Block scale terms of block `blk` of a fetched unit: d multiplies the dot
// chain, m (Q4_1 min; Q4_K minus dmin * min) multiplies the block sum of x.
// u is the unit's index in its row (Q4_K: which group of the super-block).
template <int SCH>
RLXQ_DEV void block_scales(const uint32_t* dw, int blk, float& d, float& m, int u = 0) {
  if constexpr (SCH == SCH_Q5_K) {
    // (the head copied out: a runtime index into the 21-dword unit would
    // keep the whole unit in scratch memory)
    const uint32_t head[4] = {dw[0], dw[1], dw[2], dw[3]};
    float sc, mn;
    q4k_scale_min(head, 2 * (int)dw[20] + blk, sc, mn);
    d = f16_bits_to_f32(dw[0] & 0xffffu) * sc;
    m = -(f16_bits_to_f32(dw[0] >> 16) * mn);
    return;
  }
  if constexpr (SCH == SCH_Q8_K) {
    d = __uint_as_float(dw[8]);
    m = 0.f;
    return;
  }
  if constexpr (SCH == SCH_Q2_K || SCH == SCH_Q3_K) {
    float d2, m2;
    block_scales_half<SCH>(dw, d, d2, m, m2);
    return;
  }
  if constexpr (SCH == SCH_Q6_K) {
    // d * scale of the block's first and second 16 weights (both exact)
    const float dd = f16_bits_to_f32(dw[19] & 0xffffu);
    d = dd * (float)(int8_t)(dw[18] & 0xffu);
    m = dd * (float)(int8_t)((dw[18] >> 8) & 0xffu);
    return;
  }
  if constexpr (SCH == SCH_Q4_K) {
    float sc, mn;
    q4k_scale_min(dw, 2 * (u & 3) + blk, sc, mn);
    d = f16_bits_to_f32(dw[0] & 0xffffu) * sc;
    m = -(f16_bits_to_f32(dw[0] >> 16) * mn);
    return;
  }
  if constexpr (SCH == SCH_Q4_1) {
    d = f16_bits_to_f32(dw[0] & 0xffffu);
    m = f16_bits_to_f32(dw[0] >> 16);
  } else if constexpr (SCH == SCH_Q4_0 || SCH == SCH_Q8_0) {
    constexpr int HI = SCH == SCH_Q4_0 ? 4 : 8;  // dword holding block B's d in its high half
    d = blk == 0 ? f16_bits_to_f32(dw[0] & 0xffffu) : f16_bits_to_f32(dw[HI] >> 16);
    m = 0.f;
  } else {
    d = 0.f;
    m = 0.f;
  }
}

// The 16 pair-dwords of block `blk` of a fetched unit.
template <int SCH>
RLXQ_DEV void block_pairs(const uint32_t* dw, int blk, uint32_t* pw, const UnpackK& k) {
  if constexpr (SCH == SCH_Q4_1) {
#pragma unroll
    for (int i = 0; i < 4; i++) nib_pairs(dw[1 + i], &pw[4 * i], k);
  } else if constexpr (SCH == SCH_Q4_0) {
    if (blk == 0) {
      // block A: d = bytes 0-1, qs = bytes 2..17 (re-aligned by 2 bytes)
#pragma unroll
      for (int i = 0; i < 4; i++) nib_pairs(align_bytes(dw[i + 1], dw[i], 2), &pw[4 * i], k);
    } else {
      // block B: d = bytes 18-19, qs = bytes 20..35
#pragma unroll
      for (int i = 0; i < 4; i++) nib_pairs(dw[5 + i], &pw[4 * i], k);
    }
  } else if constexpr (SCH == SCH_Q8_0) {
    if (blk == 0) {
#pragma unroll
      for (int i = 0; i < 8; i++) byte_pairs(align_bytes(dw[i + 1], dw[i], 2) ^ 0x80808080u, &pw[2 * i]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) byte_pairs(dw[9 + i] ^ 0x80808080u, &pw[2 * i]);
    }
  } else if constexpr (SCH == SCH_MLX4) {
#pragma unroll
    for (int i = 0; i < 4; i++) nib_pairs(dw[i], &pw[4 * i], k);
  } else if constexpr (SCH == SCH_MXFP4) {
    // byte t of the 16 code bytes -> the E2M1 values of elements (2t, 2t+1)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      pw[4 * i + 0] = fp4x2_to_bf16x2<0>(dw[i]);
      pw[4 * i + 1] = fp4x2_to_bf16x2<1>(dw[i]);
      pw[4 * i + 2] = fp4x2_to_bf16x2<2>(dw[i]);
      pw[4 * i + 3] = fp4x2_to_bf16x2<3>(dw[i]);
    }
  } else if constexpr (SCH == SCH_Q6_K) {
    // code = (ql nibble j >> 1) | (qh bits 2j..2j+1) << 4 for four elements
    // at once (one byte each), then f16 (1024 + code) pairs
    const uint32_t off = dw[20] & 3u, j = dw[20] >> 8;
    const uint32_t ns = 4 * (j >> 1), hs = 2 * j;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t ql = off ? align_bytes(dw[i + 1], dw[i], 2) : dw[i];
      const uint32_t qh = off ? align_bytes(dw[10 + i], dw[9 + i], 2) : dw[9 + i];
      byte_pairs(((ql >> ns) & 0x0F0F0F0Fu) | (((qh >> hs) & 0x03030303u) << 4), &pw[2 * i]);
    }
  } else if constexpr (SCH == SCH_Q5_K) {
    // sub-block 2g + blk: nibble blk of the group's qs bytes, fifth bit from
    // bit 2g + blk of the qh bytes; bf16 (128 + code) pairs
    const uint32_t hs = 2 * dw[20] + blk;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t c = ((dw[12 + i] >> (4 * blk)) & 0x0F0F0F0Fu) | (((dw[4 + i] >> hs) & 0x01010101u) << 4);
      pw[2 * i] = (c & 0x001F001Fu) | 0x43004300u;
      pw[2 * i + 1] = ((c >> 8) & 0x001F001Fu) | 0x43004300u;
    }
  } else if constexpr (SCH == SCH_Q8_K) {
#pragma unroll
    for (int i = 0; i < 8; i++) byte_pairs(dw[i] ^ 0x80808080u, &pw[2 * i]);
  } else if constexpr (SCH == SCH_Q2_K) {
    // bits 2j..2j+1 of the half's 32 qs bytes (elements 0..15: bytes 0..15)
    const uint32_t sh = 2 * dw[10];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t c = (dw[i] >> sh) & 0x03030303u;
      pw[2 * i] = (c & 0x00030003u) | 0x43004300u;
      pw[2 * i + 1] = ((c >> 8) & 0x00030003u) | 0x43004300u;
    }
  } else if constexpr (SCH == SCH_Q3_K) {
    // 2 bits (qs bit 2j) + 4 * (hmask bit 4n + j): 0..7 = code + 4
    const uint32_t off = dw[21] & 3u, j = (dw[21] >> 8) & 3u, n = dw[21] >> 16;
    const uint32_t qsh = 2 * j, hsh = 4 * n + j;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t hm = off ? align_bytes(dw[i + 1], dw[i], 2) : dw[i];
      const uint32_t qv = off ? align_bytes(dw[10 + i], dw[9 + i], 2) : dw[9 + i];
      const uint32_t c = ((qv >> qsh) & 0x03030303u) | (((hm >> hsh) & 0x01010101u) << 2);
      pw[2 * i] = (c & 0x00070007u) | 0x43004300u;
      pw[2 * i + 1] = ((c >> 8) & 0x00070007u) | 0x43004300u;
    }
  } else if constexpr (SCH == SCH_Q4_K) {
    // sub-block blk: the low (0) or high (1) nibbles of the group's 32 bytes
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t w = dw[4 + i] >> (4 * blk);
      pw[2 * i] = (w & k.mask) | k.magic;
      pw[2 * i + 1] = ((w >> 8) & k.mask) | k.magic;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) byte_pairs(dw[i], &pw[2 * i]);
  }
}

// Q6_K: the block's two 16-weight halves carry their own scale, so the
// chain runs per half from -bias times the half's sum (record word
// NPL*16+3 holds the first half's sum) and each half takes its d * scale;
// the record's power-of-two block factor scales the result.
template <int NPL>
RLXQ_DEV float q6k_block_dot(const uint32_t* pw, const uint32_t* xr, float d_lo, float d_hi) {
  const float s = __uint_as_float(xr[NPL * 16 + 0]), s_lo = __uint_as_float(xr[NPL * 16 + 3]);
  const float scl = __uint_as_float(xr[NPL * 16 + 2]);
  float lo = -chain_bias<SCH_Q6_K>() * s_lo, hi = -chain_bias<SCH_Q6_K>() * (s - s_lo);
#pragma unroll
  for (int t = 0; t < 8; t++) {
    lo = dot2_f16(pw[t], xr[t], lo);
    if constexpr (NPL == 2) lo = dot2_f16(pw[t], xr[16 + t], lo);
    hi = dot2_f16(pw[8 + t], xr[8 + t], hi);
    if constexpr (NPL == 2) hi = dot2_f16(pw[8 + t], xr[24 + t], hi);
  }
  return scl * fmaf(d_lo, lo, d_hi * hi);
}

// Q2_K / Q3_K (bf16 pairs, bias chain_bias): each 16-weight half's chain
// runs from -bias times the half's x sum (record word NPL*16+3 holds the
// first half's) and takes its own multiplier; the mins multiply the halves'
// x sums.
template <int SCH, int NPL>
RLXQ_DEV float khalf_block_dot(const uint32_t* pw, const uint32_t* xr, float d_lo, float d_hi, float m_lo,
                               float m_hi) {
  const float s = __uint_as_float(xr[NPL * 16 + 0]), s_lo = __uint_as_float(xr[NPL * 16 + 3]);
  float lo = -chain_bias<SCH>() * s_lo, hi = -chain_bias<SCH>() * (s - s_lo);
#pragma unroll
  for (int t = 0; t < 8; t++) {
    lo = dot2_bf16(pw[t], xr[t], lo);
    if constexpr (NPL == 2) lo = dot2_bf16(pw[t], xr[16 + t], lo);
    hi = dot2_bf16(pw[8 + t], xr[8 + t], hi);
    if constexpr (NPL == 2) hi = dot2_bf16(pw[8 + t], xr[24 + t], hi);
  }
  float r = fmaf(d_lo, lo, d_hi * hi);
  if constexpr (SCH == SCH_Q2_K) r = fmaf(m_lo, s_lo, fmaf(m_hi, s - s_lo, r));
  return r;
}

// sum over the block of (bias + code) * x, started at -bias * S so that it
// ends at sum(w_int * x).
template <int SCH, int NPL>
RLXQ_DEV float block_dot(const uint32_t* pw, const uint32_t* xr) {
  constexpr bool BIT8 = Unit<SCH>::BIT8;
  float c = chain_start<SCH>(__uint_as_float(xr[NPL * 16 + 0]));
#pragma unroll
  for (int t = 0; t < 16; t++) {
    if constexpr (BIT8) {
      c = dot2_f16(pw[t], xr[t], c);
      if constexpr (NPL == 2) c = dot2_f16(pw[t], xr[16 + t], c);
    } else {
      c = dot2_bf16(pw[t], xr[t], c);
      if constexpr (NPL == 2) c = dot2_bf16(pw[t], xr[16 + t], c);
    }
  }
  return c;
}

// Raw bits of MLX scale/bias idx for the register rings: two 16-bit loads
// issued unconditionally (a bf16 slab: the element, twice; an f32 slab: its
// two halves), so no branch on the slab dtype sits between the ring's loads
// and the wait counts keep them in flight; sb_decode forms the value at use.
struct SbRaw {
  uint32_t lo, hi;
};
RLXQ_DEV SbRaw load_sb_raw(const void* p, int64_t idx, bool bf16) {
  const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
  const int64_t i0 = bf16 ? idx : 2 * idx;
  return {q[i0], q[bf16 ? i0 : i0 + 1]};
}
RLXQ_DEV float sb_decode(SbRaw r, bool bf16) {
  return __uint_as_float(bf16 ? (r.lo << 16) : (r.lo | (r.hi << 16)));
}

// Slab scale of a scheme at idx for the register rings, raw: MLX (f32 or
// bf16, load_sb_raw); MXFP4 (sbt 2: E8M0 bytes, 1: bf16) as two byte loads
// from addresses chosen without a branch, both in bounds either way.
template <int SCH>
RLXQ_DEV SbRaw load_scale_raw(const void* p, int64_t idx, int sbt) {
  if constexpr (SCH == SCH_MXFP4) {
    const uint8_t* b = reinterpret_cast<const uint8_t*>(p);
    const int64_t i0 = sbt == 2 ? idx : 2 * idx;
    return {b[i0], b[sbt == 2 ? i0 : i0 + 1]};
  } else {
    return load_sb_raw(p, idx, sbt == 1);
  }
}
template <int SCH>
RLXQ_DEV float scale_decode(SbRaw r, int sbt) {
  if constexpr (SCH == SCH_MXFP4) return sbt == 2 ? e8m0_to_f32(r.lo) : bf16_bits_to_f32(r.lo | (r.hi << 8));
  return sb_decode(r, sbt == 1);
}

// MLX scale/bias for (row n, block b); sb_bf16 selects the slab dtype.
RLXQ_DEV float load_sb(const void* p, int64_t idx, bool bf16) {
  if (bf16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[idx]);
  return reinterpret_cast<const float*>(p)[idx];
}

// Sum over aligned groups of L lanes with DPP row operations; for L = 64 the
// four 16-lane row sums are combined through readlane, so every lane ends
// with its group's sum.
template <int L>
RLXQ_DEV float lane_group_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  if constexpr (L == 2) return v;
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  if constexpr (L == 4) return v;
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  if constexpr (L == 8) return v;
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  if constexpr (L == 16) return v;
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  if constexpr (L == 32) return (threadIdx.x & 32) ? r2 + r3 : r0 + r1;
  return (r0 + r1) + (r2 + r3);
}

// Plane dwords of one 32-element block from its 16 raw bf16-pair dwords
// R[i] = (x[2i], x[2i+1]), in the extraction order of plane_pair<SCH>.
template <int SCH>
RLXQ_DEV void pairs_from_raw(const uint32_t* R, uint32_t* X) {
  constexpr uint32_t LO = 0x05040100u, HI = 0x07060302u;  // low / high halves of (R[a], R[b])
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if constexpr (SCH == SCH_Q4_K || SCH == SCH_Q5_K) {
      // t = 2j + e holds (4j+e, 4j+e+2): R[2j] and R[2j+1], j = 2i, 2i+1
      X[4 * i + 0] = perm_b32(R[4 * i + 1], R[4 * i], LO);
      X[4 * i + 1] = perm_b32(R[4 * i + 1], R[4 * i], HI);
      X[4 * i + 2] = perm_b32(R[4 * i + 3], R[4 * i + 2], LO);
      X[4 * i + 3] = perm_b32(R[4 * i + 3], R[4 * i + 2], HI);
    } else if constexpr (SCH == SCH_MXFP4) {
      // t holds (2t, 2t+1): the raw pairs as they are
      X[4 * i + 0] = R[4 * i + 0];
      X[4 * i + 1] = R[4 * i + 1];
      X[4 * i + 2] = R[4 * i + 2];
      X[4 * i + 3] = R[4 * i + 3];
    } else if constexpr (SCH == SCH_MLX4) {
      // t = 4i+e holds (8i+e, 8i+e+4): R[4i + e/2] and R[4i + 2 + e/2]
      X[4 * i + 0] = perm_b32(R[4 * i + 2], R[4 * i + 0], LO);
      X[4 * i + 1] = perm_b32(R[4 * i + 2], R[4 * i + 0], HI);
      X[4 * i + 2] = perm_b32(R[4 * i + 3], R[4 * i + 1], LO);
      X[4 * i + 3] = perm_b32(R[4 * i + 3], R[4 * i + 1], HI);
    } else {
      // GGUF nibble order: t = 4i + e, e=0 (4i, 4i+2), e=1 (4i+16, 4i+18),
      // e=2 (4i+1, 4i+3), e=3 (4i+17, 4i+19)
      X[4 * i + 0] = perm_b32(R[2 * i + 1], R[2 * i], LO);
      X[4 * i + 2] = perm_b32(R[2 * i + 1], R[2 * i], HI);
      X[4 * i + 1] = perm_b32(R[2 * i + 9], R[2 * i + 8], LO);
      X[4 * i + 3] = perm_b32(R[2 * i + 9], R[2 * i + 8], HI);
    }
  }
}

}  // namespace rlxq
