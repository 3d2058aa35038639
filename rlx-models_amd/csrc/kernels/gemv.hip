// Dequant-GEMV for decode (M = 1..few rows): y[m, n] = sum_k x[m, k] * W[n, k]
// over packed GGUF Q4_1 / Q4_0 / Q8_0 blocks or MLX affine 4/8-bit codes,
// with fp32 accumulation.  Replaces the backend kernel of Op::DequantMatMul
// (crates/rlx-models-core/src/standard_decoder.rs:727-738).
//
// Work split (one wave64 = 64 lanes):
//   * L lanes own one weight row; a wave covers RP = 64/L rows per pass and
//     P passes, a workgroup of WAVES waves covers WAVES*P*RP rows.
//   * A lane decodes "units" u = li, li+L, li+2L, ... of its row.  A unit is
//     the span that can be fetched with dword-aligned loads: one 20-byte Q4_1
//     block, a pair of 18-byte Q4_0 or 34-byte Q8_0 blocks, or one 32-code MLX
//     group slice.  Consecutive lanes read consecutive units, so a wave's
//     loads cover one contiguous span of the row.
//   * The MT activation rows of the workgroup are staged once in LDS as
//     "x records", one per 32-element block, holding the activations as bf16
//     (4-bit codes) or f16 (8-bit codes) pairs in exactly the order the code
//     extraction below yields them, plus the block sums.
//   * 4-bit codes become bf16 (128 + q) with one and-or per pair; 8-bit codes
//     become f16 (1024 + u) with one byte permute per pair.  v_dot2c
//     accumulates pairs in f32 starting from -bias * (block sum of x), which
//     removes the 128 / 1024 offset, so the block dot is sum(q * x).
//   * f32 activations are split into hi + lo planes so the products keep
//     ~17 (bf16) / ~22 (f16) significant bits; bf16 activations are exact in a
//     single plane.  8-bit schemes scale each block of x by a power of two so
//     that f16 cannot overflow (the factor is folded into the block scale).
#include "common.hip.h"

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

// Offset that the code -> float trick adds to each code, and the value the
// dot chain starts from (in units of the block's plane sum) so that the chain
// ends at sum(w_int * x) where w_int is the scheme's integer weight:
//   Q4_1/MLX4: q (bias 128)    Q4_0: q - 8 (bias 136)
//   Q8_0: q (bias 1024 + 128, codes stored as q ^ 0x80)   MLX8: code (1024)
template <int SCH>
RLXQ_DEV constexpr float chain_bias() {
  return SCH == SCH_Q4_0 ? 136.f : (SCH == SCH_Q8_0 ? 1152.f : (SCH == SCH_MLX8 ? 1024.f : 128.f));
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
  } else if constexpr (SCH == SCH_MLX4) {
    // u32 word i holds codes 8i..8i+7 LSB-first; extraction e -> (8i+e, 8i+e+4).
    int i = t >> 2, e = t & 3;
    a = 8 * i + e;
    b = 8 * i + e + 4;
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

// Build the x records of MT activation rows into LDS.
template <int SCH, bool XBF16, int NPL>
RLXQ_DEV void stage_x(uint32_t* lds, const void* xv, int64_t m0, int64_t M, int K, int MT) {
  constexpr bool BIT8 = Unit<SCH>::BIT8;
  constexpr int RS = Rec<NPL>::STRIDE;
  const int bpr = K >> 5;
  const int nrec = MT * bpr;
  for (int r = threadIdx.x; r < nrec; r += blockDim.x) {
    const int m = r / bpr, b = r - m * bpr;
    float v[32];
    const int64_t row = m0 + m;
    if (row < M) {
      if constexpr (XBF16) {
        const uint4* p = reinterpret_cast<const uint4*>(
            reinterpret_cast<const uint16_t*>(xv) + row * (int64_t)K + (int64_t)b * 32);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          uint4 u = p[q];
          uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int h = 0; h < 4; h++) {
            v[q * 8 + 2 * h] = bf16_bits_to_f32(w4[h] & 0xffffu);
            v[q * 8 + 2 * h + 1] = bf16_bits_to_f32(w4[h] >> 16);
          }
        }
      } else {
        const float4* p = reinterpret_cast<const float4*>(
            reinterpret_cast<const float*>(xv) + row * (int64_t)K + (int64_t)b * 32);
#pragma unroll
        for (int q = 0; q < 8; q++) {
          float4 f = p[q];
          v[4 * q] = f.x;
          v[4 * q + 1] = f.y;
          v[4 * q + 2] = f.z;
          v[4 * q + 3] = f.w;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; i++) v[i] = 0.f;
    }
    float sx = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) sx += v[i];
    float scl = 1.f;
    if constexpr (BIT8) {
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
      if (amax > 0.f && amax < INFINITY) {
        int e = ilogbf(amax) - 14;  // scaled max lands in [2^14, 2^15)
        scl = ldexpf(1.f, e);
        const float inv = ldexpf(1.f, -e);
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] *= inv;
      }
    }
    uint32_t hi[32], lo[32];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      if constexpr (BIT8) {
        hi[i] = f32_to_f16_bits(v[i]);
        const float hv = f16_bits_to_f32(hi[i]);
        if constexpr (NPL == 2) {
          lo[i] = f32_to_f16_bits(v[i] - hv);
          s += hv + f16_bits_to_f32(lo[i]);
        } else {
          lo[i] = 0;
          s += hv;
        }
      } else {
        hi[i] = f32_to_bf16_bits(v[i]);
        const float hv = bf16_bits_to_f32(hi[i]);
        if constexpr (NPL == 2) {
          lo[i] = f32_to_bf16_bits(v[i] - hv);
          s += hv + bf16_bits_to_f32(lo[i]);
        } else {
          lo[i] = 0;
          s += hv;
        }
      }
    }
    uint32_t* rec = lds + (size_t)r * RS;
#pragma unroll
    for (int t = 0; t < 16; t++) {
      int a, bb;
      plane_pair<SCH>(t, a, bb);
      rec[t] = hi[a] | (hi[bb] << 16);
      if constexpr (NPL == 2) rec[16 + t] = lo[a] | (lo[bb] << 16);
    }
    rec[NPL * 16 + 0] = __float_as_uint(s);
    rec[NPL * 16 + 1] = __float_as_uint(sx);
    rec[NPL * 16 + 2] = __float_as_uint(scl);
    rec[NPL * 16 + 3] = 0u;
  }
}

// Decoded block: 16 pair-dwords of (bias + code) values plus its scale terms.
struct DecBlock {
  uint32_t pw[16];
  float d;  // multiplies the dot chain
  float m;  // multiplies the block sum of x (Q4_1 min, MLX bias), else 0
};

// 4-bit: four pairs per qs dword.
RLXQ_DEV void nib_pairs(uint32_t w, uint32_t* out) {
  out[0] = (w & 0x000F000Fu) | 0x43004300u;
  out[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  out[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  out[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
}

// 8-bit: two f16 pairs per dword of unsigned codes.
RLXQ_DEV void byte_pairs(uint32_t u, uint32_t* out) {
  out[0] = perm_b32(0x64646464u, u, 0x04020400u);
  out[1] = perm_b32(0x64646464u, u, 0x04030401u);
}

// Fetch one unit of row `n` (zeros when out of range).
template <int SCH>
RLXQ_DEV void load_unit(uint32_t* dw, const uint8_t* w, int64_t rb, int64_t n, int u, bool ok) {
  constexpr int DW = Unit<SCH>::DW;
  if (!ok) {
#pragma unroll
    for (int i = 0; i < DW; i++) dw[i] = 0u;
    return;
  }
  const uint8_t* p = w + n * rb + (int64_t)u * Unit<SCH>::BYTES;
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
  } else if constexpr (SCH == SCH_MLX4) {
    uint4 a = ld_u128(p);
    dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
  } else {
    uint4 a = ld_u128(p), b = ld_u128(p + 16);
    dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
    dw[4] = b.x; dw[5] = b.y; dw[6] = b.z; dw[7] = b.w;
  }
}

// Decode block `blk` (0 or 1) of a fetched unit.
template <int SCH>
RLXQ_DEV void decode_block(const uint32_t* dw, int blk, float ms, float mb, DecBlock& o) {
  if constexpr (SCH == SCH_Q4_1) {
    o.d = f16_bits_to_f32(dw[0] & 0xffffu);
    o.m = f16_bits_to_f32(dw[0] >> 16);
#pragma unroll
    for (int i = 0; i < 4; i++) nib_pairs(dw[1 + i], &o.pw[4 * i]);
  } else if constexpr (SCH == SCH_Q4_0) {
    o.m = 0.f;
    if (blk == 0) {
      // block A: d = bytes 0-1, qs = bytes 2..17 (re-aligned by 2 bytes)
      o.d = f16_bits_to_f32(dw[0] & 0xffffu);
#pragma unroll
      for (int i = 0; i < 4; i++) nib_pairs(align_bytes(dw[i + 1], dw[i], 2), &o.pw[4 * i]);
    } else {
      // block B: d = bytes 18-19, qs = bytes 20..35
      o.d = f16_bits_to_f32(dw[4] >> 16);
#pragma unroll
      for (int i = 0; i < 4; i++) nib_pairs(dw[5 + i], &o.pw[4 * i]);
    }
  } else if constexpr (SCH == SCH_Q8_0) {
    o.m = 0.f;
    if (blk == 0) {
      o.d = f16_bits_to_f32(dw[0] & 0xffffu);
#pragma unroll
      for (int i = 0; i < 8; i++) byte_pairs(align_bytes(dw[i + 1], dw[i], 2) ^ 0x80808080u, &o.pw[2 * i]);
    } else {
      o.d = f16_bits_to_f32(dw[8] >> 16);
#pragma unroll
      for (int i = 0; i < 8; i++) byte_pairs(dw[9 + i] ^ 0x80808080u, &o.pw[2 * i]);
    }
  } else if constexpr (SCH == SCH_MLX4) {
    o.d = ms;
    o.m = mb;
#pragma unroll
    for (int i = 0; i < 4; i++) nib_pairs(dw[i], &o.pw[4 * i]);
  } else {
    o.d = ms;
    o.m = mb;
#pragma unroll
    for (int i = 0; i < 8; i++) byte_pairs(dw[i], &o.pw[2 * i]);
  }
}

template <int SCH, int NPL>
RLXQ_DEV float block_dot(const DecBlock& db, const uint32_t* xr) {
  constexpr bool BIT8 = Unit<SCH>::BIT8;
  const float S = __uint_as_float(xr[NPL * 16 + 0]);
  float c = -chain_bias<SCH>() * S;
#pragma unroll
  for (int t = 0; t < 16; t++) {
    if constexpr (BIT8) {
      c = dot2_f16(db.pw[t], xr[t], c);
      if constexpr (NPL == 2) c = dot2_f16(db.pw[t], xr[16 + t], c);
    } else {
      c = dot2_bf16(db.pw[t], xr[t], c);
      if constexpr (NPL == 2) c = dot2_bf16(db.pw[t], xr[16 + t], c);
    }
  }
  return c;
}

// MLX scale/bias for (row n, block b); sb_bf16 selects the slab dtype.
RLXQ_DEV float load_sb(const void* p, int64_t idx, bool bf16) {
  if (bf16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[idx]);
  return reinterpret_cast<const float*>(p)[idx];
}

template <int SCH, bool XBF16, int L, int P, int NBC, int MT>
RLXQ_DEV void gemv_body(const void* __restrict__ x, const uint8_t* __restrict__ w,
                        const void* __restrict__ scales, const void* __restrict__ biases,
                        int sb_bf16, int group, void* __restrict__ y, int y_bf16,
                        int64_t M, int K, int64_t N, int64_t rb, const int32_t* __restrict__ row_map,
                        const float* __restrict__ row_scale, int64_t y_ld) {
  constexpr bool BIT8 = Unit<SCH>::BIT8;
  constexpr int NPL = (XBF16 ? 1 : 2);
  constexpr int RS = Rec<NPL>::STRIDE;
  constexpr int BLOCKS = Unit<SCH>::BLOCKS;
  constexpr int DW = Unit<SCH>::DW;
  constexpr int RP = 64 / L;
  constexpr bool MLX = (SCH == SCH_MLX4 || SCH == SCH_MLX8);
  extern __shared__ uint32_t lds[];

  const int bpr = K >> 5;
  const int U = bpr / BLOCKS;
  const int64_t m0 = (int64_t)blockIdx.y * MT;
  stage_x<SCH, XBF16, NPL>(lds, x, m0, M, K, MT);
  __syncthreads();

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane / L, li = lane % L;
  const int waves = blockDim.x >> 6;
  const int64_t row0 = ((int64_t)blockIdx.x * waves + wv) * (P * RP) + g;

  float acc[P][MT];
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[p][m] = 0.f;

  const int nb = (U + L - 1) / L;  // units per lane per row
  for (int j0 = 0; j0 < nb; j0 += NBC) {
    uint32_t dw[P][NBC][DW];
    float msc[P][NBC][BLOCKS], mbi[P][NBC][BLOCKS];
#pragma unroll
    for (int p = 0; p < P; p++) {
      const int64_t n = row0 + p * RP;
#pragma unroll
      for (int jj = 0; jj < NBC; jj++) {
        const int u = li + L * (j0 + jj);
        const bool ok = (n < N) && (u < U) && (j0 + jj < nb);
        load_unit<SCH>(dw[p][jj], w, rb, n, u, ok);
#pragma unroll
        for (int bl = 0; bl < BLOCKS; bl++) {
          msc[p][jj][bl] = 0.f;
          mbi[p][jj][bl] = 0.f;
          if constexpr (MLX) {
            if (ok) {
              const int64_t gi = n * (int64_t)(K / group) + ((int64_t)(u * BLOCKS + bl) * 32) / group;
              msc[p][jj][bl] = load_sb(scales, gi, sb_bf16 != 0);
              mbi[p][jj][bl] = load_sb(biases, gi, sb_bf16 != 0);
            }
          }
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < NBC; jj++) {
      const int u = li + L * (j0 + jj);
      const int uc = u < U ? u : U - 1;
#pragma unroll
      for (int bl = 0; bl < BLOCKS; bl++) {
        DecBlock db[P];
#pragma unroll
        for (int p = 0; p < P; p++) decode_block<SCH>(dw[p][jj], bl, msc[p][jj][bl], mbi[p][jj][bl], db[p]);
        const int b = uc * BLOCKS + bl;
#pragma unroll
        for (int m = 0; m < MT; m++) {
          const uint32_t* xr = lds + (size_t)(m * bpr + b) * RS;
          uint32_t xrec[RS];
#pragma unroll
          for (int t = 0; t < RS; t += 4) {
            uint4 q = *reinterpret_cast<const uint4*>(xr + t);
            xrec[t] = q.x; xrec[t + 1] = q.y; xrec[t + 2] = q.z; xrec[t + 3] = q.w;
          }
          const float sx = __uint_as_float(xrec[NPL * 16 + 1]);
          const float scl = __uint_as_float(xrec[NPL * 16 + 2]);
#pragma unroll
          for (int p = 0; p < P; p++) {
            const float c = block_dot<SCH, NPL>(db[p], xrec);
            const float dd = BIT8 ? db[p].d * scl : db[p].d;
            acc[p][m] = fmaf(dd, c, acc[p][m]);
            if constexpr (SCH == SCH_Q4_1 || MLX) acc[p][m] = fmaf(db[p].m, sx, acc[p][m]);
          }
        }
      }
    }
  }

#pragma unroll
  for (int p = 0; p < P; p++) {
    const int64_t n = row0 + p * RP;
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float v = group_sum<L>(acc[p][m]);
      const int64_t row = m0 + m;
      if (li == 0 && n < N && row < M) {
        int64_t yrow = row;
        float sc = 1.f;
        if (row_map) yrow = row_map[row];
        if (row_scale) sc = row_scale[row];
        if (yrow >= 0) {
          const int64_t off = yrow * y_ld + n;
          if (y_bf16) reinterpret_cast<uint16_t*>(y)[off] = (uint16_t)f32_to_bf16_bits(v * sc);
          else reinterpret_cast<float*>(y)[off] = v * sc;
        }
      }
    }
  }
}

}  // namespace rlxq

// ---------------------------------------------------------------------------
// Instantiations: rlxq_gemv_<scheme>_<x>_L<L>_P<P>_C<NBC>_M<MT>
// Arguments (all kernels): x, w, scales, biases, sb_bf16, group, y, y_bf16,
// M, K, N, rb (row bytes), row_map (NULL), row_scale (NULL), y_ld.
// ---------------------------------------------------------------------------
#define RLXQ_GEMV_INST(NAME, SCH, XBF, L, P, NBC, MT)                                          \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                      \
      const void* x, const uint8_t* w, const void* scales, const void* biases, int sb_bf16,    \
      int group, void* y, int y_bf16, int64_t M, int K, int64_t N, int64_t rb,                 \
      const int32_t* row_map, const float* row_scale, int64_t y_ld) {                          \
    rlxq::gemv_body<SCH, XBF, L, P, NBC, MT>(x, w, scales, biases, sb_bf16, group, y, y_bf16, \
                                             M, K, N, rb, row_map, row_scale, y_ld);           \
  }

#define RLXQ_GEMV_SCHEME(SNAME, SCH)                                              \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_bf16_L64_P4_C2_M1, SCH, true, 64, 4, 2, 1)  \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_bf16_L64_P2_C3_M1, SCH, true, 64, 2, 3, 1)  \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_bf16_L16_P4_C2_M1, SCH, true, 16, 4, 2, 1)  \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_bf16_L8_P4_C2_M1, SCH, true, 8, 4, 2, 1)    \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_bf16_L64_P2_C2_M4, SCH, true, 64, 2, 2, 4)  \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_bf16_L8_P2_C2_M4, SCH, true, 8, 2, 2, 4)    \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_f32_L64_P4_C2_M1, SCH, false, 64, 4, 2, 1)  \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_f32_L64_P2_C3_M1, SCH, false, 64, 2, 3, 1)  \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_f32_L16_P4_C2_M1, SCH, false, 16, 4, 2, 1)  \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_f32_L8_P4_C2_M1, SCH, false, 8, 4, 2, 1)    \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_f32_L64_P2_C2_M4, SCH, false, 64, 2, 2, 4)  \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_f32_L8_P2_C2_M4, SCH, false, 8, 2, 2, 4)

RLXQ_GEMV_SCHEME(q4_1, SCH_Q4_1)
RLXQ_GEMV_SCHEME(q4_0, SCH_Q4_0)
RLXQ_GEMV_SCHEME(q8_0, SCH_Q8_0)
RLXQ_GEMV_SCHEME(mlx4, SCH_MLX4)
RLXQ_GEMV_SCHEME(mlx8, SCH_MLX8)
