// Dequant-GEMV for decode (M = 1..few rows): y[m, n] = sum_k x[m, k] * W[n, k]
// over packed GGUF Q4_1 / Q4_0 / Q8_0 / Q4_K / Q6_K / Q5_K / Q3_K / Q2_K / Q8_K
// blocks, MLX affine 4/8-bit
// codes or MXFP4 codes, with fp32 accumulation.  Replaces the backend kernel of Op::DequantMatMul
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
//     become f16 (1024 + u) with one byte permute per pair; MXFP4 code bytes
//     become bf16 pairs of their signed E2M1 values with one
//     v_cvt_scalef32_pk_bf16_fp4 each (no offset to remove).  v_dot2c
//     accumulates pairs in f32 starting from -bias * (block sum of x), which
//     removes the 128 / 1024 offset, so the block dot is sum(q * x).
//   * f32 activations are split into hi + lo planes so the products keep
//     ~17 (bf16) / ~22 (f16) significant bits; bf16 activations are exact in a
//     single plane.  8-bit schemes scale each block of x by a power of two so
//     that f16 cannot overflow (the factor is folded into the block scale).
#include "gemv_core.hip.h"

namespace rlxq {

// One decode GEMV pass.
//
// A workgroup (WAVES waves) stages its MT activation rows once and then walks row
// tiles t = blockIdx.x, blockIdx.x + gridDim.x, ...; the host sizes the grid
// to what the device holds at once.  Each wave owns P*RP rows of a tile and
// covers them in steps of C unit chunks (C*L units of each row per step, so a
// step requests whole rows when C*L covers K).  A ring of D register buffers
// keeps the loads of the next D steps in flight while a step is computed; the
// first D steps are requested right after the activations, before the
// activation records are built.
template <int SCH, bool XBF16, int L, int P, int C, int MT, int D, int WAVES>
RLXQ_DEV void gemv_body(const rlxq_gemv_args& a) {
  constexpr bool BIT8 = Unit<SCH>::BIT8;
  constexpr int NPL = (XBF16 ? 1 : 2);
  constexpr int RS = Rec<NPL>::STRIDE;
  constexpr int BLOCKS = Unit<SCH>::BLOCKS;
  constexpr int DW = Unit<SCH>::DW;
  constexpr int BYTES = Unit<SCH>::BYTES;
  constexpr int RP = 64 / L;
  constexpr int TILE = WAVES * P * RP;
  constexpr bool SLAB = slab_scales<SCH>(), SBIAS = slab_bias<SCH>();
  constexpr bool HAS_MIN = (SCH == SCH_Q4_1 || SCH == SCH_Q4_K || SCH == SCH_Q5_K || SBIAS);
  constexpr bool HALF2 = SCH == SCH_Q2_K || SCH == SCH_Q3_K;   // two scales (and mins) per block
  extern __shared__ uint32_t lds[];

  const int K = a.K;
  const int bpr = K >> 5;
  const int U = bpr / BLOCKS;
  const int nchunk = (U + L - 1) / L;
  const int ng = (nchunk + C - 1) / C;  // steps per tile
  const int64_t ntiles = (a.N + TILE - 1) / TILE;
  const int64_t m0 = (int64_t)blockIdx.y * MT;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane / L, li = lane % L;
  const int gpr = SLAB ? K / a.group : 0;  // slab groups per row
  const int64_t row_off = wv * (P * RP) + g;

  struct Buf {
    uint32_t dw[P][C][DW];
    SbRaw sm[P][C][BLOCKS], bm[P][C][BLOCKS];
  };
  auto load = [&](int64_t t, int jg, Buf& bf) {
#pragma unroll
    for (int p = 0; p < P; p++) {
      int64_t n = t * TILE + row_off + p * RP;
      n = (n < a.N && t < ntiles) ? n : 0;
      const uint8_t* rp = a.w + n * a.rb;
#pragma unroll
      for (int c = 0; c < C; c++) {
        const int u = li + L * (jg * C + c);
        const int uc = u < U ? u : U - 1;
        load_unit_at<SCH>(bf.dw[p][c], rp, uc);
        if constexpr (SLAB) {
#pragma unroll
          for (int bl = 0; bl < BLOCKS; bl++) {
            const int64_t gi = n * gpr + ((uc * BLOCKS + bl) * 32) / a.group;
            bf.sm[p][c][bl] = load_scale_raw<SCH>(a.scales, gi, a.sb_bf16);
            if constexpr (SBIAS) bf.bm[p][c][bl] = load_sb_raw(a.biases, gi, a.sb_bf16 != 0);
          }
        }
      }
    }
  };

  float acc[P][MT];
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[p][m] = 0.f;

  const UnpackK kc = unpack_consts();
  auto compute = [&](int64_t t, int jg, const Buf& bf) {
#pragma unroll
    for (int c = 0; c < C; c++) {
      const int u = li + L * (jg * C + c);
      const bool uok = u < U;
      const int uc = uok ? u : U - 1;
#pragma unroll
      for (int bl = 0; bl < BLOCKS; bl++) {
        const int b = uc * BLOCKS + bl;
        float d[P], mn[P], d2[P], m2[P];
        uint32_t pw[P][16];
#pragma unroll
        for (int p = 0; p < P; p++) {
          d2[p] = m2[p] = 0.f;
          if constexpr (SLAB) {
            d[p] = scale_decode<SCH>(bf.sm[p][c][bl], a.sb_bf16);
            mn[p] = SBIAS ? sb_decode(bf.bm[p][c][bl], a.sb_bf16 != 0) : 0.f;
          } else if constexpr (HALF2) {
            block_scales_half<SCH>(bf.dw[p][c], d[p], d2[p], mn[p], m2[p]);
          } else {
            block_scales<SCH>(bf.dw[p][c], bl, d[p], mn[p], uc);
          }
          const bool rok = t * TILE + row_off + p * RP < a.N;
          if (!(rok && uok)) {
            d[p] = 0.f;
            mn[p] = 0.f;
            d2[p] = 0.f;
            m2[p] = 0.f;
          }
          block_pairs<SCH>(bf.dw[p][c], bl, pw[p], kc);
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
          const uint32_t* xr = lds + (size_t)(m * bpr + b) * RS;
          uint32_t xrec[RS];
#pragma unroll
          for (int q = 0; q < RS; q += 4) {
            const uint4 v = *reinterpret_cast<const uint4*>(xr + q);
            xrec[q] = v.x; xrec[q + 1] = v.y; xrec[q + 2] = v.z; xrec[q + 3] = v.w;
          }
          const float sx = __uint_as_float(xrec[NPL * 16 + 1]);
          const float scl = __uint_as_float(xrec[NPL * 16 + 2]);
#pragma unroll
          for (int p = 0; p < P; p++) {
            if constexpr (SCH == SCH_Q6_K) {
              acc[p][m] += q6k_block_dot<NPL>(pw[p], xrec, d[p], mn[p]);   // mn: the second half's d
            } else if constexpr (HALF2) {
              acc[p][m] += khalf_block_dot<SCH, NPL>(pw[p], xrec, d[p], d2[p], mn[p], m2[p]);
            } else {
              const float cc = block_dot<SCH, NPL>(pw[p], xrec);
              acc[p][m] = fmaf(BIT8 ? d[p] * scl : d[p], cc, acc[p][m]);
              if constexpr (HAS_MIN) acc[p][m] = fmaf(mn[p], sx, acc[p][m]);
            }
          }
        }
      }
    }
    if (jg == ng - 1) {
#pragma unroll
      for (int p = 0; p < P; p++) {
        const int64_t n = t * TILE + row_off + p * RP;
#pragma unroll
        for (int m = 0; m < MT; m++) {
          const float v = lane_group_sum<L>(acc[p][m]);
          acc[p][m] = 0.f;
          const int64_t row = m0 + m;
          if (li == 0 && n < a.N && row < a.M) {
            int64_t yrow = row;
            float sc = 1.f;
            if (a.row_map) yrow = a.row_map[row];
            if (a.row_scale) sc = a.row_scale[row];
            if (yrow >= 0) {
              const int64_t off = yrow * a.y_ld + n;
              if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[off] = (uint16_t)f32_to_bf16_bits(v * sc);
              else reinterpret_cast<float*>(a.y)[off] = v * sc;
            }
          }
        }
      }
    }
  };

  auto next = [&](int64_t& t, int& jg) {
    if (++jg == ng) {
      jg = 0;
      t += gridDim.x;
    }
  };

  // The activation loads go out first, then the first D steps of weights, so
  // the x records can be built while the weights are in flight.
  XRaw<XBF16> raw;
  stage_fetch<XBF16>(raw, a.x, m0, a.M, K, 0);
  Buf ring[D];
  int64_t lt = blockIdx.x;  // load cursor
  int lj = 0;
#pragma unroll
  for (int i = 0; i < D; i++) {
    if (lt < ntiles) load(lt, lj, ring[i]);
    next(lt, lj);
  }
  stage_store<SCH, XBF16, NPL>(lds, raw, 0, K, 0);
  for (int m = 0; m < MT; m++)
    for (int base = m == 0 ? (int)blockDim.x * XRaw<XBF16>::XB : 0; base < bpr * 8;
         base += blockDim.x * XRaw<XBF16>::XB) {
      stage_fetch<XBF16>(raw, a.x, m0 + m, a.M, K, base);
      stage_store<SCH, XBF16, NPL>(lds, raw, m, K, base);
    }
  __syncthreads();

  int64_t ct = blockIdx.x;  // compute cursor
  int cj = 0;
  while (ct < ntiles) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      if (ct < ntiles) {
        compute(ct, cj, ring[i]);
        next(ct, cj);
        if (lt < ntiles) load(lt, lj, ring[i]);
        next(lt, lj);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Register-resident activations for the single-row decode GEMV (M = 1, bf16
// activations, 4-bit codes).  Lane li owns units li + 64c (c < NU) of every
// row, so it only ever needs the activations of those units: it loads them
// once from global memory and builds their bf16 pairs (in the code-extraction
// order) and block sums in registers.  There is no LDS stage and no barrier;
// a wave starts on its first row as soon as its own activations and weights
// arrive.  Waves take rows n = global wave id + i * (total waves), with a ring
// of D rows of weight loads in flight.
// ---------------------------------------------------------------------------

// F32X: one row of f32 activations, held as two bf16 rows, the rounded row
// (hi) and what the rounding left over (lo), so that the pairs keep ~16
// significant bits of each element; both rows' sums add into the one output.
// KS > 1 (K split inside the workgroup, for rows too long for one wave's
// registers or too few to keep the CUs' loads in flight): waves KS r ..
// KS r + KS - 1 take the same weight rows, each a contiguous KS-th of the
// units; their row sums meet in LDS after the last row and are added in
// part order (fixed, so the result does not depend on timing).
template <int SCH, int NU, int D, int WAVES, bool XLDS, int MT = 1, bool F32X = false, int KS = 1>
RLXQ_DEV void gemv_xr_body(const rlxq_gemv_args& a) {
  static_assert(!F32X || (MT == 2 && XLDS), "f32 activations: hi and lo rows through LDS");
  static_assert(KS == 1 || (XLDS && (MT == 1 || F32X) && WAVES % KS == 0),
                "K split: one output row, partial sums through LDS");
  constexpr int BLOCKS = Unit<SCH>::BLOCKS;
  constexpr int DW = Unit<SCH>::DW;
  constexpr int BYTES = Unit<SCH>::BYTES;
  constexpr bool MLX = SCH == SCH_MLX4;
  constexpr bool MX = SCH == SCH_MXFP4;
  constexpr bool HAS_MIN = (SCH == SCH_Q4_1 || SCH == SCH_Q4_K || SCH == SCH_Q5_K || MLX);
  // Q2_K / Q3_K: a scale (Q2_K: and a min) per 16 weights, two dot chains
  // per block on the halves' activation sums (the records carry the first
  // half's sum after the block sums)
  constexpr bool HALF = half_scales<SCH>();
  static_assert(!HALF || (XLDS && MT == 1 && !F32X && KS == 1), "per-16 scales: one bf16 row through LDS");
  constexpr int XREC = HALF ? 18 : 17;   // LDS dwords per block: 16 pairs, the sum[, the first half's sum]
  static_assert(!Unit<SCH>::BIT8, "register activations serve 4-bit codes");

  const int K = a.K;
  const int bpr = K >> 5;
  const int U = bpr / BLOCKS;
  // the wave index through readfirstlane: the row loop below is then known
  // to be wave-uniform (scalar branches), so the compiler's wait counts can
  // keep the ring's loads in flight across iterations
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // K part and row slot of this wave; RW row slots per workgroup
  constexpr int RW = WAVES / KS;
  const int kh = wv % KS, wr = wv / KS;
  // rows of this wave: n0 + s * G, s < cnt (N < 2^31: 32-bit division)
  const uint32_t G = gridDim.x * RW, n0u = blockIdx.x * RW + wr, N32 = (uint32_t)a.N;
  const int64_t n0 = n0u;
  const int64_t cnt = n0u < N32 ? (N32 - n0u + G - 1) / G : 0;
  const int gpr = (MLX || MX) ? K / a.group : 0;
  // this wave's units [ub, ue)
  const int UH = (U + KS - 1) / KS, ub = kh * UH, ue = ub + UH < U ? ub + UH : U;

  int uc[NU];
  bool uok[NU];
#pragma unroll
  for (int c = 0; c < NU; c++) {
    const int u = ub + lane + 64 * c;
    uok[c] = u < ue;
    uc[c] = uok[c] ? u : U - 1;
  }

  struct Buf {
    uint32_t dw[NU][DW];
    SbRaw sm[NU][BLOCKS], bm[NU][BLOCKS];
  };
  auto load = [&](int64_t n, Buf& bf) {
    const int64_t nn = (n >= 0 && n < a.N) ? n : 0;  // no rows (cnt = 0): row 0
    const uint8_t* rp = a.w + nn * a.rb;
#pragma unroll
    for (int c = 0; c < NU; c++) {
      load_unit_at<SCH>(bf.dw[c], rp, uc[c]);
      if constexpr (MLX || MX) {
        const int64_t gi = nn * gpr + (uc[c] * 32) / a.group;
        bf.sm[c][0] = load_scale_raw<SCH>(a.scales, gi, a.sb_bf16);
        if constexpr (MLX) bf.bm[c][0] = load_sb_raw(a.biases, gi, a.sb_bf16 != 0);
      }
    }
  };

  // Activations of my units as bf16 pairs in the code-extraction order, and
  // their block sums.  XR: each lane loads its units' raw activations from
  // global memory and builds the pairs itself.  XLDS: the workgroup builds
  // them once in LDS (so the row of x crosses L2 once per workgroup and each
  // element is converted once): thread t takes half-blocks t, t + 64*WAVES,
  // ...; half h of block b is the 16 elements whose pairs fill dwords
  // 8h..8h+7 of the block's record (GGUF nibble order: elements 8h..8h+7 and
  // 16+8h..16+8h+7; MLX order: 16h..16h+15), and the two halves' sums are
  // added through a lane swap.  LDS: [bpr][16] pair dwords, then [bpr] sums.
  // Either way the first D rows of weights are requested right after the
  // activation loads.
  // MT activation rows (M <= MT; rows past M read row 0 and are not stored)
  uint32_t X[MT][NU][BLOCKS][16];
  float S[MT][NU][BLOCKS];
  float SL[MT][NU][BLOCKS];   // (HALF: the first half's sums)
  Buf ring[D];
  if constexpr (XLDS) {
    extern __shared__ __align__(16) uint32_t xlds[];
    constexpr int NT = 64 * WAVES;
    constexpr int XH = (2 * 64 * NU * KS * BLOCKS + NT - 1) / NT;   // half-blocks per thread and row
    constexpr uint32_t LO = 0x05040100u, HI = 0x07060302u;
    constexpr bool LINEAR = MLX || MX || SCH == SCH_Q4_K || SCH == SCH_Q5_K || HALF;   // half h = elements 16h..16h+15
    uint4 xa[MT][XH], xc[MT][XH];
    if constexpr (F32X) {
      // the half-block's 16 f32 elements, split after the first weight
      // requests: hi = bf16(v), lo = bf16(v - hi)
      const float* xg = reinterpret_cast<const float*>(a.x);
      float4 fr[XH][4];
#pragma unroll
      for (int i = 0; i < XH; i++) {
        const int hb = threadIdx.x + NT * i, b = hb >> 1, h = hb & 1;
#pragma unroll
        for (int q = 0; q < 4; q++) fr[i][q] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (hb < 2 * bpr) {
          const float* p = xg + (int64_t)b * 32;
          const int o0 = LINEAR ? 16 * h : 8 * h, o1 = LINEAR ? 16 * h + 8 : 16 + 8 * h;
          fr[i][0] = *reinterpret_cast<const float4*>(p + o0);
          fr[i][1] = *reinterpret_cast<const float4*>(p + o0 + 4);
          fr[i][2] = *reinterpret_cast<const float4*>(p + o1);
          fr[i][3] = *reinterpret_cast<const float4*>(p + o1 + 4);
        }
      }
#pragma unroll
      for (int i = 0; i < D; i++) load(n0 + (i < cnt ? i : cnt - 1) * G, ring[i]);
      auto split8 = [](float4 u, float4 v, uint4& hi, uint4& lo) {
        const float e[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        uint32_t h[8], l[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
          h[q] = f32_to_bf16_bits(e[q]);
          l[q] = f32_to_bf16_bits(e[q] - bf16_bits_to_f32(h[q]));
        }
        hi = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
        lo = make_uint4(l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16), l[6] | (l[7] << 16));
      };
#pragma unroll
      for (int i = 0; i < XH; i++) {
        split8(fr[i][0], fr[i][1], xa[0][i], xa[1][i]);
        split8(fr[i][2], fr[i][3], xc[0][i], xc[1][i]);
      }
    } else {
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const uint16_t* xg = reinterpret_cast<const uint16_t*>(a.x) + (int64_t)(m < a.M ? m : 0) * K;
#pragma unroll
        for (int i = 0; i < XH; i++) {
          const int hb = threadIdx.x + NT * i, b = hb >> 1, h = hb & 1;
          xa[m][i] = xc[m][i] = make_uint4(0u, 0u, 0u, 0u);
          if (hb < 2 * bpr) {
            const uint16_t* p = xg + (int64_t)b * 32;
            xa[m][i] = *reinterpret_cast<const uint4*>(p + (LINEAR ? 16 * h : 8 * h));
            xc[m][i] = *reinterpret_cast<const uint4*>(p + (LINEAR ? 16 * h + 8 : 16 + 8 * h));
          }
        }
      }
#pragma unroll
      for (int i = 0; i < D; i++) load(n0 + (i < cnt ? i : cnt - 1) * G, ring[i]);
    }
#pragma unroll
    for (int m = 0; m < MT; m++) {
      uint32_t* xs = xlds + (size_t)m * bpr * XREC;
      float* xsum = reinterpret_cast<float*>(xs + bpr * 16);
#pragma unroll
      for (int i = 0; i < XH; i++) {
        const int hb = threadIdx.x + NT * i, b = hb >> 1, h = hb & 1;
        const uint32_t A[4] = {xa[m][i].x, xa[m][i].y, xa[m][i].z, xa[m][i].w};
        const uint32_t C[4] = {xc[m][i].x, xc[m][i].y, xc[m][i].z, xc[m][i].w};
        uint32_t P[8];
#pragma unroll
        for (int t = 0; t < 2; t++) {
          if constexpr (MX) {
            const uint32_t* R = t == 0 ? A : C;   // elements 16h + 8t .. +7: pairs (2j, 2j+1) as loaded
            P[4 * t + 0] = R[0];
            P[4 * t + 1] = R[1];
            P[4 * t + 2] = R[2];
            P[4 * t + 3] = R[3];
          } else if constexpr (SCH == SCH_Q4_K || SCH == SCH_Q5_K || HALF) {
            const uint32_t* R = t == 0 ? A : C;   // elements 16h + 8t .. +7: pairs (4j+e, 4j+e+2)
            P[4 * t + 0] = perm_b32(R[1], R[0], LO);
            P[4 * t + 1] = perm_b32(R[1], R[0], HI);
            P[4 * t + 2] = perm_b32(R[3], R[2], LO);
            P[4 * t + 3] = perm_b32(R[3], R[2], HI);
          } else if constexpr (MLX) {
            const uint32_t* R = t == 0 ? A : C;   // elements 16h + 8t .. +7
            P[4 * t + 0] = perm_b32(R[2], R[0], LO);
            P[4 * t + 1] = perm_b32(R[2], R[0], HI);
            P[4 * t + 2] = perm_b32(R[3], R[1], LO);
            P[4 * t + 3] = perm_b32(R[3], R[1], HI);
          } else {
            P[4 * t + 0] = perm_b32(A[2 * t + 1], A[2 * t], LO);
            P[4 * t + 2] = perm_b32(A[2 * t + 1], A[2 * t], HI);
            P[4 * t + 1] = perm_b32(C[2 * t + 1], C[2 * t], LO);
            P[4 * t + 3] = perm_b32(C[2 * t + 1], C[2 * t], HI);
          }
        }
        float sh = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) sh = dot2_bf16(A[q], 0x3F803F80u, sh);
#pragma unroll
        for (int q = 0; q < 4; q++) sh = dot2_bf16(C[q], 0x3F803F80u, sh);
        const float so = __shfl_xor(sh, 1, 64);
        if (hb < 2 * bpr) {
          uint4* dst = reinterpret_cast<uint4*>(xs + b * 16 + 8 * h);
          dst[0] = make_uint4(P[0], P[1], P[2], P[3]);
          dst[1] = make_uint4(P[4], P[5], P[6], P[7]);
          if (h == 0) xsum[b] = sh + so;
          if (HALF && h == 0) xsum[bpr + b] = sh;   // (half 0: elements 0..15)
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MT; m++) {
      const uint32_t* xs = xlds + (size_t)m * bpr * XREC;
      const float* xsum = reinterpret_cast<const float*>(xs + bpr * 16);
#pragma unroll
      for (int c = 0; c < NU; c++)
#pragma unroll
        for (int bl = 0; bl < BLOCKS; bl++) {
          const int blk = uc[c] * BLOCKS + bl;
          const uint4* p = reinterpret_cast<const uint4*>(xs + blk * 16);
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const uint4 v = p[q];
            X[m][c][bl][4 * q] = v.x; X[m][c][bl][4 * q + 1] = v.y;
            X[m][c][bl][4 * q + 2] = v.z; X[m][c][bl][4 * q + 3] = v.w;
          }
          S[m][c][bl] = xsum[blk];
          if constexpr (HALF) SL[m][c][bl] = xsum[bpr + blk];
        }
    }
  } else {
    static_assert(MT == 1 || XLDS, "several activation rows go through LDS");
    const uint16_t* xg = reinterpret_cast<const uint16_t*>(a.x);
#pragma unroll
    for (int c = 0; c < NU; c++)
#pragma unroll
      for (int bl = 0; bl < BLOCKS; bl++) {
        const uint4* p = reinterpret_cast<const uint4*>(xg + (int64_t)(uc[c] * BLOCKS + bl) * 32);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const uint4 v = p[q];
          X[0][c][bl][4 * q] = v.x; X[0][c][bl][4 * q + 1] = v.y;
          X[0][c][bl][4 * q + 2] = v.z; X[0][c][bl][4 * q + 3] = v.w;
        }
      }
#pragma unroll
    for (int i = 0; i < D; i++) load(n0 + (i < cnt ? i : cnt - 1) * G, ring[i]);
#pragma unroll
    for (int c = 0; c < NU; c++)
#pragma unroll
      for (int bl = 0; bl < BLOCKS; bl++) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) s = dot2_bf16(X[0][c][bl][i], 0x3F803F80u, s);
        S[0][c][bl] = s;
        uint32_t R[16];
#pragma unroll
        for (int i = 0; i < 16; i++) R[i] = X[0][c][bl][i];
        pairs_from_raw<SCH>(R, X[0][c][bl]);
      }
  }

  // output row and factor of the activation row (scalar loads, issued after
  // the weights; used only by the stores)
  int64_t yrow = 0;
  float ysc = 1.f;
  if (a.row_map) yrow = a.row_map[0];
  if (a.row_scale) ysc = a.row_scale[0];

  // K split: every part's row sums, [RW][cmax][KS] floats after the
  // activation records
  float* kpart = nullptr;
  int64_t cmax = 0;
  if constexpr (KS > 1) {
    extern __shared__ __align__(16) uint32_t xlds[];
    kpart = reinterpret_cast<float*>(xlds + (size_t)MT * bpr * XREC);
    cmax = (N32 + G - 1) / G;
  }
  auto store = [&](int64_t off, float v) {
    if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[off] = (uint16_t)f32_to_bf16_bits(v * ysc);
    else reinterpret_cast<float*>(a.y)[off] = v * ysc;
  };

  const UnpackK kc = unpack_consts();
  // Row s of the wave uses ring slot s % D.  While D more rows follow a full
  // group, each slot is refilled right after use with the row D later (no
  // condition on the refill, so the compiler's wait counts keep the other
  // slots' loads in flight); the last rows, already in the ring, are then
  // computed without refills.
  auto row = [&](int64_t st, const Buf& bf) {
    const int64_t n = n0 + st * G;
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) acc[m] = 0.f;
#pragma unroll
    for (int c = 0; c < NU; c++)
#pragma unroll
      for (int bl = 0; bl < BLOCKS; bl++) {
        if constexpr (HALF) {
          // two 16-weight halves (planes 0..7: elements 0..15), each chain
          // from -bias times its half's activation sum, its own scale (and
          // Q2_K's min times that sum)
          float d0, d1, m0, m1;
          block_scales_half<SCH>(bf.dw[c], d0, d1, m0, m1);
          if (!uok[c]) d0 = d1 = m0 = m1 = 0.f;
          uint32_t pw[16];
          block_pairs<SCH>(bf.dw[c], bl, pw, kc);
          const float sl = SL[0][c][bl], sh = S[0][c][bl] - sl;
          float lo = -chain_bias<SCH>() * sl, hi = -chain_bias<SCH>() * sh;
#pragma unroll
          for (int t = 0; t < 8; t++) {
            lo = dot2_bf16(pw[t], X[0][c][bl][t], lo);
            hi = dot2_bf16(pw[8 + t], X[0][c][bl][8 + t], hi);
          }
          acc[0] = fmaf(d0, lo, fmaf(d1, hi, acc[0]));
          if constexpr (SCH == SCH_Q2_K) acc[0] = fmaf(m0, sl, fmaf(m1, sh, acc[0]));
          continue;
        }
        float d, mn;
        if constexpr (MLX) {
          d = sb_decode(bf.sm[c][bl], a.sb_bf16 != 0);
          mn = sb_decode(bf.bm[c][bl], a.sb_bf16 != 0);
        } else if constexpr (MX) {
          d = scale_decode<SCH>(bf.sm[c][bl], a.sb_bf16);
          mn = 0.f;
        } else {
          block_scales<SCH>(bf.dw[c], bl, d, mn, uc[c]);
        }
        if (!uok[c]) {
          d = 0.f;
          mn = 0.f;
        }
        uint32_t pw[16];
        block_pairs<SCH>(bf.dw[c], bl, pw, kc);
#pragma unroll
        for (int m = 0; m < MT; m++) {
          float ch = chain_start<SCH>(S[m][c][bl]);
#pragma unroll
          for (int t = 0; t < 16; t++) ch = dot2_bf16(pw[t], X[m][c][bl][t], ch);
          acc[m] = fmaf(d, ch, acc[m]);
          if constexpr (HAS_MIN) acc[m] = fmaf(mn, S[m][c][bl], acc[m]);
        }
      }
    if constexpr (F32X) {
      const float v = lane_group_sum<64>(acc[0] + acc[1]);
      if constexpr (KS > 1) {
        if (lane == 0) kpart[((int64_t)wr * cmax + st) * KS + kh] = v;
      } else if (lane == 0 && yrow >= 0) {
        store(yrow * a.y_ld + n, v);
      }
    } else if constexpr (KS > 1) {
      const float v = lane_group_sum<64>(acc[0]);
      if (lane == 0) kpart[((int64_t)wr * cmax + st) * KS + kh] = v;
    } else {
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const float v = lane_group_sum<64>(acc[m]);
        if (lane == 0 && yrow >= 0 && m < a.M) store((yrow + m) * a.y_ld + n, v);
      }
    }
  };
  int64_t s0 = 0;
  for (; s0 + 2 * D <= cnt; s0 += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      row(s0 + i, ring[i]);
      load(n0 + (s0 + i + D) * G, ring[i]);
    }
  }
  // at most 2D - 1 rows remain: the first D of them may still refill
#pragma unroll
  for (int i = 0; i < D; i++) {
    if (s0 + i < cnt) {
      row(s0 + i, ring[i]);
      if (s0 + i + D < cnt) load(n0 + (s0 + i + D) * G, ring[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < D; i++)
    if (s0 + D + i < cnt) row(s0 + D + i, ring[i]);
  if constexpr (KS > 1) {
    // every wave has left its row loop: part 0's wave adds the parts of its
    // rows in part order and stores them
    __syncthreads();
    if (kh == 0 && yrow >= 0)
      for (int64_t st = lane; st < cnt; st += 64) {
        const float* p = kpart + ((int64_t)wr * cmax + st) * KS;
        float v = p[0];
#pragma unroll
        for (int q = 1; q < KS; q++) v += p[q];
        store(yrow * a.y_ld + n0 + st * G, v);
      }
  }
}

}  // namespace rlxq

// ---------------------------------------------------------------------------
// Instantiations: rlxq_gemv_<scheme>_<x>_L<L>_P<P>_C<C>_M<MT>_D<D>_W<WAVES>,
// one rlxq_gemv_args argument.
// ---------------------------------------------------------------------------
#define RLXQ_GEMV_INST(NAME, SCH, XBF, L, P, C, MT, D, W)                                \
  extern "C" __global__ __launch_bounds__(64 * W) void NAME(rlxq_gemv_args a) {         \
    rlxq::gemv_body<SCH, XBF, L, P, C, MT, D, W>(a);                                     \
  }

#ifndef RLXQ_GEMV_SWEEP
#define RLXQ_GEMV_X(SNAME, SCH, XN, XBF)                                                     \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L64_P1_C2_M1_D1_W16, SCH, XBF, 64, 1, 2, 1, 1, 16) \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L64_P1_C2_M1_D2_W16, SCH, XBF, 64, 1, 2, 1, 2, 16) \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L64_P1_C2_M1_D3_W16, SCH, XBF, 64, 1, 2, 1, 3, 16) \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L64_P1_C2_M1_D2_W8, SCH, XBF, 64, 1, 2, 1, 2, 8)   \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L64_P1_C1_M1_D4_W16, SCH, XBF, 64, 1, 1, 1, 4, 16) \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L64_P2_C1_M1_D2_W8, SCH, XBF, 64, 2, 1, 1, 2, 8)   \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L32_P2_C1_M1_D2_W8, SCH, XBF, 32, 2, 1, 1, 2, 8)   \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L16_P2_C1_M1_D2_W8, SCH, XBF, 16, 2, 1, 1, 2, 8)   \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L8_P2_C1_M1_D2_W8, SCH, XBF, 8, 2, 1, 1, 2, 8)     \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L64_P2_C1_M4_D1_W8, SCH, XBF, 64, 2, 1, 4, 1, 8)   \
  RLXQ_GEMV_INST(rlxq_gemv_##SNAME##_##XN##_L8_P2_C1_M4_D1_W8, SCH, XBF, 8, 2, 1, 4, 1, 8)
#endif

#define RLXQ_GEMV_SCHEME(SNAME, SCH) \
  RLXQ_GEMV_X(SNAME, SCH, bf16, true) \
  RLXQ_GEMV_X(SNAME, SCH, f32, false)

// Register-activation variants: rlxq_gemvxr_<scheme>_U<NU>_D<D>_W<WAVES>,
// and rlxq_gemvxs_... with the activations passed through LDS.
#define RLXQ_GEMVXR_INST(NAME, SCH, NU, D, W)                                         \
  extern "C" __global__ __launch_bounds__(64 * W) void NAME(rlxq_gemv_args a) {      \
    rlxq::gemv_xr_body<SCH, NU, D, W, false>(a);                                      \
  }
#define RLXQ_GEMVXS_INST(NAME, SCH, NU, D, W)                                         \
  extern "C" __global__ __launch_bounds__(64 * W) void NAME(rlxq_gemv_args a) {      \
    rlxq::gemv_xr_body<SCH, NU, D, W, true>(a);                                       \
  }
#define RLXQ_GEMVXR_SCHEME(SNAME, SCH)                                  \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U1_D2_W4, SCH, 1, 2, 4)       \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U2_D2_W4, SCH, 2, 2, 4)       \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U2_D1_W4, SCH, 2, 1, 4)       \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U2_D3_W4, SCH, 2, 3, 4)       \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U2_D2_W2, SCH, 2, 2, 2)       \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U3_D2_W4, SCH, 3, 2, 4)       \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U4_D1_W4, SCH, 4, 1, 4)       \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U4_D2_W4, SCH, 4, 2, 4)
// six chunks (K up to 12288) for the one-block units only
#define RLXQ_GEMVXR_WIDE(SNAME, SCH)                                    \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U6_D1_W4, SCH, 6, 1, 4)       \
  RLXQ_GEMVXR_INST(rlxq_gemvxr_##SNAME##_U6_D2_W4, SCH, 6, 2, 4)
#if RLXQ_PART_IS(0)
RLXQ_GEMVXR_SCHEME(q4_1, SCH_Q4_1)
RLXQ_GEMVXR_SCHEME(q4_0, SCH_Q4_0)
RLXQ_GEMVXR_SCHEME(mlx4, SCH_MLX4)
RLXQ_GEMVXR_WIDE(q4_1, SCH_Q4_1)
RLXQ_GEMVXR_WIDE(mlx4, SCH_MLX4)
#endif
#define RLXQ_GEMVXS_SCHEME(SNAME, SCH)                                  \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U1_D2_W8, SCH, 1, 2, 8)       \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U2_D2_W8, SCH, 2, 2, 8)       \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U2_D2_W16, SCH, 2, 2, 16)     \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U2_D2_W4, SCH, 2, 2, 4)       \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U2_D1_W4, SCH, 2, 1, 4)       \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U3_D2_W8, SCH, 3, 2, 8)       \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U4_D1_W8, SCH, 4, 1, 8)       \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U4_D2_W8, SCH, 4, 2, 8)
#define RLXQ_GEMVXS_WIDE(SNAME, SCH)                                    \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U6_D1_W8, SCH, 6, 1, 8)       \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U6_D2_W8, SCH, 6, 2, 8)
// Q4_K (64-weight units, 12 dwords each): up to three units per lane (K <= 12288)
#define RLXQ_GEMVXS_Q4K                                                     \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_q4_k_U1_D2_W8, SCH_Q4_K, 1, 2, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_q4_k_U2_D2_W8, SCH_Q4_K, 2, 2, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_q4_k_U2_D1_W8, SCH_Q4_K, 2, 1, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_q4_k_U3_D1_W8, SCH_Q4_K, 3, 1, 8)
// Q5_K (64-weight units of 21 dwords: the head, the qh bytes and the
// group's qs bytes; Q4_K's pair order): up to three units per lane
#define RLXQ_GEMVXS_Q5K                                                     \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_q5_k_U1_D2_W8, SCH_Q5_K, 1, 2, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_q5_k_U1_D1_W8, SCH_Q5_K, 1, 1, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_q5_k_U2_D1_W8, SCH_Q5_K, 2, 1, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_q5_k_U3_D1_W8, SCH_Q5_K, 3, 1, 8)
// Q2_K (11-dword units) and Q3_K (22): one 32-weight block per unit, K up to
// four (Q2_K) or three (Q3_K) unit chunks
#define RLXQ_GEMVXS_KHALF(SNAME, SCH)                                       \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U1_D2_W8, SCH, 1, 2, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U2_D1_W8, SCH, 2, 1, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U2_D2_W8, SCH, 2, 2, 8)          \
  RLXQ_GEMVXS_INST(rlxq_gemvxs_##SNAME##_U3_D1_W8, SCH, 3, 1, 8)
#if RLXQ_PART_IS(0)
RLXQ_GEMVXS_Q4K
RLXQ_GEMVXS_Q5K
RLXQ_GEMVXS_KHALF(q2_k, SCH_Q2_K)
RLXQ_GEMVXS_KHALF(q3_k, SCH_Q3_K)
RLXQ_GEMVXS_INST(rlxq_gemvxs_q2_k_U4_D1_W8, SCH_Q2_K, 4, 1, 8)
#endif
// several activation rows (M = 2..4): rlxq_gemvxs_<scheme>_U<NU>_D<D>_W<W>_M<MT>,
// NU * MT <= 8 units of activations per lane
#define RLXQ_GEMVXSM_INST(NAME, SCH, NU, D, W, MT)                                    \
  extern "C" __global__ __launch_bounds__(64 * W) void NAME(rlxq_gemv_args a) {      \
    rlxq::gemv_xr_body<SCH, NU, D, W, true, MT>(a);                                   \
  }
#define RLXQ_GEMVXSM_SCHEME(SNAME, SCH)                                       \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U1_D2_W8_M2, SCH, 1, 2, 8, 2)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U2_D1_W4_M2, SCH, 2, 1, 4, 2)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U2_D2_W4_M2, SCH, 2, 2, 4, 2)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U3_D1_W8_M2, SCH, 3, 1, 8, 2)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U4_D1_W8_M2, SCH, 4, 1, 8, 2)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U1_D2_W8_M4, SCH, 1, 2, 8, 4)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U2_D1_W4_M4, SCH, 2, 1, 4, 4)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U2_D2_W4_M4, SCH, 2, 2, 4, 4)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U2_D1_W8_M2, SCH, 2, 1, 8, 2)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U2_D2_W8_M2, SCH, 2, 2, 8, 2)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U2_D1_W8_M4, SCH, 2, 1, 8, 4)      \
  RLXQ_GEMVXSM_INST(rlxq_gemvxs_##SNAME##_U2_D2_W8_M4, SCH, 2, 2, 8, 4)
// one row of f32 activations as hi and lo bf16 rows: rlxq_gemvxs_<scheme>_U<NU>_D<D>_W<W>_F
#define RLXQ_GEMVXSF_INST(NAME, SCH, NU, D, W)                                        \
  extern "C" __global__ __launch_bounds__(64 * W) void NAME(rlxq_gemv_args a) {      \
    rlxq::gemv_xr_body<SCH, NU, D, W, true, 2, true>(a);                              \
  }
#define RLXQ_GEMVXSF_SCHEME(SNAME, SCH)                                       \
  RLXQ_GEMVXSF_INST(rlxq_gemvxs_##SNAME##_U1_D2_W8_F, SCH, 1, 2, 8)          \
  RLXQ_GEMVXSF_INST(rlxq_gemvxs_##SNAME##_U2_D2_W4_F, SCH, 2, 2, 4)          \
  RLXQ_GEMVXSF_INST(rlxq_gemvxs_##SNAME##_U2_D1_W4_F, SCH, 2, 1, 4)          \
  RLXQ_GEMVXSF_INST(rlxq_gemvxs_##SNAME##_U2_D1_W8_F, SCH, 2, 1, 8)          \
  RLXQ_GEMVXSF_INST(rlxq_gemvxs_##SNAME##_U2_D2_W8_F, SCH, 2, 2, 8)          \
  RLXQ_GEMVXSF_INST(rlxq_gemvxs_##SNAME##_U2_D1_W16_F, SCH, 2, 1, 16)        \
  RLXQ_GEMVXSF_INST(rlxq_gemvxs_##SNAME##_U3_D1_W8_F, SCH, 3, 1, 8)          \
  RLXQ_GEMVXSF_INST(rlxq_gemvxs_##SNAME##_U4_D1_W8_F, SCH, 4, 1, 8)
// K split inside the workgroup (KS waves per weight row):
// rlxq_gemvxs_<scheme>_U<NU>_D<D>_W<W>[_F]_K<KS>, NU unit chunks per part
#define RLXQ_GEMVXSK_INST(NAME, SCH, NU, D, W, KS)                                    \
  extern "C" __global__ __launch_bounds__(64 * W) void NAME(rlxq_gemv_args a) {      \
    rlxq::gemv_xr_body<SCH, NU, D, W, true, 1, false, KS>(a);                         \
  }
#define RLXQ_GEMVXSFK_INST(NAME, SCH, NU, D, W, KS)                                   \
  extern "C" __global__ __launch_bounds__(64 * W) void NAME(rlxq_gemv_args a) {      \
    rlxq::gemv_xr_body<SCH, NU, D, W, true, 2, true, KS>(a);                          \
  }
#if RLXQ_PART_IS(2)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U1_D2_W8_K2, SCH_Q4_1, 1, 2, 8, 2)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U1_D3_W8_K2, SCH_Q4_1, 1, 3, 8, 2)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U1_D2_W16_K2, SCH_Q4_1, 1, 2, 16, 2)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U3_D1_W8_K2, SCH_Q4_1, 3, 1, 8, 2)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U3_D2_W8_K2, SCH_Q4_1, 3, 2, 8, 2)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U3_D1_W16_K2, SCH_Q4_1, 3, 1, 16, 2)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U2_D1_W8_K4, SCH_Q4_1, 2, 1, 8, 4)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U2_D2_W8_K4, SCH_Q4_1, 2, 2, 8, 4)
RLXQ_GEMVXSK_INST(rlxq_gemvxs_q4_1_U2_D1_W16_K4, SCH_Q4_1, 2, 1, 16, 4)
RLXQ_GEMVXSFK_INST(rlxq_gemvxs_q4_1_U3_D1_W8_F_K2, SCH_Q4_1, 3, 1, 8, 2)
RLXQ_GEMVXSFK_INST(rlxq_gemvxs_q4_1_U2_D1_W8_F_K2, SCH_Q4_1, 2, 1, 8, 2)
RLXQ_GEMVXSFK_INST(rlxq_gemvxs_q4_1_U1_D2_W8_F_K2, SCH_Q4_1, 1, 2, 8, 2)
#endif
#if RLXQ_PART_IS(1)
RLXQ_GEMVXSF_SCHEME(q4_1, SCH_Q4_1)
RLXQ_GEMVXSF_SCHEME(mlx4, SCH_MLX4)
RLXQ_GEMVXSF_SCHEME(mxfp4, SCH_MXFP4)
RLXQ_GEMVXSF_INST(rlxq_gemvxs_q4_k_U1_D2_W8_F, SCH_Q4_K, 1, 2, 8)
RLXQ_GEMVXSF_INST(rlxq_gemvxs_q4_k_U2_D1_W8_F, SCH_Q4_K, 2, 1, 8)
RLXQ_GEMVXSM_SCHEME(q4_1, SCH_Q4_1)
RLXQ_GEMVXSM_SCHEME(mlx4, SCH_MLX4)
RLXQ_GEMVXSM_SCHEME(mxfp4, SCH_MXFP4)
// Q4_K (two-block units): NU * MT <= 4
RLXQ_GEMVXSM_INST(rlxq_gemvxs_q4_k_U1_D2_W8_M2, SCH_Q4_K, 1, 2, 8, 2)
RLXQ_GEMVXSM_INST(rlxq_gemvxs_q4_k_U2_D1_W8_M2, SCH_Q4_K, 2, 1, 8, 2)
RLXQ_GEMVXSM_INST(rlxq_gemvxs_q4_k_U1_D2_W8_M4, SCH_Q4_K, 1, 2, 8, 4)
#endif
#if RLXQ_PART_IS(0)
RLXQ_GEMVXS_SCHEME(q4_1, SCH_Q4_1)
RLXQ_GEMVXS_SCHEME(q4_0, SCH_Q4_0)
RLXQ_GEMVXS_SCHEME(mlx4, SCH_MLX4)
RLXQ_GEMVXS_SCHEME(mxfp4, SCH_MXFP4)
RLXQ_GEMVXS_WIDE(q4_1, SCH_Q4_1)
RLXQ_GEMVXS_WIDE(mlx4, SCH_MLX4)
RLXQ_GEMVXS_WIDE(mxfp4, SCH_MXFP4)

#endif
#if RLXQ_PART_IS(2)
RLXQ_GEMV_SCHEME(q4_1, SCH_Q4_1)
RLXQ_GEMV_SCHEME(q4_0, SCH_Q4_0)
RLXQ_GEMV_SCHEME(q8_0, SCH_Q8_0)
RLXQ_GEMV_SCHEME(q4_k, SCH_Q4_K)
RLXQ_GEMV_SCHEME(q6_k, SCH_Q6_K)
#endif
#if RLXQ_PART_IS(3)
RLXQ_GEMV_SCHEME(mlx4, SCH_MLX4)
RLXQ_GEMV_SCHEME(mlx8, SCH_MLX8)
RLXQ_GEMV_SCHEME(mxfp4, SCH_MXFP4)
#endif
#if RLXQ_PART_IS(4)
RLXQ_GEMV_SCHEME(q5_k, SCH_Q5_K)
RLXQ_GEMV_SCHEME(q8_k, SCH_Q8_K)
#endif
#if RLXQ_PART_IS(5)
RLXQ_GEMV_SCHEME(q3_k, SCH_Q3_K)
RLXQ_GEMV_SCHEME(q2_k, SCH_Q2_K)
#endif
