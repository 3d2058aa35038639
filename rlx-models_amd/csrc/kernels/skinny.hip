// Batched-decode dequant-GEMM for small M (the multi-row decode path):
// y[m, n] = sum_k x[m, k] * dequant(W)[n, k] for up to 256 activation rows
// (512 prepared rows) and GGUF Q8_0 / Q4_0 / Q4_1 / Q4_K / Q5_K / Q6_K /
// Q3_K / Q2_K / Q8_K, MLX affine 4/8-bit and MXFP4 weights, streaming every
// weight once for all rows.
// Replaces the backend kernel of Op::DequantMatMul at decode batch sizes
// (crates/rlx-models-core/src/standard_decoder.rs:727-738, M rows per call).
//
//  * rlxq_x16_prep: each activation row to f16, scaled by a power of two so
//    its largest element lies in [2^9, 2^10) (exact; undone in the
//    epilogue), and permuted within each 32-element block to the order in
//    which a lane unpacks the codes: for the GGUF nibble formats position
//    8g + e holds element 4g + e (e < 4) or 16 + 4g + e - 4, for MLX's
//    element 8g + 2e (e < 4) or 8g + 2(e - 4) + 1.  f32 rows become a hi and
//    a lo row (split).  The block sums of the prepared values go beside them
//    (the min / bias term).
//  * rlxq_skinnyxr_* (register-streamed) and rlxq_skinnyns_* (N-split):
//    each lane turns its 8 codes into exact f16 values and the weights into
//    two f16 operands whose sum is the weight (f16dq.hip.h), both contracted
//    by v_mfma_f32_16x16x32_f16 into f32; one more MFMA per 128-element
//    chunk adds the blocks' m * sum(x).  f16 weights rounded once would be
//    ~2^-12 off each, which structured data accumulates past a 1e-3 output
//    bar.  MXFP4 codes are exact in bf16 and take one bf16 MFMA.
//  * rlxq_skinny_reduce: K splits added in split order (also the prefill
//    GEMM's split-K reduction).
#include "common.hip.h"
#include "f16dq.hip.h"
#include "gemm_dq.hip.h"
#include "skinny_args.h"
#include "moe_args.h"

namespace rlxq {

constexpr int SK_BN = 128;          // weight rows per workgroup

// Stores the sums of 16-row MFMA tiles (row chunk from x16 row m0, column
// tiles from n0): C[i][j] of a tile sits in lane j + 16 (i / 4), register
// i % 4, scaled by the row's inv_s, to the split's partial sums or to y.
// With pairs the x16 rows 2r and 2r + 1 (a lane's registers 0, 1 and 2, 3)
// are added into output row r.
template <int MT, int NT>
RLXQ_DEV void sk_store(const rlxq_skinny_args& a, const f32x4_t (&acc)[MT][NT], int64_t m0, int64_t n0, int sp,
                       int g, int j) {
  const int64_t mo_rows = a.pairs ? a.M >> 1 : a.M;
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      if (a.pairs && (r & 1)) continue;
      const int64_t m = m0 + 16 * mt + 4 * g + r;
      if (m >= a.M) continue;
      const int64_t mo = a.pairs ? m >> 1 : m;
      const float is = a.inv_s[m];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const int64_t n = n0 + 16 * t + j;
        if (n >= a.N) continue;
        const float v = (a.pairs ? acc[mt][t][r] + acc[mt][t][r < 3 ? r + 1 : r] : acc[mt][t][r]) * is;
        if (a.splits > 1) a.part[((int64_t)sp * mo_rows + mo) * a.N + n] = v;
        else if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[mo * a.y_ld + n] = (uint16_t)f32_to_bf16_bits(v);
        else reinterpret_cast<float*>(a.y)[mo * a.y_ld + n] = v;
      }
    }
}


// The MFMAs of one 128-element chunk: normalised blocks o[t] (lane (j, g):
// block 4c + g of weight row j of tile t), activation fragments xa[mt][i]
// (positions 8i .. 8i + 7 of the lane group's block, rows 16 mt + j), and,
// for the formats with a min / bias, the rows' block sums s[mt].  Each step
// contracts both weight operands (exact f16 hi + lo) into acc; then one MFMA
// per tile pair adds sum over the four blocks of s * m.
template <int SCH, int MT, int NT>
RLXQ_DEV void sk_chunk(const uint32_t (&o)[NT][sk_bdw<SCH>()], const f16x8_t (&xa)[MT][4], const float* s,
                       f32x4_t (&acc)[MT][NT]) {
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if constexpr (SCH == SCH_MXFP4) {
        const bf16x8_t b = sk_b_mxfp4(o[t], i);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[mt][i]), b, acc[mt][t],
                                                               0, 0, 0);
      } else {
        f16x8_t b1, b2;
        sk_b2<SCH>(o[t], i, b1, b2);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][i], b1, acc[mt][t], 0, 0, 0);
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][i], b2, acc[mt][t], 0, 0, 0);
        }
      }
    }
  if constexpr (sk_has_m<SCH>()) {
    f16x8_t ma[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) ma[mt] = sk_ma(s[mt]);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const f16x8_t mb = sk_mb<SCH>(o[t]);
#pragma unroll
      for (int mt = 0; mt < MT; mt++) acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ma[mt], mb, acc[mt][t], 0, 0, 0);
    }
  }
}

template <int MT, int NT>
RLXQ_DEV bool sk_wave_sum(f32x4_t (&acc)[MT][NT], float* R, int wv, int lane);

// ---------------------------------------------------------------------------
// Register-streamed variant: no LDS stage and no barrier per step.
// The four waves of a workgroup take the same NT tiles of 16 weight rows and
// split their K range in 4-block chunks (chunk c -> wave c % 4).  Lane
// (j, g) = (lane % 16, lane / 16) loads all the bytes of block 4c + g of row
// j of each tile into a ring of D chunks, so D * NT blocks per lane are in
// flight.  The four MFMA steps i of a chunk each take positions 8i .. 8i + 7
// of every lane's block: across the lane groups g a step's 32 K positions
// are positions 8i .. 8i + 7 of blocks 4c .. 4c + 3 (prepared activation
// order), and the A fragment of lane (m, g) is the 16 bytes of row m at
// block 4c + g, positions 8i .. 8i + 7, loaded with the chunk.  The waves'
// sums are added in the fixed order (w0 + w2) + (w1 + w3).
// The contraction of the register-streamed kernel for 16 MT activation rows
// from m0 (fragment-major x16 over Mp rows) against NT 16-row weight tiles
// (lane j of tile t reads weight row wrow[t] of the rows at w, stride rb)
// over K [kb, ke).  Returns true in wave 0, whose acc then holds the sums.
template <int SCH, int MT, int NT, int D>
RLXQ_DEV bool skinny_xr_core(const uint16_t* x16, const float* ssum, int64_t Mp, int64_t m0, const uint8_t* w,
                             int64_t rb, int64_t K, int64_t kb, int64_t ke, const int64_t (&wrow)[NT],
                             const bool (&wok)[NT], f32x4_t (&acc)[MT][NT], const void* scales = nullptr,
                             const void* biases = nullptr, int64_t group = 32, int32_t sb_bf16 = 0) {
  constexpr int BDW = sk_bdw<SCH>();
  constexpr bool HM = sk_has_m<SCH>();
  // wave index through readfirstlane: the chunk loop is wave-uniform
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nchunk = (int)((ke - kb) / 128);
  // chunks of this wave: wv + 4 it, it < cnt
  const int cnt = nchunk > wv ? (nchunk - wv + 3) / 4 : 0;

  rlxq_gemm_args ga;
  ga.w = w;
  ga.rb = rb;
  ga.K = K;
  ga.group = group;
  ga.sb_bf16 = sb_bf16;
  ga.scales = scales;
  ga.biases = biases;
  // activations in the fragment-major layout: piece i of chunk c for row m,
  // lane group g at ((4 c + i) Mp + m) 4 + g (16-byte pieces), so the A
  // fragment of 16 rows is one contiguous 1 KB read; the Mp rows cover every
  // 16 MT-row chunk (padding rows zero)
  // The block sums (min / bias term) in the same order, one f32 per block:
  // chunk c, row m, lane group g at (c Mp + m) 4 + g.
  const uint4* xrow[MT];
  const float* srow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    xrow[mt] = reinterpret_cast<const uint4*>(x16) + ((kb / 32) * Mp + m0 + 16 * mt + j) * 4 + g;
    srow[mt] = HM ? ssum + ((kb / 128) * Mp + m0 + 16 * mt + j) * 4 + g : nullptr;
  }

  struct Stage {
    RawBlk<SCH> w[NT];
    uint4 x[MT][4];
    float s[HM ? MT : 1];
  };
  auto load = [&](int c, Stage& st) {
#pragma unroll
    for (int t = 0; t < NT; t++) load_blk<SCH>(ga, wrow[t], kb / 32 + 4 * c + g, wok[t], st.w[t]);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) st.x[mt][i] = xrow[mt][((int64_t)c * 4 + i) * Mp * 4];
    if constexpr (HM) {
#pragma unroll
      for (int mt = 0; mt < MT; mt++) st.s[mt] = srow[mt][(int64_t)c * Mp * 4];
    }
  };

#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Chunk it uses ring slot it % D.  While D more chunks follow a full
  // group, each slot is refilled right after use with the chunk D later (no
  // condition on the refill, so the wait counts keep the other slots' loads
  // in flight); the last chunks, already in the ring, are computed after.
  auto chunk_of = [&](int it) { return wv + 4 * it; };
  auto compute = [&](const Stage& st) {
    uint32_t o[NT][BDW];
#pragma unroll
    for (int t = 0; t < NT; t++) normalise<SCH>(st.w[t], o[t]);
    f16x8_t xa[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) xa[mt][i] = __builtin_bit_cast(f16x8_t, st.x[mt][i]);
    sk_chunk<SCH, MT, NT>(o, xa, HM ? st.s : nullptr, acc);
  };
  // (slots past the wave's chunks repeat its last one: a few redundant
  // loads when it has fewer than D chunks, none otherwise; a wave with no
  // chunk at all (K under 512) loads chunk 0, never one past K)
  Stage ring[D];
#pragma unroll
  for (int d = 0; d < D; d++) load(cnt > 0 ? chunk_of(d < cnt ? d : cnt - 1) : 0, ring[d]);
  int it0 = 0;
  for (; it0 + 2 * D <= cnt; it0 += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      compute(ring[d]);
      load(chunk_of(it0 + d + D), ring[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < D; d++) {
    if (it0 + d < cnt) {
      compute(ring[d]);
      if (it0 + d + D < cnt) load(chunk_of(it0 + d + D), ring[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < D; d++)
    if (it0 + D + d < cnt) compute(ring[d]);

  extern __shared__ __align__(16) uint32_t sm[];
  return sk_wave_sum<MT, NT>(acc, reinterpret_cast<float*>(sm), wv, lane);
}

// The four waves' sums added in the fixed order (w0 + w2) + (w1 + w3)
// through R ([2][MT NT 4][64] floats of LDS); true in wave 0, whose acc then
// holds the total.
template <int MT, int NT>
RLXQ_DEV bool sk_wave_sum(f32x4_t (&acc)[MT][NT], float* R, int wv, int lane) {
  constexpr int E = MT * NT * 4;
  if (wv >= 2) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) R[((wv - 2) * E + (mt * NT + t) * 4 + r) * 64 + lane] = acc[mt][t][r];
  }
  __syncthreads();
  if (wv < 2) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[mt][t][r] += R[(wv * E + (mt * NT + t) * 4 + r) * 64 + lane];
  }
  __syncthreads();
  if (wv == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) R[((mt * NT + t) * 4 + r) * 64 + lane] = acc[mt][t][r];
  }
  __syncthreads();
  if (wv != 0) return false;
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[mt][t][r] += R[((mt * NT + t) * 4 + r) * 64 + lane];
  return true;
}

template <int SCH, int MT, int NT, int D>
RLXQ_DEV void skinny_xr_body(const rlxq_skinny_args& a) {
  const int lane = threadIdx.x & 63;
  const int j = lane & 15, g = lane >> 4;
  const int tn = blockIdx.x % a.tiles_n;
  const int sp = (blockIdx.x / a.tiles_n) % a.splits;
  const int mc = blockIdx.x / (a.tiles_n * a.splits);
  const int64_t n0 = (int64_t)tn * 16 * NT, m0 = (int64_t)mc * 16 * MT;
  const int64_t kb = (int64_t)sp * a.kslice;
  const int64_t ke = kb + a.kslice < a.K ? kb + a.kslice : a.K;
  int64_t wrow[NT];
  bool wok[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int64_t n = n0 + 16 * t + j;
    wok[t] = n < a.N;
    wrow[t] = wok[t] ? n : a.N - 1;
  }
  f32x4_t acc[MT][NT];
  if (!skinny_xr_core<SCH, MT, NT, D>(a.x16, a.ssum, a.Mp, m0, a.w, a.rb, a.K, kb, ke, wrow, wok, acc, a.scales,
                                      a.biases, a.group, a.sb_bf16))
    return;
  sk_store<MT, NT>(a, acc, m0, n0, sp, g, j);
}

// ---------------------------------------------------------------------------
// LDS-staged variant (rlxq_skinnyxl_*): the register-streamed kernel's
// contraction, with the weights reaching the lanes another way.  A wave's
// unit of K is a step of SC chunks (chunks SC s .. SC s + SC - 1 of its K
// range; the four waves take steps w, w + 4, ...).  The step's weights for
// the workgroup's 16 NT rows are one contiguous segment of SC CB bytes per
// row (CB = bytes of a 128-element chunk of a row); the wave reads them as
// 16-byte pieces, consecutive lanes on consecutive pieces of a row, and
// stores them in its own LDS region (rows LROW bytes apart, an odd number of
// 16-byte units, so the 16 rows a block read touches fall in distinct banks).
// Lane (j, g) then takes block 4c + g of row j of each tile, chunk c of the
// step, from there, as the register-streamed kernel takes it from memory.
// (Reading the weights as 16 row segments of one 20- to 34-byte block per
// lane moved 63 MB at 3.1 TB/s without any arithmetic; row-contiguous
// 16-byte pieces of the same rows moved it at 5.1-5.5 TB/s.)
// The region is the wave's own: its stores and its later loads are ordered
// by the wave's in-order LDS queue, with no barrier.  The steps' loads (the
// weight pieces, the activation fragments and the block sums) go D steps
// ahead into a register ring.
template <int SCH> constexpr int xl_chunk_bytes() {
  return SCH == SCH_Q4_1 ? 80 : SCH == SCH_Q4_0 ? 72 : SCH == SCH_Q8_0 ? 136 : SCH == SCH_Q4_K ? 72
         : SCH == SCH_Q5_K ? 88 : 0;
}
template <int SCH, int SC> constexpr int xl_lrow() {
  constexpr int seg = SC * xl_chunk_bytes<SCH>();
  return ((seg / 16) & 1) ? seg : seg + 16;
}

template <int SCH, int MT, int NT, int SC, int D>
RLXQ_DEV bool skinny_xl_core(const uint16_t* x16, const float* ssum, int64_t Mp, int64_t m0, const uint8_t* w,
                             int64_t rb, int64_t N, int64_t n0, int64_t kb, int64_t ke, f32x4_t (&acc)[MT][NT],
                             uint8_t* lds) {
  constexpr int CB = xl_chunk_bytes<SCH>(), SEG = SC * CB, PPR = SEG / 16, LROW = xl_lrow<SCH, SC>();
  static_assert(CB > 0 && SEG % 16 == 0, "a step must be whole 16-byte pieces of each row");
  static_assert(!(SCH == SCH_Q4_K || SCH == SCH_Q5_K) || SC % 2 == 0, "K-quant steps: whole super-blocks");
  constexpr int R = 16 * NT, NP = R * PPR, NL = (NP + 63) / 64;
  constexpr int BDW = sk_bdw<SCH>();
  constexpr bool HM = sk_has_m<SCH>();
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nsteps = (int)((ke - kb) / (128 * SC));   // (the host keeps K ranges whole steps)
  const int cnt = nsteps > wv ? (nsteps - wv + 3) / 4 : 0;
  uint8_t* reg = lds + wv * (R * LROW);

  // this lane's pieces: piece p = lane + 64 u is unit p % PPR of row p / PPR
  // (rows past N read row N - 1; their blocks are zeroed when read back)
  // (byte offsets from the segment of row n0: the rows past N stay within
  // the workgroup's 16 NT rows, so they fit 32 bits)
  const uint8_t* wseg = w + n0 * rb + (kb / 128) * CB;
  uint32_t src[NL];
  int dst[NL];
  bool pv[NL];
#pragma unroll
  for (int u = 0; u < NL; u++) {
    const int p = lane + 64 * u;
    pv[u] = p < NP;
    const int pp = pv[u] ? p : NP - 1, r = pp / PPR, c = pp % PPR;
    const int64_t rr = n0 + r < N ? r : N - 1 - n0;
    src[u] = (uint32_t)(rr * rb + c * 16);
    dst[u] = r * LROW + c * 16;
  }
  bool wok[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) wok[t] = n0 + 16 * t + j < N;
  rlxq_gemm_args la{};   // block reads from the LDS region
  la.w = reg;
  la.rb = LROW;

  const uint4* xrow[MT];
  const float* srow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    xrow[mt] = reinterpret_cast<const uint4*>(x16) + ((kb / 32) * Mp + m0 + 16 * mt + j) * 4 + g;
    srow[mt] = HM ? ssum + ((kb / 128) * Mp + m0 + 16 * mt + j) * 4 + g : nullptr;
  }
  // The ring holds the weight pieces and block sums of D steps; the
  // activation fragments (L2-resident) are loaded one chunk ahead of use.
  struct Stage {
    uint4 w[NL];
    float s[SC][HM ? MT : 1];
  };
  auto load = [&](int it, Stage& st) {
    const int s = wv + 4 * (it < cnt ? it : cnt - 1);
#pragma unroll
    for (int u = 0; u < NL; u++) st.w[u] = ld_u128(wseg + src[u] + (int64_t)s * SEG);
    if constexpr (HM) {
#pragma unroll
      for (int cc = 0; cc < SC; cc++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) st.s[cc][mt] = srow[mt][((int64_t)s * SC + cc) * Mp * 4];
    }
  };
  uint4 xn[MT][4];   // the next chunk's activation fragments
  auto load_x = [&](int64_t c) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) xn[mt][i] = xrow[mt][(c * 4 + i) * Mp * 4];
  };

#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // step it of the wave (ring slot st); the chunk after its last is the
  // first of step it + 1 (or its own last again, a redundant load)
  auto compute = [&](const Stage& st, int it) {
    const int s = wv + 4 * it;
    const int64_t cnext = it + 1 < cnt ? (int64_t)(s + 4) * SC : (int64_t)s * SC + SC - 1;
#pragma unroll
    for (int u = 0; u < NL; u++)
      if (pv[u]) *reinterpret_cast<uint4*>(reg + dst[u]) = st.w[u];
#pragma unroll
    for (int cc = 0; cc < SC; cc++) {
      f16x8_t xa[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) xa[mt][i] = __builtin_bit_cast(f16x8_t, xn[mt][i]);
      load_x(cc + 1 < SC ? (int64_t)s * SC + cc + 1 : cnext);
      uint32_t o[NT][BDW];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        RawBlk<SCH> b;
        load_blk<SCH>(la, 16 * t + j, 4 * cc + g, wok[t], b);
        normalise<SCH>(b, o[t]);
      }
      sk_chunk<SCH, MT, NT>(o, xa, HM ? st.s[cc] : nullptr, acc);
    }
  };
  if (cnt > 0) {
    Stage ring[D];
#pragma unroll
    for (int d = 0; d < D; d++) load(d, ring[d]);
    load_x((int64_t)wv * SC);
    int it0 = 0;
    for (; it0 + 2 * D <= cnt; it0 += D) {
#pragma unroll
      for (int d = 0; d < D; d++) {
        compute(ring[d], it0 + d);
        load(it0 + d + D, ring[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < D; d++) {
      if (it0 + d < cnt) {
        compute(ring[d], it0 + d);
        if (it0 + d + D < cnt) load(it0 + d + D, ring[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < D; d++)
      if (it0 + D + d < cnt) compute(ring[d], it0 + D + d);
  }
  return sk_wave_sum<MT, NT>(acc, reinterpret_cast<float*>(lds + 4 * R * LROW), wv, lane);
}

template <int SCH, int MT, int NT, int SC, int D>
RLXQ_DEV void skinny_xl_body(const rlxq_skinny_args& a) {
  extern __shared__ __align__(16) uint8_t smx[];
  const int lane = threadIdx.x & 63;
  const int j = lane & 15, g = lane >> 4;
  // Workgroup order: the dispatcher deals workgroups round-robin over the
  // eight XCDs, so b, b + 8, b + 16, ... share an XCD and its L2.  With a
  // grid of whole eights, consecutive workgroups of one XCD take the row
  // chunks of one (tile, split): the weight segments the first reads from
  // HBM the others find in that L2.  (A permutation of the grid; any order
  // computes the same sums.)
  const int G = (int)gridDim.x, mch = G / (a.tiles_n * a.splits);
  const int L = G % 8 == 0 ? (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
  const int mc = L % mch, rest = L / mch;
  const int tn = rest % a.tiles_n, sp = rest / a.tiles_n;
  const int64_t n0 = (int64_t)tn * 16 * NT, m0 = (int64_t)mc * 16 * MT;
  const int64_t kb = (int64_t)sp * a.kslice;
  const int64_t ke = kb + a.kslice < a.K ? kb + a.kslice : a.K;
  f32x4_t acc[MT][NT];
  if (!skinny_xl_core<SCH, MT, NT, SC, D>(a.x16, a.ssum, a.Mp, m0, a.w, a.rb, a.N, n0, kb, ke, acc, smx)) return;
  sk_store<MT, NT>(a, acc, m0, n0, sp, g, j);
}

// ---------------------------------------------------------------------------
// Grouped (MoE) variant of the register-streamed kernel for prefill-sized
// calls: a workgroup takes one chunk of 16 MT gathered rows, all of one
// expert, and NT 16-row weight tiles of that expert's slab; with SwiGLU the
// first NT / 2 tiles are gate rows and the rest the matching up rows N / 2
// further on, and the epilogue writes silu(g) * u.  Output rows go to the
// rows' entries.  Replaces the backend kernel of Op::DequantGroupedMatMul
// and the MoE expert FFN (crates/rlx-models-core/src/standard_decoder.rs:
// 12634-12760) at prefill sizes.
template <int SCH, int MT, int NT, int D, bool SW>
RLXQ_DEV void moe_sk_body(const rlxq_moe_sk_args& a) {
  constexpr int NH = SW ? NT / 2 : NT;   // output column tiles
  static_assert(!SW || NT % 2 == 0, "gate/up tile pairs");
  const int lane = threadIdx.x & 63;
  const int j = lane & 15, g = lane >> 4;
  const int chunk = blockIdx.x / a.tiles_n, tn = blockIdx.x % a.tiles_n;
  if (chunk >= a.cmap[0]) return;
  const int e = a.cmap[1 + chunk];
  const int64_t m0 = (int64_t)chunk * 16 * MT;
  const int64_t width = SW ? a.N / 2 : a.N;
  const int64_t n0 = (int64_t)tn * 16 * NH;
  int64_t wrow[NT];
  bool wok[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int64_t c = n0 + 16 * (t % NH) + j;
    wok[t] = c < width;
    const int64_t cc = wok[t] ? c : width - 1;
    wrow[t] = (SW && t >= NH) ? width + cc : cc;
  }
  f32x4_t acc[MT][NT];
  // the expert's scale slabs (MLX, MXFP4): N rows of K / group entries
  const int64_t slab = (int64_t)e * a.N * (a.K / a.group);
  const int esz = a.sb_bf16 == 0 ? 4 : (a.sb_bf16 == 1 ? 2 : 1);
  const void* sc = a.scales ? static_cast<const void*>(static_cast<const uint8_t*>(a.scales) + slab * esz) : nullptr;
  const void* bi = a.biases ? static_cast<const void*>(static_cast<const uint8_t*>(a.biases) + slab * esz) : nullptr;
  if (!skinny_xr_core<SCH, MT, NT, D>(a.x16, a.ssum, a.Mp, m0, a.bank + (int64_t)e * a.N * a.rb, a.rb, a.K, 0, a.K,
                                      wrow, wok, acc, sc, bi, a.group, a.sb_bf16))
    return;
  // C[i][j] of the 16x16 tile sits in lane j + 16*(i/4), register i%4.
  // With pairs, x16 rows 2r and 2r + 1 (a lane's registers 0, 1 and 2, 3)
  // are the hi and lo rows of gathered row r: their sums are added.
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      if (a.pairs && (r & 1)) continue;
      const int64_t m = m0 + 16 * mt + 4 * g + r;
      const int32_t ent = a.emap[a.pairs ? m >> 1 : m];
      if (ent < 0) continue;
      const float is = a.inv_s[m];
      const int r2 = a.pairs ? (r < 3 ? r + 1 : r) : r;   // (the pair's lo register)
#pragma unroll
      for (int t = 0; t < NH; t++) {
        const int64_t c = n0 + 16 * t + j;
        if (c >= width) continue;
        float o = (a.pairs ? acc[mt][t][r] + acc[mt][t][r2] : acc[mt][t][r]) * is;
        if constexpr (SW) {   // silu(g) * u
          const float u = (a.pairs ? acc[mt][t + NH][r] + acc[mt][t + NH][r2] : acc[mt][t + NH][r]) * is;
          o = o / (1.f + expf(-o)) * u;
        }
        const int64_t off = (int64_t)ent * a.y_ld + c;
        if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[off] = (uint16_t)f32_to_bf16_bits(o);
        else reinterpret_cast<float*>(a.y)[off] = o;
      }
    }
}

// ---------------------------------------------------------------------------
// N-split variant (GGUF Q4_1, Q4_0, Q8_0): the four waves of a workgroup take
// different weight rows (wave w: NT tiles of 16 rows) over the same K range,
// so each step's activations are loaded once per workgroup and shared through
// LDS; the weights stream into registers as in the register-streamed variant
// (lane (j, g): block 4c + g of row j of each tile).  A step is a
// 128-element K chunk c.  Both the weights and the activation pieces of a
// step are loaded D steps ahead into register rings (plain loads only, so
// the compiler's load-count waits stay exact); the activations of step s + 1
// go to LDS at the start of step s, into the slot step s - 1 read (two slots),
// and one barrier per step publishes them.
//
// LDS slot layout: group q = i MT + mt (piece i of the chunk's blocks, m-tile
// mt) is 1 KB, position g 16 + j holding the 16-byte piece of row 16 mt + j,
// block 4c + g, so an A fragment read is 1 KB of consecutive LDS (no bank
// conflicts).  Thread (w, lane) loads and stores piece i = w of every m-tile.
template <int SCH, int MT, int NT, int D>
RLXQ_DEV void skinny_ns_body(const rlxq_skinny_args& a) {
  constexpr int MC = 16 * MT;
  constexpr int AST = 4 * MC * 64;   // bytes of one activation slot
  constexpr int BDW = sk_bdw<SCH>();
  constexpr bool HM = sk_has_m<SCH>();
  extern __shared__ __align__(16) uint8_t sma[];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int tn = blockIdx.x % a.tiles_n;
  const int sp = (blockIdx.x / a.tiles_n) % a.splits;
  const int mc = blockIdx.x / (a.tiles_n * a.splits);
  const int64_t n0 = (int64_t)tn * 64 * NT + 16 * NT * wv, m0 = (int64_t)mc * MC;
  const int64_t kb = (int64_t)sp * a.kslice;
  const int64_t ke = kb + a.kslice < a.K ? kb + a.kslice : a.K;
  const int nsteps = (int)((ke - kb) / 128);

  rlxq_gemm_args ga;
  ga.w = a.w;
  ga.rb = a.rb;
  ga.K = a.K;
  ga.group = a.group;
  ga.sb_bf16 = a.sb_bf16;
  ga.scales = a.scales;
  ga.biases = a.biases;
  int64_t wrow[NT];
  bool wok[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int64_t n = n0 + 16 * t + j;
    wok[t] = n < a.N;
    wrow[t] = wok[t] ? n : a.N - 1;
  }
  // this thread's activation piece: row 16 u + j of the m-chunk, block 4c + g,
  // positions 8 wv .. 8 wv + 7 (fragment-major source; the Mp rows cover
  // every m-chunk)
  const u32x4_t* xsrc = reinterpret_cast<const u32x4_t*>(a.x16) + (wv * a.Mp + m0 + j) * 4 + g;
  // the block sums of rows 16 u + j, block 4c + g (min / bias term)
  const float* ssrc = HM ? a.ssum + (m0 + j) * 4 + g : nullptr;

  // ring slot d: a step's weight blocks wr[d] and activation pieces xr[d]
  // (pieces held as a clang vector type: a ring of HIP's uint4 struct, or
  // one struct of both rings, stayed in scratch memory for some schemes)
  RawBlk<SCH> wr[D][NT];
  u32x4_t xr[D][MT];
  float sr[D][HM ? MT : 1];
  // steps past the last repeat it (their data is never used), so every step
  // issues the same loads
  auto load = [&](int s, int d) {
    const int64_t c = kb / 128 + (s < nsteps ? s : nsteps - 1);
#pragma unroll
    for (int u = 0; u < MT; u++) xr[d][u] = xsrc[(4 * c * a.Mp + 16 * u) * 4];
#pragma unroll
    for (int t = 0; t < NT; t++) load_blk<SCH>(ga, wrow[t], 4 * c + g, wok[t], wr[d][t]);
    if constexpr (HM) {
#pragma unroll
      for (int u = 0; u < MT; u++) sr[d][u] = ssrc[(c * a.Mp + 16 * u) * 4];
    }
  };
  auto put = [&](int s, int d) {
    uint8_t* slot = sma + (s & 1) * AST;
#pragma unroll
    for (int u = 0; u < MT; u++) *reinterpret_cast<u32x4_t*>(slot + (wv * MT + u) * 1024 + lane * 16) = xr[d][u];
  };
  // the LDS stores of this wave have completed; then every wave's have
  auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int s, int d) {
    const uint8_t* slot = sma + (s & 1) * AST;
    uint32_t o[NT][BDW];
#pragma unroll
    for (int t = 0; t < NT; t++) normalise<SCH>(wr[d][t], o[t]);
    f16x8_t xa[MT][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) xa[mt][i] = *reinterpret_cast<const f16x8_t*>(slot + (i * MT + mt) * 1024 + lane * 16);
    sk_chunk<SCH, MT, NT>(o, xa, HM ? sr[d] : nullptr, acc);
  };
  // step s: ring slot s % D holds step s's weights (and step s's
  // activations, already in LDS slot s & 1); slot (s + 1) % D holds step
  // s + 1's activations, stored now into LDS slot (s + 1) & 1
  auto step = [&](int s, int d) {
    put(s + 1, (d + 1) % D);
    compute(s, d);
    load(s + D, d);
    barrier();
  };

#pragma unroll
  for (int d = 0; d < D; d++) load(d, d);
  put(0, 0);
  barrier();
  int s0 = 0;
  for (; s0 + D <= nsteps; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; d++) step(s0 + d, d);
  }
#pragma unroll
  for (int d = 0; d < D; d++)
    if (s0 + d < nsteps) step(s0 + d, d);

  sk_store<MT, NT>(a, acc, m0, n0, sp, g, j);
}

}  // namespace rlxq

// Activation preparation.  Workgroup (r, chunk) handles x16 row r's
// elements [2048 chunk, 2048 chunk + 2048): thread t one 16-byte piece,
// positions 8i .. 8i + 7 (i = t % 4) of block 64 chunk + t / 4 in the
// code-unpacking order.  Every workgroup of a row first reads the whole row
// for its maximum (L2 hits), so all workgroups find the same power-of-two
// scale, which puts the row maximum in [2^9, 2^10) (a block sum then stays
// below 2^15, inside f16).  The four pieces of a block are lanes 4b' .. 4b'
// + 3 of a wave: their sums add by two lane swaps.  With split, x16 rows
// 2r, 2r + 1 (split 1) or 64b + i, 64b + 32 + i (split 2) hold the
// f16 (bf16) rounding of row r's scaled elements (hi) and the remainder of
// that rounding (lo).
constexpr int X16_CHUNK = 2048;

// The 8 source elements of piece i of a block (positions 8i .. 8i + 7, code
// order `ORD`) as offsets into the block.
template <int ORD>
RLXQ_DEV int piece_src(int i, int e) {
  if constexpr (ORD == 0) return 8 * i + e;
  else if constexpr (ORD == 2) return 8 * i + (e < 4 ? 2 * e : 2 * (e - 4) + 1);
  else return e < 4 ? 4 * i + e : 16 + 4 * i + (e - 4);
}

template <int ORD>
RLXQ_DEV void load_piece(const rlxq_x16_args& a, int64_t src, int64_t b, int i, float* v) {
  if (a.x_bf16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(a.x) + src * a.K + b * 32;
    if constexpr (ORD == 1) {
      const uint2 u0 = *reinterpret_cast<const uint2*>(p + 4 * i);
      const uint2 u1 = *reinterpret_cast<const uint2*>(p + 16 + 4 * i);
      const uint32_t w[4] = {u0.x, u0.y, u1.x, u1.y};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[2 * e] = bf16_bits_to_f32(w[e] & 0xffffu);
        v[2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
      }
    } else {
      const uint4 u = *reinterpret_cast<const uint4*>(p + 8 * i);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
      float n[8];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        n[2 * e] = bf16_bits_to_f32(w[e] & 0xffffu);
        n[2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = n[piece_src<ORD>(i, e) - 8 * i];
    }
  } else {
    const float* p = reinterpret_cast<const float*>(a.x) + src * a.K + b * 32;
    if constexpr (ORD == 1) {
      const float4 f0 = *reinterpret_cast<const float4*>(p + 4 * i);
      const float4 f1 = *reinterpret_cast<const float4*>(p + 16 + 4 * i);
      v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
      v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
    } else {
      const float4 f0 = *reinterpret_cast<const float4*>(p + 8 * i);
      const float4 f1 = *reinterpret_cast<const float4*>(p + 8 * i + 4);
      const float n[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = n[piece_src<ORD>(i, e) - 8 * i];
    }
  }
}

template <int ORD>
RLXQ_DEV void x16_prep_body(const rlxq_x16_args& a) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63;
  // logical row (entry) of x16 row r and its part
  const int64_t lr = a.split == 2 ? ((r >> 6) << 5) + (r & 31) : (a.split ? r >> 1 : r);
  const bool lo_part = a.split == 2 ? ((r >> 5) & 1) != 0 : (a.split && (r & 1));
  const int64_t nblk = a.K >> 5, nchunk = (a.K + X16_CHUNK - 1) / X16_CHUNK;
  const int i = t & 3;   // this thread's piece of its block
  const int32_t ent = a.rmap ? (r < a.Mp ? a.rmap[lr] : -1) : 0;
  const int64_t src = a.rmap ? (int64_t)(ent >= 0 ? ent : 0) / a.rdiv : lr;   // x row of x16 row r
  auto store_piece = [&](int64_t b, uint4 o) {
    if (a.frag_major)
      reinterpret_cast<uint4*>(a.x16)[(((b >> 2) * 4 + i) * a.Mp + r) * 4 + (b & 3)] = o;
    else
      *reinterpret_cast<uint4*>(a.x16 + r * a.K + b * 32 + 8 * i) = o;
  };
  if (a.rmap ? ent < 0 : lr >= a.M) {
    // padding rows (fragment-major, and the row-major 64-row blocks): zeros
    if (a.frag_major || a.split == 2)
      for (int64_t cy = blockIdx.y; cy < nchunk; cy += gridDim.y) {
        const int64_t b = cy * (X16_CHUNK / 32) + (t >> 2);
        if (b >= nblk) continue;
        store_piece(b, make_uint4(0u, 0u, 0u, 0u));
        if (a.frag_major && a.ssum && i == 0) a.ssum[((b >> 2) * a.Mp + r) * 4 + (b & 3)] = 0.f;
      }
    if (!a.frag_major && a.split == 2 && blockIdx.y == 0 && t == 0) a.inv_s[r] = 0.f;
    return;
  }
  // the row maximum (every element of the row, 8 per load)
  float amax = 0.f;
  if (a.x_bf16) {
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.x) + src * a.K);
    for (int64_t q = t; q < a.K / 8; q += 256) {
      const uint4 u = p[q];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; e++)
        amax = fmaxf(amax, fmaxf(fabsf(bf16_bits_to_f32(w[e] & 0xffffu)), fabsf(bf16_bits_to_f32(w[e] >> 16))));
    }
  } else {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.x) + src * a.K);
    for (int64_t q = t; q < a.K / 4; q += 256) {
      const float4 f = p[q];
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if (lane == 0) red[t >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float s = 1.f, inv = ldexpf(1.f, a.post_exp);
  if (amax > 0.f && amax <= 3.4e38f) {
    int sh = 9 - ilogbf(amax);
    sh = sh < -126 ? -126 : (sh > 126 ? 126 : sh);
    s = ldexpf(1.f, sh);
    inv = ldexpf(ldexpf(1.f, -sh), a.post_exp);
  }
  if (blockIdx.y == 0 && t == 0) a.inv_s[r] = inv;
  // the row's chunks of 2048 elements, gridDim.y apart (one pass over the
  // row for its maximum, then each chunk, from cache, once)
  for (int64_t cy = blockIdx.y; cy < nchunk; cy += gridDim.y) {
  const int64_t b = cy * (X16_CHUNK / 32) + (t >> 2);   // this thread's block
  const bool live = b < nblk;
  float v[8];
  if (live) load_piece<ORD>(a, src, b, i, v);
  uint32_t o[4];
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    float w0 = live ? v[2 * e] * s : 0.f, w1 = live ? v[2 * e + 1] * s : 0.f;
    uint32_t h0 = a.out_bf16 ? f32_to_bf16_bits(w0) : f32_to_f16_bits(w0);
    uint32_t h1 = a.out_bf16 ? f32_to_bf16_bits(w1) : f32_to_f16_bits(w1);
    if (lo_part) {
      // the remainder w - hi is exact in f32; rounded once more
      w0 -= a.out_bf16 ? bf16_bits_to_f32(h0) : f16_bits_to_f32(h0);
      w1 -= a.out_bf16 ? bf16_bits_to_f32(h1) : f16_bits_to_f32(h1);
      h0 = a.out_bf16 ? f32_to_bf16_bits(w0) : f32_to_f16_bits(w0);
      h1 = a.out_bf16 ? f32_to_bf16_bits(w1) : f32_to_f16_bits(w1);
    }
    o[e] = h0 | (h1 << 16);
    sum += a.out_bf16 ? bf16_bits_to_f32(h0) : f16_bits_to_f32(h0);
    sum += a.out_bf16 ? bf16_bits_to_f32(h1) : f16_bits_to_f32(h1);
  }
  // block sum over the block's four pieces (lanes 4b' .. 4b' + 3), in a
  // fixed order: (p0 + p1) + (p2 + p3)
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  if (!live) continue;
  store_piece(b, make_uint4(o[0], o[1], o[2], o[3]));
  if (a.frag_major && a.ssum && i == 0) a.ssum[((b >> 2) * a.Mp + r) * 4 + (b & 3)] = sum;
  }
}

extern "C" __global__ __launch_bounds__(256) void rlxq_x16_prep(rlxq_x16_args a) {
  if (a.nibble_order == 1) x16_prep_body<1>(a);
  else if (a.nibble_order == 2) x16_prep_body<2>(a);
  else x16_prep_body<0>(a);
}

// Split-K partial sums added in split order.
// Four outputs per thread when N % 4 == 0 (up to eight slices' loads in
// flight), one otherwise; either way each output adds the slices in slice
// order, starting from zero.
extern "C" __global__ __launch_bounds__(256) void rlxq_skinny_reduce(rlxq_skinny_args a) {
  const int64_t mn = a.M * a.N;
  if ((a.N & 3) == 0) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= mn) return;
    const int64_t m = i / a.N, n = i - m * a.N;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.splits; s0 += 8) {
      const int cnt = a.splits - s0 < 8 ? a.splits - s0 : 8;
      float4 v[8];
#pragma unroll
      for (int q = 0; q < 8; q++)
        if (q < cnt) v[q] = *reinterpret_cast<const float4*>(a.part + (int64_t)(s0 + q) * mn + i);
#pragma unroll
      for (int q = 0; q < 8; q++)
        if (q < cnt) {
          s[0] += v[q].x;
          s[1] += v[q].y;
          s[2] += v[q].z;
          s[3] += v[q].w;
        }
    }
    if (a.y_bf16) {
      uint16_t* yp = reinterpret_cast<uint16_t*>(a.y) + m * a.y_ld + n;
#pragma unroll
      for (int e = 0; e < 4; e++) yp[e] = (uint16_t)f32_to_bf16_bits(s[e]);
    } else {
      float* yp = reinterpret_cast<float*>(a.y) + m * a.y_ld + n;
#pragma unroll
      for (int e = 0; e < 4; e++) yp[e] = s[e];
    }
    return;
  }
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= mn) return;
  const int64_t m = i / a.N, n = i - m * a.N;
  float v = 0.f;
  for (int sp = 0; sp < a.splits; sp++) v += a.part[(int64_t)sp * mn + i];
  if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = (uint16_t)f32_to_bf16_bits(v);
  else reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = v;
}

// Register-streamed variants: rlxq_skinnyxr_<scheme>_mt<MT>_nt<NT>_d<D>.
#define RLXQ_SKINNYXR_INST(SNAME, SCH, MT, NT, D)                                                      \
  extern "C" __global__ __launch_bounds__(256) void rlxq_skinnyxr_##SNAME##_mt##MT##_nt##NT##_d##D(     \
      rlxq_skinny_args a) {                                                                            \
    rlxq::skinny_xr_body<SCH, MT, NT, D>(a);                                                           \
  }
RLXQ_SKINNYXR_INST(q4_1, SCH_Q4_1, 1, 2, 4)
RLXQ_SKINNYXR_INST(q4_1, SCH_Q4_1, 1, 4, 2)
RLXQ_SKINNYXR_INST(q4_1, SCH_Q4_1, 1, 4, 3)
RLXQ_SKINNYXR_INST(q4_1, SCH_Q4_1, 2, 2, 3)
RLXQ_SKINNYXR_INST(q4_1, SCH_Q4_1, 2, 4, 2)
RLXQ_SKINNYXR_INST(q4_1, SCH_Q4_1, 4, 2, 2)
RLXQ_SKINNYXR_INST(q4_1, SCH_Q4_1, 4, 4, 1)
// the defaults only for the other schemes
RLXQ_SKINNYXR_INST(q4_0, SCH_Q4_0, 1, 2, 4)
RLXQ_SKINNYXR_INST(q4_0, SCH_Q4_0, 2, 2, 3)
RLXQ_SKINNYXR_INST(q4_0, SCH_Q4_0, 4, 2, 2)
RLXQ_SKINNYXR_INST(q8_0, SCH_Q8_0, 1, 2, 4)
RLXQ_SKINNYXR_INST(q8_0, SCH_Q8_0, 2, 2, 3)
RLXQ_SKINNYXR_INST(q8_0, SCH_Q8_0, 4, 2, 2)
// Q4_K sub-blocks (13-dword raw blocks: shallower rings)
RLXQ_SKINNYXR_INST(q4_k, SCH_Q4_K, 1, 2, 3)
RLXQ_SKINNYXR_INST(q4_k, SCH_Q4_K, 2, 2, 2)
RLXQ_SKINNYXR_INST(q4_k, SCH_Q4_K, 4, 2, 2)
// Q6_K (22-dword raw blocks)
RLXQ_SKINNYXR_INST(mlx4, SCH_MLX4, 1, 2, 4)
RLXQ_SKINNYXR_INST(mlx4, SCH_MLX4, 2, 2, 3)
RLXQ_SKINNYXR_INST(mlx4, SCH_MLX4, 4, 2, 2)
RLXQ_SKINNYXR_INST(mlx8, SCH_MLX8, 1, 2, 4)
RLXQ_SKINNYXR_INST(mlx8, SCH_MLX8, 2, 2, 3)
RLXQ_SKINNYXR_INST(mlx8, SCH_MLX8, 4, 2, 2)
RLXQ_SKINNYXR_INST(mxfp4, SCH_MXFP4, 1, 2, 4)
RLXQ_SKINNYXR_INST(mxfp4, SCH_MXFP4, 2, 2, 3)
RLXQ_SKINNYXR_INST(mxfp4, SCH_MXFP4, 4, 2, 2)
RLXQ_SKINNYXR_INST(q6_k, SCH_Q6_K, 1, 2, 2)
RLXQ_SKINNYXR_INST(q6_k, SCH_Q6_K, 2, 2, 2)
RLXQ_SKINNYXR_INST(q6_k, SCH_Q6_K, 4, 2, 1)
RLXQ_SKINNYXR_INST(q5_k, SCH_Q5_K, 1, 2, 2)
RLXQ_SKINNYXR_INST(q5_k, SCH_Q5_K, 2, 2, 2)
RLXQ_SKINNYXR_INST(q5_k, SCH_Q5_K, 4, 2, 1)
RLXQ_SKINNYXR_INST(q3_k, SCH_Q3_K, 1, 2, 2)
RLXQ_SKINNYXR_INST(q3_k, SCH_Q3_K, 2, 2, 2)
RLXQ_SKINNYXR_INST(q3_k, SCH_Q3_K, 4, 2, 1)
RLXQ_SKINNYXR_INST(q2_k, SCH_Q2_K, 1, 2, 3)
RLXQ_SKINNYXR_INST(q2_k, SCH_Q2_K, 2, 2, 2)
RLXQ_SKINNYXR_INST(q2_k, SCH_Q2_K, 4, 2, 2)
RLXQ_SKINNYXR_INST(q8_k, SCH_Q8_K, 1, 2, 4)
RLXQ_SKINNYXR_INST(q8_k, SCH_Q8_K, 2, 2, 3)
RLXQ_SKINNYXR_INST(q8_k, SCH_Q8_K, 4, 2, 2)

// N-split variants: rlxq_skinnyns_<scheme>_mt<MT>_nt<NT>_d<D>.
// LDS-staged variants: rlxq_skinnyxl_<scheme>_mt<MT>_nt<NT>_s<SC>_d<D>.
#define RLXQ_SKINNYXL_INST(SNAME, SCH, MT, NT, SC, D)                                                  \
  extern "C" __global__ __launch_bounds__(256) void rlxq_skinnyxl_##SNAME##_mt##MT##_nt##NT##_s##SC##_d##D( \
      rlxq_skinny_args a) {                                                                            \
    rlxq::skinny_xl_body<SCH, MT, NT, SC, D>(a);                                                       \
  }
RLXQ_SKINNYXL_INST(q4_1, SCH_Q4_1, 1, 2, 2, 1)
RLXQ_SKINNYXL_INST(q4_1, SCH_Q4_1, 1, 2, 1, 2)
RLXQ_SKINNYXL_INST(q4_1, SCH_Q4_1, 1, 2, 1, 3)
RLXQ_SKINNYXL_INST(q4_1, SCH_Q4_1, 1, 1, 2, 2)
RLXQ_SKINNYXL_INST(q4_1, SCH_Q4_1, 1, 4, 1, 2)
RLXQ_SKINNYXL_INST(q4_1, SCH_Q4_1, 2, 1, 2, 1)
RLXQ_SKINNYXL_INST(q4_0, SCH_Q4_0, 1, 2, 2, 1)
RLXQ_SKINNYXL_INST(q8_0, SCH_Q8_0, 1, 2, 2, 1)
RLXQ_SKINNYXL_INST(q4_k, SCH_Q4_K, 1, 2, 2, 1)
RLXQ_SKINNYXL_INST(q5_k, SCH_Q5_K, 1, 2, 2, 1)

#define RLXQ_SKINNYNS_INST(SNAME, SCH, MT, NT, D)                                                      \
  extern "C" __global__ __launch_bounds__(256) void rlxq_skinnyns_##SNAME##_mt##MT##_nt##NT##_d##D(     \
      rlxq_skinny_args a) {                                                                            \
    rlxq::skinny_ns_body<SCH, MT, NT, D>(a);                                                           \
  }
RLXQ_SKINNYNS_INST(q4_1, SCH_Q4_1, 1, 1, 3)
RLXQ_SKINNYNS_INST(q4_1, SCH_Q4_1, 2, 1, 3)
RLXQ_SKINNYNS_INST(q4_1, SCH_Q4_1, 2, 2, 3)
RLXQ_SKINNYNS_INST(q4_1, SCH_Q4_1, 4, 1, 3)
RLXQ_SKINNYNS_INST(q4_1, SCH_Q4_1, 4, 2, 2)
RLXQ_SKINNYNS_INST(q8_0, SCH_Q8_0, 4, 2, 2)
RLXQ_SKINNYNS_INST(q4_0, SCH_Q4_0, 4, 1, 3)
RLXQ_SKINNYNS_INST(q4_k, SCH_Q4_K, 1, 1, 3)
RLXQ_SKINNYNS_INST(q4_k, SCH_Q4_K, 2, 1, 3)
RLXQ_SKINNYNS_INST(q4_k, SCH_Q4_K, 4, 1, 3)
RLXQ_SKINNYNS_INST(mlx4, SCH_MLX4, 1, 1, 3)
RLXQ_SKINNYNS_INST(mlx4, SCH_MLX4, 2, 1, 3)
RLXQ_SKINNYNS_INST(mlx4, SCH_MLX4, 4, 1, 3)
RLXQ_SKINNYNS_INST(mlx8, SCH_MLX8, 1, 1, 3)
RLXQ_SKINNYNS_INST(mlx8, SCH_MLX8, 2, 1, 3)
RLXQ_SKINNYNS_INST(mlx8, SCH_MLX8, 4, 1, 3)
RLXQ_SKINNYNS_INST(mxfp4, SCH_MXFP4, 1, 1, 3)
RLXQ_SKINNYNS_INST(mxfp4, SCH_MXFP4, 2, 1, 3)
RLXQ_SKINNYNS_INST(mxfp4, SCH_MXFP4, 4, 1, 3)
RLXQ_SKINNYNS_INST(q6_k, SCH_Q6_K, 1, 1, 3)
RLXQ_SKINNYNS_INST(q6_k, SCH_Q6_K, 2, 1, 3)
RLXQ_SKINNYNS_INST(q6_k, SCH_Q6_K, 4, 1, 2)

// Gathered-row layout of the grouped MFMA path (see rlxq_moe_pad_args): one
// workgroup of 1024 threads, thread f for fired-expert slot f (E <= 1024).
extern "C" __global__ __launch_bounds__(1024) void rlxq_moe_pad_k(rlxq_moe_pad_args a) {
  __shared__ int32_t wsum[16];
  __shared__ int32_t cstart[1025];   // first chunk of each slot, then the total
  const int f = threadIdx.x, lane = f & 63, wv = f >> 6;
  const int F = a.table[0];
  const int32_t* off = a.table + 1 + a.E;
  const int32_t* perm = a.table + 2 + 2 * a.E;
  const int R = a.rows_per_chunk;
  const int cnt = f < F ? off[f + 1] - off[f] : 0;
  const int ch = (cnt + R - 1) / R;
  // exclusive sum of the chunk counts over the 1024 threads
  int inc = ch;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < 16; w++) {
    base += w < wv ? wsum[w] : 0;
    total += wsum[w];
  }
  const int first = base + inc - ch;
  if (f < F) cstart[f] = first;
  if (f == 0) {
    a.cmap[0] = total;
    cstart[F] = total;
  }
  __syncthreads();
  // every gathered row (and chunk) by all threads: the slot of chunk c is the
  // last slot whose first chunk is at most c
  auto slot_of = [&](int c) {
    int lo = 0, hi = F - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cstart[mid] <= c) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  };
  for (int c = f; c < total; c += 1024) a.cmap[1 + c] = a.table[1 + slot_of(c)];
  for (int64_t p = f; p < a.Mp; p += 1024) {
    const int c = (int)(p / R);
    int32_t v = -1;
    if (c < total) {
      const int s = slot_of(c);
      const int64_t local = p - (int64_t)cstart[s] * R;
      if (local < off[s + 1] - off[s]) v = perm[off[s] + local];
    }
    a.emap[p] = v;
  }
}

// Grouped MFMA variants: rlxq_moesk_<scheme>_mt<MT>_nt<NT>_d<D>[_sw].
#define RLXQ_MOESK_INST(SNAME, SCH, MT, NT, D)                                                         \
  extern "C" __global__ __launch_bounds__(256) void rlxq_moesk_##SNAME##_mt##MT##_nt##NT##_d##D(        \
      rlxq_moe_sk_args a) {                                                                            \
    rlxq::moe_sk_body<SCH, MT, NT, D, false>(a);                                                       \
  }                                                                                                    \
  extern "C" __global__ __launch_bounds__(256) void rlxq_moesk_##SNAME##_mt##MT##_nt##NT##_d##D##_sw(   \
      rlxq_moe_sk_args a) {                                                                            \
    rlxq::moe_sk_body<SCH, MT, NT, D, true>(a);                                                        \
  }
#define RLXQ_MOESK_SCHEME(SNAME, SCH, D1)   \
  RLXQ_MOESK_INST(SNAME, SCH, 1, 2, D1)     \
  RLXQ_MOESK_INST(SNAME, SCH, 1, 4, 2)      \
  RLXQ_MOESK_INST(SNAME, SCH, 1, 8, 2)      \
  RLXQ_MOESK_INST(SNAME, SCH, 2, 2, 3)      \
  RLXQ_MOESK_INST(SNAME, SCH, 2, 4, 2)      \
  RLXQ_MOESK_INST(SNAME, SCH, 2, 8, 1)      \
  RLXQ_MOESK_INST(SNAME, SCH, 4, 2, 2)      \
  RLXQ_MOESK_INST(SNAME, SCH, 4, 4, 1)
RLXQ_MOESK_SCHEME(q4_1, SCH_Q4_1, 4)
RLXQ_MOESK_SCHEME(q4_0, SCH_Q4_0, 4)
RLXQ_MOESK_SCHEME(q8_0, SCH_Q8_0, 4)
RLXQ_MOESK_SCHEME(q4_k, SCH_Q4_K, 3)
RLXQ_MOESK_SCHEME(mlx4, SCH_MLX4, 4)
RLXQ_MOESK_SCHEME(mlx8, SCH_MLX8, 4)
RLXQ_MOESK_SCHEME(mxfp4, SCH_MXFP4, 4)
// Q6_K (22-dword raw blocks: shallower rings)
RLXQ_MOESK_INST(q6_k, SCH_Q6_K, 1, 2, 2)
RLXQ_MOESK_INST(q6_k, SCH_Q6_K, 1, 4, 1)
RLXQ_MOESK_INST(q6_k, SCH_Q6_K, 2, 2, 2)
RLXQ_MOESK_INST(q6_k, SCH_Q6_K, 2, 4, 1)
RLXQ_MOESK_INST(q6_k, SCH_Q6_K, 4, 2, 1)
// Q5_K, Q3_K (21- and 24-dword raw blocks) as Q6_K; Q2_K as Q4_K, Q8_K as Q8_0
#define RLXQ_MOESK_SHALLOW(SNAME, SCH) \
  RLXQ_MOESK_INST(SNAME, SCH, 1, 2, 2) \
  RLXQ_MOESK_INST(SNAME, SCH, 1, 4, 1) \
  RLXQ_MOESK_INST(SNAME, SCH, 2, 2, 2) \
  RLXQ_MOESK_INST(SNAME, SCH, 2, 4, 1) \
  RLXQ_MOESK_INST(SNAME, SCH, 4, 2, 1)
RLXQ_MOESK_SHALLOW(q5_k, SCH_Q5_K)
RLXQ_MOESK_SHALLOW(q3_k, SCH_Q3_K)
RLXQ_MOESK_SCHEME(q2_k, SCH_Q2_K, 3)
RLXQ_MOESK_SCHEME(q8_k, SCH_Q8_K, 4)
