// Batched-decode dequant-GEMM for small M (the multi-row decode path):
// y[m, n] = sum_k x[m, k] * dequant(W)[n, k] for up to 64 activation rows and
// GGUF Q8_0 / Q4_0 / Q4_1 / Q4_K / Q6_K, MLX affine 4/8-bit and MXFP4
// weights, streaming every weight once for all
// rows.
// Replaces the backend kernel of Op::DequantMatMul at decode batch sizes
// (crates/rlx-models-core/src/standard_decoder.rs:727-738, M rows per call).
//
//  * rlxq_x16_prep: each activation row to f16, scaled by a power of two so
//    its largest element lies in [2^13, 2^14) (exact; undone in the
//    epilogue), and permuted within each 32-element block to the order in
//    which a lane unpacks the codes: for the GGUF nibble formats position
//    8g + e holds element 4g + e (e < 4) or 16 + 4g + e - 4, for MLX's
//    element 8g + 2e (e < 4) or 8g + 2(e - 4) + 1.
//  * rlxq_skinny_*: a workgroup takes 128 weight rows, a K split and all M
//    rows.  Per step the raw blocks are staged in LDS (a run of blocks per
//    thread, normalised to a dword scale word plus the code dwords) and the
//    prepared activations next to them; wave w then contracts blocks w,
//    w + 4, ... of the step: each lane turns its 8 codes into f16 weights with packed f16
//    arithmetic (exact codes, then d*q + m with one rounding) as the B operand
//    of v_mfma_f32_16x16x32_f16.  f16 weights keep the products within ~2^-12
//    of the exact dequantised weights (bf16 weights would not meet a 1e-3
//    output bound).  The four waves' partial sums are added in a fixed order.
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


// BPT blocks per thread per step: 2 threads per weight row, so a step spans
// NB = 2 * BPT blocks (KS = 32 * NB of K) and wave w contracts blocks
// w, w + 4, ...  One LDS buffer: the raw blocks of step s + 1 are in flight
// in registers while step s is contracted from LDS.
template <int SCH, int MT, int BPT>
RLXQ_DEV void skinny_body(const rlxq_skinny_args& a) {
  constexpr int NT = SK_BN / 16;   // 16-row N tiles per wave
  constexpr int NB = 2 * BPT, KS = 32 * NB;
  constexpr int BDW = sk_bdw<SCH>();
  // row stride: NB blocks + 2 dwords, so that the scale and code reads of 16
  // rows by 4 lane groups spread over the banks
  constexpr int RDW = NB * BDW + 2;
  constexpr int MC = 16 * MT;
  constexpr int XST = KS + 8;                  // activation LDS row stride (f16)
  constexpr int XC = MC * (KS / 8) / 256;      // 16-byte activation chunks per thread per step
  static_assert(XC >= 1 && (MC * (KS / 8)) % 256 == 0, "rows");
  extern __shared__ __align__(16) uint32_t sm[];
  uint32_t* Wl = sm;                                              // [SK_BN][RDW]
  uint16_t* Xl = reinterpret_cast<uint16_t*>(sm + SK_BN * RDW);    // [MC][XST]

  const int tn = blockIdx.x % a.tiles_n;
  const int sp = (blockIdx.x / a.tiles_n) % a.splits;
  const int mc = blockIdx.x / (a.tiles_n * a.splits);
  const int64_t n0 = (int64_t)tn * SK_BN, m0 = (int64_t)mc * MC;
  const int64_t kb = (int64_t)sp * a.kslice;
  const int64_t ke = kb + a.kslice < a.K ? kb + a.kslice : a.K;
  const int steps = (int)((ke - kb) / KS);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = lane >> 4, j = lane & 15;

  rlxq_gemm_args ga;
  ga.w = a.w;
  ga.rb = a.rb;
  ga.K = a.K;
  ga.group = 32;
  ga.sb_bf16 = 0;
  ga.scales = nullptr;
  ga.biases = nullptr;

  // staging: thread -> weight row tid >> 1, blocks (tid & 1) * BPT + q
  const int srow = tid >> 1, sblk = (tid & 1) * BPT;
  const bool sok = n0 + srow < a.N;
  const int64_t grow = sok ? n0 + srow : a.N - 1;
  RawBlk<SCH> rb[BPT];
  uint4 xr[XC];
  int64_t xoff[XC];
  bool xok[XC];
#pragma unroll
  for (int i = 0; i < XC; i++) {
    const int c = tid + 256 * i, row = c / (KS / 8);
    xok[i] = m0 + row < a.M;
    xoff[i] = (xok[i] ? m0 + row : a.M - 1) * a.K + (c % (KS / 8)) * 8;
  }

  auto gload = [&](int s) {
    const int64_t k0 = kb + (int64_t)s * KS;
#pragma unroll
    for (int q = 0; q < BPT; q++) load_blk<SCH>(ga, grow, k0 / 32 + sblk + q, sok, rb[q]);
#pragma unroll
    for (int i = 0; i < XC; i++) {
      const uint4 v = *reinterpret_cast<const uint4*>(a.x16 + xoff[i] + k0);
      xr[i] = xok[i] ? v : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int q = 0; q < BPT; q++) {
      uint32_t o[BDW];
      normalise<SCH>(rb[q], o);
      uint32_t* dst = Wl + srow * RDW + (sblk + q) * BDW;
#pragma unroll
      for (int i = 0; i < BDW; i++) dst[i] = o[i];
    }
#pragma unroll
    for (int i = 0; i < XC; i++) {
      const int c = tid + 256 * i;
      *reinterpret_cast<uint4*>(Xl + (c / (KS / 8)) * XST + (c % (KS / 8)) * 8) = xr[i];
    }
  };

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // wave wv contracts blocks wv + 4i of the step: A = activations, 16 rows x
  // 8 positions per lane (lane j + 16g: row j, positions 8g..8g+7 of the
  // block), B = the weights of 16 rows likewise
  auto compute = [&]() {
#pragma unroll
    for (int i = 0; i < NB / 4; i++) {
      const int blk = wv + 4 * i;
      f16x8_t af[MT];
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
        af[mt] = *reinterpret_cast<const f16x8_t*>(Xl + (16 * mt + j) * XST + 32 * blk + 8 * g);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const f16x8_t b = dequant_lane<SCH>(Wl + (16 * t + j) * RDW + blk * BDW, g);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mt], b, acc[mt][t], 0, 0, 0);
      }
    }
  };

  gload(0);
  lstore();
  __syncthreads();
  for (int s = 0; s + 1 < steps; s++) {
    gload(s + 1);
    compute();
    __syncthreads();
    lstore();
    __syncthreads();
  }
  compute();

  // Add the four waves' sums in the fixed order (w0 + w2) + (w1 + w3).
  constexpr int E = MT * NT * 4;
  float* R = reinterpret_cast<float*>(sm);   // [2][E][64], reuses the staging LDS
  __syncthreads();
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
  if (wv != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[mt][t][r] += R[((mt * NT + t) * 4 + r) * 64 + lane];
  sk_store<MT, NT>(a, acc, m0, n0, sp, g, j);
}

// Q4_1 with the weight and activation tiles copied global -> LDS by the
// gfx950 LDS-DMA load (global_load_lds_dwordx4: the 16 bytes of lane l land
// at the wave's LDS pointer + 16 l), into a ring of D stages of 256 K each, so
// D - 1 steps of loads are in flight without registers.  A stage holds
// 128 rows x 8 blocks (160 B per row, the blocks' raw bytes) and MC
// activation rows x 256 f16 (512 B per row, 16-byte chunks XOR-swizzled by
// row so the MFMA operand reads of 16 rows spread over the banks).
template <int MT, int D>
RLXQ_DEV void skinny_dma_body(const rlxq_skinny_args& a) {
  constexpr int NT = SK_BN / 16;
  constexpr int KS = 256, NB = 8;              // K and blocks per step
  constexpr int WROW = NB * 20;                // raw weight bytes per row per step
  constexpr int WCH = SK_BN * WROW / 16;       // 16-byte weight chunks per stage
  constexpr int MC = 16 * MT;
  constexpr int XCH = MC * KS * 2 / 16;        // 16-byte activation chunks per stage
  constexpr int NIW = WCH / 256, NIX = XCH / 256;   // DMA instructions per wave per stage
  static_assert(WCH % 256 == 0 && XCH % 256 == 0, "stage / waves");
  constexpr int WST = SK_BN * WROW, XSTB = MC * KS * 2, STAGE = WST + XSTB;   // bytes
  extern __shared__ __align__(16) uint8_t smb[];

  const int tn = blockIdx.x % a.tiles_n;
  const int sp = (blockIdx.x / a.tiles_n) % a.splits;
  const int mc = blockIdx.x / (a.tiles_n * a.splits);
  const int64_t n0 = (int64_t)tn * SK_BN, m0 = (int64_t)mc * MC;
  const int64_t kb = (int64_t)sp * a.kslice;
  const int64_t ke = kb + a.kslice < a.K ? kb + a.kslice : a.K;
  const int steps = (int)((ke - kb) / KS);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = lane >> 4, j = lane & 15;

  // per-lane global sources of this wave's DMA instructions (step offset added later)
  const uint8_t* wsrc[NIW];
#pragma unroll
  for (int i = 0; i < NIW; i++) {
    const int c = (wv * NIW + i) * 64 + lane;          // chunk of the stage
    const int r = c / (WROW / 16), piece = c % (WROW / 16);
    const int64_t row = n0 + r < a.N ? n0 + r : a.N - 1;
    wsrc[i] = a.w + row * a.rb + 16 * piece;
  }
  const uint16_t* xsrc[NIX];
#pragma unroll
  for (int i = 0; i < NIX; i++) {
    const int c = (wv * NIX + i) * 64 + lane;          // LDS chunk position
    const int r = c / 32, cp = c % 32;                 // 32 chunks per activation row
    const int lc = cp ^ (r & 15);                      // the logical chunk stored there
    const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;
    xsrc[i] = a.x16 + m * a.K + 8 * lc;
  }
  auto issue = [&](int s) {
    uint8_t* st = smb + (s % D) * STAGE;
    const int64_t k0 = kb + (int64_t)s * KS;
#pragma unroll
    for (int i = 0; i < NIW; i++)
      __builtin_amdgcn_global_load_lds(wsrc[i] + (k0 / 32) * 20, st + (wv * NIW + i) * 1024, 16, 0, 0);
#pragma unroll
    for (int i = 0; i < NIX; i++)
      __builtin_amdgcn_global_load_lds(xsrc[i] + k0, st + WST + (wv * NIX + i) * 1024, 16, 0, 0);
  };
  // wait until this wave's loads of step s have landed: at most `later`
  // steps' loads issued after them may still be outstanding
  auto wait_for = [&](int later) {
    constexpr int PER = NIW + NIX;
    if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER));
    else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  };

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int s) {
    const uint8_t* st = smb + (s % D) * STAGE;
    const uint32_t* Wl = reinterpret_cast<const uint32_t*>(st);
    const uint16_t* Xl = reinterpret_cast<const uint16_t*>(st + WST);
#pragma unroll
    for (int i = 0; i < NB / 4; i++) {
      const int blk = wv + 4 * i;
      f16x8_t af[MT];
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const int r = 16 * mt + j, lc = 4 * blk + g;
        af[mt] = *reinterpret_cast<const f16x8_t*>(Xl + r * KS + 8 * (lc ^ (r & 15)));
      }
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const f16x8_t b = dequant_lane<SCH_Q4_1>(Wl + (16 * t + j) * (WROW / 4) + blk * 5, g);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mt], b, acc[mt][t], 0, 0, 0);
      }
    }
  };

  static_assert(D == 3, "the wait counts below assume a ring of 3");
  for (int s = 0; s < D - 1 && s < steps; s++) issue(s);
  for (int s = 0; s < steps; s++) {
    const int later = steps - 1 - s < D - 2 ? steps - 1 - s : D - 2;
    wait_for(later);
    // this wave's operand reads of step s - 1 are complete, then the barrier:
    // step s landed for every wave, and no wave still reads step s - 1's slot
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    __builtin_amdgcn_s_barrier();
    if (s + D - 1 < steps) issue(s + D - 1);
    compute(s);
  }

  // Add the four waves' sums in the fixed order (w0 + w2) + (w1 + w3).
  constexpr int E = MT * NT * 4;
  float* R = reinterpret_cast<float*>(smb);
  __syncthreads();
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
  if (wv != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[mt][t][r] += R[((mt * NT + t) * 4 + r) * 64 + lane];
  sk_store<MT, NT>(a, acc, m0, n0, sp, g, j);
}

// ---------------------------------------------------------------------------
// Register-streamed variant (GGUF Q4_1, Q4_0, Q8_0): no LDS stage and no
// barrier per step.
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
RLXQ_DEV bool skinny_xr_core(const uint16_t* x16, int64_t Mp, int64_t m0, const uint8_t* w, int64_t rb, int64_t K,
                             int64_t kb, int64_t ke, const int64_t (&wrow)[NT], const bool (&wok)[NT],
                             f32x4_t (&acc)[MT][NT], const void* scales = nullptr,
                             const void* biases = nullptr, int64_t group = 32, int32_t sb_bf16 = 0) {
  constexpr int BDW = sk_bdw<SCH>();
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
  const uint4* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
    xrow[mt] = reinterpret_cast<const uint4*>(x16) + ((kb / 32) * Mp + m0 + 16 * mt + j) * 4 + g;

  struct Stage {
    RawBlk<SCH> w[NT];
    uint4 x[MT][4];
  };
  auto load = [&](int c, Stage& st) {
#pragma unroll
    for (int t = 0; t < NT; t++) load_blk<SCH>(ga, wrow[t], kb / 32 + 4 * c + g, wok[t], st.w[t]);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) st.x[mt][i] = xrow[mt][((int64_t)c * 4 + i) * Mp * 4];
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
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const auto b = sk_b<SCH>(o[t], i);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
          acc[mt][t] = sk_mfma<SCH>(__builtin_bit_cast(f16x8_t, st.x[mt][i]), b, acc[mt][t]);
      }
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

  // (w0 + w2) + (w1 + w3)
  constexpr int E = MT * NT * 4;
  extern __shared__ __align__(16) uint32_t sm[];
  float* R = reinterpret_cast<float*>(sm);   // [2][E][64]
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
  if (!skinny_xr_core<SCH, MT, NT, D>(a.x16, a.Mp, m0, a.w, a.rb, a.K, kb, ke, wrow, wok, acc, a.scales, a.biases,
                                      a.group, a.sb_bf16))
    return;
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
  if (!skinny_xr_core<SCH, MT, NT, D>(a.x16, a.Mp, m0, a.bank + (int64_t)e * a.N * a.rb, a.rb, a.K, 0, a.K, wrow,
                                      wok, acc, sc, bi, a.group, a.sb_bf16))
    return;
  // C[i][j] of the 16x16 tile sits in lane j + 16*(i/4), register i%4
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int64_t m = m0 + 16 * mt + 4 * g + r;
      const int32_t ent = a.emap[m];
      if (ent < 0) continue;
      const float is = a.inv_s[m];
#pragma unroll
      for (int t = 0; t < NH; t++) {
        const int64_t c = n0 + 16 * t + j;
        if (c >= width) continue;
        float o = acc[mt][t][r] * is;
        if constexpr (SW) o = o / (1.f + expf(-o)) * (acc[mt][t + NH][r] * is);   // silu(g) * u
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

  // ring slot d: a step's weight blocks wr[d] and activation pieces xr[d]
  // (pieces held as a clang vector type: a ring of HIP's uint4 struct, or
  // one struct of both rings, stayed in scratch memory for some schemes)
  RawBlk<SCH> wr[D][NT];
  u32x4_t xr[D][MT];
  // steps past the last repeat it (their data is never used), so every step
  // issues the same loads
  auto load = [&](int s, int d) {
    const int64_t c = kb / 128 + (s < nsteps ? s : nsteps - 1);
#pragma unroll
    for (int u = 0; u < MT; u++) xr[d][u] = xsrc[(4 * c * a.Mp + 16 * u) * 4];
#pragma unroll
    for (int t = 0; t < NT; t++) load_blk<SCH>(ga, wrow[t], 4 * c + g, wok[t], wr[d][t]);
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
#pragma unroll
    for (int i = 0; i < 4; i++) {
      f16x8_t af[MT];
#pragma unroll
      for (int mt = 0; mt < MT; mt++) af[mt] = *reinterpret_cast<const f16x8_t*>(slot + (i * MT + mt) * 1024 + lane * 16);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const auto b = sk_b<SCH>(o[t], i);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[mt][t] = sk_mfma<SCH>(af[mt], b, acc[mt][t]);
      }
    }
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

// One workgroup of 256 per activation row (per padded row in the
// fragment-major layout); each thread owns whole 32-element blocks (held in
// registers, so the permutation is local): blocks t, t + 256, t + 512
// (K <= 24576 keeps a row in registers; longer rows are read twice).
// With split, x16 rows 2r and 2r + 1 (two workgroups, which find the same
// row maximum and scale) hold the f16 (bf16) rounding of row r's scaled
// elements and the remainder of that rounding.
extern "C" __global__ __launch_bounds__(256) void rlxq_x16_prep(rlxq_x16_args a) {
  constexpr int RB = 3;   // register-resident blocks per thread
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int64_t lr = a.split ? r >> 1 : r;   // logical row (entry) of x16 row r
  const bool lo_part = a.split && (r & 1);
  const int64_t nblk = a.K >> 5;
  const int t = threadIdx.x;
  const int32_t ent = a.rmap ? (r < a.Mp ? a.rmap[lr] : -1) : 0;
  const int64_t src = a.rmap ? (int64_t)(ent >= 0 ? ent : 0) / a.rdiv : lr;   // x row of x16 row r
  if (a.rmap ? ent < 0 : lr >= a.M) {
    // padding rows of the fragment-major layout: zeros
    if (!a.frag_major || r >= a.Mp) return;
    uint4* dst = reinterpret_cast<uint4*>(a.x16);
    for (int64_t b = t; b < nblk; b += 256)
#pragma unroll
      for (int q = 0; q < 4; q++) dst[(((b >> 2) * 4 + q) * a.Mp + r) * 4 + (b & 3)] = make_uint4(0u, 0u, 0u, 0u);
    return;
  }
  auto load_blk32 = [&](int64_t b, float* v) {
    if (a.x_bf16) {
      const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.x) + src * a.K + b * 32);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint4 u = p[q];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[8 * q + 2 * e] = bf16_bits_to_f32(w[e] & 0xffffu);
          v[8 * q + 2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
        }
      }
    } else {
      const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.x) + src * a.K + b * 32);
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const float4 u = p[q];
        v[4 * q] = u.x; v[4 * q + 1] = u.y; v[4 * q + 2] = u.z; v[4 * q + 3] = u.w;
      }
    }
  };
  float v[RB][32];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < RB; i++) {
    const int64_t b = t + 256 * i;
    if (b < nblk) {
      load_blk32(b, v[i]);
#pragma unroll
      for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(v[i][e]));
    }
  }
  for (int64_t b = t + 256 * RB; b < nblk; b += 256) {
    float w[32];
    load_blk32(b, w);
#pragma unroll
    for (int e = 0; e < 32; e++) amax = fmaxf(amax, fabsf(w[e]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if ((t & 63) == 0) red[t >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // a power-of-two scale putting the row maximum in [2^13, 2^14)
  float s = 1.f, inv = 1.f;
  if (amax > 0.f && amax <= 3.4e38f) {
    int sh = 13 - ilogbf(amax);
    sh = sh < -126 ? -126 : (sh > 126 ? 126 : sh);
    s = ldexpf(1.f, sh);
    inv = ldexpf(1.f, -sh);
  }
  const int nib = a.nibble_order;
  auto store_blk32 = [&](int64_t b, const float* w) {
    uint32_t o[16];
#pragma unroll
    for (int p = 0; p < 32; p += 2) {
      float w0 = w[rlxq::perm_k(p, nib)] * s, w1 = w[rlxq::perm_k(p + 1, nib)] * s;
      uint32_t h0 = a.out_bf16 ? f32_to_bf16_bits(w0) : f32_to_f16_bits(w0);
      uint32_t h1 = a.out_bf16 ? f32_to_bf16_bits(w1) : f32_to_f16_bits(w1);
      if (lo_part) {
        // the remainder w - hi is exact in f32; rounded once more
        w0 -= a.out_bf16 ? bf16_bits_to_f32(h0) : f16_bits_to_f32(h0);
        w1 -= a.out_bf16 ? bf16_bits_to_f32(h1) : f16_bits_to_f32(h1);
        h0 = a.out_bf16 ? f32_to_bf16_bits(w0) : f32_to_f16_bits(w0);
        h1 = a.out_bf16 ? f32_to_bf16_bits(w1) : f32_to_f16_bits(w1);
      }
      o[p / 2] = h0 | (h1 << 16);
    }
    if (a.frag_major) {
      uint4* dst = reinterpret_cast<uint4*>(a.x16);
#pragma unroll
      for (int q = 0; q < 4; q++)
        dst[(((b >> 2) * 4 + q) * a.Mp + r) * 4 + (b & 3)] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    } else {
      uint4* dst = reinterpret_cast<uint4*>(a.x16 + r * a.K + b * 32);
#pragma unroll
      for (int q = 0; q < 4; q++) dst[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    }
  };
#pragma unroll
  for (int i = 0; i < RB; i++) {
    const int64_t b = t + 256 * i;
    if (b < nblk) store_blk32(b, v[i]);
  }
  for (int64_t b = t + 256 * RB; b < nblk; b += 256) {
    float w[32];
    load_blk32(b, w);
    store_blk32(b, w);
  }
  if (t == 0) a.inv_s[r] = inv;
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

#define RLXQ_SKINNY_INST(SNAME, SCH, MT, BPT)                                                      \
  extern "C" __global__ __launch_bounds__(256, 2) void rlxq_skinny_##SNAME##_mt##MT##_b##BPT(       \
      rlxq_skinny_args a) {                                                                        \
    rlxq::skinny_body<SCH, MT, BPT>(a);                                                            \
  }
#define RLXQ_SKINNY_SCHEME(SNAME, SCH) \
  RLXQ_SKINNY_INST(SNAME, SCH, 1, 2)   \
  RLXQ_SKINNY_INST(SNAME, SCH, 1, 8)   \
  RLXQ_SKINNY_INST(SNAME, SCH, 2, 2)   \
  RLXQ_SKINNY_INST(SNAME, SCH, 2, 8)   \
  RLXQ_SKINNY_INST(SNAME, SCH, 4, 2)   \
  RLXQ_SKINNY_INST(SNAME, SCH, 4, 4)
RLXQ_SKINNY_SCHEME(q4_1, SCH_Q4_1)
RLXQ_SKINNY_SCHEME(q4_0, SCH_Q4_0)
RLXQ_SKINNY_SCHEME(q8_0, SCH_Q8_0)

#define RLXQ_SKINNY_DMA_INST(MT)                                                                  \
  extern "C" __global__ __launch_bounds__(256, 2) void rlxq_skinny_q4_1_mt##MT##_dma(rlxq_skinny_args a) { \
    rlxq::skinny_dma_body<MT, 3>(a);                                                              \
  }
RLXQ_SKINNY_DMA_INST(1)
RLXQ_SKINNY_DMA_INST(2)
RLXQ_SKINNY_DMA_INST(4)

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

// N-split variants: rlxq_skinnyns_<scheme>_mt<MT>_nt<NT>_d<D>.
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
