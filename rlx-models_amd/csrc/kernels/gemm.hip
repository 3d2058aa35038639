// Prefill dequant-GEMM on bf16 MFMA: y[m, n] = sum_k x[m, k] * dequant(W)[n, k]
// for M >= 64 rows of bf16 activations, with fp32 accumulation and bf16 or
// f32 output.  Replaces the backend kernel of Op::DequantMatMul on the
// prefill path (crates/rlx-models-core/src/standard_decoder.rs:12421-12433).
//
// A workgroup (4 waves) owns a BM x BN output tile and walks K in steps of
// BK = 64:
//   * the activation tile [BM, BK] is copied global -> LDS (bf16, rows padded
//     to BK + 8 elements so the MFMA operand reads spread over the banks);
//   * the weight tile [BN, BK] is dequantized into LDS as bf16: each thread
//     turns one 32-weight block into f32 (d*q + m, the same arithmetic as the
//     CPU decoder) and rounds to bf16 (nearest even);
//   * every wave computes a (BM/2) x (BN/2) sub-tile with
//     v_mfma_f32_32x32x16_bf16 from the two LDS tiles.
// The global loads of step k+1 are in flight while the MFMAs of step k run;
// the LDS tiles are double-buffered, one barrier per step.
#include "common.hip.h"
#include "gemm_args.h"
#include "gemm_dq.hip.h"
#include "f16dq.hip.h"

namespace rlxq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int GBK = 64;        // K per step
constexpr int GLD = GBK + 8;   // LDS row stride (bf16 elements)


template <int SCH, int BM, int BN>
RLXQ_DEV void gemm_body(const rlxq_gemm_args& a) {
  static_assert(BM == 128 && BN == 128, "tile shape");
  constexpr int WM = BM / 2, WN = BN / 2;    // wave sub-tile
  constexpr int TM = WM / 32, TN = WN / 32;  // 32x32 MFMA tiles per wave
  extern __shared__ uint16_t smem[];
  uint16_t* As = smem;                        // [2][BM][GLD]
  uint16_t* Bs = smem + 2 * BM * GLD;         // [2][BN][GLD]

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv & 1, wn = wv >> 1;

  // Tile order: consecutive workgroups share the same weight columns (n), so
  // the weight tile is reused from L2 across the M tiles.
  const int64_t tiles_m = (a.M + BM - 1) / BM;
  const int64_t tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int KT = a.K / GBK;

  // activation tile: BM rows x 128 B; 256 threads x 4 chunks of 16 B
  uint4 areg[4];
  auto load_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = tid + 256 * i, r = c >> 3, c16 = c & 7;
      const int64_t row = m0 + r;
      areg[i] = make_uint4(0u, 0u, 0u, 0u);
      if (row < a.M)
        areg[i] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.x) + row * a.K +
                                                  (int64_t)kt * GBK + c16 * 8);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = tid + 256 * i, r = c >> 3, c16 = c & 7;
      *reinterpret_cast<uint4*>(As + (buf * BM + r) * GLD + c16 * 8) = areg[i];
    }
  };
  // weight tile: BN rows x 2 blocks; thread -> (row, block)
  const int brow = tid >> 1, bblk = tid & 1;
  auto dequant_b = [&](int kt, int buf) {
    uint32_t o[16];
    const int64_t row = n0 + brow;
    dequant_block_bf16<SCH>(a, row < a.N ? row : 0, (int64_t)kt * 2 + bblk, row < a.N, o);
    uint16_t* dst = Bs + (buf * BN + brow) * GLD + bblk * 32;
#pragma unroll
    for (int i = 0; i < 4; i++)
      *reinterpret_cast<uint4*>(dst + 8 * i) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  load_a(0);
  dequant_b(0, 0);
  store_a(0);
  __syncthreads();

  for (int kt = 0; kt < KT; kt++) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) load_a(kt + 1);
    const uint16_t* Ab = As + (cur * BM + wm * WM) * GLD;
    const uint16_t* Bb = Bs + (cur * BN + wn * WN) * GLD;
#pragma unroll
    for (int ks = 0; ks < GBK / 16; ks++) {
      bf16x8_t af[TM], bfr[TN];
      const int kof = ks * 16 + 8 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < TM; i++)
        af[i] = *reinterpret_cast<const bf16x8_t*>(Ab + (i * 32 + (lane & 31)) * GLD + kof);
#pragma unroll
      for (int j = 0; j < TN; j++)
        bfr[j] = *reinterpret_cast<const bf16x8_t*>(Bb + (j * 32 + (lane & 31)) * GLD + kof);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      dequant_b(kt + 1, cur ^ 1);
      store_a(cur ^ 1);
    }
    __syncthreads();
  }

  // epilogue: C[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), reg 4*(i/8) + i%4
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int64_t m = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
        const int64_t n = n0 + wn * WN + j * 32 + (lane & 31);
        if (m < a.M && n < a.N) {
          const float v = acc[i][j][r];
          if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = (uint16_t)f32_to_bf16_bits(v);
          else reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = v;
        }
      }
}

// 256 x 256 output tile, one workgroup per CU (144 KB of LDS), WGM x WGN
// waves each owning a (256/WGM) x (256/WGN) sub-tile of 32x32 MFMA tiles with
// f32 accumulators in AGPRs.  With 4 waves (2 x 2, 128 x 128 each) a wave
// issues 64 MFMAs per K step against 32 KB of LDS operand reads, half the LDS
// bytes per MFMA of a 64 x 64 wave tile; with 8 waves (2 x 4) two waves share
// each SIMD, so one wave's dequantisation and waits overlap the other's
// MFMAs.  The loop body has no branches (row bounds are clamped addresses plus
// selects), and the next step's LDS stores and conversions sit between the
// MFMA groups of the current step.
// EXACT (f16 MFMA, f32 output at the 1e-3 bar on any data): each weight's
// f32 value, computed with the CPU decoder's arithmetic, is held as an f16
// hi and lo half in B rows 32 apart (B rows 64c' + i and 64c' + 32 + i: real
// column 32c' + i, so a tile covers 128 real columns and a wave's two 32-row
// MFMA tiles hold the hi and the lo halves of the same 32 columns); the
// epilogue adds the two tiles' sums in registers.  SPLITX (f32 activations):
// the activation rows are prepared the same way, hi and lo rows in 32-row
// blocks, so a wave's four row tiles are (hi, lo) of two row groups; the
// lo x lo products (~2^-22 of a term) are skipped, three MFMAs per pair.
// With f16 weights rounded once instead, structured data (the reference's
// sin / cos parity inputs at K = 1792) already reaches 1.4e-3.  MLX, Q8_K and
// Q2_K weights are held times 2^8 (sk_wscale; undone through the activation
// row factors) so that small scales stay normal f16.
// BNT = 128 (bf16 variant only): 256 x 128 tiles, twice the tiles of a
// shape, so half the K slices where the tiles do not cover the CUs (half the
// split-K partial sums written and added).
template <int SCH, int WGM, int WGN, int PF, bool F16, bool LATE = false, bool EXACT = false, bool SPLITX = false,
          int BNT = 256>
RLXQ_DEV void gemm256_body(const rlxq_gemm_args& a) {
  static_assert(EXACT == F16, "f16 MFMA runs the exact variant on the prepared f16 activations");
  static_assert(!SPLITX || EXACT, "hi / lo activation rows on the exact variant");
  static_assert(BNT == 256 || (BNT == 128 && !EXACT), "256 x 128 tiles on the bf16 variant");
  constexpr int BM = 256, BN = BNT;
  constexpr int NREAL = EXACT ? BN / 2 : BN;   // output columns per tile
  constexpr float WSCALE = sk_wscale<SCH>();
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AP = 2048 / NT;   // 16-byte activation chunks per thread per step
  // weight blocks per step: 2 BN; per thread BPT, or one in the first 2 BN
  // threads when there are more threads than blocks (whole waves)
  constexpr int WB = 2 * BN;
  constexpr bool WALL = WB >= NT;
  constexpr int BPT = WALL ? WB / NT : 1;
  static_assert(AP % 2 == 0 && BPT >= 1 && WB % 64 == 0, "threads");
  extern __shared__ uint16_t smem[];
  uint16_t* As = smem;                // [2][BM][GLD]
  uint16_t* Bs = smem + 2 * BM * GLD;  // [2][BN][GLD]

  // workgroup = (K slice, tile): the slice is the slowest index, so the
  // tiles of one slice keep the XCD-aware order
  const int tiles_pad = 8 * ((a.tiles_m * a.tiles_n + 7) / 8);
  const int sp = blockIdx.x / tiles_pad;
  int tm, tn;
  if (!tile_of(blockIdx.x % tiles_pad, a.tiles_m, a.tiles_n, 4, tm, tn)) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv % WGM, wn = wv / WGM;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * NREAL;
  const int64_t kbeg = (int64_t)sp * a.kslice;
  const int64_t kend = kbeg + a.kslice < a.K ? kbeg + a.kslice : a.K;
  const int KT = (int)((kend - kbeg) / GBK);
  const int kt0 = (int)(kbeg / GBK);
  const uint16_t* xg = reinterpret_cast<const uint16_t*>(a.x);

  // activation tile: 256 rows x 128 B = 2048 chunks of 16 B.  Rows past M
  // read row M - 1 and weight rows past N read row N - 1: they only feed
  // output rows and columns that are not stored, so no select zeroes them.
  int64_t arow[AP];
#pragma unroll
  for (int i = 0; i < AP; i++) {
    const int c = tid + NT * i, r = c >> 3;
    arow[i] = (m0 + r < a.M ? m0 + r : a.M - 1) * a.K + (c & 7) * 8;
  }
  // weight tile: BN rows x 2 blocks; thread -> row n0 + tid % BN, blocks
  // tid / BN + q * (NT / BN)
  // (EXACT: B row brl holds half (brl >> 5) & 1 of real column
  // n0 + 32 (brl >> 6) + brl % 32)
  const int brl = tid & (BN - 1);
  const bool wthread = WALL || tid < WB;
  auto wblk = [&](int q) { return tid / BN + q * (NT / BN); };
  const int64_t bcol = n0 + (EXACT ? ((brl >> 6) << 5) + (brl & 31) : brl);
  const int64_t brow = bcol < a.N ? bcol : a.N - 1;

  // Global loads run PF steps ahead of the MFMAs (PF register stages); the
  // LDS stores and conversions of the next step sit between the MFMA groups
  // of the current one.
  // (activation chunks as a clang vector type: HIP's uint4 struct copied in
  // from memory kept the stages in scratch memory)
  struct Stage {
    u32x4_t a[AP];
    RawBlk<SCH> b[BPT];
  };
  auto gload = [&](int kt, Stage& P) {
    kt += kt0;
#pragma unroll
    for (int i = 0; i < AP; i++) P.a[i] = *reinterpret_cast<const u32x4_t*>(xg + arow[i] + (int64_t)kt * GBK);
    if (wthread) {
#pragma unroll
      for (int q = 0; q < BPT; q++) load_blk<SCH>(a, brow, 2 * (int64_t)kt + wblk(q), true, P.b[q]);
    }
  };
  auto store_a = [&](const Stage& P, int buf, int half) {
#pragma unroll
    for (int i = half * AP / 2; i < (half + 1) * AP / 2; i++) {
      const int c = tid + NT * i;
      *reinterpret_cast<u32x4_t*>(As + (buf * BM + (c >> 3)) * GLD + (c & 7) * 8) = P.a[i];
    }
  };
  auto store_b = [&](const Stage& P, int buf, int q) {
    if (!wthread) return;
    uint16_t* dst = Bs + (buf * BN + brl) * GLD + wblk(q) * 32;
    if constexpr (EXACT) {
      // The two threads of a real column (B rows brl and brl ^ 32, the same
      // raw block) split the block's K range: thread half h converts
      // elements 16h .. 16h + 15 and writes their hi halves to the column's
      // hi row and their lo halves to its lo row.
      const int h = (brl >> 5) & 1;
      // (the half as a bit mask, opaque to the optimiser)
      uint32_t mh = 0u - (uint32_t)h;
      asm volatile("" : "+v"(mh));
      float w[16];
      blk_f32_half<SCH>(P.b[q], mh, w);
#pragma unroll
      for (int e = 0; e < 16; e++) w[e] *= WSCALE;
      uint32_t hi[8], lo[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float a0 = w[2 * i], a1 = w[2 * i + 1];
        const uint32_t h0 = f32_to_f16_bits(a0), h1 = f32_to_f16_bits(a1);
        hi[i] = h0 | (h1 << 16);
        lo[i] = f32_to_f16_bits(a0 - f16_bits_to_f32(h0)) | (f32_to_f16_bits(a1 - f16_bits_to_f32(h1)) << 16);
      }
      const int kof = wblk(q) * 32 + 16 * h;
      uint16_t* dh = Bs + (buf * BN + (brl & ~32)) * GLD + kof;
      uint16_t* dl = Bs + (buf * BN + (brl | 32)) * GLD + kof;
      *reinterpret_cast<uint4*>(dh) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
      *reinterpret_cast<uint4*>(dh + 8) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
      *reinterpret_cast<uint4*>(dl) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
      *reinterpret_cast<uint4*>(dl + 8) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
    } else {
      uint32_t o[16];
      conv_blk<SCH>(P.b[q], o);
#pragma unroll
      for (int i = 0; i < 4; i++)
        *reinterpret_cast<uint4*>(dst + 8 * i) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  auto compute_ks = [&](int cur, int ks) {
    const uint16_t* Ab = As + (cur * BM + wm * WM) * GLD;
    const uint16_t* Bb = Bs + (cur * BN + wn * WN) * GLD;
    const int kof = ks * 16 + 8 * (lane >> 5);
    if constexpr (F16) {
      f16x8_t af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) af[i] = *reinterpret_cast<const f16x8_t*>(Ab + (i * 32 + (lane & 31)) * GLD + kof);
#pragma unroll
      for (int j = 0; j < TN; j++) bfr[j] = *reinterpret_cast<const f16x8_t*>(Bb + (j * 32 + (lane & 31)) * GLD + kof);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
          if (!(SPLITX && (i & 1) && (j & 1)))   // (lo activations x lo weights: skipped)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    } else {
      bf16x8_t af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) af[i] = *reinterpret_cast<const bf16x8_t*>(Ab + (i * 32 + (lane & 31)) * GLD + kof);
#pragma unroll
      for (int j = 0; j < TN; j++) bfr[j] = *reinterpret_cast<const bf16x8_t*>(Bb + (j * 32 + (lane & 31)) * GLD + kof);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  };
  auto store_all = [&](const Stage& P, int buf) {
    store_a(P, buf, 0);
    store_a(P, buf, 1);
#pragma unroll
    for (int q = 0; q < BPT; q++) store_b(P, buf, q);
  };
  // one K step: MFMAs from buffer `cur` while stage `Pn` goes into cur ^ 1
  auto step = [&](int cur, const Stage& Pn) {
    compute_ks(cur, 0);
    compute_ks(cur, 1);
    store_a(Pn, cur ^ 1, 0);
    compute_ks(cur, 2);
    store_a(Pn, cur ^ 1, 1);
    store_b(Pn, cur ^ 1, 0);
    compute_ks(cur, 3);
#pragma unroll
    for (int q = 1; q < BPT; q++) store_b(Pn, cur ^ 1, q);
  };

  if constexpr (PF == 1) {
    Stage P;
    gload(0, P);
    store_all(P, 0);
    __syncthreads();
    for (int kt = 0; kt + 1 < KT; kt++) {
      gload(kt + 1, P);
      if constexpr (LATE) {
        // the stage's LDS stores after all four MFMA groups: the loads have
        // the whole step to arrive
#pragma unroll
        for (int ks = 0; ks < GBK / 16; ks++) compute_ks(kt & 1, ks);
        store_all(P, (kt & 1) ^ 1);
      } else {
        step(kt & 1, P);
      }
      __syncthreads();
    }
  } else {
    // two stages, the loop unrolled by two so each stage is a fixed register set
    Stage P0, P1;
    gload(0, P0);
    gload(KT > 1 ? 1 : 0, P1);
    store_all(P0, 0);
    __syncthreads();
    int kt = 0;
    for (; kt + 2 < KT; kt += 2) {
      gload(kt + 2, P0);
      step(0, P1);
      __syncthreads();
      gload(kt + 3 < KT ? kt + 3 : KT - 1, P1);
      step(1, P0);
      __syncthreads();
    }
    if (kt + 1 < KT) {
      step(0, P1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int ks = 0; ks < GBK / 16; ks++) compute_ks((KT - 1) & 1, ks);

  // epilogue: C[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), reg
  // 4*(i/8) + i%4.  The tiles are walked with compile-time indices: a runtime
  // loop over them would index the accumulators dynamically and move them to
  // scratch memory.  The destination (partial sums, bf16 or f32 output) and
  // whether the tile lies wholly inside M x N are decided once per
  // workgroup; a lane then stores through one base pointer at offsets that
  // are wave-uniform (row offset x leading dimension), so a whole tile needs
  // no per-element bounds checks, branches or 64-bit multiplies (the
  // per-element form cost 8% of the kernel at M=4096).
  const int64_t mb = m0 + wm * WM + 4 * (lane >> 5);   // the lane's first row
  if constexpr (EXACT) {
    static_assert(TN == 2 && WN == 64, "a wave's two column tiles are the hi and lo halves of 32 columns");
    // Output: the wave's 32 real columns n0 + 32 wn + (lane & 31); rows of
    // row tile i (or, with SPLITX, of row group g = tiles 2g (hi), 2g + 1
    // (lo)).  C[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), reg
    // 4*(i/8) + i%4.
    constexpr int RT = SPLITX ? TM / 2 : TM;          // output row tiles per wave
    const int64_t m0r = SPLITX ? (int64_t)tm * (BM / 2) : m0;   // first output row of the tile
    const int64_t mbo = m0r + wm * (WM / (SPLITX ? 2 : 1)) + 4 * (lane >> 5);
    const int64_t nbo = n0 + wn * (WN / 2) + (lane & 31);
    const bool whole = m0r + (SPLITX ? BM / 2 : BM) <= a.m_out && n0 + NREAL <= a.N;
    auto epx = [&](auto put, auto checked) {
      static_for<RT>([&](auto G) {
        constexpr int g = G.value;
        const f32x16_t v = SPLITX ? acc[2 * g][0] + acc[2 * g + 1][0] + acc[2 * g][1] : acc[g][0] + acc[g][1];
        // the row factor of the tile's (hi) x16 rows
        const int64_t mp = m0 + wm * WM + (SPLITX ? 64 * g : 32 * g) + 4 * (lane >> 5);
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int dm = 32 * g + 8 * (r / 4) + (r % 4);
          const float o = v[r] * a.inv_s[mp + 8 * (r / 4) + (r % 4)];
          if (!checked.value || (mbo + dm < a.m_out && nbo < a.N)) put(dm, o);
        }
      });
    };
    auto epx_any = [&](auto put) {
      if (whole) epx(put, std::false_type{});
      else epx(put, std::true_type{});
    };
    if (a.splits > 1) {
      float* p = a.part + ((int64_t)sp * a.m_out + mbo) * a.N + nbo;
      epx_any([&](int dm, float o) { p[(int64_t)dm * a.N] = o; });
    } else if (a.y_bf16) {
      uint16_t* p = reinterpret_cast<uint16_t*>(a.y) + mbo * a.y_ld + nbo;
      epx_any([&](int dm, float o) { p[(int64_t)dm * a.y_ld] = (uint16_t)f32_to_bf16_bits(o); });
    } else {
      float* p = reinterpret_cast<float*>(a.y) + mbo * a.y_ld + nbo;
      epx_any([&](int dm, float o) { p[(int64_t)dm * a.y_ld] = o; });
    }
    return;
  }
  const int64_t nb = n0 + wn * WN + (lane & 31);       // its column in tile 0
  const bool whole = m0 + BM <= a.M && n0 + BN <= a.N;
  auto epi = [&](auto put, auto checked) {
    static_for<TM>([&](auto I) {
      static_for<TN>([&](auto J) {
        const f32x16_t v = acc[I.value][J.value];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          constexpr int dn = J.value * 32;
          const int dm = I.value * 32 + 8 * (r / 4) + (r % 4);
          if (!checked.value || (mb + dm < a.M && nb + dn < a.N))
            put(dm, dn, v[r]);
        }
      });
    });
  };
  auto epi_any = [&](auto put) {
    if (whole) epi(put, std::false_type{});
    else epi(put, std::true_type{});
  };
  if (a.splits > 1) {
    float* p = a.part + ((int64_t)sp * a.M + mb) * a.N + nb;
    epi_any([&](int dm, int dn, float o) { p[(int64_t)dm * a.N + dn] = o; });
  } else if (a.y_bf16) {
    uint16_t* p = reinterpret_cast<uint16_t*>(a.y) + mb * a.y_ld + nb;
    epi_any([&](int dm, int dn, float o) { p[(int64_t)dm * a.y_ld + dn] = (uint16_t)f32_to_bf16_bits(o); });
  } else {
    float* p = reinterpret_cast<float*>(a.y) + mb * a.y_ld + nb;
    epi_any([&](int dm, int dn, float o) { p[(int64_t)dm * a.y_ld + dn] = o; });
  }
}

}  // namespace rlxq

#define RLXQ_GEMM_INST(NAME, SCH)                                                         \
  extern "C" __global__ __launch_bounds__(256) void NAME(rlxq_gemm_args a) {             \
    rlxq::gemm_body<SCH, 128, 128>(a);                                                     \
  }
RLXQ_GEMM_INST(rlxq_gemm_q4_1_t128, SCH_Q4_1)
RLXQ_GEMM_INST(rlxq_gemm_q4_0_t128, SCH_Q4_0)
RLXQ_GEMM_INST(rlxq_gemm_q8_0_t128, SCH_Q8_0)
RLXQ_GEMM_INST(rlxq_gemm_mlx4_t128, SCH_MLX4)
RLXQ_GEMM_INST(rlxq_gemm_mlx8_t128, SCH_MLX8)
RLXQ_GEMM_INST(rlxq_gemm_q4_k_t128, SCH_Q4_K)
RLXQ_GEMM_INST(rlxq_gemm_q6_k_t128, SCH_Q6_K)
RLXQ_GEMM_INST(rlxq_gemm_q8_k_t128, SCH_Q8_K)
RLXQ_GEMM_INST(rlxq_gemm_mxfp4_t128, SCH_MXFP4)
RLXQ_GEMM_INST(rlxq_gemm_q5_k_t128, SCH_Q5_K)
RLXQ_GEMM_INST(rlxq_gemm_q3_k_t128, SCH_Q3_K)
RLXQ_GEMM_INST(rlxq_gemm_q2_k_t128, SCH_Q2_K)

#define RLXQ_GEMM256_INST(SNAME, SCH)                                                        \
  extern "C" __global__ __launch_bounds__(256, 1) void rlxq_gemm_##SNAME##_t256(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 2, 1, false>(a);                                                    \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(512, 1) void rlxq_gemm_##SNAME##_t256w8(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 4, 1, false>(a);                                                    \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(512, 1) void rlxq_gemm_##SNAME##_t256w8p2(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 4, 2, false>(a);                                                    \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(512, 1) void rlxq_gemm_##SNAME##_t256w8l(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 4, 1, false, true>(a);                                              \
  }
// 256 x 128 tiles (bf16 variant): rlxq_gemm_<scheme>_t256n128 (4 waves, 2 x 2,
// 128 x 64 each) and ..._t256n128w8 (8 waves, 4 x 2, 64 x 64 each; the first
// four convert the weight blocks)
#define RLXQ_GEMM256N_INST(SNAME, SCH, PF, LATE)                                              \
  extern "C" __global__ __launch_bounds__(256, 1) void rlxq_gemm_##SNAME##_t256n128(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 2, PF, false, LATE, false, false, 128>(a);                          \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(512, 1) void rlxq_gemm_##SNAME##_t256n128w8(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 4, 2, PF, false, LATE, false, false, 128>(a);                          \
  }
// Exact f32-output variant (EXACT above): rlxq_gemm_<scheme>_t256w8[p2|l]x,
// f16 MFMA on the prepared activations (natural order), f16 hi + lo weights
// and rlxq_gemm_<scheme>_t256w8[p2|l]xs for f32 activations (hi / lo rows)
#define RLXQ_GEMM256XN_INST(SNAME, SCH, PF, SUFFIX, LATE)                                    \
  extern "C" __global__ __launch_bounds__(512, 1) void rlxq_gemm_##SNAME##_t256w8##SUFFIX##x(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 4, PF, true, LATE, true, false>(a);                                 \
  }
#define RLXQ_GEMM256XS_INST(SNAME, SCH, PF, SUFFIX, LATE)                                    \
  extern "C" __global__ __launch_bounds__(512, 1) void rlxq_gemm_##SNAME##_t256w8##SUFFIX##xs(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 4, PF, true, LATE, true, true>(a);                                  \
  }
#define RLXQ_GEMM256X_INST(SNAME, SCH, PF, SUFFIX, LATE) \
  RLXQ_GEMM256XN_INST(SNAME, SCH, PF, SUFFIX, LATE)      \
  RLXQ_GEMM256XS_INST(SNAME, SCH, PF, SUFFIX, LATE)
RLXQ_GEMM256_INST(q4_1, SCH_Q4_1)
RLXQ_GEMM256_INST(q4_0, SCH_Q4_0)
RLXQ_GEMM256_INST(q8_0, SCH_Q8_0)
RLXQ_GEMM256_INST(mlx4, SCH_MLX4)
RLXQ_GEMM256_INST(mlx8, SCH_MLX8)
RLXQ_GEMM256_INST(q4_k, SCH_Q4_K)
RLXQ_GEMM256_INST(q6_k, SCH_Q6_K)
RLXQ_GEMM256_INST(q8_k, SCH_Q8_K)
RLXQ_GEMM256_INST(mxfp4, SCH_MXFP4)
RLXQ_GEMM256_INST(q5_k, SCH_Q5_K)
RLXQ_GEMM256_INST(q3_k, SCH_Q3_K)
RLXQ_GEMM256_INST(q2_k, SCH_Q2_K)
RLXQ_GEMM256N_INST(q4_1, SCH_Q4_1, 2, false)
RLXQ_GEMM256N_INST(q4_0, SCH_Q4_0, 2, false)
RLXQ_GEMM256N_INST(q8_0, SCH_Q8_0, 2, false)
RLXQ_GEMM256N_INST(mlx4, SCH_MLX4, 2, false)
RLXQ_GEMM256N_INST(mlx8, SCH_MLX8, 2, false)
RLXQ_GEMM256N_INST(q4_k, SCH_Q4_K, 2, false)
RLXQ_GEMM256N_INST(q6_k, SCH_Q6_K, 1, true)
RLXQ_GEMM256N_INST(q8_k, SCH_Q8_K, 2, false)
RLXQ_GEMM256N_INST(mxfp4, SCH_MXFP4, 2, false)
RLXQ_GEMM256N_INST(q5_k, SCH_Q5_K, 2, false)
RLXQ_GEMM256N_INST(q3_k, SCH_Q3_K, 1, false)
RLXQ_GEMM256N_INST(q2_k, SCH_Q2_K, 2, false)
// (Q4_1 and Q8_K: the all-real-tiles variant for bf16 activations keeps one
// register stage; with two it spilled)
RLXQ_GEMM256XN_INST(q4_1, SCH_Q4_1, 1, , false)
RLXQ_GEMM256XS_INST(q4_1, SCH_Q4_1, 2, p2, false)
RLXQ_GEMM256X_INST(q4_0, SCH_Q4_0, 2, p2, false)
RLXQ_GEMM256X_INST(q8_0, SCH_Q8_0, 1, , false)
RLXQ_GEMM256X_INST(q4_k, SCH_Q4_K, 2, p2, false)
RLXQ_GEMM256X_INST(q6_k, SCH_Q6_K, 1, l, true)
RLXQ_GEMM256X_INST(q5_k, SCH_Q5_K, 1, , false)
RLXQ_GEMM256X_INST(q3_k, SCH_Q3_K, 1, , false)
RLXQ_GEMM256X_INST(q2_k, SCH_Q2_K, 2, p2, false)
RLXQ_GEMM256XN_INST(q8_k, SCH_Q8_K, 1, , false)
RLXQ_GEMM256XS_INST(q8_k, SCH_Q8_K, 2, p2, false)
RLXQ_GEMM256X_INST(mlx4, SCH_MLX4, 1, , false)
RLXQ_GEMM256X_INST(mlx8, SCH_MLX8, 2, p2, false)
