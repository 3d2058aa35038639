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

namespace rlxq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int GBK = 64;        // K per step
constexpr int GLD = GBK + 8;   // LDS row stride (bf16 elements)


// Raw bytes of one 32-weight block, loaded ahead of their conversion so the
// global loads of a K step can be in flight while the previous step computes.
// All-zero raw bytes convert to zero weights (d = 0, or scale = bias = 0).
template <int SCH> struct RawBlk;
template <> struct RawBlk<SCH_Q4_1> { uint32_t h; uint4 q; };
template <> struct RawBlk<SCH_Q4_0> { uint32_t w[5]; uint32_t off; };
template <> struct RawBlk<SCH_Q8_0> { uint32_t w[9]; uint32_t off; };
template <> struct RawBlk<SCH_MLX4> { uint4 q; float s, b; };
template <> struct RawBlk<SCH_MLX8> { uint4 q0, q1; float s, b; };

// Loads block `kb` of weight row `row` (a valid row); `ok` = false zeroes it
// with selects, so the caller's loop body stays free of branches.
template <int SCH>
RLXQ_DEV void load_blk(const rlxq_gemm_args& a, int64_t row, int64_t kb, bool ok, RawBlk<SCH>& r) {
  const uint8_t* rp = a.w + row * a.rb;
  if constexpr (SCH == SCH_Q4_1) {
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

// Converts a raw block into 16 dwords of bf16 pairs in natural element order:
// f32 d*q + m (the CPU decoder's arithmetic), rounded to bf16 (nearest even).
template <int SCH>
RLXQ_DEV void conv_blk(const RawBlk<SCH>& r, uint32_t* out) {
  float v[32];
  if constexpr (SCH == SCH_Q4_1 || SCH == SCH_Q4_0) {
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
#pragma unroll
  for (int i = 0; i < 16; i++) out[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
}

// Dequantize one 32-weight block of row `row` (K-block `kb`) into 16 dwords of
// bf16 pairs in natural element order.  `ok` = false yields zeros.
template <int SCH>
RLXQ_DEV void dequant_block_bf16(const rlxq_gemm_args& a, int64_t row, int64_t kb, bool ok, uint32_t* out) {
  RawBlk<SCH> r;
  load_blk<SCH>(a, row, kb, ok, r);
  conv_blk<SCH>(r, out);
}

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
template <int SCH, int WGM, int WGN, int PF>
RLXQ_DEV void gemm256_body(const rlxq_gemm_args& a) {
  constexpr int BM = 256, BN = 256;
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AP = 2048 / NT;   // 16-byte activation chunks per thread per step
  constexpr int BPT = 512 / NT;   // weight blocks per thread per step
  static_assert(AP % 2 == 0 && BPT >= 1, "threads");
  extern __shared__ uint16_t smem[];
  uint16_t* As = smem;                // [2][BM][GLD]
  uint16_t* Bs = smem + 2 * BM * GLD;  // [2][BN][GLD]

  int tm, tn;
  if (!tile_of(blockIdx.x, a.tiles_m, a.tiles_n, 4, tm, tn)) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv % WGM, wn = wv / WGM;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int KT = (int)(a.K / GBK);
  const uint16_t* xg = reinterpret_cast<const uint16_t*>(a.x);

  // activation tile: 256 rows x 128 B = 2048 chunks of 16 B
  int64_t arow[AP];
  bool aok[AP];
#pragma unroll
  for (int i = 0; i < AP; i++) {
    const int c = tid + NT * i, r = c >> 3;
    aok[i] = m0 + r < a.M;
    arow[i] = (aok[i] ? m0 + r : a.M - 1) * a.K + (c & 7) * 8;
  }
  // weight tile: 256 rows x 2 blocks; thread -> row n0 + (tid & 255), blocks
  // (tid >> 8) + q * (NT / 256)
  const int brl = tid & 255;
  const bool bok = n0 + brl < a.N;
  const int64_t brow = bok ? n0 + brl : a.N - 1;

  // Global loads run PF steps ahead of the MFMAs (PF register stages); the
  // LDS stores and conversions of the next step sit between the MFMA groups
  // of the current one.
  struct Stage {
    uint4 a[AP];
    RawBlk<SCH> b[BPT];
  };
  auto gload = [&](int kt, Stage& P) {
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const uint4 v = *reinterpret_cast<const uint4*>(xg + arow[i] + (int64_t)kt * GBK);
      P.a[i] = aok[i] ? v : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int q = 0; q < BPT; q++) load_blk<SCH>(a, brow, 2 * (int64_t)kt + (tid >> 8) + q, bok, P.b[q]);
  };
  auto store_a = [&](const Stage& P, int buf, int half) {
#pragma unroll
    for (int i = half * AP / 2; i < (half + 1) * AP / 2; i++) {
      const int c = tid + NT * i;
      *reinterpret_cast<uint4*>(As + (buf * BM + (c >> 3)) * GLD + (c & 7) * 8) = P.a[i];
    }
  };
  auto store_b = [&](const Stage& P, int buf, int q) {
    uint32_t o[16];
    conv_blk<SCH>(P.b[q], o);
    uint16_t* dst = Bs + (buf * BN + brl) * GLD + ((tid >> 8) + q) * 32;
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

  auto compute_ks = [&](int cur, int ks) {
    const uint16_t* Ab = As + (cur * BM + wm * WM) * GLD;
    const uint16_t* Bb = Bs + (cur * BN + wn * WN) * GLD;
    bf16x8_t af[TM], bfr[TN];
    const int kof = ks * 16 + 8 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; i++) af[i] = *reinterpret_cast<const bf16x8_t*>(Ab + (i * 32 + (lane & 31)) * GLD + kof);
#pragma unroll
    for (int j = 0; j < TN; j++) bfr[j] = *reinterpret_cast<const bf16x8_t*>(Bb + (j * 32 + (lane & 31)) * GLD + kof);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
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
      step(kt & 1, P);
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

  // epilogue: C[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), reg 4*(i/8) + i%4
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int64_t n = n0 + wn * WN + j * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int64_t m = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
        if (m < a.M && n < a.N) {
          const float v = acc[i][j][r];
          if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = (uint16_t)f32_to_bf16_bits(v);
          else reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = v;
        }
      }
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

#define RLXQ_GEMM256_INST(SNAME, SCH)                                                        \
  extern "C" __global__ __launch_bounds__(256, 1) void rlxq_gemm_##SNAME##_t256(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 2, 1>(a);                                                           \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(512, 1) void rlxq_gemm_##SNAME##_t256w8(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 4, 1>(a);                                                           \
  }                                                                                                \
  extern "C" __global__ __launch_bounds__(512, 1) void rlxq_gemm_##SNAME##_t256w8p2(rlxq_gemm_args a) { \
    rlxq::gemm256_body<SCH, 2, 4, 2>(a);                                                           \
  }
RLXQ_GEMM256_INST(q4_1, SCH_Q4_1)
RLXQ_GEMM256_INST(q4_0, SCH_Q4_0)
RLXQ_GEMM256_INST(q8_0, SCH_Q8_0)
RLXQ_GEMM256_INST(mlx4, SCH_MLX4)
RLXQ_GEMM256_INST(mlx8, SCH_MLX8)
