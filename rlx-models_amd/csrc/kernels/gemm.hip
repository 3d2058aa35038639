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

// Two f32 -> one dword of two bf16 (round to nearest even).
RLXQ_DEV uint32_t pack_bf16x2(float a, float b) { return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16); }

// Dequantize one 32-weight block of row `row` (K-block `kb`) into 16 dwords of
// bf16 pairs in natural element order.  `ok` = false yields zeros.
template <int SCH>
RLXQ_DEV void dequant_block_bf16(const rlxq_gemm_args& a, int64_t row, int64_t kb, bool ok, uint32_t* out) {
  if (!ok) {
#pragma unroll
    for (int i = 0; i < 16; i++) out[i] = 0u;
    return;
  }
  const uint8_t* rp = a.w + row * a.rb;
  float v[32];
  if constexpr (SCH == SCH_Q4_1 || SCH == SCH_Q4_0) {
    constexpr int BB = SCH == SCH_Q4_1 ? 20 : 18;
    const uint8_t* p = rp + kb * BB;
    uint32_t qs[4];
    float d, m;
    if constexpr (SCH == SCH_Q4_1) {
      const uint32_t h = ld_u32(p);
      const uint4 q = ld_u128(p + 4);
      qs[0] = q.x; qs[1] = q.y; qs[2] = q.z; qs[3] = q.w;
      d = f16_bits_to_f32(h & 0xffffu);
      m = f16_bits_to_f32(h >> 16);
    } else {
      // 18-byte blocks are 2-byte aligned: read the dwords covering the
      // block without touching a byte beyond it (the tail is a 16-bit load
      // when the block starts dword aligned).
      const uint32_t off = (uint32_t)(kb * BB) & 3u;
      const uint8_t* base = p - off;
      uint32_t w5[5];
#pragma unroll
      for (int i = 0; i < 4; i++) w5[i] = ld_u32(base + 4 * i);
      w5[4] = off ? ld_u32(base + 16) : (uint32_t)*reinterpret_cast<const uint16_t*>(base + 16);
      const uint32_t hd = off ? (w5[0] >> 16) : (w5[0] & 0xffffu);
#pragma unroll
      // qs starts 2 bytes after the block start: byte off + 2 of the span
      // (v_alignbyte takes shifts 0..3, so a 4-byte shift is the next dword)
      for (int i = 0; i < 4; i++) qs[i] = off ? w5[i + 1] : align_bytes(w5[i + 1], w5[i], 2);
      d = f16_bits_to_f32(hd);
      m = -8.f * d;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t lo = qs[i] & 0x0F0F0F0Fu, hi = (qs[i] >> 4) & 0x0F0F0F0Fu;
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
    // 34-byte blocks: as for Q4_0, no byte beyond the block is read.
    const uint32_t off = (uint32_t)(kb * 34) & 3u;
    const uint8_t* base = rp + kb * 34 - off;
    uint32_t w9[9];
#pragma unroll
    for (int i = 0; i < 8; i++) w9[i] = ld_u32(base + 4 * i);
    w9[8] = off ? ld_u32(base + 32) : (uint32_t)*reinterpret_cast<const uint16_t*>(base + 32);
    const float d = f16_bits_to_f32(off ? (w9[0] >> 16) : (w9[0] & 0xffffu));
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t q = off ? w9[i + 1] : align_bytes(w9[i + 1], w9[i], 2);
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * i + e] = d * (float)(int8_t)((q >> (8 * e)) & 0xffu);
    }
  } else {
    // MLX affine: codes LSB-first in u32 words, one scale/bias per group.
    constexpr int BITS = SCH == SCH_MLX4 ? 4 : 8;
    const uint32_t* wq = reinterpret_cast<const uint32_t*>(rp) + kb * BITS;
    const int64_t gi = row * (int64_t)(a.K / a.group) + (kb * 32) / a.group;
    float s, bi;
    if (a.sb_bf16) {
      s = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.scales)[gi]);
      bi = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.biases)[gi]);
    } else {
      s = reinterpret_cast<const float*>(a.scales)[gi];
      bi = reinterpret_cast<const float*>(a.biases)[gi];
    }
#pragma unroll
    for (int i = 0; i < BITS; i++) {
      const uint32_t w = wq[i];
      constexpr int PER = 32 / BITS;
#pragma unroll
      for (int e = 0; e < PER; e++) v[PER * i + e] = fmaf(s, (float)((w >> (BITS * e)) & ((1u << BITS) - 1u)), bi);
    }
  }
#pragma unroll
  for (int i = 0; i < 16; i++) out[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
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
