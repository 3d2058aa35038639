// Grouped-expert dequant-GEMV driven by a device routing table.
//
// Replaces the backend kernels of Op::DequantGroupedMatMul (one expert index
// per activation row, crates/rlx-qwen35/src/builder.rs:2955-2973) and of the
// top-k MoE FFN built from it (crates/rlx-unlimited-ocr/tests/quant_parity_backends.rs:338-373),
// where the reference issues one grouped op per top-k slot, each re-reading
// the expert rows of its tokens.  Here:
//   1. rlxq_moe_table_k (one workgroup) groups the (token, slot) entries by
//      expert: counts, prefix offsets, the list of fired experts and the
//      entries of each, plus zero output rows for invalid indices;
//   2. rlxq_moe_gemv_* workgroups each take (fired expert, tile of rows),
//      stage the activations of that expert's entries (MT at a time) in LDS
//      and stream the expert's weight rows once per MT entries;
//   3. for the probability-weighted combine, rlxq_moe_combine_k sums the
//      per-entry rows of each token in slot order (deterministic).
#include "gemv_core.hip.h"
#include "moe_args.h"

// One workgroup of 1024 threads.  E <= 1024.
extern "C" __global__ __launch_bounds__(1024) void rlxq_moe_table_k(rlxq_moe_table_args a) {
  __shared__ int32_t cnt[1024], cur[1024], scan[1024];
  const int t = threadIdx.x;
  const int E = a.E;
  cnt[t] = 0;
  __syncthreads();
  auto expert_of = [&](int64_t i) -> int {
    if (a.ids) {
      const int32_t e = a.ids[i];
      return (e >= 0 && e < E) ? e : -1;
    }
    const float f = a.idx_f32[i];
    if (!(f >= 0.f) || f >= (float)E || (float)(int)f != f) return -1;
    return (int)f;
  };
  for (int64_t i = t; i < a.n; i += blockDim.x) {
    const int e = expert_of(i);
    if (e >= 0) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // fired flags -> slot numbers (inclusive scan of flags over 1024 experts)
  const int fired = (t < E && cnt[t] > 0) ? 1 : 0;
  scan[t] = fired;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int v = t >= off ? scan[t - off] : 0;
    __syncthreads();
    scan[t] += v;
    __syncthreads();
  }
  const int slot = scan[t] - fired;  // exclusive
  const int nf = scan[1023];
  int32_t* fired_list = a.table + 1;
  int32_t* offs = a.table + 1 + E;
  int32_t* perm = a.table + 2 + 2 * E;
  // entry offsets per expert (exclusive scan of counts)
  __syncthreads();
  scan[t] = t < E ? cnt[t] : 0;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int v = t >= off ? scan[t - off] : 0;
    __syncthreads();
    scan[t] += v;
    __syncthreads();
  }
  const int base = scan[t] - (t < E ? cnt[t] : 0);
  if (fired) {
    fired_list[slot] = t;
    offs[slot] = base;
  }
  cur[t] = base;
  if (t == 0) {
    a.table[0] = nf;
    offs[nf] = scan[1023];
  }
  __syncthreads();
  for (int64_t i = t; i < a.n; i += blockDim.x) {
    const int e = expert_of(i);
    if (e >= 0) {
      perm[atomicAdd(&cur[e], 1)] = (int32_t)i;
    } else if (a.zero_rows) {
      for (int64_t c = 0; c < a.N; c++) {
        if (a.zero_bf16) reinterpret_cast<uint16_t*>(a.zero_rows)[i * a.zero_ld + c] = 0;
        else reinterpret_cast<float*>(a.zero_rows)[i * a.zero_ld + c] = 0.f;
      }
    }
  }
}

// y[r, :] = sum_j probs[r, j] * tmp[r * top_k + j, :], j in order.
extern "C" __global__ __launch_bounds__(256) void rlxq_moe_combine_k(const float* __restrict__ tmp,
                                                                      const float* __restrict__ probs, int64_t rows,
                                                                      int32_t top_k, int64_t N, void* __restrict__ y,
                                                                      int32_t y_bf16) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * N) return;
  const int64_t r = i / N, c = i - r * N;
  float s = 0.f;
  for (int j = 0; j < top_k; j++) s = fmaf(probs[r * top_k + j], tmp[(r * top_k + j) * N + c], s);
  if (y_bf16) reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)f32_to_bf16_bits(s);
  else reinterpret_cast<float*>(y)[i] = s;
}

namespace rlxq {

// Workgroup (4 waves) = (fired expert slot, tile of TILE weight rows).  The
// activations of the expert's entries are staged MT at a time; each wave
// walks RPW rows of the tile, L lanes per row, every lane decoding units
// li, li+L, ... of the row against the MT staged records.
template <int SCH, bool XBF16, int L, int MT>
RLXQ_DEV void moe_gemv_body(const rlxq_moe_gemv_args& a) {
  constexpr bool BIT8 = Unit<SCH>::BIT8;
  constexpr int NPL = XBF16 ? 1 : 2;
  constexpr int RS = Rec<NPL>::STRIDE;
  constexpr int BLOCKS = Unit<SCH>::BLOCKS;
  constexpr int DW = Unit<SCH>::DW;
  constexpr int BYTES = Unit<SCH>::BYTES;
  constexpr int RP = 64 / L;
  constexpr int TILE = 32;
  constexpr int RPW = TILE / 4 / RP;  // row passes per wave
  constexpr bool MLX = (SCH == SCH_MLX4 || SCH == SCH_MLX8);
  constexpr bool HAS_MIN = (SCH == SCH_Q4_1 || MLX);
  extern __shared__ uint32_t lds[];

  const int slot = blockIdx.x / a.tiles_n, tn = blockIdx.x % a.tiles_n;
  const int nf = a.table[0];
  if (slot >= nf) return;
  const int e = a.table[1 + slot];
  const int beg = a.table[1 + a.E + slot], end = a.table[1 + a.E + slot + 1];
  const int32_t* perm = a.table + 2 + 2 * a.E;

  const int K = a.K;
  const int bpr = K >> 5;
  const int U = bpr / BLOCKS;
  const int nchunk = (U + L - 1) / L;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane / L, li = lane % L;
  const uint8_t* wbase = a.bank + (int64_t)e * a.N * a.rb;
  const int gpr = MLX ? K / a.group : 0;
  const UnpackK kc = unpack_consts();

  for (int c0 = beg; c0 < end; c0 += MT) {
    // stage the activation rows of entries c0 .. c0+MT-1
    for (int m = 0; m < MT; m++) {
      const int ent = c0 + m < end ? perm[c0 + m] : -1;
      const int64_t xrow = ent >= 0 ? ent / a.x_div : 0;
      for (int base = 0; base < bpr * 8; base += blockDim.x * XRaw<XBF16>::XB) {
        XRaw<XBF16> raw;
        stage_fetch<XBF16>(raw, reinterpret_cast<const char*>(a.x) + xrow * a.x_ld * (XBF16 ? 2 : 4), 0,
                           ent >= 0 ? 1 : 0, K, base);
        stage_store<SCH, XBF16, NPL>(lds, raw, m, K, base);
      }
    }
    __syncthreads();
    for (int rp = 0; rp < RPW; rp++) {
      const int64_t n = (int64_t)tn * TILE + (wv * RPW + rp) * RP + g;
      const bool rok = n < a.N;
      const int64_t nn = rok ? n : 0;
      const uint8_t* rowp = wbase + nn * a.rb;
      float acc[MT];
#pragma unroll
      for (int m = 0; m < MT; m++) acc[m] = 0.f;
      for (int j = 0; j < nchunk; j++) {
        const int u = li + L * j;
        const bool uok = u < U;
        const int uc = uok ? u : U - 1;
        uint32_t dw[DW];
        load_unit<SCH>(dw, rowp + (int64_t)uc * BYTES);
#pragma unroll
        for (int bl = 0; bl < BLOCKS; bl++) {
          float d, mn;
          if constexpr (MLX) {
            const int64_t gi = ((int64_t)e * a.N + nn) * gpr + ((uc * BLOCKS + bl) * 32) / a.group;
            d = load_sb(a.scales, gi, a.sb_bf16 != 0);
            mn = load_sb(a.biases, gi, a.sb_bf16 != 0);
          } else {
            block_scales<SCH>(dw, bl, d, mn);
          }
          if (!(rok && uok)) {
            d = 0.f;
            mn = 0.f;
          }
          uint32_t pw[16];
          block_pairs<SCH>(dw, bl, pw, kc);
          const int b = uc * BLOCKS + bl;
#pragma unroll
          for (int m = 0; m < MT; m++) {
            const uint32_t* xr = lds + (size_t)(m * bpr + b) * RS;
            uint32_t xrec[RS];
#pragma unroll
            for (int q = 0; q < RS; q += 4) {
              const uint4 v = *reinterpret_cast<const uint4*>(xr + q);
              xrec[q] = v.x; xrec[q + 1] = v.y; xrec[q + 2] = v.z; xrec[q + 3] = v.w;
            }
            const float cc = block_dot<SCH, NPL>(pw, xrec);
            const float scl = __uint_as_float(xrec[NPL * 16 + 2]);
            acc[m] = fmaf(BIT8 ? d * scl : d, cc, acc[m]);
            if constexpr (HAS_MIN) acc[m] = fmaf(mn, __uint_as_float(xrec[NPL * 16 + 1]), acc[m]);
          }
        }
      }
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const float v = lane_group_sum<L>(acc[m]);
        if (li == 0 && rok && c0 + m < end) {
          const int64_t off = (int64_t)perm[c0 + m] * a.y_ld + n;
          if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[off] = (uint16_t)f32_to_bf16_bits(v);
          else reinterpret_cast<float*>(a.y)[off] = v;
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace rlxq

#define RLXQ_MOE_INST(NAME, SCH, XBF, L, MT)                                           \
  extern "C" __global__ __launch_bounds__(256) void NAME(rlxq_moe_gemv_args a) {      \
    rlxq::moe_gemv_body<SCH, XBF, L, MT>(a);                                            \
  }
#define RLXQ_MOE_X(SNAME, SCH, XN, XBF)                                          \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L64_M1, SCH, XBF, 64, 1)         \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L64_M2, SCH, XBF, 64, 2)         \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L64_M4, SCH, XBF, 64, 4)         \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L8_M1, SCH, XBF, 8, 1)           \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L8_M2, SCH, XBF, 8, 2)           \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L8_M4, SCH, XBF, 8, 4)
#define RLXQ_MOE_SCHEME(SNAME, SCH) \
  RLXQ_MOE_X(SNAME, SCH, bf16, true) \
  RLXQ_MOE_X(SNAME, SCH, f32, false)

RLXQ_MOE_SCHEME(q4_1, SCH_Q4_1)
RLXQ_MOE_SCHEME(q4_0, SCH_Q4_0)
RLXQ_MOE_SCHEME(q8_0, SCH_Q8_0)
RLXQ_MOE_SCHEME(mlx4, SCH_MLX4)
RLXQ_MOE_SCHEME(mlx8, SCH_MLX8)
