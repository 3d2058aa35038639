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

#if RLXQ_PART_IS(0)
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
#endif

namespace rlxq {

constexpr int MOE_TILE_MAX = 256;  // most weight rows per workgroup tile
constexpr int MOE_RING = 4;        // weight units in flight per lane

// Weight row of local tile row lr of tile tn, and whether it exists.  Plain:
// tile_rows consecutive rows.  SwiGLU: tile_rows/2 gate rows and the
// matching up rows N/2 further on.
template <bool SWIGLU>
RLXQ_DEV int64_t tile_row(const rlxq_moe_gemv_args& a, int tn, int lr, bool& ok) {
  if constexpr (SWIGLU) {
    const int H = a.tile_rows / 2;
    const int64_t half = a.N / 2, c = (int64_t)tn * H + (lr % H);
    ok = c < half;
    return lr < H ? c : half + c;
  } else {
    const int64_t n = (int64_t)tn * a.tile_rows + lr;
    ok = n < a.N;
    return n;
  }
}

// One tile of expert e's weight rows against the entries perm[beg .. end)
// (perm in global or LDS memory).  The activations of MT entries at a time
// are staged in LDS as records once; the waves then walk the tile's rows,
// RP rows per pass with L lanes per row, every lane decoding units li,
// li + L, ... of its row.  The (pass, unit) steps are flattened and the
// weight units run MOE_RING steps ahead of the arithmetic in a register ring.
template <int SCH, bool XBF16, int L, int MT, bool SWIGLU>
RLXQ_DEV void moe_tile(const rlxq_moe_gemv_args& a, int e, const int32_t* perm, int beg, int end, int tn) {
  constexpr bool BIT8 = Unit<SCH>::BIT8;
  constexpr int NPL = XBF16 ? 1 : 2;
  constexpr int RS = Rec<NPL>::STRIDE;
  constexpr int BLOCKS = Unit<SCH>::BLOCKS;
  constexpr int DW = Unit<SCH>::DW;
  constexpr int BYTES = Unit<SCH>::BYTES;
  constexpr int RP = 64 / L;
  const int NPASS = a.tile_rows / 4 / RP;  // row passes per wave
  constexpr int D = MOE_RING;
  constexpr bool SLAB = slab_scales<SCH>(), SBIAS = slab_bias<SCH>();
  constexpr bool HAS_MIN = (SCH == SCH_Q4_1 || SCH == SCH_Q4_K || SCH == SCH_Q5_K || SBIAS);
  constexpr bool HALF2 = SCH == SCH_Q2_K || SCH == SCH_Q3_K;   // two scales (and mins) per block
  extern __shared__ uint32_t lds[];
  __shared__ float res[SWIGLU ? MT * MOE_TILE_MAX : 1];

  const int K = a.K;
  const int bpr = K >> 5;
  const int U = bpr / BLOCKS;
  const int nchunk = (U + L - 1) / L;
  const int S = NPASS * nchunk;   // steps per c0 chunk
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane / L, li = lane % L;
  const uint8_t* wbase = a.bank + (int64_t)e * a.N * a.rb;
  const int gpr = SLAB ? K / a.group : 0;
  const UnpackK kc = unpack_consts();

  auto step_row = [&](int s, int& lr, int& j) {
    const int p = s / nchunk;
    j = s - p * nchunk;
    lr = (p * 4 + wv) * RP + g;
  };
  auto load_step = [&](int s, uint32_t* dw) {
    int lr, j;
    step_row(s, lr, j);
    bool rok;
    const int64_t n = tile_row<SWIGLU>(a, tn, lr, rok);
    const int u = li + L * j;
    load_unit_at<SCH>(dw, wbase + (rok ? n : 0) * a.rb, u < U ? u : U - 1);
  };

  for (int c0 = beg; c0 < end; c0 += MT) {
    uint32_t ring[D][DW];
#pragma unroll
    for (int d = 0; d < D - 1; d++)
      if (d < S) load_step(d, ring[d]);
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
    float acc[MT];
    for (int s0 = 0; s0 < S; s0 += D) {
#pragma unroll
      for (int d = 0; d < D; d++) {
        const int s = s0 + d;
        if (s + D - 1 < S) load_step(s + D - 1, ring[(d + D - 1) % D]);
        if (s < S) {
          int lr, j;
          step_row(s, lr, j);
          bool rok;
          const int64_t n = tile_row<SWIGLU>(a, tn, lr, rok);
          const int64_t nn = rok ? n : 0;
          const int u = li + L * j;
          const bool uok = u < U;
          const int uc = uok ? u : U - 1;
          if (j == 0) {
#pragma unroll
            for (int m = 0; m < MT; m++) acc[m] = 0.f;
          }
#pragma unroll
          for (int bl = 0; bl < BLOCKS; bl++) {
            float dd, mn, d2 = 0.f, m2 = 0.f;
            if constexpr (SLAB) {
              const int64_t gi = ((int64_t)e * a.N + nn) * gpr + ((uc * BLOCKS + bl) * 32) / a.group;
              dd = scale_decode<SCH>(load_scale_raw<SCH>(a.scales, gi, a.sb_bf16), a.sb_bf16);
              mn = SBIAS ? load_sb(a.biases, gi, a.sb_bf16 != 0) : 0.f;
            } else if constexpr (HALF2) {
              block_scales_half<SCH>(ring[d], dd, d2, mn, m2);
            } else {
              block_scales<SCH>(ring[d], bl, dd, mn, uc);
            }
            if (!(rok && uok)) {
              dd = 0.f;
              mn = 0.f;
              d2 = 0.f;
              m2 = 0.f;
            }
            uint32_t pw[16];
            block_pairs<SCH>(ring[d], bl, pw, kc);
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
              if constexpr (SCH == SCH_Q6_K) {   // per-half scales: dd, mn = d * scale of each half
                acc[m] += q6k_block_dot<NPL>(pw, xrec, dd, mn);
                continue;
              }
              if constexpr (HALF2) {
                acc[m] += khalf_block_dot<SCH, NPL>(pw, xrec, dd, d2, mn, m2);
                continue;
              }
              const float cc = block_dot<SCH, NPL>(pw, xrec);
              const float scl = __uint_as_float(xrec[NPL * 16 + 2]);
              acc[m] = fmaf(BIT8 ? dd * scl : dd, cc, acc[m]);
              if constexpr (HAS_MIN) acc[m] = fmaf(mn, __uint_as_float(xrec[NPL * 16 + 1]), acc[m]);
            }
          }
          if (j == nchunk - 1) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
              const float v = lane_group_sum<L>(acc[m]);
              if constexpr (SWIGLU) {
                if (li == 0) res[m * MOE_TILE_MAX + lr] = v;
              } else if (li == 0 && rok && c0 + m < end) {
                const int64_t off = (int64_t)perm[c0 + m] * a.y_ld + n;
                if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[off] = (uint16_t)f32_to_bf16_bits(v);
                else reinterpret_cast<float*>(a.y)[off] = v;
              }
            }
          }
        }
      }
    }
    if constexpr (SWIGLU) {
      // out = silu(g) * u = g / (1 + exp(-g)) * u, the GroupedSwiglu rule
      const int H = a.tile_rows / 2;
      __syncthreads();
      for (int t = threadIdx.x; t < MT * H; t += blockDim.x) {
        const int m = t / H, c = t % H;
        const int64_t col = (int64_t)tn * H + c;
        if (c0 + m < end && col < a.N / 2) {
          const float gv = res[m * MOE_TILE_MAX + c], uv = res[m * MOE_TILE_MAX + H + c];
          const float o = gv / (1.f + expf(-gv)) * uv;
          const int64_t off = (int64_t)perm[c0 + m] * a.y_ld + col;
          if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[off] = (uint16_t)f32_to_bf16_bits(o);
          else reinterpret_cast<float*>(a.y)[off] = o;
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Register-activation tile (4-bit codes, bf16 activations).  Lane li of an
// L-lane group owns units li + L c (c < NU) of every row of the expert, so it
// needs only the activations of those units: it loads the bf16 values of the
// MT entries being served straight from global memory and builds their
// pairs (in the code-extraction order) and block sums in registers.  There
// is no LDS stage and no barrier.  The nw waves given to an expert take its
// output columns (a row, or a gate/up row pair for SwiGLU) in a stride of
// RP * nw, with D column steps of weight loads in flight.
// ---------------------------------------------------------------------------
template <int SCH, int L, int NU, int MT, int D, bool SWIGLU>
RLXQ_DEV void moe_xr_wave(const rlxq_moe_gemv_args& a, int e, const int32_t* perm, int beg, int end, int wq,
                          int nw, int64_t cb = 0, int64_t ce = -1, float* vout = nullptr) {
  constexpr int BLOCKS = Unit<SCH>::BLOCKS;
  constexpr int DW = Unit<SCH>::DW;
  constexpr int BYTES = Unit<SCH>::BYTES;
  constexpr int RP = 64 / L;
  constexpr int R2 = SWIGLU ? 2 : 1;
  constexpr bool MLX = SCH == SCH_MLX4;
  constexpr bool MX = SCH == SCH_MXFP4;
  constexpr bool HAS_MIN = (SCH == SCH_Q4_1 || SCH == SCH_Q4_K || MLX);
  static_assert(!Unit<SCH>::BIT8, "register activations serve 4-bit codes");

  const int K = a.K;
  const int U = (K >> 5) / BLOCKS;
  const int lane = threadIdx.x & 63, g = lane / L, li = lane % L;
  const int64_t width = SWIGLU ? a.N / 2 : a.N;
  // output columns [cb, ce) (default: all); vout != NULL: the single entry's
  // values go to vout[col - cb] instead of y
  if (ce < 0) ce = width;
  const uint8_t* wbase = a.bank + (int64_t)e * a.N * a.rb;
  const int gpr = (MLX || MX) ? K / a.group : 0;
  const int64_t cstride = (int64_t)nw * RP;

  int uc[NU];
  bool uok[NU];
#pragma unroll
  for (int c = 0; c < NU; c++) {
    const int u = li + L * c;
    uok[c] = u < U;
    uc[c] = uok[c] ? u : U - 1;
  }

  struct Buf {
    uint32_t dw[R2][NU][DW];
    SbRaw sm[R2][NU], bm[R2][NU];
  };
  // rows of output column col: col (and width + col, the up row, for SwiGLU)
  auto load = [&](int64_t col, Buf& bf) {
    const int64_t cc = col < ce ? col : cb;
#pragma unroll
    for (int r = 0; r < R2; r++) {
      const int64_t n = r == 0 ? cc : width + cc;
      const uint8_t* rp = wbase + n * a.rb;
#pragma unroll
      for (int c = 0; c < NU; c++) {
        load_unit_at<SCH>(bf.dw[r][c], rp, uc[c]);
        if constexpr (MLX || MX) {
          const int64_t gi = ((int64_t)e * a.N + n) * gpr + (uc[c] * 32) / a.group;
          bf.sm[r][c] = load_scale_raw<SCH>(a.scales, gi, a.sb_bf16);
          if constexpr (MLX) bf.bm[r][c] = load_sb_raw(a.biases, gi, a.sb_bf16 != 0);
        }
      }
    }
  };

  const UnpackK kc = unpack_consts();
  const int64_t base = cb + (int64_t)wq * RP;  // the wave's first column (wave-uniform)
  // column steps of this wave: base + s * cstride, s < cnt
  const int64_t cnt = base < ce ? (ce - base + cstride - 1) / cstride : 0;
  auto step_col = [&](int64_t st) { return base + (st < cnt ? st : (cnt > 0 ? cnt - 1 : 0)) * cstride + g; };
  for (int c0 = beg; c0 < end; c0 += MT) {
    // activations of the MT entries (raw bf16), requested before the ring so
    // that waiting for them does not wait for the weights
    int ent[MT];
    uint32_t X[MT][NU][BLOCKS][16];
    float S[MT][NU][BLOCKS];
#pragma unroll
    for (int m = 0; m < MT; m++) {
      ent[m] = c0 + m < end ? perm[c0 + m] : -1;
      const int64_t xrow = ent[m] >= 0 ? ent[m] / a.x_div : 0;
      const uint16_t* xb = reinterpret_cast<const uint16_t*>(a.x) + xrow * a.x_ld;
#pragma unroll
      for (int c = 0; c < NU; c++)
#pragma unroll
        for (int bl = 0; bl < BLOCKS; bl++) {
          const uint4* p = reinterpret_cast<const uint4*>(xb + (int64_t)(uc[c] * BLOCKS + bl) * 32);
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const uint4 v = p[q];
            X[m][c][bl][4 * q] = v.x;
            X[m][c][bl][4 * q + 1] = v.y;
            X[m][c][bl][4 * q + 2] = v.z;
            X[m][c][bl][4 * q + 3] = v.w;
          }
        }
    }
    // keep the activation loads ahead of the weight loads in the issue order
    __builtin_amdgcn_sched_barrier(0);
    Buf ring[D];
#pragma unroll
    for (int i = 0; i < D; i++) load(step_col(i), ring[i]);
    // pairs and block sums of my units (zero for absent entries)
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int c = 0; c < NU; c++)
#pragma unroll
        for (int bl = 0; bl < BLOCKS; bl++) {
          uint32_t R[16];
#pragma unroll
          for (int t = 0; t < 16; t++) R[t] = ent[m] >= 0 ? X[m][c][bl][t] : 0u;
          float sum = 0.f;
#pragma unroll
          for (int t = 0; t < 16; t++) sum = dot2_bf16(R[t], 0x3F803F80u, sum);
          S[m][c][bl] = sum;
          pairs_from_raw<SCH>(R, X[m][c][bl]);
        }

    // Column step s uses ring slot s % D.  While D more steps follow a full
    // group, each slot is refilled right after use with the step D later (no
    // condition on the refill, so the wait counts keep the other slots'
    // loads in flight); the last steps, already in the ring, follow.
    auto step = [&](int64_t st, const Buf& rb) {
      const int64_t col = base + st * cstride;
      float acc[R2][MT];
#pragma unroll
      for (int r = 0; r < R2; r++)
#pragma unroll
        for (int m = 0; m < MT; m++) acc[r][m] = 0.f;
#pragma unroll
      for (int r = 0; r < R2; r++)
#pragma unroll
        for (int c = 0; c < NU; c++)
#pragma unroll
          for (int bl = 0; bl < BLOCKS; bl++) {
            float d, mn;
            if constexpr (MLX) {
              d = sb_decode(rb.sm[r][c], a.sb_bf16 != 0);
              mn = sb_decode(rb.bm[r][c], a.sb_bf16 != 0);
            } else if constexpr (MX) {
              d = scale_decode<SCH>(rb.sm[r][c], a.sb_bf16);
              mn = 0.f;
            } else {
              block_scales<SCH>(rb.dw[r][c], bl, d, mn, uc[c]);
            }
            if (!uok[c]) {
              d = 0.f;
              mn = 0.f;
            }
            uint32_t pw[16];
            block_pairs<SCH>(rb.dw[r][c], bl, pw, kc);
#pragma unroll
            for (int m = 0; m < MT; m++) {
              float ch = chain_start<SCH>(S[m][c][bl]);
#pragma unroll
              for (int t = 0; t < 16; t++) ch = dot2_bf16(pw[t], X[m][c][bl][t], ch);
              acc[r][m] = fmaf(d, ch, acc[r][m]);
              if constexpr (HAS_MIN) acc[r][m] = fmaf(mn, S[m][c][bl], acc[r][m]);
            }
          }
      float v[R2][MT];
#pragma unroll
      for (int r = 0; r < R2; r++)
#pragma unroll
        for (int m = 0; m < MT; m++) v[r][m] = lane_group_sum<L>(acc[r][m]);
      const int64_t mycol = col + g;
      if (vout) {
        if (li == 0 && mycol < ce) vout[mycol - cb] = v[0][0];
      } else if (li == 0 && mycol < ce) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (ent[m] >= 0) {
            float o = v[0][m];
            if constexpr (SWIGLU) o = o / (1.f + expf(-o)) * v[1][m];  // silu(g) * u
            const int64_t off = (int64_t)ent[m] * a.y_ld + mycol;
            if (a.counters)   // (combine in this launch: written through to the device-coherent level)
              __hip_atomic_store(reinterpret_cast<float*>(a.y) + off, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[off] = (uint16_t)f32_to_bf16_bits(o);
            else reinterpret_cast<float*>(a.y)[off] = o;
          }
        }
      }
    };
    int64_t s0 = 0;
    for (; s0 + 2 * D <= cnt; s0 += D) {
#pragma unroll
      for (int i = 0; i < D; i++) {
        step(s0 + i, ring[i]);
        load(step_col(s0 + i + D), ring[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < D; i++) {
      if (s0 + i < cnt) {
        step(s0 + i, ring[i]);
        if (s0 + i + D < cnt) load(step_col(s0 + i + D), ring[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < D; i++)
      if (s0 + D + i < cnt) step(s0 + D + i, ring[i]);
  }
}

// Table-driven: workgroup = (fired expert slot, tile); work(e, perm, beg,
// end, tn) serves entries perm[beg .. end) of expert e.
template <class Work>
RLXQ_DEV void table_dispatch(const rlxq_moe_gemv_args& a, Work work) {
  const int slot = blockIdx.x / a.tiles_n, tn = blockIdx.x % a.tiles_n;
  const int nf = a.table[0];
  if (slot >= nf) return;
  const int e = a.table[1 + slot];
  const int beg = a.table[1 + a.E + slot], end = a.table[1 + a.E + slot + 1];
  work(e, a.table + 2 + 2 * a.E, beg, end, tn);
}

// Expert of entry i of the id list (int32 ids or f32 indices), -1 if invalid.
RLXQ_DEV int entry_expert(const rlxq_moe_gemv_args& a, int i) {
  if (a.ids) {
    const int32_t v = a.ids[i];
    return (v >= 0 && v < a.E) ? v : -1;
  }
  const float f = a.idx_f32[i];
  return (!(f >= 0.f) || f >= (float)a.E || (float)(int)f != f) ? -1 : (int)f;
}

// Exclusive sum over the 256 threads of v (every thread gets its prefix and
// the total).  ws: 4 ints of LDS not in use by other threads.
RLXQ_DEV int block_exclusive_sum(int v, int32_t* ws, int& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(inc, off, 64);
    if (lane >= off) inc += o;
  }
  if (lane == 63) ws[wv] = inc;
  __syncthreads();
  int base = 0;
#pragma unroll
  for (int w = 0; w < 4; w++) base += w < wv ? ws[w] : 0;
  total = ws[0] + ws[1] + ws[2] + ws[3];
  return base + inc - v;
}

// Routing in the workgroup, balanced over experts: the entries of each expert
// (in increasing order) are cut into chunks of MT, and workgroup = (chunk,
// tile) over the chunks of all experts in expert order, so that every
// workgroup serves at most MT entries of one expert whatever the skew.
// Chunk number C (the count of chunks; the grid always holds it) zeroes the
// output rows of invalid entries, its tiles splitting the rows.  Chunks past
// C exit.  E <= 1024, n_entries <= 1024, 256 threads.
template <int MT, class Work, class After>
RLXQ_DEV void balanced_dispatch(const rlxq_moe_gemv_args& a, Work work, After after) {
  __shared__ int32_t cnt[1024];
  __shared__ int32_t ent[1024];
  __shared__ int32_t ws0[4], ws1[4], pick[2];
  const int chunk = blockIdx.x / a.tiles_n, tn = blockIdx.x % a.tiles_n;
  const int t = threadIdx.x;
  const int E = a.E;
#pragma unroll
  for (int q = 0; q < 4; q++)
    if (4 * t + q < E) cnt[4 * t + q] = 0;
  if (t == 0) {
    pick[0] = -1;
    pick[1] = 0;
  }
  __syncthreads();
  int ex[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int i = 4 * t + q;
    ex[q] = i < a.n_entries ? entry_expert(a, i) : -2;
    if (ex[q] >= 0) atomicAdd(&cnt[ex[q]], 1);
  }
  __syncthreads();
  // chunk offsets: exclusive sum of ceil(count / MT) over the experts
  int c4[4], s = 0;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int e = 4 * t + q;
    c4[q] = e < E ? (cnt[e] + MT - 1) / MT : 0;
    s += c4[q];
  }
  int nchunks;
  int off = block_exclusive_sum(s, ws0, nchunks);
#pragma unroll
  for (int q = 0; q < 4; q++) {
    if (chunk >= off && chunk < off + c4[q]) {
      pick[0] = 4 * t + q;
      pick[1] = chunk - off;
    }
    off += c4[q];
  }
  if (t == 0 && chunk == nchunks) pick[0] = E;
  __syncthreads();
  const int e = pick[0], j = pick[1];
  if (e < 0) return;
  // entries of e (e == E: the invalid ones) in increasing order
  int mine[4], c = 0;
#pragma unroll
  for (int q = 0; q < 4; q++)
    if (ex[q] == e || (e == E && ex[q] == -1)) mine[c++] = 4 * t + q;
  int total;
  const int first = block_exclusive_sum(c, ws1, total);
#pragma unroll
  for (int q = 0; q < 4; q++)
    if (q < c) ent[first + q] = mine[q];
  __syncthreads();
  if (e == E) {
    // (with the combine in this launch the rows of invalid entries are not
    // read: only their counts are needed)
    if (a.counters) {
      after(ent, 0, total, tn);
      return;
    }
    const int64_t width = a.swiglu ? a.N / 2 : a.N;
    for (int64_t idx = (int64_t)tn * blockDim.x + t; idx < (int64_t)total * width;
         idx += (int64_t)blockDim.x * a.tiles_n) {
      const int64_t o = (int64_t)ent[idx / width] * a.y_ld + idx % width;
      if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[o] = 0;
      else reinterpret_cast<float*>(a.y)[o] = 0.f;
    }
    return;
  }
  const int beg = j * MT;
  const int end = beg + MT < total ? beg + MT : total;
  work(e, ent, beg, end, tn);
  if (a.counters) after(ent, beg, end, tn);
}

// The combine step of a fused down launch (see rlxq_moe_gemv_args): this
// workgroup has written the rows of entries ent[beg .. end) for the columns
// of tile tn (waves 4 tn .. 4 tn + 3 of nw = 4 tiles_n, RP columns per wave
// step, steps nw * RP apart).  Each entry counts once for its (token row,
// tile); the workgroup that brings a count to top_k sums the row's entries
// over the tile's columns in slot order and resets the count.
// Ordering: every thread's entry-row stores complete before the barrier
// that precedes the counts, and the count is an agent-scope acquire-release
// read-modify-write, so the workgroup that completes a row has seen (through
// the release of each earlier count and the barriers) every other
// workgroup's stores of that row before its sum's agent-scope loads.
template <int RP>
RLXQ_DEV void combine_tail(const rlxq_moe_gemv_args& a, const int32_t* ent, int beg, int end, int tn) {
  __shared__ int32_t done[1024];
  __shared__ int32_t ndone;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    int nd = 0;
    for (int i = beg; i < end; i++) {
      const int r = ent[i] / a.top_k;
      int32_t* c = a.counters + (int64_t)r * a.tiles_n + tn;
      if (__hip_atomic_fetch_add(c, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == a.top_k - 1) {
        __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        done[nd++] = r;
      }
    }
    ndone = nd;
  }
  __syncthreads();
  const int nd = ndone;
  if (nd == 0) return;
  const int64_t width = a.N;
  const int64_t nw = 4 * (int64_t)a.tiles_n;
  float* tmp = reinterpret_cast<float*>(a.y);
  for (int d = 0; d < nd; d++) {
    const int64_t r = done[d];
    for (int64_t jj = threadIdx.x;; jj += blockDim.x) {
      const int64_t st = jj / (4 * RP), rem = jj % (4 * RP);
      if ((st * nw + 4 * tn) * RP >= width) break;
      const int64_t col = (st * nw + 4 * tn + rem / RP) * RP + rem % RP;
      if (col >= width) continue;
      float acc = 0.f;
      for (int q = 0; q < a.top_k; q++) {
        const int64_t en = r * a.top_k + q;
        if (entry_expert(a, (int)en) < 0) continue;
        acc = fmaf(a.probs[en], __hip_atomic_load(tmp + en * a.y_ld + col, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                   acc);
      }
      if (a.out_bf16) reinterpret_cast<uint16_t*>(a.out)[r * width + col] = (uint16_t)f32_to_bf16_bits(acc);
      else reinterpret_cast<float*>(a.out)[r * width + col] = acc;
    }
  }
}

template <int SCH, bool XBF16, int L, int MT, bool SWIGLU, bool FUSED>
RLXQ_DEV void moe_gemv_body(const rlxq_moe_gemv_args& a) {
  auto work = [&](int e, const int32_t* perm, int beg, int end, int tn) {
    moe_tile<SCH, XBF16, L, MT, SWIGLU>(a, e, perm, beg, end, tn);
  };
  if constexpr (FUSED) balanced_dispatch<MT>(a, work, [](const int32_t*, int, int, int) {});
  else table_dispatch(a, work);
}

template <int SCH, int L, int NU, int MT, int D, bool SWIGLU, bool FUSED>
RLXQ_DEV void moe_xr_body(const rlxq_moe_gemv_args& a) {
  auto work = [&](int e, const int32_t* perm, int beg, int end, int tn) {
    moe_xr_wave<SCH, L, NU, MT, D, SWIGLU>(a, e, perm, beg, end,
                                           tn * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), a.tiles_n * 4);
  };
  auto after = [&](const int32_t* perm, int beg, int end, int tn) {
    if constexpr (!SWIGLU) combine_tail<64 / L>(a, perm, beg, end, tn);
  };
  if constexpr (FUSED) balanced_dispatch<MT>(a, work, after);
  else table_dispatch(a, work);
}

// Down projection and combine of decode-sized MoE calls in one launch,
// token-major: workgroup = (token row r, tile of tile_rows output columns),
// wave j = top-k slot j (64 * top_k threads, top_k <= 8).  Wave j computes
// entry r * top_k + j's values for the tile's columns exactly as the
// expert-major register kernel computes them for one entry (the same
// moe_xr_wave, one entry per pass) into LDS, then the workgroup sums the
// slots in slot order, y[r, c] = fma(probs[r, j], v[j][c], ...) for j = 0,
// 1, ... as rlxq_moe_combine_k does, so the output matches the two-launch
// path bit for bit.  An invalid expert id contributes zero (as its zeroed
// row does there).  No per-entry rows in memory, no counters, no atomics.
template <int SCH, int L, int NU, int D>
RLXQ_DEV void moe_xc_body(const rlxq_moe_gemv_args& a) {
  extern __shared__ float vals[];   // [top_k][tile_rows]
  __shared__ int32_t ents[8];
  const int tk = a.top_k, TC = a.tile_rows;
  const int64_t r = blockIdx.x / a.tiles_n;
  const int tn = blockIdx.x % a.tiles_n;
  const int64_t cb = (int64_t)tn * TC, ce = cb + TC < a.N ? cb + TC : a.N;
  const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (threadIdx.x < tk) ents[threadIdx.x] = (int32_t)(r * tk + threadIdx.x);
  __syncthreads();
  float* vj = vals + j * TC;
  const int e = entry_expert(a, (int)(r * tk + j));
  if (e >= 0) {
    moe_xr_wave<SCH, L, NU, 1, D, false>(a, e, ents, j, j + 1, 0, 1, cb, ce, vj);
  } else {
    for (int64_t c = threadIdx.x & 63; c < ce - cb; c += 64) vj[c] = 0.f;
  }
  __syncthreads();
  for (int64_t c = threadIdx.x; c < ce - cb; c += blockDim.x) {
    float acc = 0.f;
    for (int q = 0; q < tk; q++) acc = fmaf(a.probs[r * tk + q], vals[q * TC + c], acc);
    if (a.out_bf16) reinterpret_cast<uint16_t*>(a.out)[r * a.N + cb + c] = (uint16_t)f32_to_bf16_bits(acc);
    else reinterpret_cast<float*>(a.out)[r * a.N + cb + c] = acc;
  }
}

}  // namespace rlxq

#define RLXQ_MOE_INST(NAME, SCH, XBF, L, MT, SW)                                        \
  extern "C" __global__ __launch_bounds__(256) void NAME(rlxq_moe_gemv_args a) {      \
    rlxq::moe_gemv_body<SCH, XBF, L, MT, SW, false>(a);                                 \
  }
#define RLXQ_MOEF_INST(NAME, SCH, XBF, L, MT, SW)                                       \
  extern "C" __global__ __launch_bounds__(256) void NAME(rlxq_moe_gemv_args a) {      \
    rlxq::moe_gemv_body<SCH, XBF, L, MT, SW, true>(a);                                  \
  }
#define RLXQ_MOE_X(SNAME, SCH, XN, XBF)                                                   \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L64_M1, SCH, XBF, 64, 1, false)           \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L64_M2, SCH, XBF, 64, 2, false)           \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L64_M4, SCH, XBF, 64, 4, false)           \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L8_M1, SCH, XBF, 8, 1, false)             \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L8_M2, SCH, XBF, 8, 2, false)             \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L8_M4, SCH, XBF, 8, 4, false)             \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L64_M2_sw, SCH, XBF, 64, 2, true)         \
  RLXQ_MOE_INST(rlxq_moe_gemv_##SNAME##_##XN##_L8_M2_sw, SCH, XBF, 8, 2, true)           \
  RLXQ_MOEF_INST(rlxq_moe_gemvf_##SNAME##_##XN##_L64_M2, SCH, XBF, 64, 2, false)         \
  RLXQ_MOEF_INST(rlxq_moe_gemvf_##SNAME##_##XN##_L8_M2, SCH, XBF, 8, 2, false)           \
  RLXQ_MOEF_INST(rlxq_moe_gemvf_##SNAME##_##XN##_L64_M2_sw, SCH, XBF, 64, 2, true)       \
  RLXQ_MOEF_INST(rlxq_moe_gemvf_##SNAME##_##XN##_L8_M2_sw, SCH, XBF, 8, 2, true)
#define RLXQ_MOE_SCHEME(SNAME, SCH) \
  RLXQ_MOE_X(SNAME, SCH, bf16, true) \
  RLXQ_MOE_X(SNAME, SCH, f32, false)

#if RLXQ_PART_IS(0)
RLXQ_MOE_SCHEME(q4_1, SCH_Q4_1)
RLXQ_MOE_SCHEME(q4_0, SCH_Q4_0)
RLXQ_MOE_SCHEME(q8_0, SCH_Q8_0)
RLXQ_MOE_SCHEME(mlx4, SCH_MLX4)
#endif
#if RLXQ_PART_IS(1)
RLXQ_MOE_SCHEME(mlx8, SCH_MLX8)
RLXQ_MOE_SCHEME(mxfp4, SCH_MXFP4)
RLXQ_MOE_SCHEME(q4_k, SCH_Q4_K)
RLXQ_MOE_SCHEME(q6_k, SCH_Q6_K)
#endif
#if RLXQ_PART_IS(4)
RLXQ_MOE_SCHEME(q5_k, SCH_Q5_K)
RLXQ_MOE_SCHEME(q8_k, SCH_Q8_K)
RLXQ_MOE_SCHEME(q3_k, SCH_Q3_K)
RLXQ_MOE_SCHEME(q2_k, SCH_Q2_K)
#endif

// Register-activation variants (4-bit codes, bf16 activations):
// rlxq_moexr[f]_<scheme>_L<L>_U<NU>_M<MT>[_sw]; f = routing in the workgroup.
// The ring depth D shrinks as the units per lane grow.
#define RLXQ_MOEXR_INST(NAME, SCH, L, NU, MT, D, SW, F)                                \
  extern "C" __global__ __launch_bounds__(256) void NAME(rlxq_moe_gemv_args a) {      \
    rlxq::moe_xr_body<SCH, L, NU, MT, D, SW, F>(a);                                     \
  }
#define RLXQ_MOEXR_LU(SNAME, SCH, L, NU, MT, D)                                                       \
  RLXQ_MOEXR_INST(rlxq_moexr_##SNAME##_L##L##_U##NU##_M##MT, SCH, L, NU, MT, D, false, false)        \
  RLXQ_MOEXR_INST(rlxq_moexr_##SNAME##_L##L##_U##NU##_M##MT##_sw, SCH, L, NU, MT, D, true, false)    \
  RLXQ_MOEXR_INST(rlxq_moexrf_##SNAME##_L##L##_U##NU##_M##MT, SCH, L, NU, MT, D, false, true)        \
  RLXQ_MOEXR_INST(rlxq_moexrf_##SNAME##_L##L##_U##NU##_M##MT##_sw, SCH, L, NU, MT, D, true, true)
// Token-major down + combine: rlxq_moexc_<scheme>_L<L>_U<NU> (the lane
// groups and ring depths of the one-entry register kernels)
#define RLXQ_MOEXC_INST(SNAME, SCH, L, NU, D)                                                  \
  extern "C" __global__ __launch_bounds__(512) void rlxq_moexc_##SNAME##_L##L##_U##NU(rlxq_moe_gemv_args a) { \
    rlxq::moe_xc_body<SCH, L, NU, D>(a);                                                         \
  }
#define RLXQ_MOEXC_SCHEME(SNAME, SCH)   \
  RLXQ_MOEXC_INST(SNAME, SCH, 64, 1, 4) \
  RLXQ_MOEXC_INST(SNAME, SCH, 64, 2, 2) \
  RLXQ_MOEXC_INST(SNAME, SCH, 64, 4, 1) \
  RLXQ_MOEXC_INST(SNAME, SCH, 8, 1, 4)  \
  RLXQ_MOEXC_INST(SNAME, SCH, 8, 2, 2)  \
  RLXQ_MOEXC_INST(SNAME, SCH, 8, 3, 2)  \
  RLXQ_MOEXC_INST(SNAME, SCH, 8, 4, 1)
#define RLXQ_MOEXR_SCHEME(SNAME, SCH)        \
  RLXQ_MOEXR_LU(SNAME, SCH, 64, 1, 1, 4)     \
  RLXQ_MOEXR_LU(SNAME, SCH, 64, 1, 2, 2)     \
  RLXQ_MOEXR_LU(SNAME, SCH, 64, 1, 4, 4)     \
  RLXQ_MOEXR_LU(SNAME, SCH, 64, 2, 1, 2)     \
  RLXQ_MOEXR_LU(SNAME, SCH, 64, 2, 2, 2)     \
  RLXQ_MOEXR_LU(SNAME, SCH, 64, 2, 4, 2)     \
  RLXQ_MOEXR_LU(SNAME, SCH, 64, 4, 1, 1)     \
  RLXQ_MOEXR_LU(SNAME, SCH, 64, 4, 2, 1)     \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 1, 1, 4)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 1, 2, 4)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 1, 4, 4)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 2, 1, 2)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 2, 2, 2)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 2, 4, 2)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 3, 1, 2)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 3, 2, 2)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 4, 1, 1)      \
  RLXQ_MOEXR_LU(SNAME, SCH, 8, 4, 2, 1)
#if RLXQ_PART_IS(2)
RLXQ_MOEXR_SCHEME(q4_1, SCH_Q4_1)
RLXQ_MOEXR_SCHEME(mlx4, SCH_MLX4)
#endif
#if RLXQ_PART_IS(3)
RLXQ_MOEXR_SCHEME(mxfp4, SCH_MXFP4)
#endif
#if RLXQ_PART_IS(4)
RLXQ_MOEXC_SCHEME(q4_1, SCH_Q4_1)
RLXQ_MOEXC_SCHEME(mlx4, SCH_MLX4)
RLXQ_MOEXC_SCHEME(mxfp4, SCH_MXFP4)
RLXQ_MOEXC_INST(q4_1, SCH_Q4_1, 32, 2, 2)
RLXQ_MOEXC_INST(mlx4, SCH_MLX4, 32, 2, 2)
RLXQ_MOEXC_INST(mxfp4, SCH_MXFP4, 32, 2, 2)
RLXQ_MOEXC_INST(q4_k, SCH_Q4_K, 32, 1, 4)
RLXQ_MOEXC_INST(q4_k, SCH_Q4_K, 64, 1, 4)
RLXQ_MOEXC_INST(q4_k, SCH_Q4_K, 64, 2, 2)
RLXQ_MOEXC_INST(q4_k, SCH_Q4_K, 8, 1, 4)
RLXQ_MOEXC_INST(q4_k, SCH_Q4_K, 8, 2, 2)
RLXQ_MOEXC_INST(q4_0, SCH_Q4_0, 64, 1, 4)
RLXQ_MOEXC_INST(q4_0, SCH_Q4_0, 64, 2, 2)
RLXQ_MOEXC_INST(q4_0, SCH_Q4_0, 8, 1, 4)
RLXQ_MOEXC_INST(q4_0, SCH_Q4_0, 8, 2, 2)
#endif
#if RLXQ_PART_IS(2)
// Q4_1 at 33..64 units (K = 2048): 32-lane groups of two units
RLXQ_MOEXR_LU(q4_1, SCH_Q4_1, 32, 2, 1, 2)
RLXQ_MOEXR_LU(q4_1, SCH_Q4_1, 32, 2, 2, 2)
RLXQ_MOEXR_LU(q4_1, SCH_Q4_1, 32, 2, 4, 2)
RLXQ_MOEXR_LU(mlx4, SCH_MLX4, 32, 2, 1, 2)
RLXQ_MOEXR_LU(mlx4, SCH_MLX4, 32, 2, 2, 2)
RLXQ_MOEXR_LU(mlx4, SCH_MLX4, 32, 2, 4, 2)
RLXQ_MOEXR_LU(mxfp4, SCH_MXFP4, 32, 2, 1, 2)
RLXQ_MOEXR_LU(mxfp4, SCH_MXFP4, 32, 2, 2, 2)
RLXQ_MOEXR_LU(mxfp4, SCH_MXFP4, 32, 2, 4, 2)
#endif
#if RLXQ_PART_IS(3)
// Q4_K: 64-weight units (two blocks, 12 dwords): at most two units per lane;
// 32-lane groups for the 32 units of K = 2048
RLXQ_MOEXR_LU(q4_k, SCH_Q4_K, 32, 1, 1, 4)
RLXQ_MOEXR_LU(q4_k, SCH_Q4_K, 32, 1, 2, 2)
RLXQ_MOEXR_LU(q4_k, SCH_Q4_K, 64, 1, 1, 4)
RLXQ_MOEXR_LU(q4_k, SCH_Q4_K, 64, 1, 2, 2)
RLXQ_MOEXR_LU(q4_k, SCH_Q4_K, 64, 2, 1, 2)
RLXQ_MOEXR_LU(q4_k, SCH_Q4_K, 8, 1, 1, 4)
RLXQ_MOEXR_LU(q4_k, SCH_Q4_K, 8, 1, 2, 4)
RLXQ_MOEXR_LU(q4_k, SCH_Q4_K, 8, 2, 1, 2)
// Q4_0 units hold two blocks: at most four blocks of activations per lane
// and entry (NU * MT <= 2).
RLXQ_MOEXR_LU(q4_0, SCH_Q4_0, 64, 1, 1, 4)
RLXQ_MOEXR_LU(q4_0, SCH_Q4_0, 64, 1, 2, 4)
RLXQ_MOEXR_LU(q4_0, SCH_Q4_0, 64, 2, 1, 2)
RLXQ_MOEXR_LU(q4_0, SCH_Q4_0, 8, 1, 1, 4)
RLXQ_MOEXR_LU(q4_0, SCH_Q4_0, 8, 1, 2, 4)
RLXQ_MOEXR_LU(q4_0, SCH_Q4_0, 8, 2, 1, 2)
#endif
