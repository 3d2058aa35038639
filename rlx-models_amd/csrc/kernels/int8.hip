// Int8 kernels on gfx950 MFMA.  Both read weights stored the reference's way,
// int8 [K, N] row-major with one f32 scale per column
// (crates/rlx-kimi-k3/src/common.rs:466-482):
//
//  * rlxq_w8a8_*: the W8A8 GEMM.  Activations are quantised per row to int8
//    (rlxq_quant_act_i8, crates/rlx-quant-calib/src/bitnet.rs:76-93); the
//    product runs on v_mfma_i32_32x32x32_i8 with int32 accumulation (exact),
//    and the epilogue is y = (float(acc) * sx[m]) * sw[n].
//  * rlxq_i8b_*: QuantScheme::Int8Block (crates/rlx-kimi-k3/examples/int8_kernel.rs:59-89),
//    y = x . ((Wq - zp) * s) with f32 or bf16 activations.  x is split into
//    two bf16 terms hi + lo (16 significant bits); int8 codes are exact in
//    bf16, so v_mfma_f32_16x16x32_bf16 forms the products to ~2^-17 relative
//    with fp32 accumulation.  Evaluated as s * (sum x*q - zp * sum x).
//
// The weight tile is copied into LDS unchanged ([k][n], N contiguous).  The
// MFMA B operand needs consecutive k in each lane; it is read with the LDS
// transpose read ds_read_b64_tr_b8: in each group of 16 lanes, lanes 2r and
// 2r+1 name the two 8-byte halves of a 16-byte row r, and lane i receives
// byte i of rows 0..7 (8 consecutive k of column i).
#include "common.hip.h"
#include "int8_args.h"

namespace rlxq {

typedef int32_t i32x2_t __attribute__((ext_vector_type(2)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef int32_t i32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef i32x2_t __attribute__((address_space(3))) lds_i32x2_t;

RLXQ_DEV i32x2_t lds_tr8(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t*)(p));
}

// ---------------------------------------------------------------- W8A8 GEMM

// y[m, n] = (float(acc) * sx[m]) * sw[n], two roundings in this order.  The
// output dtype and whether the workgroup's tile lies wholly inside M x N are
// decided once; a lane stores through one base pointer at wave-uniform
// offsets, so a whole tile needs no per-element bounds checks or 64-bit
// multiplies.
template <int TM, int TN>
RLXQ_DEV void w8a8_epilogue(const rlxq_w8a8_args& a, const i32x16_t (&acc)[TM][TN], int64_t mb, int64_t nb,
                            int lane, bool whole) {
#pragma clang fp contract(off)
  const int64_t m1 = mb + 4 * (lane >> 5), n1 = nb + (lane & 31);   // the lane's first row, column
  auto epi = [&](auto put, auto checked) {
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int64_t n = n1 + j * 32;
      if (checked.value && n >= a.N) continue;
      const float sw = a.sw[n];
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int dm = i * 32 + 8 * (r / 4) + (r % 4);
          if (!checked.value || m1 + dm < a.M) put(dm, j * 32, ((float)acc[i][j][r] * a.sx[m1 + dm]) * sw);
        }
    }
  };
  auto epi_any = [&](auto put) {
    if (whole) epi(put, std::false_type{});
    else epi(put, std::true_type{});
  };
  if (a.y_bf16) {
    uint16_t* p = reinterpret_cast<uint16_t*>(a.y) + m1 * a.y_ld + n1;
    epi_any([&](int dm, int dn, float v) { p[(int64_t)dm * a.y_ld + dn] = (uint16_t)f32_to_bf16_bits(v); });
  } else {
    float* p = reinterpret_cast<float*>(a.y) + m1 * a.y_ld + n1;
    epi_any([&](int dm, int dn, float v) { p[(int64_t)dm * a.y_ld + dn] = v; });
  }
}

// Workgroup of WGM x WGN waves owns a BM x BN output tile and walks K in steps
// of BK bytes; each wave computes a (BM/WGM) x (BN/WGN) sub-tile from 32x32
// MFMA tiles.  Global loads of step k+1 are in flight during the MFMAs of step
// k; LDS tiles are double-buffered with one barrier per step.
// KF: K is a whole number of BK steps, so every load is in range along K and
// none is zeroed; rows past M and columns past N read the clamped row or
// column and only feed outputs that are not stored.
template <int BM, int BN, int BK, int WGM, int WGN, int GM, int PF, bool KF = false>
RLXQ_DEV void w8a8_body(const rlxq_w8a8_args& a) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AST = BK + 16;  // A row stride (bytes): 16-byte reads of 8 rows hit distinct banks
  // B row stride: a transpose read covers 8 rows x 32 bytes per 32 lanes, so
  // the stride is an odd multiple of 32 bytes (8 banks per row, the 8 rows on
  // distinct banks); BN + 16 had each row's second 16 bytes on the next
  // row's banks
  constexpr int BST = BN + 32;
  constexpr int ACH = BK / 16, BCH = BN / 16;
  constexpr int AP = BM * ACH / NT, BP = BK * BCH / NT;
  static_assert((BM * ACH) % NT == 0 && (BK * BCH) % NT == 0, "tile / threads");
  static_assert(WM % 32 == 0 && WN % 32 == 0 && BK % 32 == 0, "tile shape");
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* As = smem;                 // [2][BM][AST]
  uint8_t* Bs = smem + 2 * BM * AST;  // [2][BK][BST]

  int tm, tn;
  if (!tile_of(blockIdx.x, a.tiles_m, a.tiles_n, GM, tm, tn)) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv % WGM, wn = wv / WGM;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int KT = (int)((a.K + BK - 1) / BK);

  // Loads are branch-free: out-of-range chunks read a clamped, valid address
  // and are replaced by zeros with selects (K and N are multiples of 16).
  struct Stage {
    uint4 a[AP], b[BP];
  };
  // loop-invariant parts of the chunk addresses: activation row (clamped),
  // K offset of the chunk within the step; weight column (clamped), K row
  // of the chunk within the step
  const int8_t* abase[AP];
  bool amok[AP];
  int akof[AP];
#pragma unroll
  for (int i = 0; i < AP; i++) {
    const int c = tid + NT * i, r = c / ACH, cc = c % ACH;
    amok[i] = m0 + r < a.M;
    abase[i] = a.qx + (amok[i] ? m0 + r : a.M - 1) * a.K;
    akof[i] = 16 * cc;
  }
  const int8_t* bbase[BP];
  bool bnok[BP];
  int bkr[BP];
#pragma unroll
  for (int i = 0; i < BP; i++) {
    const int c = tid + NT * i, r = c / BCH, cc = c % BCH;
    bnok[i] = n0 + 16 * cc < a.N;
    bbase[i] = a.wq + (bnok[i] ? n0 + 16 * cc : a.N - 16);
    bkr[i] = r;
  }
  auto load = [&](int kt, Stage& P) {
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int64_t k = k0 + akof[i];
      if constexpr (KF) {
        P.a[i] = *reinterpret_cast<const uint4*>(abase[i] + k);
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(abase[i] + (k < a.K ? k : a.K - 16));
        P.a[i] = (amok[i] && k < a.K) ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int i = 0; i < BP; i++) {
      const int64_t k = k0 + bkr[i];
      if constexpr (KF) {
        P.b[i] = *reinterpret_cast<const uint4*>(bbase[i] + k * a.N);
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(bbase[i] + (k < a.K ? k : a.K - 1) * a.N);
        P.b[i] = (bnok[i] && k < a.K) ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  auto store_a = [&](const Stage& P, int buf) {
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int c = tid + NT * i, r = c / ACH, cc = c % ACH;
      *reinterpret_cast<uint4*>(As + (buf * BM + r) * AST + 16 * cc) = P.a[i];
    }
  };
  auto store_b = [&](const Stage& P, int buf) {
#pragma unroll
    for (int i = 0; i < BP; i++) {
      const int c = tid + NT * i, r = c / BCH, cc = c % BCH;
      *reinterpret_cast<uint4*>(Bs + (buf * BK + r) * BST + 16 * cc) = P.b[i];
    }
  };
  auto store = [&](const Stage& P, int buf) {
    store_a(P, buf);
    store_b(P, buf);
  };

  i32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

  const int g = lane >> 4, s = lane & 15;
  auto compute_ks = [&](int cur, int ks) {
    const uint8_t* Ab = As + (cur * BM + wm * WM) * AST;
    const uint8_t* Bb = Bs + cur * BK * BST + wn * WN;
    {
      i32x4_t af[TM], bq[TN];
#pragma unroll
      for (int i = 0; i < TM; i++)
        af[i] = *reinterpret_cast<const i32x4_t*>(Ab + (i * 32 + (lane & 31)) * AST + ks * 32 + 16 * (lane >> 5));
#pragma unroll
      for (int j = 0; j < TN; j++) {
        // B[k][j] of the 32x32x32 tile sits in lane j + 32*(k/16), byte k%16:
        // group g covers columns 16*(g&1).., k = 16*(g>>1) + 0..7 and + 8..15.
        const uint8_t* p = Bb + (ks * 32 + 16 * (g >> 1) + (s >> 1)) * BST + j * 32 + 16 * (g & 1) + 8 * (s & 1);
        const i32x2_t lo = lds_tr8(p), hi = lds_tr8(p + 8 * BST);
        bq[j] = i32x4_t{lo.x, lo.y, hi.x, hi.y};
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bq[j], acc[i][j], 0, 0, 0);
    }
  };
  auto compute = [&](int cur) {
#pragma unroll
    for (int ks = 0; ks < BK / 32; ks++) compute_ks(cur, ks);
  };
  if constexpr (PF == 1) {
    // the next step's LDS stores sit between the MFMA groups of this one
    // (activation rows after the first, weight rows after the second), so
    // they overlap the MFMAs instead of following them
    Stage P;
    load(0, P);
    store(P, 0);
    __syncthreads();
    for (int kt = 0; kt + 1 < KT; kt++) {
      load(kt + 1, P);
      const int cur = kt & 1;
#pragma unroll
      for (int ks = 0; ks < BK / 32; ks++) {
        compute_ks(cur, ks);
        if (ks == 0) store_a(P, cur ^ 1);
        if (ks == 1) store_b(P, cur ^ 1);
      }
      __syncthreads();
    }
    compute((KT - 1) & 1);
  } else {
    // global loads two K steps ahead in two register stages, the loop
    // unrolled by two so each stage is a fixed register set
    Stage P0, P1;
    load(0, P0);
    load(KT > 1 ? 1 : 0, P1);
    store(P0, 0);
    __syncthreads();
    int kt = 0;
    for (; kt + 2 < KT; kt += 2) {
      load(kt + 2, P0);
      compute(0);
      store(P1, 1);
      __syncthreads();
      load(kt + 3 < KT ? kt + 3 : KT - 1, P1);
      compute(1);
      store(P0, 0);
      __syncthreads();
    }
    if (kt + 1 < KT) {
      compute(0);
      store(P1, 1);
      __syncthreads();
      compute(1);
    } else {
      compute(0);
    }
  }
  w8a8_epilogue<TM, TN>(a, acc, m0 + wm * WM, n0 + wn * WN, lane, m0 + BM <= a.M && n0 + BN <= a.N);
}

// ------------------------------------------------------------- Int8Block

constexpr int I8B_BN = 256;   // columns per workgroup (64 per wave)
constexpr int I8B_KST = 128;  // K rows per LDS step
constexpr int I8B_WST = I8B_BN + 16;
constexpr int I8B_XST = I8B_KST + 8;

RLXQ_DEV uint32_t i8_pair_bf16(uint32_t w, int sh) {
  const float f0 = (float)(int8_t)((w >> sh) & 0xffu);
  const float f1 = (float)(int8_t)((w >> (sh + 8)) & 0xffu);
  // small integers: the bf16 is the high half of the f32, exactly
  return perm_b32(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}

RLXQ_DEV float i8b_finish(const rlxq_i8b_args& a, float v, int64_t m, int64_t n) {
  if (a.zp) v = fmaf(-a.zp[n], a.xsum[m], v);
  return v * a.scale[n];
}

// Workgroup = (256-column block, K split, chunk of 16*MT rows); each wave owns
// 64 columns as four 16-column MFMA tiles.
template <int MT, bool XBF16>
RLXQ_DEV void i8b_body(const rlxq_i8b_args& a) {
  constexpr int MC = 16 * MT;
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* Ws = smem;                                                     // [KST][WST]
  uint16_t* Xh = reinterpret_cast<uint16_t*>(smem + I8B_KST * I8B_WST);  // [MC][XST]
  uint16_t* Xl = Xh + MC * I8B_XST;

  const int tn = blockIdx.x % a.tiles_n;
  const int sp = (blockIdx.x / a.tiles_n) % a.splits;
  const int mc = blockIdx.x / (a.tiles_n * a.splits);
  const int64_t n0 = (int64_t)tn * I8B_BN, m0 = (int64_t)mc * MC;
  const int64_t kb = (int64_t)sp * a.kslice;
  const int64_t ke = kb + a.kslice < a.K ? kb + a.kslice : a.K;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = lane >> 4, s = lane & 15;

  f32x4_t acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[t][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int64_t k0 = kb; k0 < ke; k0 += I8B_KST) {
    uint4 wr[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int c = tid + 256 * i, r = c >> 4, cc = c & 15;
      const int64_t k = k0 + r, n = n0 + 16 * cc;
      wr[i] = make_uint4(0u, 0u, 0u, 0u);
      if (k < ke && n < a.N) wr[i] = *reinterpret_cast<const uint4*>(a.wq + k * a.N + n);
    }
    for (int u = tid; u < MC * (I8B_KST / 8); u += 256) {
      const int row = u / (I8B_KST / 8), c8 = u % (I8B_KST / 8);
      const int64_t m = m0 + row, k = k0 + 8 * c8;
      uint32_t h[4], l[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float v[2];
#pragma unroll
        for (int q = 0; q < 2; q++) {
          const int64_t kk = k + e + q;
          v[q] = 0.f;
          if (m < a.M && kk < ke) {
            if constexpr (XBF16) v[q] = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.x)[m * a.K + kk]);
            else v[q] = reinterpret_cast<const float*>(a.x)[m * a.K + kk];
          }
        }
        const uint32_t h0 = f32_to_bf16_bits(v[0]), h1 = f32_to_bf16_bits(v[1]);
        h[e / 2] = h0 | (h1 << 16);
        if constexpr (!XBF16) {
          const uint32_t l0 = f32_to_bf16_bits(v[0] - bf16_bits_to_f32(h0));
          const uint32_t l1 = f32_to_bf16_bits(v[1] - bf16_bits_to_f32(h1));
          l[e / 2] = l0 | (l1 << 16);
        }
      }
      *reinterpret_cast<uint4*>(Xh + row * I8B_XST + 8 * c8) = make_uint4(h[0], h[1], h[2], h[3]);
      if constexpr (!XBF16)
        *reinterpret_cast<uint4*>(Xl + row * I8B_XST + 8 * c8) = make_uint4(l[0], l[1], l[2], l[3]);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int c = tid + 256 * i, r = c >> 4, cc = c & 15;
      *reinterpret_cast<uint4*>(Ws + r * I8B_WST + 16 * cc) = wr[i];
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < I8B_KST / 32; ks++) {
      // A[i][k] of the 16x16x32 tile: lane i%16 + 16*(k/8); B[k][j]: lane j + 16*(k/8)
      bf16x8_t ah[MT], al[MT];
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const int off = (t * 16 + s) * I8B_XST + ks * 32 + 8 * g;
        ah[t] = *reinterpret_cast<const bf16x8_t*>(Xh + off);
        if constexpr (!XBF16) al[t] = *reinterpret_cast<const bf16x8_t*>(Xl + off);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint8_t* p = Ws + (ks * 32 + 8 * g + (s >> 1)) * I8B_WST + 64 * wv + 16 * j + 8 * (s & 1);
        const i32x2_t q = lds_tr8(p);
        const uint32_t q0 = (uint32_t)q.x, q1 = (uint32_t)q.y;
        uint32_t bw[4] = {i8_pair_bf16(q0, 0), i8_pair_bf16(q0, 16), i8_pair_bf16(q1, 0), i8_pair_bf16(q1, 16)};
        const bf16x8_t b = __builtin_bit_cast(bf16x8_t, bw);
#pragma unroll
        for (int t = 0; t < MT; t++) {
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[t], b, acc[t][j], 0, 0, 0);
          if constexpr (!XBF16) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[t], b, acc[t][j], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }
  // C[i][j] of the 16x16 tile sits in lane j + 16*(i/4), register i%4
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int64_t m = m0 + t * 16 + 4 * g + r;
        const int64_t n = n0 + 64 * wv + 16 * j + s;
        if (m >= a.M || n >= a.N) continue;
        const float v = acc[t][j][r];
        if (a.splits > 1) {
          a.part[((int64_t)sp * a.M + m) * a.N + n] = v;
        } else {
          const float o = i8b_finish(a, v, m, n);
          if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = (uint16_t)f32_to_bf16_bits(o);
          else reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = o;
        }
      }
}

// Decode-size Int8Block (M <= 4): a streaming GEMV over the [K, N] int8
// rows, fp32 FMA on the exact integer values.  A lane owns 16 consecutive
// columns (one 16-byte load per K row), a wave 1024 columns; the W waves of
// a workgroup take interleaved rows kb + w, kb + w + W, ... of the
// workgroup's K slice (the workgroup reads W rows' 1 KB pieces per step),
// each with a ring of D rows of loads in flight, and their sums are added
// in wave order through LDS, one activation row at a time.  K slices go to
// the partial buffer (added in slice order by rlxq_i8b_reduce) unless there
// is one.
constexpr int I8BV_KMAX = 1024;  // most K rows per workgroup slice

template <int MR, bool XBF16, int W, int D>
RLXQ_DEV void i8b_gemv_body(const rlxq_i8b_args& a) {
  __shared__ float red[W][1024];
  __shared__ float xs[MR][I8BV_KMAX];   // the slice's activations, as f32
  constexpr int NT = 64 * W;
  const int tn = blockIdx.x % a.tiles_n;
  const int sp = blockIdx.x / a.tiles_n;
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n0 = (int64_t)tn * 1024 + 16 * lane;
  const bool nok = n0 < a.N;
  const int64_t kb = (int64_t)sp * a.kslice;
  const int64_t ke = kb + a.kslice < a.K ? kb + a.kslice : a.K;
  const int klen = (int)(ke - kb);
  // rows of this wave: kb + wv + W s, s < cnt
  const int cnt = wv < klen ? (klen - wv + W - 1) / W : 0;
  const int8_t* wp = a.wq + (nok ? n0 : 0) + (kb + wv) * a.N;

  float acc[MR][16];
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int j = 0; j < 16; j++) acc[m][j] = 0.f;

  auto load = [&](int st) {
    const int s2 = st < cnt ? st : (cnt > 0 ? cnt - 1 : 0);
    return *reinterpret_cast<const uint4*>(wp + (int64_t)s2 * W * a.N);
  };
  auto step = [&](int st, const uint4& w) {
    const int kl = wv + W * st;
    float xv[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) xv[m] = xs[m][kl];
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const float q = (float)(int)(int8_t)((wd[j >> 2] >> (8 * (j & 3))) & 0xffu);
#pragma unroll
      for (int m = 0; m < MR; m++) acc[m][j] = fmaf(xv[m], q, acc[m][j]);
    }
  };

  // the slice's activations (issued first, so waiting for them does not
  // wait for the ring), then D rows of weights
  constexpr int XPT = (MR * I8BV_KMAX + NT - 1) / NT;
  float xl[XPT];
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int e = threadIdx.x + NT * i, m = e / I8BV_KMAX, kl = e % I8BV_KMAX;
    xl[i] = 0.f;
    if (m < MR && m < a.M && kl < klen) {
      const int64_t off = m * a.K + kb + kl;
      if constexpr (XBF16) xl[i] = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.x)[off]);
      else xl[i] = reinterpret_cast<const float*>(a.x)[off];
    }
  }
  uint4 ring[D];
#pragma unroll
  for (int i = 0; i < D; i++) ring[i] = load(i);
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int e = threadIdx.x + NT * i;
    if (e < MR * I8BV_KMAX) xs[e / I8BV_KMAX][e % I8BV_KMAX] = xl[i];
  }
  __syncthreads();
  int s0 = 0;
  for (; s0 + 2 * D <= cnt; s0 += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      step(s0 + i, ring[i]);
      ring[i] = load(s0 + i + D);
    }
  }
#pragma unroll
  for (int i = 0; i < D; i++) {
    if (s0 + i < cnt) {
      step(s0 + i, ring[i]);
      if (s0 + i + D < cnt) ring[i] = load(s0 + i + D);
    }
  }
#pragma unroll
  for (int i = 0; i < D; i++)
    if (s0 + D + i < cnt) step(s0 + D + i, ring[i]);

  // the waves' sums, added in wave order, one activation row at a time
#pragma unroll
  for (int m = 0; m < MR; m++) {
#pragma unroll
    for (int j = 0; j < 16; j += 4)
      *reinterpret_cast<float4*>(&red[wv][16 * lane + j]) =
          make_float4(acc[m][j], acc[m][j + 1], acc[m][j + 2], acc[m][j + 3]);
    __syncthreads();
    for (int c = threadIdx.x; c < 1024; c += NT) {
      const int64_t n = (int64_t)tn * 1024 + c;
      float v = red[0][c];
#pragma unroll
      for (int w = 1; w < W; w++) v += red[w][c];
      if (m < a.M && n < a.N) {
        if (a.splits > 1) {
          a.part[((int64_t)sp * a.M + m) * a.N + n] = v;
        } else {
          const float o = i8b_finish(a, v, m, n);
          if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = (uint16_t)f32_to_bf16_bits(o);
          else reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = o;
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace rlxq

#define RLXQ_W8A8_INST(BM, BN, BK, WGM, WGN)                                                        \
  extern "C" __global__ __launch_bounds__(WGM * WGN * 64) void rlxq_w8a8_m##BM##n##BN##k##BK##w##WGM##WGN( \
      rlxq_w8a8_args a) {                                                                          \
    rlxq::w8a8_body<BM, BN, BK, WGM, WGN, 8, 1>(a);                                                \
  }
// global loads two K steps ahead: ..._p2
#define RLXQ_W8A8_INST_P2(BM, BN, BK, WGM, WGN)                                                     \
  extern "C" __global__ __launch_bounds__(WGM * WGN * 64, 1) void rlxq_w8a8_m##BM##n##BN##k##BK##w##WGM##WGN##_p2( \
      rlxq_w8a8_args a) {                                                                          \
    rlxq::w8a8_body<BM, BN, BK, WGM, WGN, 8, 2>(a);                                                \
  }
RLXQ_W8A8_INST(128, 128, 64, 2, 2)
RLXQ_W8A8_INST(128, 128, 128, 2, 2)
RLXQ_W8A8_INST(256, 128, 64, 2, 2)
RLXQ_W8A8_INST(128, 256, 64, 2, 2)
RLXQ_W8A8_INST(256, 256, 64, 2, 4)
RLXQ_W8A8_INST_P2(128, 128, 128, 2, 2)
RLXQ_W8A8_INST(256, 256, 128, 2, 4)
// K a whole number of steps: ..._kf (no zeroing selects in the loads)
#define RLXQ_W8A8_INST_KF(BM, BN, BK, WGM, WGN)                                                     \
  extern "C" __global__ __launch_bounds__(WGM * WGN * 64) void rlxq_w8a8_m##BM##n##BN##k##BK##w##WGM##WGN##_kf( \
      rlxq_w8a8_args a) {                                                                          \
    rlxq::w8a8_body<BM, BN, BK, WGM, WGN, 8, 1, true>(a);                                          \
  }
RLXQ_W8A8_INST_KF(256, 256, 64, 2, 4)
RLXQ_W8A8_INST_KF(256, 256, 128, 2, 4)

#define RLXQ_I8B_INST(MT, XN, XBF)                                                        \
  extern "C" __global__ __launch_bounds__(256) void rlxq_i8b_##XN##_mt##MT(rlxq_i8b_args a) { \
    rlxq::i8b_body<MT, XBF>(a);                                                           \
  }
RLXQ_I8B_INST(1, f32, false)
RLXQ_I8B_INST(2, f32, false)
RLXQ_I8B_INST(4, f32, false)
RLXQ_I8B_INST(1, bf16, true)
RLXQ_I8B_INST(2, bf16, true)
RLXQ_I8B_INST(4, bf16, true)

#define RLXQ_I8BV_INST(MR, XN, XBF)                                                           \
  extern "C" __global__ __launch_bounds__(1024) void rlxq_i8bv_##XN##_m##MR(rlxq_i8b_args a) { \
    rlxq::i8b_gemv_body<MR, XBF, 16, 8>(a);                                                     \
  }
RLXQ_I8BV_INST(1, f32, false)
RLXQ_I8BV_INST(2, f32, false)
RLXQ_I8BV_INST(4, f32, false)
RLXQ_I8BV_INST(1, bf16, true)
RLXQ_I8BV_INST(2, bf16, true)
RLXQ_I8BV_INST(4, bf16, true)

// Split-K reduction of the Int8Block partials, summed in split order.  Four
// outputs per thread when N % 4 == 0, with sixteen slices' loads in flight
// at a time (the sums stay in slice order).
extern "C" __global__ __launch_bounds__(256) void rlxq_i8b_reduce(rlxq_i8b_args a) {
  const int64_t mn = a.M * a.N;
  if ((a.N & 3) == 0) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= mn) return;
    const int64_t m = i / a.N, n = i - m * a.N;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.splits; s0 += 16) {
      const int c = a.splits - s0 < 16 ? a.splits - s0 : 16;
      float4 p[16];
#pragma unroll
      for (int q = 0; q < 16; q++)
        if (q < c) p[q] = *reinterpret_cast<const float4*>(a.part + (int64_t)(s0 + q) * mn + i);
#pragma unroll
      for (int q = 0; q < 16; q++)
        if (q < c) {
          v[0] += p[q].x;
          v[1] += p[q].y;
          v[2] += p[q].z;
          v[3] += p[q].w;
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float o = rlxq::i8b_finish(a, v[e], m, n + e);
      if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n + e] = (uint16_t)f32_to_bf16_bits(o);
      else reinterpret_cast<float*>(a.y)[m * a.y_ld + n + e] = o;
    }
    return;
  }
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= mn) return;
  const int64_t m = i / a.N, n = i - m * a.N;
  float v = 0.f;
  for (int sp = 0; sp < a.splits; sp++) v += a.part[(int64_t)sp * mn + i];
  const float o = rlxq::i8b_finish(a, v, m, n);
  if (a.y_bf16) reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = (uint16_t)f32_to_bf16_bits(o);
  else reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = o;
}

// Row sums of x (f32 accumulation), for the zero-point term.  One workgroup
// of 256 per row.
extern "C" __global__ __launch_bounds__(256) void rlxq_row_sum(const void* __restrict__ x, int x_bf16, int64_t M,
                                                               int64_t K, float* __restrict__ out) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  if (r >= M) return;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < K; c += 256)
    s += x_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(x)[r * K + c])
                : reinterpret_cast<const float*>(x)[r * K + c];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[r] = (red[0] + red[1]) + (red[2] + red[3]);
}
