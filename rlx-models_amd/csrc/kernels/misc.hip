// Small kernels around the quantized matmuls: weight dequantization (the
// bit-exact check entry), SwiGLU between fused gate|up and down, per-row int8
// activation quantisation, and the MoE router (softmax + top-k).
#include "common.hip.h"

// One thread per eight consecutive weights (a quarter of a 32-weight block),
// so that a wave writes 2 KB of contiguous f32 with 16-byte stores.  Q8_0:
// d*q; Q4_0: d*(q-8); Q4_1: d*q + m (d*q is exact in f32, so the single
// rounding is the add); Q4_K, Q5_K, Q2_K: (d*sc)*q - dmin*mn (GGML block_q4_K
// / q5_K / q2_K); Q3_K: (d*(sc-32))*q; Q8_K: d*q; MXFP4:
// E2M1(code) * 2^(e - 127) (exact); MLX:
// scale*code rounded, then + bias rounded (no contraction), as
// crates/rlx-moshi/src/mlx_dequant.rs:66-71 evaluates it.
extern "C" __global__ __launch_bounds__(256) void rlxq_dequant_rows(
    int scheme, const uint8_t* __restrict__ w, const void* __restrict__ scales,
    const void* __restrict__ biases, int sb_bf16, int group, int64_t rows, int K, int64_t rb,
    float* __restrict__ out) {
  // Two roundings (multiply, then add), never a fused multiply-add: the
  // pragma governs the expressions written below.
#pragma clang fp contract(off)
  const int bpr = K >> 5;
  const int64_t qid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (qid >= rows * bpr * 4) return;
  const int64_t blk = qid >> 2;
  const int q = (int)(qid & 3);
  const int64_t r = blk / bpr;
  const int b = (int)(blk - r * bpr);
  float v[8];
  if (scheme == SCH_Q6_K) {
    // weight 128h + 32j + l of super-block b / 8 (b % 8 = 4h + j):
    // code = ql nibble | qh 2 bits << 4, w = (d * scale) * (code - 32)
    const int h = (b >> 2) & 1, j = b & 3;
    const uint8_t* p = w + r * rb + (int64_t)(b >> 3) * 210;
    const float d = f16_bits_to_f32((uint32_t)p[208] | ((uint32_t)p[209] << 8));
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int l = 8 * q + i;
      const int lo = (p[64 * h + l + 32 * (j & 1)] >> (4 * (j >> 1))) & 15;
      const int hi = (p[128 + 32 * h + l] >> (2 * j)) & 3;
      const float ds = d * (float)(int8_t)p[192 + 8 * h + 2 * j + l / 16];
      v[i] = ds * (float)((lo | (hi << 4)) - 32);
    }
  } else if (scheme == SCH_Q4_K) {
    // sub-block s of super-block b / 8: the low (s even) or high nibbles of
    // the 32 code bytes of group s / 2; w = (d*sc)*q - dmin*mn
    const int s = b & 7, g = s >> 1;
    const uint8_t* p = w + r * rb + (int64_t)(b >> 3) * 144;
    const float d = f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8));
    const float dmin = f16_bits_to_f32((uint32_t)p[2] | ((uint32_t)p[3] << 8));
    const uint8_t* q12 = p + 4;
    int sc, mn;
    if (s < 4) {
      sc = q12[s] & 63;
      mn = q12[s + 4] & 63;
    } else {
      sc = (q12[s + 4] & 15) | ((q12[s - 4] >> 6) << 4);
      mn = (q12[s + 4] >> 4) | ((q12[s] >> 6) << 4);
    }
    const float d1 = d * (float)sc, m1 = dmin * (float)mn;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int byte = p[16 + 32 * g + 8 * q + i];
      const float prod = d1 * (float)((s & 1) ? byte >> 4 : byte & 15);
      v[i] = prod - m1;
    }
  } else if (scheme == SCH_Q5_K) {
    // sub-block s of super-block b / 8: nibble s & 1 of the group's qs
    // bytes, fifth bit from qh bit s; w = (d*sc)*code - dmin*mn
    const int s = b & 7, g = s >> 1;
    const uint8_t* p = w + r * rb + (int64_t)(b >> 3) * 176;
    const float d = f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8));
    const float dmin = f16_bits_to_f32((uint32_t)p[2] | ((uint32_t)p[3] << 8));
    const uint8_t* q12 = p + 4;
    int sc, mn;
    if (s < 4) {
      sc = q12[s] & 63;
      mn = q12[s + 4] & 63;
    } else {
      sc = (q12[s + 4] & 15) | ((q12[s - 4] >> 6) << 4);
      mn = (q12[s + 4] >> 4) | ((q12[s] >> 6) << 4);
    }
    const float d1 = d * (float)sc, m1 = dmin * (float)mn;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int l = 8 * q + i;
      const int code = ((p[48 + 32 * g + l] >> (4 * (s & 1))) & 15) | (((p[16 + l] >> s) & 1) << 4);
      const float prod = d1 * (float)code;
      v[i] = prod - m1;
    }
  } else if (scheme == SCH_Q3_K || scheme == SCH_Q2_K) {
    // block (n, j) = (b % 8 / 4, b % 4) of super-block b / 8; its weights
    // 16i + l (i < 2) have code bits 2j of qs byte 32n + 16i + l and
    // scale 8n + 2j + i
    const int bb = b & 7, n = bb >> 2, j = bb & 3, i = q >> 1;
    const int s = 8 * n + 2 * j + i;
    if (scheme == SCH_Q3_K) {
      // w = (d * (scale - 32)) * (2 bits - (hmask bit 4n + j ? 0 : 4))
      const uint8_t* p = w + r * rb + (int64_t)(b >> 3) * 110;
      const uint8_t* sc12 = p + 96;
      const int sc = ((sc12[s & 7] >> (4 * (s >> 3))) & 15) | (((sc12[8 + (s & 3)] >> (2 * (s >> 2))) & 3) << 4);
      const float dl = f16_bits_to_f32((uint32_t)p[108] | ((uint32_t)p[109] << 8)) * (float)(sc - 32);
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const int l = 8 * (q & 1) + t;
        const int lo = (p[32 + 32 * n + 16 * i + l] >> (2 * j)) & 3;
        const int hi = (p[16 * i + l] >> (4 * n + j)) & 1;
        v[t] = dl * (float)(lo - (hi ? 0 : 4));
      }
    } else {
      // w = (d * (c & 15)) * code - dmin * (c >> 4), c = scales[s]
      const uint8_t* p = w + r * rb + (int64_t)(b >> 3) * 84;
      const int c = p[s];
      const float d = f16_bits_to_f32((uint32_t)p[80] | ((uint32_t)p[81] << 8));
      const float dmin = f16_bits_to_f32((uint32_t)p[82] | ((uint32_t)p[83] << 8));
      const float dl = d * (float)(c & 15), ml = dmin * (float)(c >> 4);
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const int l = 8 * (q & 1) + t;
        const float prod = dl * (float)((p[16 + 32 * n + 16 * i + l] >> (2 * j)) & 3);
        v[t] = prod - ml;
      }
    }
  } else if (scheme == SCH_Q8_K) {
    // w = d * q, d the super-block's f32
    const uint8_t* p = w + r * rb + (int64_t)(b >> 3) * 292;
    const float d = __uint_as_float((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                                    ((uint32_t)p[3] << 24));
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = d * (float)(int8_t)p[4 + 32 * (b & 7) + 8 * q + i];
  } else if (scheme == SCH_MXFP4) {
    // codes 8q..8q+7 of the block are dword 4b + q of the row (low nibble =
    // even element); w = E2M1(code) * scale, exact.  sb_bf16: 2 = E8M0 bytes,
    // 1 = the decoded scales as bf16.
    const int64_t gi = r * (int64_t)bpr + b;
    const float sc = sb_bf16 == 2 ? e8m0_to_f32(reinterpret_cast<const uint8_t*>(scales)[gi])
                                  : bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(scales)[gi]);
    const uint32_t cw = reinterpret_cast<const uint32_t*>(w + r * rb)[4 * b + q];
    const uint32_t pr[4] = {fp4x2_to_bf16x2<0>(cw), fp4x2_to_bf16x2<1>(cw), fp4x2_to_bf16x2<2>(cw),
                            fp4x2_to_bf16x2<3>(cw)};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = bf16_bits_to_f32(pr[i] & 0xffffu) * sc;
      v[2 * i + 1] = bf16_bits_to_f32(pr[i] >> 16) * sc;
    }
  } else if (scheme == SCH_Q8_0 || scheme == SCH_Q4_0 || scheme == SCH_Q4_1) {
    const int bb = scheme == SCH_Q8_0 ? 34 : (scheme == SCH_Q4_0 ? 18 : 20);
    const uint8_t* p = w + r * rb + (int64_t)b * bb;
    const float d = f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8));
    if (scheme == SCH_Q8_0) {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = d * (float)(int8_t)p[2 + 8 * q + i];
    } else {
      // element e = 8q + i: low nibble of byte e (e < 16), else high nibble of byte e - 16
      const int hdr = scheme == SCH_Q4_0 ? 2 : 4;
      const int byte0 = (8 * q) & 15, shift = q >= 2 ? 4 : 0;
      const float m = scheme == SCH_Q4_1 ? f16_bits_to_f32((uint32_t)p[2] | ((uint32_t)p[3] << 8)) : 0.f;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int c = (p[hdr + byte0 + i] >> shift) & 15;
        v[i] = scheme == SCH_Q4_0 ? d * (float)(c - 8) : d * (float)c + m;
      }
    }
  } else {
    // MLX affine: codes of this block; one scale/bias per group.
    const int bits = scheme == SCH_MLX4 ? 4 : 8;
    const int64_t gi = r * (int64_t)(K / group) + ((int64_t)b * 32) / group;
    float s, bi;
    if (sb_bf16) {
      s = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(scales)[gi]);
      bi = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(biases)[gi]);
    } else {
      s = reinterpret_cast<const float*>(scales)[gi];
      bi = reinterpret_cast<const float*>(biases)[gi];
    }
    const uint32_t* wq = reinterpret_cast<const uint32_t*>(w + r * rb) + (b * 32 * bits) / 32;
    const int per = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int e = 8 * q + i;
      const uint32_t code = (wq[e / per] >> ((e % per) * bits)) & mask;
      v[i] = s * (float)code + bi;
    }
  }
  float* o = out + r * (int64_t)K + (int64_t)b * 32 + 8 * q;
  if ((reinterpret_cast<uintptr_t>(out) & 15) == 0) {
    reinterpret_cast<float4*>(o)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(o)[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = v[i];
  }
}

// out[r, i] = silu(gu[r, i]) * gu[r, inter + i] with silu(v) = v / (1 + e^-v)
// (crates/rlx-laguna/src/mlx_affine.rs:126-128), f32 arithmetic.
extern "C" __global__ __launch_bounds__(256) void rlxq_swiglu_k(
    const void* __restrict__ gu, int gu_bf16, int64_t rows, int64_t inter, void* __restrict__ out,
    int out_bf16) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * inter) return;
  const int64_t r = i / inter, c = i - r * inter;
  const int64_t gi = r * 2 * inter + c, ui = gi + inter;
  float g, u;
  if (gu_bf16) {
    g = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(gu)[gi]);
    u = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(gu)[ui]);
  } else {
    g = reinterpret_cast<const float*>(gu)[gi];
    u = reinterpret_cast<const float*>(gu)[ui];
  }
  const float v = g / (1.0f + expf(-g)) * u;
  if (out_bf16) reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(v);
  else reinterpret_cast<float*>(out)[i] = v;
}

// Per-row int8 activation quantisation (crates/rlx-quant-calib/src/bitnet.rs:76-93):
// s = amax/127 (1 when the row is all zero), q = round_half_away(x * (1/s))
// clamped to +-127.  One workgroup of 256 threads per row.
extern "C" __global__ __launch_bounds__(256) void rlxq_quant_act_i8(
    const void* __restrict__ x, int x_bf16, int64_t M, int K, int8_t* __restrict__ q,
    float* __restrict__ scales, int vec) {
  // 16-element chunks (vec: 16-byte aligned rows, else every element goes
  // through the scalar loops): RB per thread stay in registers between the amax pass
  // and the quantisation (one 16-byte store each); chunks past 256 * RB and
  // the K % 16 tail are read again.  Per element the arithmetic is the
  // scalar rule: q = clamp(round(x * (1 / (amax / 127))), -127, 127).
  constexpr int RB = 3;
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  if (r >= M) return;
  const int t = threadIdx.x;
  const int nch = vec ? K >> 4 : 0;
  auto ld16 = [&](int c, float* v) {
    if (x_bf16) {
      const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + r * K + 16 * c);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const uint4 u = p[h];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[8 * h + 2 * e] = bf16_bits_to_f32(w[e] & 0xffffu);
          v[8 * h + 2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
        }
      }
    } else {
      const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + r * K + 16 * c);
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const float4 u = p[h];
        v[4 * h] = u.x; v[4 * h + 1] = u.y; v[4 * h + 2] = u.z; v[4 * h + 3] = u.w;
      }
    }
  };
  auto ld1 = [&](int c) -> float {
    if (x_bf16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(x)[r * K + c]);
    return reinterpret_cast<const float*>(x)[r * K + c];
  };
  float v[RB][16];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < RB; i++) {
    const int c = t + 256 * i;
    if (c < nch) {
      ld16(c, v[i]);
#pragma unroll
      for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(v[i][e]));
    }
  }
  for (int c = t + 256 * RB; c < nch; c += 256) {
    float w[16];
    ld16(c, w);
#pragma unroll
    for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(w[e]));
  }
  for (int c = 16 * nch + t; c < K; c += 256) amax = fmaxf(amax, fabsf(ld1(c)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if ((t & 63) == 0) red[t >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax > 0.f ? __fdiv_rn(amax, 127.0f) : 1.0f;
  const float inv = __fdiv_rn(1.0f, s);
  auto quant = [&](float xv) -> uint32_t {
    const float qv = fminf(fmaxf(roundf(__fmul_rn(xv, inv)), -127.f), 127.f);
    return (uint32_t)(uint8_t)(int8_t)qv;
  };
  auto st16 = [&](int c, const float* w) {
    uint32_t o[4];
#pragma unroll
    for (int d = 0; d < 4; d++)
      o[d] = quant(w[4 * d]) | (quant(w[4 * d + 1]) << 8) | (quant(w[4 * d + 2]) << 16) | (quant(w[4 * d + 3]) << 24);
    *reinterpret_cast<uint4*>(q + r * K + 16 * c) = make_uint4(o[0], o[1], o[2], o[3]);
  };
#pragma unroll
  for (int i = 0; i < RB; i++) {
    const int c = t + 256 * i;
    if (c < nch) st16(c, v[i]);
  }
  for (int c = t + 256 * RB; c < nch; c += 256) {
    float w[16];
    ld16(c, w);
    st16(c, w);
  }
  for (int c = 16 * nch + t; c < K; c += 256) q[r * K + c] = (int8_t)(int)fminf(fmaxf(roundf(__fmul_rn(ld1(c), inv)), -127.f), 127.f);
  if (t == 0) scales[r] = s;
}

namespace rlxq {

// DPP moves within 16-lane rows: xor 1 and xor 2 (quad_perm), the 8-lane half
// mirror and the 16-lane mirror; after the four, every lane of a row holds
// the row's reduction.
#define RLXQ_DPP(v, ctrl) __builtin_amdgcn_mov_dpp((v), (ctrl), 0xF, 0xF, false)

template <typename Op>
RLXQ_DEV float wave_reduce(float v, Op op) {
  v = op(v, __int_as_float(RLXQ_DPP(__float_as_int(v), 0xB1)));
  v = op(v, __int_as_float(RLXQ_DPP(__float_as_int(v), 0x4E)));
  v = op(v, __int_as_float(RLXQ_DPP(__float_as_int(v), 0x141)));
  v = op(v, __int_as_float(RLXQ_DPP(__float_as_int(v), 0x140)));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return op(op(r0, r1), op(r2, r3));
}

// (probability, expert) maximum over the wave: larger probability, then the
// lower expert id.  The result is the same in every lane.
RLXQ_DEV void wave_argmax(float& v, int& e) {
  auto take = [&](float ov, int oe) {
    if (ov > v || (ov == v && oe < e)) {
      v = ov;
      e = oe;
    }
  };
  take(__int_as_float(RLXQ_DPP(__float_as_int(v), 0xB1)), RLXQ_DPP(e, 0xB1));
  take(__int_as_float(RLXQ_DPP(__float_as_int(v), 0x4E)), RLXQ_DPP(e, 0x4E));
  take(__int_as_float(RLXQ_DPP(__float_as_int(v), 0x141)), RLXQ_DPP(e, 0x141));
  take(__int_as_float(RLXQ_DPP(__float_as_int(v), 0x140)), RLXQ_DPP(e, 0x140));
  float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  int be = __builtin_amdgcn_readlane(e, 0);
#pragma unroll
  for (int row = 1; row < 4; row++) {
    const float ov = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * row));
    const int oe = __builtin_amdgcn_readlane(e, 16 * row);
    if (ov > bv || (ov == bv && oe < be)) {
      bv = ov;
      be = oe;
    }
  }
  v = bv;
  e = be;
}

}  // namespace rlxq

// Router: softmax over E logits then top-k by probability, ties to the lower
// expert id; optional renormalisation of the kept probabilities.  One wave per
// row, E <= 64 * NPER (lane l holds experts l, l + 64, ...); the reductions
// use DPP row moves and readlane.
namespace rlxq {
template <int NPER>
RLXQ_DEV void moe_route_body(const float* __restrict__ logits, int64_t rows, int E, int topk, int renorm,
                             int32_t* __restrict__ ids, float* __restrict__ probs) {
  const int64_t r = blockIdx.x;
  if (r >= rows) return;
  const int lane = threadIdx.x;
  const float* l = logits + r * E;
  float p[NPER];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NPER; i++) {
    const int e = lane + 64 * i;
    p[i] = e < E ? l[e] : -INFINITY;
    mx = fmaxf(mx, p[i]);
  }
  mx = wave_reduce(mx, [](float x, float y) { return fmaxf(x, y); });
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NPER; i++) {
    const int e = lane + 64 * i;
    p[i] = e < E ? expf(p[i] - mx) : 0.f;
    s += p[i];
  }
  s = wave_reduce(s, [](float x, float y) { return x + y; });
#pragma unroll
  for (int i = 0; i < NPER; i++) {
    const int e = lane + 64 * i;
    p[i] = e < E ? p[i] / s : -1.f;
  }
  float kept = 0.f, sel_p = 0.f;
  int sel_e = 0;
  for (int j = 0; j < topk; j++) {
    // lane-local best (highest probability, lowest id on ties), then the wave's
    float bv = -2.f;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < NPER; i++) {
      const int e = lane + 64 * i;
      if (p[i] > bv || (p[i] == bv && e < be)) {
        bv = p[i];
        be = e;
      }
    }
    wave_argmax(bv, be);
    if (lane == j) {
      sel_p = bv;
      sel_e = be;
    }
    kept += bv;
#pragma unroll
    for (int i = 0; i < NPER; i++)
      if (lane + 64 * i == be) p[i] = -1.f;
  }
  if (lane < topk) {
    ids[r * topk + lane] = sel_e;
    probs[r * topk + lane] = renorm ? sel_p / kept : sel_p;
  }
}
}  // namespace rlxq

#define RLXQ_ROUTE_INST(NPER)                                                                         \
  extern "C" __global__ __launch_bounds__(64) void rlxq_moe_route_k##NPER(                            \
      const float* __restrict__ logits, int64_t rows, int E, int topk, int renorm,                      \
      int32_t* __restrict__ ids, float* __restrict__ probs) {                                           \
    rlxq::moe_route_body<NPER>(logits, rows, E, topk, renorm, ids, probs);                             \
  }
RLXQ_ROUTE_INST(1)
RLXQ_ROUTE_INST(2)
RLXQ_ROUTE_INST(4)
RLXQ_ROUTE_INST(8)
RLXQ_ROUTE_INST(16)

// ---------------------------------------------------------------------------
// Peak probes for the measurement (the denominators a roofline fraction can
// be quoted against besides the data-sheet peaks).
//
// MFMA: each wave runs `iters` rounds of four independent
// v_mfma_f32_32x32x16_bf16 on register operands (no memory traffic, four
// chains hide the instruction's latency); 32768 flops per instruction.  The
// accumulators are stored only when a sum nobody can reach is hit, which
// keeps the chains live.
typedef __bf16 rlxq_probe_bf16x8 __attribute__((ext_vector_type(8)));
typedef float rlxq_probe_f32x16 __attribute__((ext_vector_type(16)));
extern "C" __global__ __launch_bounds__(256) void rlxq_probe_mfma(int64_t iters, float* __restrict__ sink) {
  const float f = 1.0f + 1e-3f * (float)(threadIdx.x & 7);
  rlxq_probe_bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (__bf16)(f * (float)(i + 1) * 1e-3f);
    b[i] = (__bf16)(f * (float)(8 - i) * 1e-3f);
  }
  rlxq_probe_f32x16 acc[4];
#pragma unroll
  for (int c = 0; c < 4; c++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[c][r] = 0.f;
  for (int64_t it = 0; it < iters; it++) {
#pragma unroll
    for (int c = 0; c < 4; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 4; c++)
#pragma unroll
    for (int r = 0; r < 16; r++) s += acc[c][r];
  if (s == -1234.5f) sink[threadIdx.x] = s;
}

// Streaming read: every byte of `bytes` (a multiple of 4096) read once with
// 16-byte loads, grid-stride, one load per iteration (the pattern that
// measured fastest on MI355X: deeper unrolls of the stride loop, and
// contiguous spans per workgroup, read 2-15% slower); each workgroup's xor
// of the data goes to sink[blockIdx.x] (keeps the loads live).
// The same bytes, four independent 16-byte loads per thread issued before
// any is used, over a grid sized to them (4 * gridDim.x * 256 >= n16).
extern "C" __global__ __launch_bounds__(256) void rlxq_probe_read4(const uint4* __restrict__ src, int64_t n16,
                                                                   uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint4 v[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int64_t i = i0 + u * stride;
    v[u] = i < n16 ? src[i] : make_uint4(0u, 0u, 0u, 0u);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int k = 0; k < 256; k++) t ^= red[k];
    sink[blockIdx.x] = t;
  }
}

// The register-streamed batched-decode kernel's weight reads with no
// arithmetic: rows of 2560 bytes (4096 Q4_1 codes, 128 blocks of 20 bytes);
// workgroup b takes rows 32 b .. 32 b + 31 as two 16-row tiles, wave w the
// 80-byte chunks w, w + 4, ... of them, and lane (j, g) block 4 c + g of
// row j of each tile as one dword and one 16-byte load, four chunks in
// flight: 16 rows x 80 bytes per wave instruction.
extern "C" __global__ __launch_bounds__(256) void rlxq_probe_tile20(const uint8_t* __restrict__ w,
                                                                    uint32_t* __restrict__ sink) {
  constexpr int RB = 2560, CH = 8, D = 4;   // CH chunks per wave (32 per row)
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, j = lane & 15, g = lane >> 4;
  const uint8_t* base = w + (int64_t)blockIdx.x * 32 * RB;
  uint32_t h[D][2];
  uint4 q[D][2];
  auto load = [&](int it, int d) {
    const int c = wv + 4 * it;
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const uint8_t* p = base + (16 * t + j) * RB + (4 * c + g) * 20;
      h[d][t] = ld_u32(p);
      q[d][t] = ld_u128(p + 4);
    }
  };
#pragma unroll
  for (int d = 0; d < D; d++) load(d, d);
  uint32_t acc = 0;
#pragma unroll
  for (int it0 = 0; it0 < CH; it0 += D)
#pragma unroll
    for (int d = 0; d < D; d++) {
#pragma unroll
      for (int t = 0; t < 2; t++) acc ^= h[d][t] ^ q[d][t].x ^ q[d][t].y ^ q[d][t].z ^ q[d][t].w;
      if (it0 + d + D < CH) load(it0 + d + D, d);
    }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int k = 0; k < 256; k++) t ^= red[k];
    sink[blockIdx.x] = t;
  }
}

extern "C" __global__ __launch_bounds__(256) void rlxq_probe_read(const uint4* __restrict__ src, int64_t n16,
                                                                  uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const uint4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int k = 0; k < 256; k++) t ^= red[k];
    sink[blockIdx.x] = t;
  }
}
