// Host side of the batched-decode (small M) dequant-GEMM: activation
// preparation, then the skinny kernel, then (small N only) the split-K sum.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "rlxq.h"
#include "rlxq_internal.hpp"
#include "skinny_args.h"

namespace rlxq {

namespace {
size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }
}  // namespace

// x -> prepared f16 activations and row scales in the workspace (x16 at
// the start, inv_s after it; `extra` more bytes follow for the caller).
int splits_reduce(rlxq_ctx* ctx, rlxq_skinny_args& a, void* stream) {
  hipFunction_t fn;
  int rc;
  if ((rc = get_fn(ctx, "rlxq_skinny_reduce", &fn))) return rc;
  const int64_t per = a.N % 4 == 0 ? 4 : 1, threads = (a.M * a.N + per - 1) / per;
  void* rargs[] = {&a};
  return launch(ctx, fn, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, rargs, "rlxq_skinny_reduce");
}

int prep_x16(rlxq_ctx* ctx, const void* x, int x_dtype, int64_t m, int64_t k, int order, size_t extra,
             rlxq_x16_args& xa, char** rest, void* stream, bool frag_major, int64_t mp, bool out_bf16, int split,
             int post_exp) {
  // x16 rows: 2m (split 1), m rounded up to 32 times 2 (split 2), else m
  const int64_t rows = split == 2 ? (m + 31) / 32 * 64 : (split ? 2 * m : m);
  if (!frag_major || mp < rows) mp = rows;
  // fragment-major: the block sums (one f32 per 32 elements) after inv_s
  const size_t x16_bytes = round256((size_t)(mp * k) * 2), s_bytes = round256((size_t)rows * 4);
  const size_t sum_bytes = frag_major ? round256((size_t)(mp * (k / 32)) * 4) : 0;
  void* ws = nullptr;
  int rc;
  if ((rc = workspace(ctx, x16_bytes + s_bytes + sum_bytes + extra, &ws, stream))) return rc;
  char* wsb = static_cast<char*>(ws);
  std::memset(&xa, 0, sizeof xa);
  xa.x = x;
  xa.x16 = reinterpret_cast<uint16_t*>(wsb);
  xa.inv_s = reinterpret_cast<float*>(wsb + x16_bytes);
  xa.M = m;
  xa.K = k;
  xa.Mp = mp;
  xa.x_bf16 = x_dtype == RLXQ_BF16;
  xa.nibble_order = order;
  xa.frag_major = frag_major ? 1 : 0;
  xa.out_bf16 = out_bf16 ? 1 : 0;
  xa.split = split;
  xa.post_exp = post_exp;
  xa.ssum = frag_major ? reinterpret_cast<float*>(wsb + x16_bytes + s_bytes) : nullptr;
  *rest = wsb + x16_bytes + s_bytes + sum_bytes;
  hipFunction_t fn;
  if ((rc = get_fn(ctx, "rlxq_x16_prep", &fn))) return rc;
  void* xargs[] = {&xa};
  // workgroup (x16 row, 2048-element chunks of K gy apart): a chunk each
  // while rows are few, whole rows (one read for the row maximum) once the
  // rows alone fill the chip
  const int64_t nchunk = (k + 2047) / 2048, cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  const int64_t gy = std::max<int64_t>(1, std::min<int64_t>(nchunk, (8 * cus + mp - 1) / mp));
  if (gy > 65535 || mp > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, "activation preparation grid");
  return launch(ctx, fn, dim3((unsigned)mp, (unsigned)gy), dim3(256), 0, stream, xargs, "rlxq_x16_prep");
}

namespace {

// Bytes of one weight row per 128-element chunk (the LDS-staged kernel's
// formats; 0 for the others).
int64_t xl_chunk_bytes(int scheme) {
  switch (scheme) {
    case RLXQ_GGUF_Q4_1: return 80;
    case RLXQ_GGUF_Q4_0: return 72;
    case RLXQ_GGUF_Q8_0: return 136;
    case RLXQ_GGUF_Q4_K: return 72;
    case RLXQ_GGUF_Q5_K: return 88;
    default: return 0;
  }
}

// Register-streamed kernel (SC = 0), or its LDS-staged form (SC chunks a
// step): workgroups (NT x 16 weight rows, K split, 16*MT-row chunk); K
// splits (powers of two, whole 128-element chunks, whole steps) until the
// grid holds about two workgroups per CU (RLXQ_SKINNY_WGS scales that).
int skinny_xr_dispatch(rlxq_ctx* ctx, int scheme, const void* x, int x_dtype, const void* w, int64_t rb, int64_t m,
                       int64_t k, int64_t n, void* y, int y_dtype, void* stream, int MT, int NT, int D,
                       const SkinnySb& sb, int SC = 0) {
  // f32 activations: hi and lo rows (2m x16 rows), added in the epilogue
  const bool split = x_dtype == RLXQ_F32;
  const int64_t mr = split ? 2 * m : m;
  const int64_t tiles_n = (n + 16 * NT - 1) / (16 * NT), mch = (mr + 16 * MT - 1) / (16 * MT);
  const int64_t chunks = k / 128;
  const int64_t cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  // 64-row chunks with a two-deep ring (the byte-code formats past 32 rows):
  // one workgroup per CU, half the K splits (down 12288->4096 at M=64: Q8_0
  // 51.7 -> 43.0 us, Q8_K 51.2 -> 43.1, Q2_K 61.0 -> 52.9; with a one-deep
  // ring, or 16-row chunks, fewer splits measured the same or slower)
  int64_t target = (MT >= 4 && D >= 2) ? cus : 2 * cus;
  if (const char* e = std::getenv("RLXQ_SKINNY_WGS")) target = (int64_t)(cus * std::atof(e));
  int64_t splits = 1;
  while (tiles_n * mch * splits < target && splits * 2 * 4 <= chunks && splits < 32) splits *= 2;
  // (LDS-staged: each split whole steps of SC chunks; the caller keeps K a
  // whole number of steps)
  const int64_t unit = SC > 0 ? SC : 1, steps = chunks / unit;
  const int64_t kslice = ((steps + splits - 1) / splits) * unit * 128;
  splits = (k + kslice - 1) / kslice;
  if (tiles_n * mch * splits > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: batched-decode grid");
  const size_t part_bytes = splits > 1 ? round256((size_t)(splits * m * n) * 4) : 0;
  rlxq_x16_args xa;
  char* rest = nullptr;
  int rc;
  const int64_t mp = mch * 16 * MT;
  if ((rc = prep_x16(ctx, x, x_dtype, m, k, sk_order(scheme), part_bytes, xa, &rest, stream, true, mp,
                     scheme == RLXQ_MLX_MXFP4, split ? 1 : 0, sk_post_exp(scheme))))
    return rc;
  rlxq_skinny_args a;
  std::memset(&a, 0, sizeof a);
  a.x16 = xa.x16;
  a.inv_s = xa.inv_s;
  a.ssum = xa.ssum;
  a.w = static_cast<const uint8_t*>(w);
  a.part = part_bytes ? reinterpret_cast<float*>(rest) : nullptr;
  a.y = y;
  a.M = mr;
  a.pairs = split ? 1 : 0;
  a.N = n;
  a.K = k;
  a.rb = rb;
  a.y_ld = n;
  a.Mp = mp;
  a.kslice = (int32_t)kslice;
  a.splits = (int32_t)splits;
  a.tiles_n = (int32_t)tiles_n;
  a.y_bf16 = y_dtype == RLXQ_BF16;
  a.scales = sb.scales;
  a.biases = sb.biases;
  a.group = sb.group;
  a.sb_bf16 = sb.sb_bf16;
  char name[64];
  size_t lds = 2 * (size_t)(MT * NT * 4) * 64 * 4;   // the waves' sums
  if (SC > 0) {
    // four wave regions of 16 NT rows, each LROW bytes (an odd number of
    // 16-byte units), before the sums
    const int64_t seg = SC * xl_chunk_bytes(scheme), lrow = (seg / 16) % 2 ? seg : seg + 16;
    lds += (size_t)(4 * 16 * NT * lrow);
    std::snprintf(name, sizeof name, "rlxq_skinnyxl_%s_mt%d_nt%d_s%d_d%d", scheme_name(scheme), MT, NT, SC, D);
  } else {
    std::snprintf(name, sizeof name, "rlxq_skinnyxr_%s_mt%d_nt%d_d%d", scheme_name(scheme), MT, NT, D);
  }
  hipFunction_t fn;
  if ((rc = get_fn(ctx, name, &fn))) return rc;
  void* args[] = {&a};
  if ((rc = launch(ctx, fn, dim3((unsigned)(tiles_n * splits * mch)), dim3(256), lds, stream, args, name))) return rc;
  if (splits > 1) {
    rlxq_skinny_args r = a;   // the partial sums hold the m output rows
    r.M = m;
    rc = splits_reduce(ctx, r, stream);
    if (!rc) ctx->last_kernel = name;
  }
  return rc;
}
// N-split kernel: workgroups (4 NT x 16 weight rows, K split, 16*MT-row
// chunk), the activations of a step shared by the four waves through LDS; K
// splits as for the register-streamed kernel.
int skinny_ns_dispatch(rlxq_ctx* ctx, int scheme, const void* x, int x_dtype, const void* w, int64_t rb, int64_t m,
                       int64_t k, int64_t n, void* y, int y_dtype, void* stream, int MT, int NT, int D,
                       const SkinnySb& sb) {
  // f32 activations: hi and lo rows (2m x16 rows), added in the epilogue
  const bool split = x_dtype == RLXQ_F32;
  const int64_t mr = split ? 2 * m : m;
  const int64_t tiles_n = (n + 64 * NT - 1) / (64 * NT), mch = (mr + 16 * MT - 1) / (16 * MT);
  const int64_t chunks = k / 128;
  const int64_t cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  int64_t target = 2 * cus;
  if (const char* e = std::getenv("RLXQ_SKINNY_WGS")) target = (int64_t)(cus * std::atof(e));
  int64_t splits = 1;
  while (tiles_n * mch * splits < target && splits * 2 * 4 <= chunks && splits < 32) splits *= 2;
  const int64_t kslice = ((chunks + splits - 1) / splits) * 128;
  splits = (k + kslice - 1) / kslice;
  if (tiles_n * mch * splits > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: batched-decode grid");
  const size_t part_bytes = splits > 1 ? round256((size_t)(splits * m * n) * 4) : 0;
  rlxq_x16_args xa;
  char* rest = nullptr;
  int rc;
  const int64_t mp = mch * 16 * MT;
  if ((rc = prep_x16(ctx, x, x_dtype, m, k, sk_order(scheme), part_bytes, xa, &rest, stream, true, mp,
                     scheme == RLXQ_MLX_MXFP4, split ? 1 : 0, sk_post_exp(scheme))))
    return rc;
  rlxq_skinny_args a;
  std::memset(&a, 0, sizeof a);
  a.x16 = xa.x16;
  a.inv_s = xa.inv_s;
  a.ssum = xa.ssum;
  a.w = static_cast<const uint8_t*>(w);
  a.part = part_bytes ? reinterpret_cast<float*>(rest) : nullptr;
  a.y = y;
  a.M = mr;
  a.pairs = split ? 1 : 0;
  a.N = n;
  a.K = k;
  a.rb = rb;
  a.y_ld = n;
  a.Mp = mp;
  a.kslice = (int32_t)kslice;
  a.splits = (int32_t)splits;
  a.tiles_n = (int32_t)tiles_n;
  a.y_bf16 = y_dtype == RLXQ_BF16;
  a.scales = sb.scales;
  a.biases = sb.biases;
  a.group = sb.group;
  a.sb_bf16 = sb.sb_bf16;
  char name[64];
  std::snprintf(name, sizeof name, "rlxq_skinnyns_%s_mt%d_nt%d_d%d", scheme_name(scheme), MT, NT, D);
  hipFunction_t fn;
  if ((rc = get_fn(ctx, name, &fn))) return rc;
  const size_t lds = 2 * (size_t)(4 * 16 * MT * 64);
  void* args[] = {&a};
  if ((rc = launch(ctx, fn, dim3((unsigned)(tiles_n * splits * mch)), dim3(256), lds, stream, args, name))) return rc;
  if (splits > 1) {
    rlxq_skinny_args r = a;   // the partial sums hold the m output rows
    r.M = m;
    rc = splits_reduce(ctx, r, stream);
    if (!rc) ctx->last_kernel = name;
  }
  return rc;
}
}  // namespace

// (the formats whose f16 weight operands carry a 2^8 factor, sk_wscale)
int sk_post_exp(int scheme) {
  return (scheme == RLXQ_MLX_AFFINE4 || scheme == RLXQ_MLX_AFFINE8 || scheme == RLXQ_GGUF_Q8_K ||
          scheme == RLXQ_GGUF_Q2_K)
             ? -8
             : 0;
}

// Code order of the prepared activations: the GGUF nibble formats 1, MLX's
// 4-bit codes 2, the one-code-per-byte forms natural (0).
int sk_order(int scheme) {
  if (scheme == RLXQ_MLX_AFFINE4) return 2;
  return scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_GGUF_Q4_K ? 1 : 0;
}

bool skinny_applies(int scheme, int group, int sb_dtype, int64_t m, int64_t k) {
  return (scheme == RLXQ_GGUF_Q8_0 || scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_GGUF_Q4_1 ||
          ((scheme == RLXQ_GGUF_Q4_K || scheme == RLXQ_GGUF_Q6_K || scheme == RLXQ_GGUF_Q5_K ||
            scheme == RLXQ_GGUF_Q3_K || scheme == RLXQ_GGUF_Q2_K || scheme == RLXQ_GGUF_Q8_K) &&
           k % 256 == 0) ||
          ((scheme == RLXQ_MLX_AFFINE4 || scheme == RLXQ_MLX_AFFINE8) && group >= 32 && group % 32 == 0 &&
           k % group == 0) ||
          // (E8M0 scales only: a bf16 scale times a code is not exact in bf16)
          (scheme == RLXQ_MLX_MXFP4 && sb_dtype == RLXQ_U8)) &&
         m >= 1 && m <= 256 && k % 128 == 0;
}

// Workgroups: (128 weight rows, K split, 64-row chunk).  K splits only where
// the row tiles do not cover the CUs: the smallest power of two that does,
// at most 32 and at most one split per K step; their partial sums (f32,
// [splits, M, N]) are added in split order.
int skinny_dispatch(rlxq_ctx* ctx, int scheme, const void* x, int x_dtype, const void* w, int64_t rb, int64_t m_out,
                    int64_t k, int64_t n, void* y, int y_dtype, void* stream, const SkinnySb& sb) {
  const bool mlx = scheme == RLXQ_MLX_AFFINE4 || scheme == RLXQ_MLX_AFFINE8 || scheme == RLXQ_MLX_MXFP4;
  // f32 activations run as hi and lo x16 rows (the register-streamed and
  // N-split kernels add each pair): the tilings below are chosen on those
  // rows
  const bool f32x = x_dtype == RLXQ_F32;
  const int64_t m = f32x ? 2 * m_out : m_out;
  auto run_xr = [&](int MT, int NT, int D) {
    return skinny_xr_dispatch(ctx, scheme, x, x_dtype, w, rb, m_out, k, n, y, y_dtype, stream, MT, NT, D, sb);
  };
  auto run_ns = [&](int MT, int NT, int D) {
    return skinny_ns_dispatch(ctx, scheme, x, x_dtype, w, rb, m_out, k, n, y, y_dtype, stream, MT, NT, D, sb);
  };
  // The LDS-staged kernels (Q4_1, Q4_0, Q8_0, Q4_K, Q5_K; K whole 2-chunk
  // steps), MT 1, NT 2, 2-chunk steps, ring depth 1 (three waves per SIMD):
  // up to 16 x16 rows, and to 32 for Q4_1, Q4_0 and Q5_K, where they
  // measured faster than the register-streamed and N-split kernels (config-3
  // shapes at M = 16, bf16 x: Q4_1 gate_up 28.8 -> 23.0 us, down 22.9 ->
  // 20.2; Q4_K 36.8 -> 28.0 and 25.8 -> 21.0; Q5_K 45.0 -> 30.1 and 30.4 ->
  // 22.6; at 64 rows most were slower).  RLXQ_SKINNY_XL="MT,NT,SC,D" picks a
  // compiled one, "0" turns the default off, and a RLXQ_SKINNY_XR or
  // RLXQ_SKINNY_NS choice does too.
  {
    const bool fmt = xl_chunk_bytes(scheme) > 0;
    int lmt = 1, lnt = 2, lsc = 2, ld = 1;
    bool xl = fmt && (m <= 16 || (m <= 32 && (scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_GGUF_Q4_0 ||
                                              scheme == RLXQ_GGUF_Q5_K)));
    if (std::getenv("RLXQ_SKINNY_XR") || std::getenv("RLXQ_SKINNY_NS")) xl = false;
    if (const char* e = std::getenv("RLXQ_SKINNY_XL")) {
      int a1, a2, a3, a4;
      if (std::sscanf(e, "%d,%d,%d,%d", &a1, &a2, &a3, &a4) == 4 && fmt && a3 > 0) lmt = a1, lnt = a2, lsc = a3, ld = a4, xl = true;
      else if (e[0] == '0') xl = false;
    }
    if (xl && (k / 128) % lsc == 0)
      return skinny_xr_dispatch(ctx, scheme, x, x_dtype, w, rb, m_out, k, n, y, y_dtype, stream, lmt, lnt, ld, sb, lsc);
  }
  // The register-streamed kernels (no LDS stage).  RLXQ_SKINNY_XR="MT,NT,D"
  // picks a compiled one (every combination for Q4_1, the defaults for the
  // other formats).
  // The N-split kernel (activations shared through LDS): Q4_1 (and Q4_K) past 16 rows,
  // where it measured 5-13% faster than the register-streamed one (at 16 rows
  // and below, and for Q8_0, it was slower).  RLXQ_SKINNY_NS="MT,NT,D" picks
  // a compiled one for any scheme, "0" turns the default off.
  {
    const bool q6k = scheme == RLXQ_GGUF_Q6_K;
    int nmt = m <= 32 ? 2 : 4, nnt = 1, nd = q6k && m > 32 ? 2 : 3;
    bool ns = (scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_GGUF_Q4_K || q6k || mlx) && m > 16;
    if (const char* e = std::getenv("RLXQ_SKINNY_NS")) {
      int a1, a2, a3;
      if (std::sscanf(e, "%d,%d,%d", &a1, &a2, &a3) == 3) nmt = a1, nnt = a2, nd = a3, ns = true;
      else if (e[0] == '0') ns = false;
    }
    if (std::getenv("RLXQ_SKINNY_XR") && !std::getenv("RLXQ_SKINNY_NS")) ns = false;
    if (ns) return run_ns(nmt, nnt, nd);
  }
  int xmt = m <= 16 ? 1 : (m <= 32 ? 2 : 4), xnt = 2, xd = m <= 16 ? 4 : (m <= 32 ? 3 : 2);
  // ring depth by raw block size: Q4_K 13 dwords, Q2_K 11; Q6_K 22, Q5_K 21,
  // Q3_K 24 (Q8_K's 9 and the legacy blocks take the default)
  if (scheme == RLXQ_GGUF_Q4_K || scheme == RLXQ_GGUF_Q2_K) xd = m <= 16 ? 3 : 2;
  if (scheme == RLXQ_GGUF_Q6_K || scheme == RLXQ_GGUF_Q5_K || scheme == RLXQ_GGUF_Q3_K) xd = m <= 32 ? 2 : 1;
  if (const char* e = std::getenv("RLXQ_SKINNY_XR")) {
    int a1, a2, a3;
    if (std::sscanf(e, "%d,%d,%d", &a1, &a2, &a3) == 3) xmt = a1, xnt = a2, xd = a3;
  }
  return run_xr(xmt, xnt, xd);
}

}  // namespace rlxq
