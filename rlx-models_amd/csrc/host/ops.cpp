// Host-side dispatch of the dense GEMV, the dequantize check entry, SwiGLU,
// int8 activation quantisation and the MoE router.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "rlxq.h"
#include "rlxq_internal.hpp"
#include "gemv_args.h"
#include "gemm_args.h"

namespace rlxq {

namespace {

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

const char* scheme_name(int s) {
  switch (s) {
    case RLXQ_GGUF_Q8_0: return "q8_0";
    case RLXQ_GGUF_Q4_0: return "q4_0";
    case RLXQ_GGUF_Q4_1: return "q4_1";
    case RLXQ_MLX_AFFINE4: return "mlx4";
    case RLXQ_MLX_AFFINE8: return "mlx8";
    case RLXQ_GGUF_Q4_K: return "q4_k";
    case RLXQ_GGUF_Q6_K: return "q6_k";
    case RLXQ_MLX_MXFP4: return "mxfp4";
    case RLXQ_GGUF_Q5_K: return "q5_k";
    case RLXQ_GGUF_Q3_K: return "q3_k";
    case RLXQ_GGUF_Q2_K: return "q2_k";
    case RLXQ_GGUF_Q8_K: return "q8_k";
    default: return nullptr;
  }
}

namespace {

struct GemvCfg {
  int L, P, C, MT, D, W;
};

// Lanes per row: the candidate that leaves the fewest idle unit slots
// (ties to the wider group, which reads longer contiguous spans).
int pick_lanes(int64_t units, const int* cands, int ncand) {
  int best = cands[0];
  int64_t best_slots = -1;
  for (int i = 0; i < ncand; i++) {
    const int L = cands[i];
    const int64_t slots = (units + L - 1) / L * L;
    if (best_slots < 0 || slots < best_slots) {
      best = L;
      best_slots = slots;
    }
  }
  return best;
}

// Variant selection for the decode GEMV, from MI355X measurements.  For the
// single-row family, RLXQ_GEMV_CFG="L,P,C,D,W" overrides it (tuning sweeps and
// the per-variant parity test); a variant that was not compiled fails with
// RLXQ_E_NOKERNEL.
GemvCfg pick_gemv(int64_t m, int64_t units, int64_t lds_rec_bytes_m4, size_t max_lds, int scheme) {
  GemvCfg c;
  if (m >= 2 && lds_rec_bytes_m4 <= (int64_t)max_lds) {
    static const int c4[] = {64, 8};
    c = {pick_lanes(units, c4, 2), 2, 1, 4, 1, 8};
  } else {
    static const int c1[] = {64, 32, 16, 8};
    const int L = pick_lanes(units, c1, 4);
    // The K-quants' wide units (12 dwords for Q4_K, 21 for Q6_K) spill in the
    // two-chunk 16-wave variant with two steps in flight: Q4_K takes one
    // chunk with four steps in flight, Q6_K two chunks with one step (97
    // VGPRs; 30.6 us against 35.1 for the 8-wave two-step variant on
    // 4096->24576, 16.9 against 18.4 on 12288->4096).
    // The other K-quants, measured on 4096->24576 and 12288->4096: Q3_K, Q2_K
    // and Q8_K also run best on Q6_K's variant (Q3_K's 22-dword units spill
    // in the two-step one); Q5_K on two rows per wave of 8-wave workgroups
    // (28.8 against 38.1 us for gate_up).
    c = L != 64 ? GemvCfg{L, 2, 1, 1, 2, 8}
                : scheme == RLXQ_GGUF_Q4_K ? GemvCfg{64, 1, 1, 1, 4, 16}
                : scheme == RLXQ_GGUF_Q5_K ? GemvCfg{64, 2, 1, 1, 2, 8}
                : (scheme == RLXQ_GGUF_Q6_K || scheme == RLXQ_GGUF_Q3_K || scheme == RLXQ_GGUF_Q2_K ||
                   scheme == RLXQ_GGUF_Q8_K)
                    ? GemvCfg{64, 1, 2, 1, 1, 16}
                    : GemvCfg{64, 1, 2, 1, 2, 16};
  }
  const char* e = c.MT == 1 ? std::getenv("RLXQ_GEMV_CFG") : nullptr;
  if (e) {
    int L, P, C, D, W;
    if (std::sscanf(e, "%d,%d,%d,%d,%d", &L, &P, &C, &D, &W) == 5) c = {L, P, C, 1, D, W};
  }
  return c;
}

}  // namespace

// Validates a weight operand of a dense or grouped call and returns the
// packed row stride in bytes.
int check_weights(rlxq_ctx* ctx, const char* what, int scheme, int group, const void* w,
                  const void* scales, const void* biases, int sb_dtype, int64_t k, int64_t* rb) {
  if (k % 32) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": K must be a multiple of 32");
  if (scheme == RLXQ_GGUF_Q4_K) {
    if (k % 256) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": Q4_K needs K % 256 == 0 (super-blocks)");
    if (!aligned(w, 16)) return fail(ctx, RLXQ_E_ALIGN, std::string(what) + ": Q4_K rows must be 16-byte aligned");
    *rb = k / 256 * 144;
    return RLXQ_OK;
  }
  if (const int64_t sb = kquant_bytes(scheme); sb > 0) {
    // Q6_K, Q5_K, Q3_K, Q2_K, Q8_K (Q5_K's 176-byte super-blocks are read
    // with 16-byte loads; the others with dword-aligned ones)
    const char* nm = scheme_name(scheme);
    if (k % 256) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": " + nm + " needs K % 256 == 0 (super-blocks)");
    const uintptr_t al = scheme == RLXQ_GGUF_Q5_K ? 16 : 4;
    if (!aligned(w, al))
      return fail(ctx, RLXQ_E_ALIGN, std::string(what) + ": " + nm + " weights must be " + std::to_string(al) +
                                         "-byte aligned");
    *rb = k / 256 * sb;
    return RLXQ_OK;
  }
  if (is_gguf(scheme)) {
    if ((scheme == RLXQ_GGUF_Q8_0 || scheme == RLXQ_GGUF_Q4_0) && k % 64)
      return fail(ctx, RLXQ_E_ALIGN,
                  std::string(what) + ": Q8_0/Q4_0 need K % 64 == 0 (block pairs are read dword aligned)");
    if (!aligned(w, 4)) return fail(ctx, RLXQ_E_ALIGN, std::string(what) + ": w must be 4-byte aligned");
    *rb = k / 32 * gguf_block_bytes(scheme);
    return RLXQ_OK;
  }
  if (scheme == RLXQ_MLX_MXFP4) {
    // MlxMxfp4 (crates/rlx-models-core/src/mxfp4_pack.rs:16-50): codes [N, K/2],
    // one scale per 32 codes (E8M0 bytes, the dense op's U8 operand, or the
    // decoded bf16 the grouped op takes); no bias (biases are not read)
    if (group != 32) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": MXFP4 group_size must be 32");
    if (!scales) return fail(ctx, RLXQ_E_NULL, std::string(what) + ": MXFP4 needs scales");
    if (sb_dtype != RLXQ_U8 && sb_dtype != RLXQ_BF16)
      return fail(ctx, RLXQ_E_DTYPE, std::string(what) + ": MXFP4 scales are U8 (E8M0) or BF16");
    if (!aligned(w, 16)) return fail(ctx, RLXQ_E_ALIGN, std::string(what) + ": MXFP4 codes must be 16-byte aligned");
    *rb = k / 2;
    return RLXQ_OK;
  }
  if (is_mlx(scheme)) {
    if (group != 32 && group != 64 && group != 128)
      return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": MLX group_size must be 32, 64 or 128");
    if (k % group) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": K must be a multiple of group_size");
    if (!scales || !biases) return fail(ctx, RLXQ_E_NULL, std::string(what) + ": MLX needs scales and biases");
    if (sb_dtype != RLXQ_F32 && sb_dtype != RLXQ_BF16)
      return fail(ctx, RLXQ_E_DTYPE, std::string(what) + ": sb_dtype must be F32 or BF16");
    if (!aligned(w, 16)) return fail(ctx, RLXQ_E_ALIGN, std::string(what) + ": MLX codes must be 16-byte aligned");
    *rb = scheme == RLXQ_MLX_AFFINE4 ? k / 2 : k;
    return RLXQ_OK;
  }
  return fail(ctx, RLXQ_E_SCHEME, std::string(what) + ": unsupported scheme " + std::to_string(scheme));
}

// Schemes with the exact f32-output variant of the prefill GEMM (each
// weight's f32 value as f16 hi + lo, f16 MFMA on prepared activations):
// every format but MXFP4, whose E8M0-scaled codes are exact in bf16 and take
// the bf16 kernels.
bool has_exact_gemm(int scheme) { return scheme != RLXQ_MLX_MXFP4; }

// Prefill dequant-GEMM launch (tilings and split-K below).  f32 output or
// f32 activations take the exact variant; f32 activations are prepared as a
// hi and a lo f16 row per row (the epilogue adds the pair).
int gemm_dispatch(rlxq_ctx* ctx, int scheme, int group, const void* x, int x_dtype, const void* w,
                  const void* scales, const void* biases, int sb_dtype, int64_t rb, int64_t m, int64_t k, int64_t n,
                  void* y, int y_dtype, void* stream) {
  // 256 x 256 tiles, 8 waves, global loads two K steps ahead (one for Q6_K
  // and Q3_K, whose larger raw blocks do not fit two stages in 256 VGPRs;
  // Q6_K with its LDS stores after the step's MFMAs, which measured 15%
  // faster for it and slower for the others).  When the tiles do not cover the CUs, K is split so that they do
  // (at most 8 slices of at least 8 K steps) and the slices' f32 partial sums
  // are added in slice order.  RLXQ_GEMM_TILE=128|256|256w8|256w8l|256w8p2|...x|
  // 256n128|256n128w8 forces a tiling (the 128 x 128 one never splits);
  // RLXQ_GEMM_SPLITS=<n> forces the slice count.
  const int64_t cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  int tile = 256;
  const bool one_stage = scheme == RLXQ_GGUF_Q6_K || scheme == RLXQ_GGUF_Q3_K;
  const char* var = scheme == RLXQ_GGUF_Q6_K ? "w8l" : (one_stage ? "w8" : "w8p2");
  const char* te = std::getenv("RLXQ_GEMM_TILE");
  if (te) {
    tile = std::atoi(te) == 128 ? 128 : 256;
    var = tile == 128 ? "" : ((std::strncmp(te, "256w8", 5) == 0 || std::strncmp(te, "256n128", 7) == 0) ? te + 3 : "");
  }
  // f32 output or f32 activations: the exact variant (bf16 weights, or f16
  // weights rounded once, do not keep 1e-3 on structured data).  Its
  // register stages: one for the raw blocks of Q8_0, Q5_K, Q3_K, MLX 4-bit
  // (and Q6_K, late stores) and for Q4_1 and Q8_K with bf16 activations,
  // two for the others.
  const bool split = x_dtype == RLXQ_F32;
  const bool want_exact = split || y_dtype == RLXQ_F32;
  // (the "...xs" kernels take f32 activations as hi / lo x16 rows)
  std::string vs = var;
  if (!te && want_exact && has_exact_gemm(scheme))
    vs = scheme == RLXQ_GGUF_Q6_K ? "w8lx"
         : (scheme == RLXQ_GGUF_Q8_0 || scheme == RLXQ_GGUF_Q5_K || scheme == RLXQ_GGUF_Q3_K ||
            scheme == RLXQ_MLX_AFFINE4 ||
            // (Q4_1 and Q8_K: one stage for bf16 activations, two for f32)
            (!split && (scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_GGUF_Q8_K))) ? "w8x" : "w8p2x";
  if (split && !vs.empty() && vs.back() == 'x') vs += 's';
  const bool exact = vs.find('x') != std::string::npos;
  bool n128 = tile == 256 && vs.compare(0, 4, "n128") == 0;   // 256 x 128 tiles
  if (exact && !has_exact_gemm(scheme))
    return fail(ctx, RLXQ_E_SCHEME, "dequant_matmul: MXFP4 has no exact f16 GEMM variant");
  if (split && !(exact && vs.back() == 's'))
    return fail(ctx, RLXQ_E_DTYPE, "dequant_matmul: f32 activations need the exact GEMM variant");
  // x16 rows: 64-row blocks of 32 hi and 32 lo rows for f32 activations;
  // the exact variant's tiles cover 128 output columns (hi and lo weight
  // rows), and with f32 activations 128 output rows
  const int64_t mr = split ? (m + 31) / 32 * 64 : m;
  const int64_t tiles_m = (mr + tile - 1) / tile, ksteps = k / 64;
  if (tiles_m * ((n + 63) / 64) > 0x7ffffff0) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: too many GEMM tiles");
  auto auto_splits = [&](int64_t t) {
    int64_t s = 1;
    while (t * s * 2 <= cus && s < 8 && ksteps / (s * 2) >= 8) s *= 2;
    return s;
  };
  // bf16 variant: 256 x 128 tiles (8 waves) where the 256 x 256 tiles would
  // split K (half the slices and partial sums; 12288->4096 at M=512 76 -> 67
  // us, 4096->4096 at M=512 / 2048 43 -> 33 / 88 -> 75) or leave a partly
  // filled last round of workgroups that the narrower tiles fill (4096->24576
  // at M=1024: 384 vs 768 tiles on 256 CUs, 235 -> 221 us)
  if (!te && tile == 256 && !exact) {
    const int64_t t256 = tiles_m * ((n + 255) / 256), t128 = tiles_m * ((n + 127) / 128);
    if (auto_splits(t256) > 1 || 2 * ((t256 + cus - 1) / cus) > (t128 + cus - 1) / cus) {
      n128 = true;
      vs = "n128w8";
    }
  }
  const bool w8 = tile == 256 && vs.find("w8") != std::string::npos;
  const int64_t tn_cols = exact ? tile / 2 : (n128 ? 128 : tile);
  const int64_t tiles_n = (n + tn_cols - 1) / tn_cols, tiles = tiles_m * tiles_n;
  int64_t splits = 1;
  if (tile == 256) {
    splits = auto_splits(tiles);
    if (const char* e = std::getenv("RLXQ_GEMM_SPLITS")) splits = std::max<int64_t>(1, std::min<int64_t>(std::atoi(e), ksteps));
  }
  const int64_t kslice = ((ksteps + splits - 1) / splits) * 64;
  splits = (k + kslice - 1) / kslice;
  char name[64];
  std::snprintf(name, sizeof name, "rlxq_gemm_%s_t%d%s", scheme_name(scheme), tile, vs.c_str());
  hipFunction_t fn;
  int rc;
  if ((rc = get_fn(ctx, name, &fn))) return rc;
  rlxq_gemm_args a;
  std::memset(&a, 0, sizeof a);
  a.x = x;
  const size_t part_bytes = splits > 1 ? (((size_t)(splits * m * n) * 4 + 255) & ~(size_t)255) : 0;
  char* part = nullptr;
  if (exact) {
    // prepared f16 activations in natural order (the exact variant's weights
    // are in natural order); MLX's 2^8 weight factor undone in the row factors
    rlxq_x16_args xa;
    if ((rc = prep_x16(ctx, x, x_dtype, m, k, 0, part_bytes, xa, &part, stream, false, 0, false, split ? 2 : 0,
                       sk_post_exp(scheme))))
      return rc;
    a.x = xa.x16;
    a.inv_s = xa.inv_s;
  } else if (part_bytes) {
    void* ws = nullptr;
    if ((rc = workspace(ctx, part_bytes, &ws, stream))) return rc;
    part = static_cast<char*>(ws);
  }
  a.w = static_cast<const uint8_t*>(w);
  a.scales = scales;
  a.biases = biases;
  a.y = y;
  a.M = mr;
  a.m_out = m;
  a.pairs = split ? 1 : 0;
  a.N = n;
  a.K = k;
  a.rb = rb;
  a.y_ld = n;
  a.group = is_mlx(scheme) ? group : 32;
  a.sb_bf16 = sb_code(sb_dtype);
  a.y_bf16 = y_dtype == RLXQ_BF16 ? 1 : 0;
  a.tiles_m = (int32_t)tiles_m;
  a.tiles_n = (int32_t)tiles_n;
  a.part = splits > 1 ? reinterpret_cast<float*>(part) : nullptr;
  a.kslice = (int32_t)kslice;
  a.splits = (int32_t)splits;
  void* args[] = {&a};
  if (tile == 128) {
    const size_t lds = 2 * (128 + 128) * 72 * sizeof(uint16_t);
    return launch(ctx, fn, dim3((unsigned)tiles), dim3(256), lds, stream, args, name);
  }
  const size_t lds = 2 * (256 + (n128 ? 128 : 256)) * 72 * sizeof(uint16_t);
  const int64_t grid = 8 * ((tiles + 7) / 8) * splits;
  if ((rc = launch(ctx, fn, dim3((unsigned)grid), dim3(w8 ? 512 : 256), lds, stream, args, name))) return rc;
  if (splits > 1) {
    // slice partial sums, added in slice order (the batched-decode reduction)
    rlxq_skinny_args r;
    std::memset(&r, 0, sizeof r);
    r.part = a.part;
    r.y = y;
    r.M = m;
    r.N = n;
    r.y_ld = n;
    r.splits = (int32_t)splits;
    r.y_bf16 = a.y_bf16;
    rc = splits_reduce(ctx, r, stream);
    if (!rc) ctx->last_kernel = name;
  }
  return rc;
}

int gemv_dispatch(rlxq_ctx* ctx, int scheme, int group, const void* x, int x_dtype, const void* w,
                  const void* scales, const void* biases, int sb_dtype, int64_t m, int64_t k,
                  int64_t n, void* y, int y_dtype, void* stream) {
  if (scheme == RLXQ_INT8_BLOCK)
    return i8b_dispatch(ctx, group, x, x_dtype, w, scales, biases, sb_dtype, m, k, n, y, y_dtype, stream);
  int64_t rb = 0;
  int rc = check_weights(ctx, "dequant_matmul", scheme, group, w, scales, biases, sb_dtype, k, &rb);
  if (rc) return rc;
  if (!aligned(x, 16)) return fail(ctx, RLXQ_E_ALIGN, "dequant_matmul: x must be 16-byte aligned");
  if (k > (int64_t)1 << 30 || n > ((int64_t)1 << 40))
    return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: K or N too large");

  const bool xbf = x_dtype == RLXQ_BF16;
  const int blocks = (scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_GGUF_Q8_0 || scheme == RLXQ_GGUF_Q4_K ||
                      scheme == RLXQ_GGUF_Q5_K) ? 2 : 1;
  const int64_t units = (k / 32) / blocks;

  // Prefill routing.  bf16 activations and bf16 output from 64 rows: the
  // bf16 GEMM (weights rounded to bf16, the 2e-2 prefill bar).  f32 output
  // past 256 rows, or f32 activations (the reference's operand type) from 64
  // rows with bf16 output: the exact variant (f16 hi + lo weights; f32
  // activations as hi + lo rows).  MXFP4 with E8M0 scales and bf16
  // activations is exact on the bf16 GEMM for f32 output too; MXFP4 with f32
  // activations or bf16 scales stays on the GEMV for f32 output.
  // RLXQ_PREFILL=gemv|gemm forces one of them where both apply (tests).
  {
    const bool mx_exact_bf16 = scheme == RLXQ_MLX_MXFP4 && sb_dtype == RLXQ_U8 && xbf;
    const bool gemm_ok = k % 64 == 0 && (xbf || has_exact_gemm(scheme));
    bool use_gemm;
    if (xbf && y_dtype == RLXQ_BF16) use_gemm = m >= 64;
    else if (y_dtype == RLXQ_BF16) use_gemm = m >= 64;                 // f32 x: exact variant
    else use_gemm = m > 256 && (has_exact_gemm(scheme) || mx_exact_bf16);
    use_gemm = use_gemm && gemm_ok;
    if (const char* e = std::getenv("RLXQ_PREFILL")) {
      if (!std::strcmp(e, "gemv")) use_gemm = false;
      if (!std::strcmp(e, "gemm")) use_gemm = gemm_ok;
    }
    if (use_gemm)
      return gemm_dispatch(ctx, scheme, group, x, x_dtype, w, scales, biases, sb_dtype, rb, m, k, n, y, y_dtype,
                           stream);
  }
  // Batched decode: from 5 rows, GGUF and MLX affine 4/8-bit weights stream
  // once for all rows through the f16-MFMA kernel (MXFP4 with E8M0 scales
  // through its bf16-MFMA twin).  bf16 activations are exact in f16 once
  // scaled; f32 activations run as hi + lo row pairs (~22 significant bits).
  // RLXQ_DECODE=gemv|skinny forces one where both apply.
  {
    const bool sk_ok = skinny_applies(scheme, group, sb_dtype, m, k);
    bool use_sk = sk_ok && m >= 5;
    if (const char* e = std::getenv("RLXQ_DECODE")) {
      if (!std::strcmp(e, "gemv")) use_sk = false;
      if (!std::strcmp(e, "skinny")) use_sk = sk_ok;
    }
    if (use_sk) {
      SkinnySb sb;
      sb.scales = scales;
      sb.biases = biases;
      sb.group = is_mlx(scheme) ? group : 32;
      sb.sb_bf16 = sb_code(sb_dtype);
      return skinny_dispatch(ctx, scheme, x, x_dtype, w, rb, m, k, n, y, y_dtype, stream, sb);
    }
  }

  rlxq_gemv_args a;
  a.x = x;
  a.w = static_cast<const uint8_t*>(w);
  a.scales = scales;
  a.biases = biases;
  a.y = y;
  a.row_map = nullptr;
  a.row_scale = nullptr;
  a.M = m;
  a.N = n;
  a.rb = rb;
  a.y_ld = n;
  a.K = (int32_t)k;
  a.group = is_mlx(scheme) ? group : 32;
  a.sb_bf16 = sb_code(sb_dtype);
  a.y_bf16 = y_dtype == RLXQ_BF16 ? 1 : 0;
  void* args[] = {&a};
  char name[96];
  hipFunction_t fn;

  // Single activation row, bf16, 4-bit codes, at most 4 unit chunks of 64 per
  // row (6 for the one-block units): activations held in registers.  By
  // default they reach the registers through LDS, once per 8-wave workgroup
  // (the row of x then crosses L2 once per workgroup, not once per wave).
  // RLXQ_GEMV_XR="NU,D,W[,XS]" picks the variant (XS=1: through LDS), "0"
  // turns the path off (tuning).
  const bool q4k = scheme == RLXQ_GGUF_Q4_K;
  // (Q5_K: 64-weight units as Q4_K's, with the qh bytes beside the codes)
  const bool q5k = scheme == RLXQ_GGUF_Q5_K, u64 = q4k || q5k;
  // (Q2_K, Q3_K: a scale per 16 weights, two chains per block; their records
  // carry the first half's activation sum as well)
  const bool khalf = scheme == RLXQ_GGUF_Q2_K || scheme == RLXQ_GGUF_Q3_K;
  const bool xr_scheme = scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_MLX_AFFINE4 ||
                         scheme == RLXQ_MLX_MXFP4 || u64 || khalf;
  const int64_t nchunk64 = (units + 63) / 64;
  const int64_t xr_max = scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_GGUF_Q2_K ? 4
                         : (u64 || scheme == RLXQ_GGUF_Q3_K ? 3 : 6);
  // two chunks (K = 4096 for the one-block units): 4-wave workgroups with one
  // row in flight per wave measured 0.2-0.3 us faster on the small shapes
  const bool two = nchunk64 == 2 && !u64;
  // (Q5_K's 21-dword units: a one-deep ring from two chunks up)
  int xr_nu = (int)(nchunk64 == 5 ? 6 : nchunk64), xr_d = (two || nchunk64 > (q5k ? 1 : (u64 ? 2 : 3))) ? 1 : 2,
      xr_w = two ? 4 : 8;
  // (gate_up 4096 -> 24576: Q2_K 14.5 us one-deep, 16.0 two-deep, 16.8 on
  // the LDS-record kernel; Q3_K 25.9, 24.5, 26.8)
  if (khalf) xr_d = (nchunk64 <= 1 || (scheme == RLXQ_GGUF_Q3_K && nchunk64 == 2)) ? 2 : 1, xr_w = 8;
  bool use_xr = m == 1 && xbf && xr_scheme && nchunk64 <= xr_max && n < (int64_t(1) << 31);
  int xr_lds = 1;   // 1: the activations pass through LDS once per workgroup
  // The K-split register kernels (KS waves per weight row, their row sums
  // added in part order in LDS; Q4_1): grid and LDS (activation records,
  // then [W / KS][rows per wave][KS] partial sums).
  auto launch_ks = [&](int nu, int d, int wv, int ks, bool f32x) -> int {
    std::snprintf(name, sizeof name, "rlxq_gemvxs_%s_U%d_D%d_W%d%s_K%d", scheme_name(scheme), nu, d, wv,
                  f32x ? "_F" : "", ks);
    int rc2;
    if ((rc2 = get_fn(ctx, name, &fn))) return rc2;
    const int rw = wv / ks;
    const size_t lds0 = (f32x ? 2 : 1) * (size_t)(k / 32) * 68;
    int per_cu = blocks_per_cu(ctx, name, fn, 64 * wv, lds0 + 1024);
    int64_t gx = std::min<int64_t>((int64_t)ctx->cu_count * std::max(per_cu, 1), (n + rw - 1) / rw);
    size_t part = (size_t)rw * ((n + gx * rw - 1) / (gx * rw)) * ks * 4;
    if (part > 1024) {
      per_cu = blocks_per_cu(ctx, name, fn, 64 * wv, lds0 + part);
      gx = std::min<int64_t>((int64_t)ctx->cu_count * std::max(per_cu, 1), (n + rw - 1) / rw);
      part = (size_t)rw * ((n + gx * rw - 1) / (gx * rw)) * ks * 4;
    }
    if (lds0 + part > ctx->max_lds) return 1;   // (not applicable: the caller goes on)
    return launch(ctx, fn, dim3((unsigned)gx, 1, 1), dim3(64 * wv, 1, 1), lds0 + part, stream, args, name);
  };
  // RLXQ_GEMV_XSK="NU,D,W,KS" (bf16) / RLXQ_GEMV_XSFK (f32 activations)
  // picks a K-split variant for one Q4_1 row whose K fits NU * KS unit
  // chunks (tuning).
  if (m == 1 && scheme == RLXQ_GGUF_Q4_1 && n < (int64_t(1) << 31)) {
    if (const char* e = std::getenv(xbf ? "RLXQ_GEMV_XSK" : "RLXQ_GEMV_XSFK")) {
      int nu, d, wv, ks;
      if (std::sscanf(e, "%d,%d,%d,%d", &nu, &d, &wv, &ks) == 4 && nchunk64 <= (int64_t)nu * ks) {
        const int r = launch_ks(nu, d, wv, ks, !xbf);
        if (r <= 0) return r;
      }
    }
  }
  // One row of f32 activations on Q4_1 with many rows at K = 4096 (gate_up:
  // 14.5 against 15.3 us) or K past four unit chunks (down, K = 12288: 10.3
  // against 10.6 us on the LDS-record kernel): the two-wave K split.  (bf16
  // activations measured no gain from it: down 8.0-8.5 us two-way and
  // 8.3-8.8 four-way against 8.1 on one wave per row.)
  if (m == 1 && !xbf && scheme == RLXQ_GGUF_Q4_1 && n < (int64_t(1) << 31) &&
      !(std::getenv("RLXQ_GEMV_XR") && std::getenv("RLXQ_GEMV_XR")[0] == '0')) {
    int r = 1;
    if (nchunk64 == 2 && n >= 16384) r = launch_ks(1, 2, 8, 2, true);
    else if (nchunk64 > 4 && nchunk64 <= 6) r = launch_ks(3, 1, 8, 2, true);
    if (r <= 0) return r;
  }
  // One row of f32 activations: the two-row kernel on its hi and lo bf16
  // rows (Q4_1, MLX 4-bit, MXFP4 up to four unit chunks, Q4_K up to two),
  // both rows' sums added into the one output.  RLXQ_GEMV_XR=0 turns it off.
  {
    const char* e = std::getenv("RLXQ_GEMV_XR");
    const bool one_block4 = scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_MLX_AFFINE4 || scheme == RLXQ_MLX_MXFP4;
    if (m == 1 && !xbf && (one_block4 || q4k) && nchunk64 <= (q4k ? 2 : 4) && n < (int64_t(1) << 31) &&
        !(e && e[0] == '0')) {
      // (8-wave workgroups: every workgroup stages the whole f32 row of x,
      // 16 KB at K = 4096, so fewer, wider workgroups read it fewer times:
      // o 6.3-6.5 -> 5.1 us, qkv 7.0 -> 6.0 against 4-wave ones)
      const int nu = (int)nchunk64;
      int d = nu <= 2 ? 2 : 1, wv = 8;
      if (q4k) d = nu == 1 ? 2 : 1, wv = 8;
      if (const char* t = std::getenv("RLXQ_GEMV_XSF")) std::sscanf(t, "%d,%d", &d, &wv);   // "D,W" (tuning)
      std::snprintf(name, sizeof name, "rlxq_gemvxs_%s_U%d_D%d_W%d_F", scheme_name(scheme), nu, d, wv);
      if ((rc = get_fn(ctx, name, &fn))) return rc;
      const size_t lds = 2 * (size_t)(k / 32) * 68;
      if (lds <= ctx->max_lds) {
        const int per_cu = blocks_per_cu(ctx, name, fn, 64 * wv, lds);
        int64_t gx = (int64_t)ctx->cu_count * per_cu;
        gx = std::min<int64_t>(gx, (n + wv - 1) / wv);
        return launch(ctx, fn, dim3((unsigned)gx, 1, 1), dim3(64 * wv, 1, 1), lds, stream, args, name);
      }
    }
  }
  if (const char* e = std::getenv("RLXQ_GEMV_XR")) {
    int nu, d, wv, xs = 0;
    if (std::sscanf(e, "%d,%d,%d,%d", &nu, &d, &wv, &xs) >= 3) {
      xr_d = d;
      xr_w = wv;
      xr_lds = xs;
      if (nu < xr_nu) use_xr = false;
      else xr_nu = nu;
    } else if (e[0] == '0') {
      use_xr = false;
    }
  }
  if (use_xr) {
    std::snprintf(name, sizeof name, "rlxq_gemvx%s_%s_U%d_D%d_W%d", xr_lds ? "s" : "r", scheme_name(scheme), xr_nu,
                  xr_d, xr_w);
    if ((rc = get_fn(ctx, name, &fn))) return rc;
    // pair records + block sums (+ the first halves' sums)
    const size_t lds = xr_lds ? (size_t)(k / 32) * (khalf ? 72 : 68) : 0;
    const int per_cu = blocks_per_cu(ctx, name, fn, 64 * xr_w, lds);
    const int64_t wgs_needed = (n + xr_w - 1) / xr_w;
    int64_t gx = (int64_t)ctx->cu_count * per_cu;
    if (gx > wgs_needed) gx = wgs_needed;
    return launch(ctx, fn, dim3((unsigned)gx, 1, 1), dim3(64 * xr_w, 1, 1), lds, stream, args, name);
  }

  // Two to four activation rows (bf16; Q4_1, MLX 4-bit, MXFP4, Q4_K): the
  // same register kernel with
  // the rows' activations side by side in registers (MT = 2 or 4 rows, at
  // most 8 units of activations per lane), so every weight row is fetched
  // once for all of them.  RLXQ_GEMV_XR=0 turns it off as well.
  {
    const char* e = std::getenv("RLXQ_GEMV_XR");
    const int mt = m <= 2 ? 2 : 4;
    const bool one_block4 = scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_MLX_AFFINE4 || scheme == RLXQ_MLX_MXFP4;
    // Q4_K's 64-weight units hold twice the activations: NU * MT <= 4
    const int64_t max_nu = q4k ? (mt == 2 ? 2 : 1) : (mt == 2 ? 4 : 2);
    if (m >= 2 && m <= 4 && xbf && (one_block4 || q4k) && n < (int64_t(1) << 31) && !(e && e[0] == '0') &&
        nchunk64 <= max_nu) {
      // (two steps in flight up to two chunks; 4-wave groups for two rows at
      // K = 4096: gate_up 15.5 us at M = 2, 23.4 at M = 4 on 8 waves)
      const int nu = (int)nchunk64;
      int d = nu <= 2 ? 2 : 1, wv = (nu == 2 && mt == 2) ? 4 : 8;
      if (q4k) d = nu == 1 ? 2 : 1, wv = 8;
      if (const char* t = std::getenv("RLXQ_GEMV_XSM")) std::sscanf(t, "%d,%d", &d, &wv);   // "D,W" (tuning)
      std::snprintf(name, sizeof name, "rlxq_gemvxs_%s_U%d_D%d_W%d_M%d", scheme_name(scheme), nu, d, wv, mt);
      if ((rc = get_fn(ctx, name, &fn))) return rc;
      const size_t lds = (size_t)mt * (k / 32) * 68;
      if (lds <= ctx->max_lds) {
        const int per_cu = blocks_per_cu(ctx, name, fn, 64 * wv, lds);
        int64_t gx = (int64_t)ctx->cu_count * per_cu;
        gx = std::min<int64_t>(gx, (n + wv - 1) / wv);
        return launch(ctx, fn, dim3((unsigned)gx, 1, 1), dim3(64 * wv, 1, 1), lds, stream, args, name);
      }
    }
  }

  const int64_t rec_bytes = (xbf ? 20 : 36) * 4;
  const int64_t bpr = k / 32;
  const GemvCfg cfg = pick_gemv(m, units, 4 * bpr * rec_bytes, ctx->max_lds, scheme);
  const int waves = cfg.W;
  const int64_t tile = (int64_t)waves * cfg.P * (64 / cfg.L);
  const int64_t lds = cfg.MT * bpr * rec_bytes;
  if (lds > (int64_t)ctx->max_lds)
    return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: K too large for the LDS activation stage");

  std::snprintf(name, sizeof name, "rlxq_gemv_%s_%s_L%d_P%d_C%d_M%d_D%d_W%d", scheme_name(scheme),
                xbf ? "bf16" : "f32", cfg.L, cfg.P, cfg.C, cfg.MT, cfg.D, cfg.W);
  if ((rc = get_fn(ctx, name, &fn))) return rc;

  // Persistent grid: as many workgroups as the device holds at once, with the
  // row tiles spread evenly over them.
  const int per_cu = blocks_per_cu(ctx, name, fn, 64 * waves, (size_t)lds);
  const int64_t ntiles = (n + tile - 1) / tile;
  const int64_t maxgrid = (int64_t)ctx->cu_count * per_cu;
  const int64_t tpw = (ntiles + maxgrid - 1) / maxgrid;
  const int64_t gx = (ntiles + tpw - 1) / tpw;
  const int64_t gy = (m + cfg.MT - 1) / cfg.MT;
  if (gx > 0x7fffffff || gy > 65535) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: grid too large");
  return launch(ctx, fn, dim3((unsigned)gx, (unsigned)gy, 1), dim3(64 * waves, 1, 1), (size_t)lds, stream, args,
                name);
}

}  // namespace rlxq

using namespace rlxq;

extern "C" {

int rlxq_dequantize(rlxq_ctx* ctx, int scheme, int group_size, const void* w, const void* scales,
                    const void* biases, int sb_dtype, int64_t rows, int64_t k, float* out, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!w || !out) return fail(ctx, RLXQ_E_NULL, "dequantize: w and out must be non-null");
  if (rows < 0 || k <= 0) return fail(ctx, RLXQ_E_SHAPE, "dequantize: need rows >= 0, k > 0");
  int64_t rb = 0;
  int rc = check_weights(ctx, "dequantize", scheme, group_size, w, scales, biases, sb_dtype, k, &rb);
  if (rc) return rc;
  if (rows == 0) return RLXQ_OK;
  DeviceGuard g(ctx->device);
  hipFunction_t fn;
  if ((rc = get_fn(ctx, "rlxq_dequant_rows", &fn))) return rc;
  int sch = scheme, sb = sb_code(sb_dtype), grp = is_mlx(scheme) ? group_size : 32, K = (int)k;
  int64_t R = rows, RB = rb;
  void* args[] = {&sch, (void*)&w, (void*)&scales, (void*)&biases, &sb, &grp, &R, &K, &RB, (void*)&out};
  const int64_t quarters = rows * (k / 32) * 4;   // one thread per 8 weights
  if ((quarters + 255) / 256 > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, "dequantize: too many weights");
  return launch(ctx, fn, dim3((unsigned)((quarters + 255) / 256)), dim3(256), 0, stream, args, "dequantize");
}

int rlxq_swiglu(rlxq_ctx* ctx, const void* gu, int gu_dtype, int64_t rows, int64_t inter, void* out,
                int out_dtype, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!gu || !out) return fail(ctx, RLXQ_E_NULL, "swiglu: null pointer");
  if (rows < 0 || inter < 0) return fail(ctx, RLXQ_E_SHAPE, "swiglu: negative size");
  if ((gu_dtype != RLXQ_F32 && gu_dtype != RLXQ_BF16) || (out_dtype != RLXQ_F32 && out_dtype != RLXQ_BF16))
    return fail(ctx, RLXQ_E_DTYPE, "swiglu: dtype");
  if (rows == 0 || inter == 0) return RLXQ_OK;
  DeviceGuard g(ctx->device);
  hipFunction_t fn;
  int rc;
  if ((rc = get_fn(ctx, "rlxq_swiglu_k", &fn))) return rc;
  int gb = gu_dtype == RLXQ_BF16, ob = out_dtype == RLXQ_BF16;
  int64_t R = rows, I = inter;
  void* args[] = {(void*)&gu, &gb, &R, &I, &out, &ob};
  const int64_t total = rows * inter;
  return launch(ctx, fn, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, args, "swiglu");
}

int rlxq_quantize_act_int8(rlxq_ctx* ctx, const void* x, int x_dtype, int64_t m, int64_t k, int8_t* q,
                           float* scales, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!x || !q || !scales) return fail(ctx, RLXQ_E_NULL, "quantize_act_int8: null pointer");
  if (m < 0 || k <= 0 || k > (1 << 30) || m > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, "quantize_act_int8: shape");
  if (x_dtype != RLXQ_F32 && x_dtype != RLXQ_BF16) return fail(ctx, RLXQ_E_DTYPE, "quantize_act_int8: x_dtype");
  if (m == 0) return RLXQ_OK;
  DeviceGuard g(ctx->device);
  hipFunction_t fn;
  int rc;
  if ((rc = get_fn(ctx, "rlxq_quant_act_i8", &fn))) return rc;
  int xb = x_dtype == RLXQ_BF16, K = (int)k;
  // 16-element vector chunks need 16-byte aligned rows of x and q
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  int vec = (k % 16 == 0 && a16(x) && a16(q)) ? 1 : 0;
  int64_t M = m;
  void* args[] = {(void*)&x, &xb, &M, &K, (void*)&q, (void*)&scales, &vec};
  return launch(ctx, fn, dim3((unsigned)m), dim3(256), 0, stream, args, "quantize_act_int8");
}

int rlxq_moe_route(rlxq_ctx* ctx, const float* logits, int64_t rows, int64_t num_experts, int64_t top_k,
                   int renorm, int32_t* ids, float* probs, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!logits || !ids || !probs) return fail(ctx, RLXQ_E_NULL, "moe_route: null pointer");
  if (rows < 0 || num_experts <= 0 || num_experts > 1024 || top_k <= 0 || top_k > num_experts || top_k > 64 ||
      rows > 0x7fffffff)
    return fail(ctx, RLXQ_E_SHAPE, "moe_route: need 0 < top_k <= min(num_experts, 64), num_experts <= 1024");
  if (rows == 0) return RLXQ_OK;
  DeviceGuard g(ctx->device);
  hipFunction_t fn;
  int rc;
  // register slots per lane: the smallest compiled count covering E
  const int nper = num_experts <= 64 ? 1 : num_experts <= 128 ? 2 : num_experts <= 256 ? 4 : num_experts <= 512 ? 8 : 16;
  char name[32];
  std::snprintf(name, sizeof name, "rlxq_moe_route_k%d", nper);
  if ((rc = get_fn(ctx, name, &fn))) return rc;
  int64_t R = rows;
  int E = (int)num_experts, K = (int)top_k, rn = renorm ? 1 : 0;
  void* args[] = {(void*)&logits, &R, &E, &K, &rn, (void*)&ids, (void*)&probs};
  return launch(ctx, fn, dim3((unsigned)rows), dim3(64), 0, stream, args, name);
}

int rlxq_peak_probe(rlxq_ctx* ctx, int kind, const void* buf, int64_t work, void* sink, int64_t* count,
                    void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!sink || !count) return fail(ctx, RLXQ_E_NULL, "peak_probe: sink and count must be non-null");
  if (work <= 0) return fail(ctx, RLXQ_E_SHAPE, "peak_probe: work must be positive");
  DeviceGuard g(ctx->device);
  const int64_t grid = (int64_t)(ctx->cu_count > 0 ? ctx->cu_count : 256) * 8;
  hipFunction_t fn;
  int rc;
  if (kind == RLXQ_PROBE_MFMA) {
    if ((rc = get_fn(ctx, "rlxq_probe_mfma", &fn))) return rc;
    int64_t iters = work;
    void* args[] = {&iters, &sink};
    *count = grid * 4 * iters * 4 * 32768;
    return launch(ctx, fn, dim3((unsigned)grid), dim3(256), 0, stream, args, "rlxq_probe_mfma");
  }
  if (kind == RLXQ_PROBE_READ) {
    if (!buf) return fail(ctx, RLXQ_E_NULL, "peak_probe: buf must be non-null");
    if (work % 4096 || !aligned(buf, 16)) return fail(ctx, RLXQ_E_ALIGN, "peak_probe: buf 16-byte aligned, 4 KiB multiple");
    if ((rc = get_fn(ctx, "rlxq_probe_read", &fn))) return rc;
    int64_t n16 = work / 16;
    void* args[] = {(void*)&buf, &n16, &sink};
    *count = work;
    return launch(ctx, fn, dim3((unsigned)grid), dim3(256), 0, stream, args, "rlxq_probe_read");
  }
  if (kind == RLXQ_PROBE_READ4) {
    if (!buf) return fail(ctx, RLXQ_E_NULL, "peak_probe: buf must be non-null");
    if (work % 4096 || !aligned(buf, 16)) return fail(ctx, RLXQ_E_ALIGN, "peak_probe: buf 16-byte aligned, 4 KiB multiple");
    if (work > ((int64_t)1 << 30)) return fail(ctx, RLXQ_E_SHAPE, "peak_probe: READ4 reads at most 1 GiB");
    if ((rc = get_fn(ctx, "rlxq_probe_read4", &fn))) return rc;
    int64_t n16 = work / 16;
    void* args[] = {(void*)&buf, &n16, &sink};
    *count = work;
    return launch(ctx, fn, dim3((unsigned)((n16 + 1023) / 1024)), dim3(256), 0, stream, args, "rlxq_probe_read4");
  }
  if (kind == RLXQ_PROBE_TILE20) {
    if (!buf) return fail(ctx, RLXQ_E_NULL, "peak_probe: buf must be non-null");
    if (work % 81920 || !aligned(buf, 16)) return fail(ctx, RLXQ_E_ALIGN, "peak_probe: buf 16-byte aligned, 80 KiB multiple");
    if (work / 81920 > 65536) return fail(ctx, RLXQ_E_SHAPE, "peak_probe: TILE20 reads at most 65536 x 80 KiB");
    if ((rc = get_fn(ctx, "rlxq_probe_tile20", &fn))) return rc;
    void* args[] = {(void*)&buf, &sink};
    *count = work;
    return launch(ctx, fn, dim3((unsigned)(work / 81920)), dim3(256), 0, stream, args, "rlxq_probe_tile20");
  }
  return fail(ctx, RLXQ_E_SHAPE, "peak_probe: unknown kind");
}

}  // extern "C"
