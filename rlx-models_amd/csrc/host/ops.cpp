// Host-side dispatch of the dense GEMV, the dequantize check entry, SwiGLU,
// int8 activation quantisation and the MoE router.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "rlxq.h"
#include "rlxq_internal.hpp"

namespace rlxq {

namespace {

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

const char* scheme_name(int s) {
  switch (s) {
    case RLXQ_GGUF_Q8_0: return "q8_0";
    case RLXQ_GGUF_Q4_0: return "q4_0";
    case RLXQ_GGUF_Q4_1: return "q4_1";
    case RLXQ_MLX_AFFINE4: return "mlx4";
    case RLXQ_MLX_AFFINE8: return "mlx8";
    default: return nullptr;
  }
}

struct GemvCfg {
  int L, P, C, MT;
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

}  // namespace

// Validates a weight operand of a dense or grouped call and returns the
// packed row stride in bytes.
int check_weights(rlxq_ctx* ctx, const char* what, int scheme, int group, const void* w,
                  const void* scales, const void* biases, int sb_dtype, int64_t k, int64_t* rb) {
  if (k % 32) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": K must be a multiple of 32");
  if (is_gguf(scheme)) {
    if ((scheme == RLXQ_GGUF_Q8_0 || scheme == RLXQ_GGUF_Q4_0) && k % 64)
      return fail(ctx, RLXQ_E_ALIGN,
                  std::string(what) + ": Q8_0/Q4_0 need K % 64 == 0 (block pairs are read dword aligned)");
    if (!aligned(w, 4)) return fail(ctx, RLXQ_E_ALIGN, std::string(what) + ": w must be 4-byte aligned");
    *rb = k / 32 * gguf_block_bytes(scheme);
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

int gemv_dispatch(rlxq_ctx* ctx, int scheme, int group, const void* x, int x_dtype, const void* w,
                  const void* scales, const void* biases, int sb_dtype, int64_t m, int64_t k,
                  int64_t n, void* y, int y_dtype, void* stream) {
  if (scheme == RLXQ_INT8_BLOCK)
    return fail(ctx, RLXQ_E_NOKERNEL, "dequant_matmul: Int8Block is served by a later kernel");
  int64_t rb = 0;
  int rc = check_weights(ctx, "dequant_matmul", scheme, group, w, scales, biases, sb_dtype, k, &rb);
  if (rc) return rc;
  if (!aligned(x, 16)) return fail(ctx, RLXQ_E_ALIGN, "dequant_matmul: x must be 16-byte aligned");
  if (k > (int64_t)1 << 30 || n > ((int64_t)1 << 40))
    return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: K or N too large");

  const bool xbf = x_dtype == RLXQ_BF16;
  const int blocks = (scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_GGUF_Q8_0) ? 2 : 1;
  const int64_t units = (k / 32) / blocks;
  const int64_t rec_bytes = (xbf ? 20 : 36) * 4;
  const int64_t bpr = k / 32;

  GemvCfg cfg;
  if (m >= 2 && 4 * bpr * rec_bytes <= (int64_t)ctx->max_lds) {
    static const int c4[] = {64, 8};
    cfg = {pick_lanes(units, c4, 2), 2, 2, 4};
  } else {
    static const int c1[] = {64, 16, 8};
    const int L = pick_lanes(units, c1, 3);
    if (L == 64 && (units + 63) / 64 > 2) cfg = {64, 2, 3, 1};
    else cfg = {L, 4, 2, 1};
  }
  const int64_t lds = cfg.MT * bpr * rec_bytes;
  if (lds > (int64_t)ctx->max_lds)
    return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: K too large for the LDS activation stage");

  char name[96];
  std::snprintf(name, sizeof name, "rlxq_gemv_%s_%s_L%d_P%d_C%d_M%d", scheme_name(scheme),
                xbf ? "bf16" : "f32", cfg.L, cfg.P, cfg.C, cfg.MT);
  hipFunction_t fn;
  if ((rc = get_fn(ctx, name, &fn))) return rc;

  const int waves = 4;
  const int64_t rows_per_wg = (int64_t)waves * cfg.P * (64 / cfg.L);
  const int64_t gx = (n + rows_per_wg - 1) / rows_per_wg;
  const int64_t gy = (m + cfg.MT - 1) / cfg.MT;
  if (gx > 0x7fffffff || gy > 65535) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: grid too large");

  int sb_bf16 = sb_dtype == RLXQ_BF16 ? 1 : 0;
  int grp = is_mlx(scheme) ? group : 32;
  int y_bf16 = y_dtype == RLXQ_BF16 ? 1 : 0;
  int64_t M = m, N = n, RB = rb, YLD = n;
  int K = (int)k;
  const int32_t* row_map = nullptr;
  const float* row_scale = nullptr;
  void* args[] = {(void*)&x,   (void*)&w,      (void*)&scales, (void*)&biases,   (void*)&sb_bf16,
                  (void*)&grp, (void*)&y,      (void*)&y_bf16, (void*)&M,        (void*)&K,
                  (void*)&N,   (void*)&RB,     (void*)&row_map, (void*)&row_scale, (void*)&YLD};
  return launch(ctx, fn, dim3((unsigned)gx, (unsigned)gy, 1), dim3(64 * waves, 1, 1), (size_t)lds, stream,
                args, name);
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
  int sch = scheme, sb = sb_dtype == RLXQ_BF16, grp = is_mlx(scheme) ? group_size : 32, K = (int)k;
  int64_t R = rows, RB = rb;
  void* args[] = {&sch, (void*)&w, (void*)&scales, (void*)&biases, &sb, &grp, &R, &K, &RB, (void*)&out};
  const int64_t blocks = rows * (k / 32);
  return launch(ctx, fn, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, stream, args, "dequantize");
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
  int64_t M = m;
  void* args[] = {(void*)&x, &xb, &M, &K, (void*)&q, (void*)&scales};
  return launch(ctx, fn, dim3((unsigned)m), dim3(256), 0, stream, args, "quantize_act_int8");
}

int rlxq_moe_route(rlxq_ctx* ctx, const float* logits, int64_t rows, int64_t num_experts, int64_t top_k,
                   int renorm, int32_t* ids, float* probs, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!logits || !ids || !probs) return fail(ctx, RLXQ_E_NULL, "moe_route: null pointer");
  if (rows < 0 || num_experts <= 0 || num_experts > 1024 || top_k <= 0 || top_k > num_experts ||
      rows > 0x7fffffff)
    return fail(ctx, RLXQ_E_SHAPE, "moe_route: need 0 < top_k <= num_experts <= 1024");
  if (rows == 0) return RLXQ_OK;
  DeviceGuard g(ctx->device);
  hipFunction_t fn;
  int rc;
  if ((rc = get_fn(ctx, "rlxq_moe_route_k", &fn))) return rc;
  int64_t R = rows;
  int E = (int)num_experts, K = (int)top_k, rn = renorm ? 1 : 0;
  void* args[] = {(void*)&logits, &R, &E, &K, &rn, (void*)&ids, (void*)&probs};
  return launch(ctx, fn, dim3((unsigned)rows), dim3(64), 0, stream, args, "moe_route");
}

int rlxq_dequant_grouped_matmul(rlxq_ctx* ctx, int, int, const void*, int, const void*, const void*,
                                const void*, int, const float*, int64_t, int64_t, int64_t, int64_t, void*,
                                int, void*) {
  if (!ctx) return RLXQ_E_NULL;
  return fail(ctx, RLXQ_E_NOKERNEL, "dequant_grouped_matmul: not built yet");
}

int rlxq_moe_grouped(rlxq_ctx* ctx, int, int, const void*, int, const void*, const int32_t*, const float*,
                     int64_t, int64_t, int64_t, int64_t, int64_t, void*, int, void*) {
  if (!ctx) return RLXQ_E_NULL;
  return fail(ctx, RLXQ_E_NOKERNEL, "moe_grouped: not built yet");
}

int rlxq_w8a8_gemm(rlxq_ctx* ctx, const void*, int, const int8_t*, const float*, int64_t, int64_t, int64_t,
                   void*, int, void*) {
  if (!ctx) return RLXQ_E_NULL;
  return fail(ctx, RLXQ_E_NOKERNEL, "w8a8_gemm: not built yet");
}

}  // extern "C"
