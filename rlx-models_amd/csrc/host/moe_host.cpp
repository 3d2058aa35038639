// Host side of the grouped-expert entry points: rlxq_dequant_grouped_matmul
// and rlxq_moe_grouped.  Both build the device routing table from the expert
// indices, then run the grouped GEMV over the fired experts.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "moe_args.h"
#include "rlxq.h"
#include "rlxq_internal.hpp"

namespace rlxq {

namespace {

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Table + grouped GEMV (+ combine).  `ids` (int32) or `idx` (f32) give the
// expert of each of the n entries; entry i reads activation row i / x_div.
int grouped_run(rlxq_ctx* ctx, const char* what, int scheme, int group, const void* x, int x_dtype,
                const void* bank, const void* scales, const void* biases, int sb_dtype, const int32_t* ids,
                const float* idx, int64_t n_entries, int64_t x_rows, int32_t x_div, int64_t k, int64_t n,
                int64_t num_experts, void* y, int y_dtype, const float* probs, int64_t rows, int32_t top_k,
                void* stream) {
  if (!x || !bank || !y || (!ids && !idx)) return fail(ctx, RLXQ_E_NULL, std::string(what) + ": null pointer");
  if (k <= 0 || n < 0 || n_entries < 0 || x_rows < 0) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": bad sizes");
  if (num_experts <= 0 || num_experts > 1024)
    return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": need 0 < num_experts <= 1024");
  if (n_entries > ((int64_t)1 << 28)) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": too many rows");
  if (x_dtype != RLXQ_F32 && x_dtype != RLXQ_BF16) return fail(ctx, RLXQ_E_DTYPE, std::string(what) + ": x_dtype");
  if (y_dtype != RLXQ_F32 && y_dtype != RLXQ_BF16) return fail(ctx, RLXQ_E_DTYPE, std::string(what) + ": y_dtype");
  int64_t rb = 0;
  int rc = check_weights(ctx, what, scheme, group, bank, scales, biases, sb_dtype, k, &rb);
  if (rc) return rc;
  if (!aligned(x, 16)) return fail(ctx, RLXQ_E_ALIGN, std::string(what) + ": x must be 16-byte aligned");
  if (n_entries == 0 || n == 0) return RLXQ_OK;
  DeviceGuard g(ctx->device);
  if (!g.ok()) return fail(ctx, RLXQ_E_HIP, std::string(what) + ": hipSetDevice");

  const bool combine = probs != nullptr;
  const size_t table_bytes = ((size_t)(2 + 2 * num_experts + n_entries) * 4 + 255) & ~size_t(255);
  const size_t tmp_bytes = combine ? (size_t)n_entries * n * 4 : 0;
  void* ws = nullptr;
  if ((rc = workspace(ctx, table_bytes + tmp_bytes, &ws))) return rc;
  int32_t* table = static_cast<int32_t*>(ws);
  float* tmp = combine ? reinterpret_cast<float*>(static_cast<char*>(ws) + table_bytes) : nullptr;

  // 1. routing table
  hipFunction_t ft;
  if ((rc = get_fn(ctx, "rlxq_moe_table_k", &ft))) return rc;
  rlxq_moe_table_args ta;
  ta.ids = ids;
  ta.idx_f32 = idx;
  ta.table = table;
  ta.zero_rows = combine ? static_cast<void*>(tmp) : y;
  ta.n = n_entries;
  ta.N = n;
  ta.zero_ld = n;
  ta.E = (int32_t)num_experts;
  ta.zero_bf16 = (!combine && y_dtype == RLXQ_BF16) ? 1 : 0;
  void* targs[] = {&ta};
  if ((rc = launch(ctx, ft, dim3(1), dim3(1024), 0, stream, targs, "rlxq_moe_table_k"))) return rc;

  // 2. grouped GEMV over (fired expert, 32-row tile)
  const int blocks = (scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_GGUF_Q8_0) ? 2 : 1;
  const int64_t units = (k / 32) / blocks;
  const int L = units >= 48 ? 64 : 8;
  const int MT = 2;
  const bool xbf = x_dtype == RLXQ_BF16;
  char name[80];
  std::snprintf(name, sizeof name, "rlxq_moe_gemv_%s_%s_L%d_M%d", scheme_name(scheme), xbf ? "bf16" : "f32", L, MT);
  hipFunction_t fg;
  if ((rc = get_fn(ctx, name, &fg))) return rc;
  rlxq_moe_gemv_args ga;
  ga.x = x;
  ga.bank = static_cast<const uint8_t*>(bank);
  ga.scales = scales;
  ga.biases = biases;
  ga.table = table;
  ga.y = combine ? static_cast<void*>(tmp) : y;
  ga.N = n;
  ga.rb = rb;
  ga.y_ld = n;
  ga.x_ld = k;
  ga.K = (int32_t)k;
  ga.E = (int32_t)num_experts;
  ga.group = is_mlx(scheme) ? group : 32;
  ga.sb_bf16 = sb_dtype == RLXQ_BF16 ? 1 : 0;
  ga.y_bf16 = (!combine && y_dtype == RLXQ_BF16) ? 1 : 0;
  ga.x_div = x_div;
  ga.tiles_n = (int32_t)((n + 31) / 32);
  ga.pad = 0;
  const int64_t slots = num_experts < n_entries ? num_experts : n_entries;
  const int64_t grid = slots * ga.tiles_n;
  if (grid > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": grid too large");
  const size_t lds = (size_t)MT * (k / 32) * (xbf ? 20 : 36) * 4;
  void* gargs[] = {&ga};
  if ((rc = launch(ctx, fg, dim3((unsigned)grid), dim3(256), lds, stream, gargs, name))) return rc;

  // 3. probability-weighted sum over the top-k slots
  if (combine) {
    hipFunction_t fc;
    if ((rc = get_fn(ctx, "rlxq_moe_combine_k", &fc))) return rc;
    int64_t R = rows, N = n;
    int32_t tk = top_k, yb = y_dtype == RLXQ_BF16 ? 1 : 0;
    void* cargs[] = {&tmp, (void*)&probs, &R, &tk, &N, &y, &yb};
    const int64_t total = rows * n;
    if ((rc = launch(ctx, fc, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, cargs,
                     "rlxq_moe_combine_k")))
      return rc;
  }
  return RLXQ_OK;
}

}  // namespace

}  // namespace rlxq

using namespace rlxq;

extern "C" {

int rlxq_dequant_grouped_matmul(rlxq_ctx* ctx, int scheme, int group_size, const void* x, int x_dtype,
                                const void* bank, const void* scales, const void* biases, int sb_dtype,
                                const float* expert_idx, int64_t rows, int64_t k, int64_t n, int64_t num_experts,
                                void* y, int y_dtype, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!expert_idx) return fail(ctx, RLXQ_E_NULL, "dequant_grouped_matmul: expert_idx is null");
  return grouped_run(ctx, "dequant_grouped_matmul", scheme, group_size, x, x_dtype, bank, scales, biases, sb_dtype,
                     nullptr, expert_idx, rows, rows, 1, k, n, num_experts, y, y_dtype, nullptr, rows, 1, stream);
}

int rlxq_moe_grouped(rlxq_ctx* ctx, int scheme, int mode, const void* x, int x_dtype, const void* bank,
                     const int32_t* ids, const float* probs, int64_t rows, int64_t top_k, int64_t k, int64_t n,
                     int64_t num_experts, void* y, int y_dtype, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!ids) return fail(ctx, RLXQ_E_NULL, "moe_grouped: ids is null");
  if (!is_gguf(scheme)) return fail(ctx, RLXQ_E_SCHEME, "moe_grouped: GGUF schemes only");
  if (rows < 0 || top_k <= 0 || top_k > 64) return fail(ctx, RLXQ_E_SHAPE, "moe_grouped: need 0 < top_k <= 64");
  if (mode == RLXQ_MOE_EXPAND)
    return grouped_run(ctx, "moe_grouped", scheme, 32, x, x_dtype, bank, nullptr, nullptr, RLXQ_F32, ids, nullptr,
                       rows * top_k, rows, (int32_t)top_k, k, n, num_experts, y, y_dtype, nullptr, rows,
                       (int32_t)top_k, stream);
  if (mode == RLXQ_MOE_COMBINE) {
    if (!probs) return fail(ctx, RLXQ_E_NULL, "moe_grouped: COMBINE needs probs");
    return grouped_run(ctx, "moe_grouped", scheme, 32, x, x_dtype, bank, nullptr, nullptr, RLXQ_F32, ids, nullptr,
                       rows * top_k, rows * top_k, 1, k, n, num_experts, y, y_dtype, probs, rows, (int32_t)top_k,
                       stream);
  }
  return fail(ctx, RLXQ_E_SHAPE, "moe_grouped: mode must be EXPAND or COMBINE");
}

}  // extern "C"
