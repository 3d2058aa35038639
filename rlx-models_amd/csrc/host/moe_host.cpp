// Host side of the grouped-expert entry points: rlxq_dequant_grouped_matmul
// and rlxq_moe_grouped.  Both route the entries by expert (a device routing
// table, or inside the GEMV's workgroups for decode-sized calls), then run
// the grouped GEMV over the fired experts.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
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
                bool swiglu, void* stream) {
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
  const int64_t width = swiglu ? n / 2 : n;   // output columns
  // Routing inside the grouped GEMV's workgroups for decode-sized calls (no
  // table launch; the entries of each expert cut into chunks of MT, one
  // workgroup per chunk and tile); the device table for larger ones.
  // RLXQ_MOE_ROUTE=table|fused forces one (fused only where it applies).
  const bool fusable = n_entries <= 1024 && num_experts <= 1024;
  bool fused = fusable, route_forced = false;
  if (const char* e = std::getenv("RLXQ_MOE_ROUTE")) {
    if (!std::strcmp(e, "table")) fused = false, route_forced = true;
    if (!std::strcmp(e, "fused")) fused = fusable, route_forced = true;
  }
  // kernel choice
  const int blocks = (scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_GGUF_Q8_0 || scheme == RLXQ_GGUF_Q4_K ||
                      scheme == RLXQ_GGUF_Q5_K) ? 2 : 1;
  const int64_t units = (k / 32) / blocks;
  const bool xbf = x_dtype == RLXQ_BF16;
  const int64_t fired_est = num_experts < n_entries ? num_experts : n_entries;
  const int64_t cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  rlxq_moe_gemv_args ga;
  std::memset(&ga, 0, sizeof ga);
  char name[80];
  int MT = 2;   // entries served per weight pass
  // Register-activation kernels (4-bit codes: Q4_1, Q4_0, Q4_K, MLX affine
  // 4-bit, MXFP4; bf16 activations; up to 256 units per row): lane groups of L
  // lanes x NU units cover a row with the least padding, MT entries are served
  // per weight pass.  The LDS-record kernels serve everything else (Q8_0, MLX
  // 8-bit, Q6_K, f32 activations).
  const bool q40 = scheme == RLXQ_GGUF_Q4_0;   // two blocks per unit
  const bool q4k = scheme == RLXQ_GGUF_Q4_K;   // two blocks per unit (64 weights)
  const bool wide = q40 || q4k;                // units of two blocks: at most two per lane
  bool xr = xbf &&
            (scheme == RLXQ_GGUF_Q4_1 || wide || scheme == RLXQ_MLX_AFFINE4 || scheme == RLXQ_MLX_MXFP4) &&
            units <= (wide ? 128 : 256) && !(is_mlx(scheme) && group % 32);
  // lane groups: L lanes x NU units, the least padding over the instantiated shapes
  // (32-lane groups: Q4_K only)
  static const int cand[][2] = {{64, 1}, {64, 2}, {64, 4}, {8, 1}, {8, 2}, {8, 3}, {8, 4}, {32, 1}};
  int L = 0, NU = 0;
  for (const auto& c : cand)
    if (!(wide && c[1] > 2) && !(c[0] == 32 && !q4k) && c[0] * c[1] >= units && (L == 0 || c[0] * c[1] < L * NU))
      L = c[0], NU = c[1];
  // one-block 4-bit units, 33..64 of them: 32-lane groups of two units rather
  // than 64 lanes of one (config 5's Q4_1 gate|up, K = 2048: 40.4 against
  // 44.1 us)
  const bool one_block4 = scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_MLX_AFFINE4 || scheme == RLXQ_MLX_MXFP4;
  if (one_block4 && units > 32 && units <= 64) L = 32, NU = 2;
  // Q4_K with under 70% of the lanes holding a unit (K = 2048 on 64-lane
  // groups: 32 units) measured slower than the LDS-record kernel (gate|up 79
  // against 58 us at config 5); RLXQ_MOE_KERNEL=xr|lds forces one (tests)
  if (q4k && units * 10 < 7 * (int64_t)L * NU) xr = false;
  if (const char* ev = std::getenv("RLXQ_MOE_KERNEL")) {
    if (!std::strcmp(ev, "lds")) xr = false;
    if (!std::strcmp(ev, "xr") && q4k && xbf && units <= 128) xr = true;
  }
  // The balanced in-workgroup routing pays for the register kernels (every
  // workgroup one chunk of MT entries); the LDS-record kernels measure faster
  // with the device table.
  if (!xr && fused && !route_forced) fused = false;
  if (xr) {
    // one entry per pass while experts hold few entries: the chunks of one
    // expert then run side by side and share its rows through the caches
    const double avg = (double)n_entries / (double)fired_est;
    MT = avg < 3.0 ? 1 : (avg < 6.0 ? 2 : 4);
    if (const char* ev = std::getenv("RLXQ_MOE_MT")) MT = std::atoi(ev);
    if (MT != 1 && MT != 2 && MT != 4) MT = 2;
    if (NU >= 3 && MT > 2) MT = 2;          // register budget of the instantiated kernels
    if (wide) MT = std::min(MT, 2 / NU);
    // workgroups (4 waves) per expert: about 16 waves per CU over the fired
    // experts, and no more waves than column steps
    const int64_t rp = 64 / L;
    int64_t tiles = (4 * cus + fired_est - 1) / fired_est;
    if (const char* ev = std::getenv("RLXQ_MOE_WGS")) tiles = std::max<int64_t>(1, tiles * std::atof(ev));
    tiles = std::min<int64_t>(tiles, (width + 4 * rp - 1) / (4 * rp));
    ga.tiles_n = (int32_t)std::max<int64_t>(tiles, 1);
    ga.tile_rows = 0;
    std::snprintf(name, sizeof name, "rlxq_moexr%s_%s_L%d_U%d_M%d%s", fused ? "f" : "", scheme_name(scheme), L, NU,
                  MT, swiglu ? "_sw" : "");
  } else {
    L = units >= 48 ? 64 : 8;
    std::snprintf(name, sizeof name, "rlxq_moe_gemv%s_%s_%s_L%d_M%d%s", fused ? "f" : "", scheme_name(scheme),
                  xbf ? "bf16" : "f32", L, MT, swiglu ? "_sw" : "");
    // Rows per workgroup tile; RLXQ_MOE_TILE=64|128|192|256 forces it.
    int tile = 64;
    if (const char* ev = std::getenv("RLXQ_MOE_TILE")) {
      const int t = std::atoi(ev);
      if (t == 64 || t == 128 || t == 192 || t == 256) tile = t;
    }
    ga.tile_rows = tile;
    ga.tiles_n = (int32_t)(swiglu ? (width + tile / 2 - 1) / (tile / 2) : (n + tile - 1) / tile);
  }
  const size_t table_bytes = fused ? 0 : ((size_t)(2 + 2 * num_experts + n_entries) * 4 + 255) & ~size_t(255);
  const size_t tmp_bytes = combine ? (size_t)n_entries * width * 4 : 0;
  void* ws = nullptr;
  if (table_bytes + tmp_bytes && (rc = workspace(ctx, table_bytes + tmp_bytes, &ws, stream))) return rc;
  int32_t* table = fused ? nullptr : static_cast<int32_t*>(ws);
  float* tmp = combine ? reinterpret_cast<float*>(static_cast<char*>(ws) + table_bytes) : nullptr;

  // 1. routing table
  if (!fused) {
    hipFunction_t ft;
    if ((rc = get_fn(ctx, "rlxq_moe_table_k", &ft))) return rc;
    rlxq_moe_table_args ta;
    ta.ids = ids;
    ta.idx_f32 = idx;
    ta.table = table;
    ta.zero_rows = combine ? static_cast<void*>(tmp) : y;
    ta.n = n_entries;
    ta.N = width;
    ta.zero_ld = width;
    ta.E = (int32_t)num_experts;
    ta.zero_bf16 = (!combine && y_dtype == RLXQ_BF16) ? 1 : 0;
    void* targs[] = {&ta};
    if ((rc = launch(ctx, ft, dim3(1), dim3(1024), 0, stream, targs, "rlxq_moe_table_k"))) return rc;
  }

  // 2. grouped GEMV over (expert or chunk, tile)
  hipFunction_t fg;
  if ((rc = get_fn(ctx, name, &fg))) return rc;
  ga.x = x;
  ga.bank = static_cast<const uint8_t*>(bank);
  ga.scales = scales;
  ga.biases = biases;
  ga.table = table;
  ga.y = combine ? static_cast<void*>(tmp) : y;
  ga.N = n;
  ga.rb = rb;
  ga.y_ld = width;
  ga.x_ld = k;
  ga.K = (int32_t)k;
  ga.E = (int32_t)num_experts;
  ga.group = is_mlx(scheme) ? group : 32;
  ga.sb_bf16 = sb_code(sb_dtype);
  ga.y_bf16 = (!combine && y_dtype == RLXQ_BF16) ? 1 : 0;
  ga.x_div = x_div;
  ga.swiglu = swiglu ? 1 : 0;
  ga.ids = ids;
  ga.idx_f32 = idx;
  ga.n_entries = (int32_t)n_entries;
  // fused: chunks number at most min(n, min(E, n) + n / MT) (each holds an
  // entry), plus the one that zeroes the rows of invalid entries
  const int64_t chunk_bound = std::min<int64_t>(n_entries, fired_est + (n_entries + MT - 1) / MT);
  const int64_t slots = fused ? chunk_bound + 1 : fired_est;
  const int64_t grid = slots * ga.tiles_n;
  if (grid > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": grid too large");
  // The combine in the down launch itself (register kernels with the
  // routing in the workgroups): the workgroup completing a (token row, tile)
  // sums it.  RLXQ_MOE_COMBINE=launch keeps the separate combine kernel.
  bool fuse_combine = combine && xr && fused && rows * ga.tiles_n <= rlxq_ctx::kCounterSlots;
  if (const char* ev = std::getenv("RLXQ_MOE_COMBINE"))
    if (!std::strcmp(ev, "launch")) fuse_combine = false;
  if (fuse_combine) {
    if ((rc = zeroed_counters(ctx, stream, &ga.counters))) return rc;
    ga.probs = probs;
    ga.out = y;
    ga.top_k = top_k;
    ga.out_bf16 = y_dtype == RLXQ_BF16 ? 1 : 0;
  }
  const size_t lds = xr ? 0 : (size_t)2 * (k / 32) * (xbf ? 20 : 36) * 4;
  void* gargs[] = {&ga};
  if ((rc = launch(ctx, fg, dim3((unsigned)grid), dim3(256), lds, stream, gargs, name))) return rc;

  // 3. probability-weighted sum over the top-k slots (in the GEMV launch
  // above when it took the counters)
  if (combine && !ga.counters) {
    hipFunction_t fc;
    if ((rc = get_fn(ctx, "rlxq_moe_combine_k", &fc))) return rc;
    int64_t R = rows, N = width;
    int32_t tk = top_k, yb = y_dtype == RLXQ_BF16 ? 1 : 0;
    void* cargs[] = {&tmp, (void*)&probs, &R, &tk, &N, &y, &yb};
    const int64_t total = rows * width;
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
                     nullptr, expert_idx, rows, rows, 1, k, n, num_experts, y, y_dtype, nullptr, rows, 1, false,
                     stream);
}

int rlxq_moe_grouped(rlxq_ctx* ctx, int scheme, int mode, const void* x, int x_dtype, const void* bank,
                     const int32_t* ids, const float* probs, int64_t rows, int64_t top_k, int64_t k, int64_t n,
                     int64_t num_experts, void* y, int y_dtype, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!ids) return fail(ctx, RLXQ_E_NULL, "moe_grouped: ids is null");
  if (!is_gguf(scheme) && kquant_bytes(scheme) < 0)
    return fail(ctx, RLXQ_E_SCHEME, "moe_grouped: GGUF schemes only");
  if (rows < 0 || top_k <= 0 || top_k > 64) return fail(ctx, RLXQ_E_SHAPE, "moe_grouped: need 0 < top_k <= 64");
  if (mode == RLXQ_MOE_EXPAND || mode == RLXQ_MOE_EXPAND_SWIGLU) {
    const bool sw = mode == RLXQ_MOE_EXPAND_SWIGLU;
    if (sw && n % 2) return fail(ctx, RLXQ_E_SHAPE, "moe_grouped: EXPAND_SWIGLU needs an even N (gate | up)");
    return grouped_run(ctx, "moe_grouped", scheme, 32, x, x_dtype, bank, nullptr, nullptr, RLXQ_F32, ids, nullptr,
                       rows * top_k, rows, (int32_t)top_k, k, n, num_experts, y, y_dtype, nullptr, rows,
                       (int32_t)top_k, sw, stream);
  }
  if (mode == RLXQ_MOE_COMBINE) {
    if (!probs) return fail(ctx, RLXQ_E_NULL, "moe_grouped: COMBINE needs probs");
    return grouped_run(ctx, "moe_grouped", scheme, 32, x, x_dtype, bank, nullptr, nullptr, RLXQ_F32, ids, nullptr,
                       rows * top_k, rows * top_k, 1, k, n, num_experts, y, y_dtype, probs, rows, (int32_t)top_k,
                       false, stream);
  }
  return fail(ctx, RLXQ_E_SHAPE, "moe_grouped: mode must be EXPAND, COMBINE or EXPAND_SWIGLU");
}

}  // extern "C"
