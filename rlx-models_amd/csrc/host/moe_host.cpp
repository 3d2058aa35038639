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
#include "skinny_args.h"
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
  // Prefill-sized calls (at least 8 entries per fired expert on average) on
  // GGUF Q4_1, Q4_0, Q8_0 or Q4_K codes with bf16 activations: the grouped
  // f16-MFMA kernels over gathered activation rows, one weight pass per chunk
  // of 16 MT entries of an expert (device table, then the gathered-row
  // layout, then the prepared rows).  RLXQ_MOE_KERNEL=sk forces them where
  // they apply; xr or lds keeps the GEMV kernels.
  const bool q6k = scheme == RLXQ_GGUF_Q6_K;
  // (MLX: groups of whole 32-blocks; MXFP4: E8M0 scale bytes only, whose
  // products with the codes are exact in bf16)
  // (f32 activations run as hi + lo row pairs, added in the epilogue)
  const bool kq_other = scheme == RLXQ_GGUF_Q5_K || scheme == RLXQ_GGUF_Q3_K || scheme == RLXQ_GGUF_Q2_K ||
                        scheme == RLXQ_GGUF_Q8_K;
  const bool sk_ok = k % 128 == 0 &&
                     (scheme == RLXQ_GGUF_Q4_1 || scheme == RLXQ_GGUF_Q4_0 || scheme == RLXQ_GGUF_Q8_0 ||
                      ((q4k || q6k || kq_other) && k % 256 == 0) ||
                      ((scheme == RLXQ_MLX_AFFINE4 || scheme == RLXQ_MLX_AFFINE8) && group >= 32 &&
                       group % 32 == 0 && k % group == 0) ||
                      (scheme == RLXQ_MLX_MXFP4 && sb_dtype == RLXQ_U8));
  // (the gathered f16 rows take about 2 K bytes per entry, twice that for
  // f32 activations: calls needing more than 1 GiB of them stay on the GEMV
  // kernels)
  const bool sk_fits =
      (double)(n_entries + fired_est * 63) * (double)k * (xbf ? 2.0 : 4.0) <= (double)(1u << 30);
  bool sk = sk_ok && sk_fits && n_entries >= 8 * fired_est;
  if (const char* ev = std::getenv("RLXQ_MOE_KERNEL")) {
    if (!std::strcmp(ev, "sk")) sk = sk_ok && sk_fits;
    else sk = false;
  }
  if (sk) {
    fused = false;
    xr = false;
  }
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
  // COMBINE on the register kernels at decode sizes: down and combine in one
  // token-major launch (rlxq_moexc_*: workgroup = token row and column tile,
  // wave = top-k slot, the slots summed in slot order in the workgroup; the
  // same bits as the expert-major kernel plus rlxq_moe_combine_k).
  // RLXQ_MOE_COMBINE=launch keeps the two launches, =fused the combine in the
  // expert-major launch (counters); RLXQ_MOE_XC_TILE=<columns> sets the tile.
  bool xc = combine && xr && fused && top_k <= 8 && x_div == 1 && rows <= 0x7fffffff;
  if (const char* ev = std::getenv("RLXQ_MOE_COMBINE"))
    if (!std::strcmp(ev, "launch") || !std::strcmp(ev, "fused")) xc = false;
  if (xc) {
    int64_t tc = 128;
    if (const char* ev = std::getenv("RLXQ_MOE_XC_TILE")) tc = std::max<int64_t>(16, std::min<int64_t>(1024, std::atoi(ev)));
    tc = std::min<int64_t>(tc, ((n + 15) / 16) * 16);
    std::snprintf(name, sizeof name, "rlxq_moexc_%s_L%d_U%d", scheme_name(scheme), L, NU);
    hipFunction_t fx;
    if ((rc = get_fn(ctx, name, &fx))) return rc;
    ga.x = x;
    ga.bank = static_cast<const uint8_t*>(bank);
    ga.N = n;
    ga.rb = rb;
    ga.x_ld = k;
    ga.K = (int32_t)k;
    ga.E = (int32_t)num_experts;
    ga.group = is_mlx(scheme) ? group : 32;
    ga.sb_bf16 = sb_code(sb_dtype);
    ga.scales = scales;
    ga.biases = biases;
    ga.x_div = 1;
    ga.ids = ids;
    ga.idx_f32 = idx;
    ga.n_entries = (int32_t)n_entries;
    ga.probs = probs;
    ga.out = y;
    ga.out_bf16 = y_dtype == RLXQ_BF16 ? 1 : 0;
    ga.top_k = top_k;
    ga.tile_rows = (int32_t)tc;
    ga.tiles_n = (int32_t)((n + tc - 1) / tc);
    const int64_t grid = rows * ga.tiles_n;
    if (grid > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": grid too large");
    void* xargs[] = {&ga};
    return launch(ctx, fx, dim3((unsigned)grid), dim3(64 * top_k), (size_t)top_k * tc * 4, stream, xargs, name);
  }
  const size_t table_bytes = fused ? 0 : ((size_t)(2 + 2 * num_experts + n_entries) * 4 + 255) & ~size_t(255);
  const size_t tmp_bytes = combine ? (((size_t)n_entries * width * 4 + 255) & ~size_t(255)) : 0;
  // grouped MFMA path: chunks of RPC gathered rows, each expert's entries
  // padded to whole chunks
  const double avg_e = (double)n_entries / (double)fired_est;
  // (chunks of 16 rows with 4 weight tiles measured best at 16 entries per
  // expert: gate|up 115 us and down 83 us at config 5 with 256 tokens,
  // against 131 and 130 with 2 tiles; 64-row chunks keep 2 tiles)
  // (f32 activations, whose chunks hold half the entries, measured best on
  // the same chunk sizes: 312 us for the 256-token layer on 16-row chunks,
  // against 340 on 32-row ones)
  int sk_mt = avg_e <= 24.0 ? 1 : (avg_e <= 48.0 ? 2 : 4), sk_nt = 0, sk_d = 0;
  if (const char* ev = std::getenv("RLXQ_MOE_SK")) std::sscanf(ev, "%d,%d,%d", &sk_mt, &sk_nt, &sk_d);   // tuning
  if (sk_mt != 1 && sk_mt != 2 && sk_mt != 4) sk_mt = 1;
  if (sk_nt != 2 && sk_nt != 4 && sk_nt != 8) sk_nt = sk_mt == 4 ? 2 : 4;
  // gathered rows per chunk (f32 activations: x16 row pairs, so half the
  // entries per 16 MT-row chunk)
  const bool sk_pairs = !xbf;
  const int64_t rpc = sk_pairs ? 8 * sk_mt : 16 * sk_mt;
  const int64_t sk_mp = sk ? ((n_entries + fired_est * (rpc - 1) + rpc - 1) / rpc) * rpc : 0;   // gathered rows
  const int64_t sk_xr = sk_pairs ? 2 * sk_mp : sk_mp;                                            // x16 rows
  auto r256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  const size_t cmap_bytes = sk ? r256((size_t)(1 + sk_mp / rpc) * 4) : 0, emap_bytes = sk ? r256((size_t)sk_mp * 4) : 0;
  const size_t x16_bytes = sk ? r256((size_t)sk_xr * k * 2) : 0, is_bytes = sk ? r256((size_t)sk_xr * 4) : 0;
  const size_t sum_bytes = sk ? r256((size_t)sk_xr * (k / 32) * 4) : 0;   // block sums of the x16 rows
  const size_t total_ws = table_bytes + tmp_bytes + cmap_bytes + emap_bytes + x16_bytes + is_bytes + sum_bytes;
  void* ws = nullptr;
  if (total_ws && (rc = workspace(ctx, total_ws, &ws, stream))) return rc;
  int32_t* table = fused ? nullptr : static_cast<int32_t*>(ws);
  float* tmp = combine ? reinterpret_cast<float*>(static_cast<char*>(ws) + table_bytes) : nullptr;
  char* skb = static_cast<char*>(ws) + table_bytes + tmp_bytes;

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

  if (sk) {
    // 2a. gathered-row layout of the table's entries
    rlxq_moe_pad_args pa;
    pa.table = table;
    pa.cmap = reinterpret_cast<int32_t*>(skb);
    pa.emap = reinterpret_cast<int32_t*>(skb + cmap_bytes);
    pa.Mp = sk_mp;
    pa.E = (int32_t)num_experts;
    pa.rows_per_chunk = (int32_t)rpc;
    hipFunction_t fp;
    if ((rc = get_fn(ctx, "rlxq_moe_pad_k", &fp))) return rc;
    void* pargs[] = {&pa};
    if ((rc = launch(ctx, fp, dim3(1), dim3(1024), 0, stream, pargs, "rlxq_moe_pad_k"))) return rc;
    // 2b. the gathered rows to f16 (scaled per row, code-unpacking order)
    rlxq_x16_args xa;
    std::memset(&xa, 0, sizeof xa);
    xa.x = x;
    xa.x16 = reinterpret_cast<uint16_t*>(skb + cmap_bytes + emap_bytes);
    xa.inv_s = reinterpret_cast<float*>(skb + cmap_bytes + emap_bytes + x16_bytes);
    xa.ssum = reinterpret_cast<float*>(skb + cmap_bytes + emap_bytes + x16_bytes + is_bytes);
    xa.M = sk_xr;
    xa.K = k;
    xa.Mp = sk_xr;
    xa.x_bf16 = xbf ? 1 : 0;
    xa.split = sk_pairs ? 1 : 0;   // (rows 2r, 2r + 1: hi and lo of gathered row r)
    xa.nibble_order = sk_order(scheme);
    xa.frag_major = 1;
    xa.rdiv = x_div;
    xa.rmap = pa.emap;
    xa.out_bf16 = scheme == RLXQ_MLX_MXFP4 ? 1 : 0;
    xa.post_exp = sk_post_exp(scheme);
    hipFunction_t fx;
    if ((rc = get_fn(ctx, "rlxq_x16_prep", &fx))) return rc;
    void* xargs[] = {&xa};
    if ((rc = launch(ctx, fx, dim3((unsigned)sk_xr, (unsigned)((k + 2047) / 2048)), dim3(256), 0, stream, xargs,
                     "rlxq_x16_prep")))
      return rc;
    // 2c. the grouped MFMA kernel over (chunk, tile): NT weight tiles of 16
    // rows (SwiGLU: NT / 2 gate tiles and their up tiles)
    const int NT = sk_nt;
    const int nh = swiglu ? NT / 2 : NT;
    // ring depth of the compiled variant (Q6_K's larger raw blocks: one
    // shallower)
    int D = sk_d;
    if (D <= 0) D = NT >= 4 ? (NT == 8 && sk_mt == 2 ? 1 : (sk_mt == 4 ? 1 : 2))
                            : (sk_mt == 1 ? (q4k ? 3 : 4) : (sk_mt == 2 ? 3 : 2));
    if (sk_d <= 0 && (q6k || scheme == RLXQ_GGUF_Q5_K || scheme == RLXQ_GGUF_Q3_K)) D = NT >= 4 || sk_mt == 4 ? 1 : 2;
    if (sk_d <= 0 && scheme == RLXQ_GGUF_Q2_K && NT < 4 && sk_mt == 1) D = 3;
    rlxq_moe_sk_args ka;
    std::memset(&ka, 0, sizeof ka);
    ka.x16 = xa.x16;
    ka.inv_s = xa.inv_s;
    ka.ssum = xa.ssum;
    ka.cmap = pa.cmap;
    ka.emap = pa.emap;
    ka.bank = static_cast<const uint8_t*>(bank);
    ka.y = combine ? static_cast<void*>(tmp) : y;
    ka.N = n;
    ka.K = k;
    ka.rb = rb;
    ka.y_ld = width;
    ka.Mp = sk_xr;
    ka.pairs = sk_pairs ? 1 : 0;
    ka.tiles_n = (int32_t)((width + 16 * nh - 1) / (16 * nh));
    ka.y_bf16 = (!combine && y_dtype == RLXQ_BF16) ? 1 : 0;
    ka.swiglu = swiglu ? 1 : 0;
    ka.scales = scales;
    ka.biases = biases;
    ka.group = is_mlx(scheme) ? group : 32;
    ka.sb_bf16 = sb_code(sb_dtype);
    std::snprintf(name, sizeof name, "rlxq_moesk_%s_mt%d_nt%d_d%d%s", scheme_name(scheme), sk_mt, NT, D,
                  swiglu ? "_sw" : "");
    hipFunction_t fk;
    if ((rc = get_fn(ctx, name, &fk))) return rc;
    const int64_t grid = (sk_mp / rpc) * ka.tiles_n;   // chunks x tiles
    if (grid > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, std::string(what) + ": grid too large");
    const size_t lds = 2 * (size_t)(sk_mt * NT * 4) * 64 * 4;
    void* kargs[] = {&ka};
    if ((rc = launch(ctx, fk, dim3((unsigned)grid), dim3(256), lds, stream, kargs, name))) return rc;
  } else {
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
  // routing in the workgroups: the workgroup completing a (token row, tile)
  // sums it) is selected by RLXQ_MOE_COMBINE=fused.  The separate combine
  // kernel stays the default: on one box, three runs each, the config-5
  // layer took 75.6-77.8 us fused against 72.3-76.6 with the extra launch
  // (the last workgroup of each token adds the sum to the kernel's tail).
  bool fuse_combine = false;
  if (const char* ev = std::getenv("RLXQ_MOE_COMBINE"))
    if (!std::strcmp(ev, "fused")) fuse_combine = combine && xr && fused && rows * ga.tiles_n <= rlxq_ctx::kCounterSlots;
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
  }

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
