// Host side of the int8 paths: the W8A8 GEMM entry point and the Int8Block
// branch of rlxq_dequant_matmul.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "rlxq.h"
#include "rlxq_internal.hpp"
#include "int8_args.h"

namespace rlxq {

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

struct W8a8Cfg {
  const char* name;  // kernel name suffix
  int BM, BN, BK, WGM, WGN;
  bool kf;           // K must be a multiple of BK (no zeroing along K)
};

// Compiled W8A8 tilings (kernel rlxq_w8a8_<name>).
const W8a8Cfg kW8a8[] = {
    {"m128n128k64w22", 128, 128, 64, 2, 2, false},   {"m128n128k128w22", 128, 128, 128, 2, 2, false},
    {"m256n128k64w22", 256, 128, 64, 2, 2, false},   {"m128n256k64w22", 128, 256, 64, 2, 2, false},
    {"m256n256k64w24", 256, 256, 64, 2, 4, false},   {"m128n128k128w22_p2", 128, 128, 128, 2, 2, false},
    {"m256n256k128w24", 256, 256, 128, 2, 4, false}, {"m256n256k64w24_kf", 256, 256, 64, 2, 4, true},
    {"m256n256k128w24_kf", 256, 256, 128, 2, 4, true},
};

// Tiling choice; RLXQ_W8A8_CFG=<name> selects one (tuning sweeps and the
// per-variant parity test).
// Default: 256 x 256 tiles (8 waves) once they cover the CUs, else 128 x 128;
// the 256 x 256 tiles take 128-byte K steps where K allows (Qwen3-8B at
// M=4096 after 20 ms of sustained launches: gate_up 451 us against 485 with
// 64-byte steps, down 227.5 against 232; the two-stage variants of both
// measured 5-30% slower).
const W8a8Cfg* pick_w8a8(int64_t m, int64_t n, int64_t k, int cus) {
  if (const char* e = std::getenv("RLXQ_W8A8_CFG")) {
    for (const auto& c : kW8a8)
      if (std::strcmp(c.name, e) == 0) return &c;
    return nullptr;
  }
  const int64_t t256 = ((m + 255) / 256) * ((n + 255) / 256);
  if (t256 < (cus > 0 ? cus : 256)) return &kW8a8[0];
  // (the _kf forms where K is a whole number of steps)
  return k % 128 == 0 ? &kW8a8[8] : (k % 64 == 0 ? &kW8a8[7] : &kW8a8[4]);
}

}  // namespace

// Int8Block{block_size: K}: w = i8 [K, N], scales = f32 [N], biases = zero
// points f32 [N] or NULL.  Workgroups take (256 columns, K split, 16*MT rows);
// the K splits are sized so the grid covers the chip, and their partial sums
// are added in split order by rlxq_i8b_reduce.
int i8b_dispatch(rlxq_ctx* ctx, int group, const void* x, int x_dtype, const void* w, const void* scales,
                 const void* zp, int sb_dtype, int64_t m, int64_t k, int64_t n, void* y, int y_dtype,
                 void* stream) {
  if (!scales) return fail(ctx, RLXQ_E_NULL, "dequant_matmul: Int8Block needs scales [N]");
  if (sb_dtype != RLXQ_F32) return fail(ctx, RLXQ_E_DTYPE, "dequant_matmul: Int8Block scales/zp are F32");
  if (group != 0 && group != k)
    return fail(ctx, RLXQ_E_SCHEME, "dequant_matmul: Int8Block block_size must equal K (one scale per column)");
  if (n % 16) return fail(ctx, RLXQ_E_ALIGN, "dequant_matmul: Int8Block needs N % 16 == 0");
  if (!aligned16(w)) return fail(ctx, RLXQ_E_ALIGN, "dequant_matmul: Int8Block weights must be 16-byte aligned");
  if (k > ((int64_t)1 << 31) || n > ((int64_t)1 << 31) || m > ((int64_t)1 << 31))
    return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: Int8Block shape too large");

  // M = 1: the streaming GEMV (rlxq_i8bv_*, which also serves M <= 4 when
  // RLXQ_I8B_GEMV=1; RLXQ_I8B_MFMA=1 forces the MFMA kernel); larger M: the
  // MFMA kernel, which reads each weight once for up to 16 rows.
  const char* force_mfma = std::getenv("RLXQ_I8B_MFMA");
  // partial sums kept under 256 MiB (under the fixed scratch of the
  // no-allocation entry point, less room for the zero-point row sums)
  const int64_t cap = ctx->fixed_active ? std::min<int64_t>((int64_t)256 << 20, (int64_t)ctx->fixed_bytes / 2)
                                        : (int64_t)256 << 20;
  const char* force_gemv = std::getenv("RLXQ_I8B_GEMV");
  const int64_t gemv_m = force_gemv && force_gemv[0] == '1' ? 4 : 1;
  const bool gemv = m <= gemv_m && !(force_mfma && force_mfma[0] == '1') && ((k + 1023) / 1024) * m * n * 4 <= cap;
  const int MT = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
  const int MR = m <= 1 ? 1 : (m <= 2 ? 2 : 4);
  const int64_t MC = 16 * MT;
  const int64_t tiles_n = gemv ? (n + 1023) / 1024 : (n + 255) / 256, mch = gemv ? 1 : (m + MC - 1) / MC;
  const int64_t unit = gemv ? 16 : 128;   // K rows per slice granule
  const int64_t ksteps = (k + unit - 1) / unit;
  const int64_t base = tiles_n * mch;
  // workgroups: four (of four waves) per CU for the MFMA kernel; one (of
  // sixteen) per CU for the GEMV
  const int64_t target = (gemv ? 1 : 4) * (int64_t)(ctx->cu_count > 0 ? ctx->cu_count : 256);
  int64_t splits = (target + base - 1) / base;
  if (gemv) splits = std::max<int64_t>(splits, (k + 1023) / 1024);   // at most 1024 rows per slice
  if (splits > ksteps) splits = ksteps;
  if (splits > 1 && splits * m * n * 4 > cap) splits = cap / (m * n * 4);
  if (splits < 1) splits = 1;
  const int64_t kslice = ((ksteps + splits - 1) / splits) * unit;
  splits = (k + kslice - 1) / kslice;
  if (gemv && kslice > 1024) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: Int8Block decode slice");
  if (tiles_n * mch * splits > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: Int8Block grid");

  const size_t part_bytes = splits > 1 ? round256((size_t)(splits * m * n) * 4) : 0;
  const size_t xsum_bytes = zp ? round256((size_t)m * 4) : 0;
  void* ws = nullptr;
  int rc;
  if (part_bytes + xsum_bytes && (rc = workspace(ctx, part_bytes + xsum_bytes, &ws, stream))) return rc;

  rlxq_i8b_args a;
  std::memset(&a, 0, sizeof a);
  a.x = x;
  a.wq = static_cast<const int8_t*>(w);
  a.scale = static_cast<const float*>(scales);
  a.zp = static_cast<const float*>(zp);
  a.part = part_bytes ? static_cast<float*>(ws) : nullptr;
  a.xsum = zp ? reinterpret_cast<const float*>(static_cast<char*>(ws) + part_bytes) : nullptr;
  a.y = y;
  a.M = m;
  a.N = n;
  a.K = k;
  a.y_ld = n;
  a.kslice = (int32_t)kslice;
  a.splits = (int32_t)splits;
  a.tiles_n = (int32_t)tiles_n;
  a.x_bf16 = x_dtype == RLXQ_BF16;
  a.y_bf16 = y_dtype == RLXQ_BF16;

  hipFunction_t fn;
  if (zp) {
    if ((rc = get_fn(ctx, "rlxq_row_sum", &fn))) return rc;
    int xb = a.x_bf16;
    int64_t M = m, K = k;
    float* out = const_cast<float*>(a.xsum);
    void* args[] = {(void*)&x, &xb, &M, &K, &out};
    if ((rc = launch(ctx, fn, dim3((unsigned)m), dim3(256), 0, stream, args, "rlxq_row_sum"))) return rc;
  }
  char name[48];
  if (gemv) std::snprintf(name, sizeof name, "rlxq_i8bv_%s_m%d", a.x_bf16 ? "bf16" : "f32", MR);
  else std::snprintf(name, sizeof name, "rlxq_i8b_%s_mt%d", a.x_bf16 ? "bf16" : "f32", MT);
  if ((rc = get_fn(ctx, name, &fn))) return rc;
  const size_t lds = gemv ? 0 : 128 * (256 + 16) + 2 * (size_t)MC * (128 + 8) * 2;
  void* args[] = {&a};
  if ((rc = launch(ctx, fn, dim3((unsigned)(tiles_n * splits * mch)), dim3(gemv ? 1024 : 256), lds, stream, args,
                   name)))
    return rc;
  if (splits > 1) {
    if ((rc = get_fn(ctx, "rlxq_i8b_reduce", &fn))) return rc;
    const int64_t total = (m * n + 3) / 4;   // threads: four outputs each (N % 16 == 0)
    if ((total + 255) / 256 > 0x7fffffff) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: Int8Block output");
    void* rargs[] = {&a};
    // the last kernel launched names the path in rlxq_last_kernel: keep the
    // matmul's name there, the reduction is its tail
    rc = launch(ctx, fn, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, rargs, "rlxq_i8b_reduce");
    if (!rc) ctx->last_kernel = name;
  }
  return rc;
}

}  // namespace rlxq

using namespace rlxq;

extern "C" {

int rlxq_w8a8_gemm(rlxq_ctx* ctx, const void* x, int x_dtype, const int8_t* wq, const float* w_scale, int64_t m,
                   int64_t k, int64_t n, void* y, int y_dtype, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  // with no rows nothing is read or written: x and y may be NULL then
  if (!wq || !w_scale || (m > 0 && (!x || !y))) return fail(ctx, RLXQ_E_NULL, "w8a8_gemm: null pointer");
  if (m < 0 || k <= 0 || n <= 0) return fail(ctx, RLXQ_E_SHAPE, "w8a8_gemm: need m >= 0, k > 0, n > 0");
  // |acc| <= 127 * 127 * K must stay inside int32
  if (k > 131072 || m > 0x7fffffff || n > 0x7fffffff)
    return fail(ctx, RLXQ_E_SHAPE, "w8a8_gemm: K above 131072 or M, N above 2^31");
  if (k % 16 || n % 16) return fail(ctx, RLXQ_E_ALIGN, "w8a8_gemm: K and N must be multiples of 16");
  if (x_dtype != RLXQ_F32 && x_dtype != RLXQ_BF16) return fail(ctx, RLXQ_E_DTYPE, "w8a8_gemm: x_dtype");
  if (y_dtype != RLXQ_F32 && y_dtype != RLXQ_BF16) return fail(ctx, RLXQ_E_DTYPE, "w8a8_gemm: y_dtype");
  if (!aligned16(wq)) return fail(ctx, RLXQ_E_ALIGN, "w8a8_gemm: wq must be 16-byte aligned");
  if (m == 0) return RLXQ_OK;

  const W8a8Cfg* c = pick_w8a8(m, n, k, ctx->cu_count);
  if (!c) return fail(ctx, RLXQ_E_NOKERNEL, "w8a8_gemm: RLXQ_W8A8_CFG names no compiled tiling");
  if (c->kf && k % c->BK) return fail(ctx, RLXQ_E_SHAPE, "w8a8_gemm: this tiling needs K to be a multiple of its K step");
  const int64_t tiles_m = (m + c->BM - 1) / c->BM, tiles_n = (n + c->BN - 1) / c->BN;
  if (tiles_m * tiles_n > 0x7ffffff0) return fail(ctx, RLXQ_E_SHAPE, "w8a8_gemm: too many tiles");

  DeviceGuard g(ctx->device);
  const size_t q_bytes = round256((size_t)(m * k));
  void* ws = nullptr;
  int rc;
  if ((rc = workspace(ctx, q_bytes + round256((size_t)m * 4), &ws, stream))) return rc;
  int8_t* qx = static_cast<int8_t*>(ws);
  float* sx = reinterpret_cast<float*>(static_cast<char*>(ws) + q_bytes);
  if ((rc = rlxq_quantize_act_int8(ctx, x, x_dtype, m, k, qx, sx, stream))) return rc;

  char name[48];
  std::snprintf(name, sizeof name, "rlxq_w8a8_%s", c->name);
  hipFunction_t fn;
  if ((rc = get_fn(ctx, name, &fn))) return rc;
  rlxq_w8a8_args a;
  std::memset(&a, 0, sizeof a);
  a.qx = qx;
  a.sx = sx;
  a.wq = wq;
  a.sw = w_scale;
  a.y = y;
  a.M = m;
  a.N = n;
  a.K = k;
  a.y_ld = n;
  a.tiles_m = (int32_t)tiles_m;
  a.tiles_n = (int32_t)tiles_n;
  a.y_bf16 = y_dtype == RLXQ_BF16;
  const int64_t grid = 8 * ((tiles_m * tiles_n + 7) / 8);
  const size_t lds = 2 * (size_t)c->BM * (c->BK + 16) + 2 * (size_t)c->BK * (c->BN + 32);
  void* args[] = {&a};
  return launch(ctx, fn, dim3((unsigned)grid), dim3(64 * c->WGM * c->WGN), lds, stream, args, name);
}

}  // extern "C"
