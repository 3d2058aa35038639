// librlxq: context, code-object loading, argument validation and the C ABI
// entry points of include/rlxq.h.
//
// The gfx950 code objects are assembled into this shared library at build
// time (.incbin) and loaded with hipModuleLoadData; kernels are launched with
// hipModuleLaunchKernel.  Nothing here allocates on the hot path except the
// per-stream context scratch, which grows to the largest size a call on that
// stream has needed (rlxq_reserve_workspace sizes it ahead).
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "rlxq.h"
#include "rlxq_internal.hpp"

#ifndef RLXQ_CO_DIR
#error "RLXQ_CO_DIR must name the directory holding the built code objects"
#endif

#define RLXQ_EMBED(sym, file)                                                                  \
  asm(".pushsection .rodata." #sym ",\"a\",@progbits\n"                                        \
      ".balign 64\n"                                                                           \
      ".globl " #sym "_begin\n"                                                                \
      ".hidden " #sym "_begin\n" #sym "_begin:\n"                                              \
      ".incbin \"" RLXQ_CO_DIR "/" file "\"\n"                                                 \
      ".globl " #sym "_end\n"                                                                  \
      ".hidden " #sym "_end\n" #sym "_end:\n"                                                  \
      ".byte 0\n"                                                                              \
      ".popsection\n");                                                                        \
  extern "C" __attribute__((visibility("hidden"))) const unsigned char sym##_begin[];         \
  extern "C" __attribute__((visibility("hidden"))) const unsigned char sym##_end[];

RLXQ_EMBED(rlxq_co_gemv0, "gemv0.co")
RLXQ_EMBED(rlxq_co_gemv1, "gemv1.co")
RLXQ_EMBED(rlxq_co_gemv2, "gemv2.co")
RLXQ_EMBED(rlxq_co_gemv3, "gemv3.co")
RLXQ_EMBED(rlxq_co_gemv4, "gemv4.co")
RLXQ_EMBED(rlxq_co_gemv5, "gemv5.co")
RLXQ_EMBED(rlxq_co_misc, "misc.co")
RLXQ_EMBED(rlxq_co_gemm, "gemm.co")
RLXQ_EMBED(rlxq_co_moe0, "moe0.co")
RLXQ_EMBED(rlxq_co_moe1, "moe1.co")
RLXQ_EMBED(rlxq_co_moe2, "moe2.co")
RLXQ_EMBED(rlxq_co_moe3, "moe3.co")
RLXQ_EMBED(rlxq_co_moe4, "moe4.co")
RLXQ_EMBED(rlxq_co_int8, "int8.co")
RLXQ_EMBED(rlxq_co_skinny, "skinny.co")

namespace {

struct Image {
  const unsigned char* begin;
  const unsigned char* end;
  const char* name;
};

const Image kImages[] = {
    {rlxq_co_gemv0_begin, rlxq_co_gemv0_end, "gemv0"},
    {rlxq_co_gemv1_begin, rlxq_co_gemv1_end, "gemv1"},
    {rlxq_co_gemv2_begin, rlxq_co_gemv2_end, "gemv2"},
    {rlxq_co_gemv3_begin, rlxq_co_gemv3_end, "gemv3"},
    {rlxq_co_gemv4_begin, rlxq_co_gemv4_end, "gemv4"},
    {rlxq_co_gemv5_begin, rlxq_co_gemv5_end, "gemv5"},
    {rlxq_co_misc_begin, rlxq_co_misc_end, "misc"},
    {rlxq_co_gemm_begin, rlxq_co_gemm_end, "gemm"},
    {rlxq_co_moe0_begin, rlxq_co_moe0_end, "moe0"},
    {rlxq_co_moe1_begin, rlxq_co_moe1_end, "moe1"},
    {rlxq_co_moe2_begin, rlxq_co_moe2_end, "moe2"},
    {rlxq_co_moe3_begin, rlxq_co_moe3_end, "moe3"},
    {rlxq_co_moe4_begin, rlxq_co_moe4_end, "moe4"},
    {rlxq_co_int8_begin, rlxq_co_int8_end, "int8"},
    {rlxq_co_skinny_begin, rlxq_co_skinny_end, "skinny"},
};

std::string hip_msg(hipError_t e) { return std::string(hipGetErrorName(e)) + ": " + hipGetErrorString(e); }

}  // namespace

namespace rlxq {

int fail(rlxq_ctx* ctx, int code, const std::string& msg) {
  if (ctx) ctx->last_error = msg;
  return code;
}

DeviceGuard::DeviceGuard(int dev) {
  if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
  if (prev_ == dev) {
    ok_ = true;
    return;
  }
  ok_ = hipSetDevice(dev) == hipSuccess;
}

DeviceGuard::~DeviceGuard() {
  int cur = -1;
  if (prev_ >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev_) (void)hipSetDevice(prev_);
}

int get_fn(rlxq_ctx* ctx, const std::string& name, hipFunction_t* out) {
  auto it = ctx->fn_cache.find(name);
  if (it != ctx->fn_cache.end()) {
    *out = it->second;
    return RLXQ_OK;
  }
  for (hipModule_t m : ctx->modules) {
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, m, name.c_str()) == hipSuccess && f) {
      ctx->fn_cache.emplace(name, f);
      *out = f;
      return RLXQ_OK;
    }
    // A miss in one module is expected; do not leave it as the thread's
    // last HIP error for the caller's runtime to report later.
    (void)hipGetLastError();
  }
  return fail(ctx, RLXQ_E_NOKERNEL, "kernel not found in the gfx950 code objects: " + name);
}

int blocks_per_cu(rlxq_ctx* ctx, const std::string& name, hipFunction_t fn, int threads, size_t lds) {
  const std::string key = name + "@" + std::to_string(lds);
  auto it = ctx->occ_cache.find(key);
  if (it != ctx->occ_cache.end()) return it->second;
  int per_cu = 0;
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) != hipSuccess || per_cu < 1) {
    (void)hipGetLastError();
    per_cu = 1;
  }
  ctx->occ_cache.emplace(key, per_cu);
  return per_cu;
}

int launch(rlxq_ctx* ctx, hipFunction_t fn, dim3 grid, dim3 block, size_t lds, void* stream,
           void** args, const char* what) {
  ctx->last_kernel = what;
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return RLXQ_OK;
  if (lds > ctx->max_lds)
    return fail(ctx, RLXQ_E_SHAPE,
                std::string(what) + ": needs " + std::to_string(lds) + " B of LDS, device has " +
                    std::to_string(ctx->max_lds));
  hipError_t e = hipModuleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                       (unsigned)lds, (hipStream_t)stream, args, nullptr);
  if (e != hipSuccess) return fail(ctx, RLXQ_E_HIP, std::string(what) + ": launch failed: " + hip_msg(e));
  return RLXQ_OK;
}

int workspace(rlxq_ctx* ctx, size_t bytes, void** out, void* stream) {
  if (ctx->fixed_active) {
    if (bytes > ctx->fixed_bytes)
      return fail(ctx, RLXQ_E_SCRATCH,
                  "this call needs " + std::to_string(bytes) + " B of scratch; the no-allocation entry point holds " +
                      std::to_string(ctx->fixed_bytes) + " B");
    *out = ctx->fixed_p;
    return RLXQ_OK;
  }
  rlxq_ctx::Scratch& w = ctx->ws[stream];
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  bool capturing = true;   // (unknown status: treat as captured, keep buffers)
  if (hipStreamIsCapturing(hs, &st) == hipSuccess) capturing = st != hipStreamCaptureStatusNone;
  else (void)hipGetLastError();
  if (!capturing) reclaim_retired(w);
  if (bytes <= w.bytes) {
    w.captured = w.captured || capturing;
    *out = w.p;
    return RLXQ_OK;
  }
  // Geometric growth: an ascending run of sizes replaces O(log) buffers.
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  if (want < w.bytes + w.bytes / 2) want = w.bytes + w.bytes / 2;
  want = (want + 4095) & ~size_t(4095);
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ctx, RLXQ_E_NOMEM,
                "workspace: hipMalloc(" + std::to_string(want) + "): " + hip_msg(e) +
                    " (under stream capture, size the scratch first with rlxq_reserve_workspace)");
  }
  // The buffer being replaced may still be read by queued work: an event
  // behind that work frees it later.  One that a captured graph may name is
  // kept until the stream is released.  Nothing waits here.
  if (w.p) {
    rlxq_ctx::Retired r{w.p, w.bytes, nullptr};
    if (!w.captured && !capturing) {
      hipEvent_t ev = nullptr;
      if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess) {
        if (hipEventRecord(ev, hs) == hipSuccess) r.done = ev;
        else (void)hipEventDestroy(ev);
      }
      (void)hipGetLastError();
    }
    w.retired.push_back(r);
  }
  w.p = p;
  w.bytes = want;
  w.captured = capturing;
  *out = w.p;
  return RLXQ_OK;
}

void reclaim_retired(rlxq_ctx::Scratch& w) {
  size_t keep = 0;
  for (size_t i = 0; i < w.retired.size(); i++) {
    rlxq_ctx::Retired& r = w.retired[i];
    if (r.done && hipEventQuery(r.done) == hipSuccess) {
      (void)hipFree(r.p);
      (void)hipEventDestroy(r.done);
      continue;
    }
    (void)hipGetLastError();   // (hipErrorNotReady)
    w.retired[keep++] = r;
  }
  w.retired.resize(keep);
}

void free_retired(rlxq_ctx::Scratch& w) {
  for (rlxq_ctx::Retired& r : w.retired) {
    (void)hipFree(r.p);
    if (r.done) (void)hipEventDestroy(r.done);
  }
  w.retired.clear();
}

int zeroed_counters(rlxq_ctx* ctx, void* stream, int32_t** out) {
  rlxq_ctx::Scratch& w = ctx->ws[stream];
  if (!w.counters) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &st) != hipSuccess ||
        st != hipStreamCaptureStatusNone) {
      (void)hipGetLastError();
      return fail(ctx, RLXQ_E_SCRATCH,
                  "counters: first use under stream capture (call rlxq_reserve_workspace on the stream first)");
    }
    void* p = nullptr;
    const size_t bytes = (size_t)rlxq_ctx::kCounterSlots * sizeof(int32_t);
    hipError_t e = hipMalloc(&p, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(p, 0, bytes, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
      (void)hipGetLastError();
      if (p) (void)hipFree(p);
      return fail(ctx, RLXQ_E_NOMEM, "counters: " + hip_msg(e));
    }
    w.counters = static_cast<int32_t*>(p);
  }
  *out = w.counters;
  return RLXQ_OK;
}

bool is_gguf(int s) { return s == RLXQ_GGUF_Q8_0 || s == RLXQ_GGUF_Q4_0 || s == RLXQ_GGUF_Q4_1; }
bool is_mlx(int s) { return s == RLXQ_MLX_AFFINE4 || s == RLXQ_MLX_AFFINE8; }

int64_t kquant_bytes(int s) {
  switch (s) {
    case RLXQ_GGUF_Q4_K: return 144;
    case RLXQ_GGUF_Q6_K: return 210;
    case RLXQ_GGUF_Q5_K: return 176;
    case RLXQ_GGUF_Q3_K: return 110;
    case RLXQ_GGUF_Q2_K: return 84;
    case RLXQ_GGUF_Q8_K: return 292;
    default: return -1;
  }
}

int64_t gguf_block_bytes(int s) {
  switch (s) {
    case RLXQ_GGUF_Q8_0: return 34;
    case RLXQ_GGUF_Q4_0: return 18;
    case RLXQ_GGUF_Q4_1: return 20;
    default: return -1;
  }
}

}  // namespace rlxq

using namespace rlxq;

extern "C" {

const char* rlxq_version(void) { return "rlxq 0.1.0 gfx950"; }

const char* rlxq_strerror(int s) {
  switch (s) {
    case RLXQ_OK: return "ok";
    case RLXQ_E_NULL: return "null pointer";
    case RLXQ_E_SHAPE: return "bad shape";
    case RLXQ_E_SCHEME: return "unsupported scheme";
    case RLXQ_E_ALIGN: return "misaligned pointer or K";
    case RLXQ_E_DTYPE: return "unsupported dtype";
    case RLXQ_E_HIP: return "HIP runtime error";
    case RLXQ_E_NOMEM: return "out of memory";
    case RLXQ_E_INDEX: return "expert index out of range";
    case RLXQ_E_NOKERNEL: return "kernel variant not available";
    case RLXQ_E_DEVICE: return "device is not gfx950";
    case RLXQ_E_IO: return "checkpoint file cannot be opened or read";
    case RLXQ_E_FORMAT: return "not a valid GGUF file";
    case RLXQ_E_NOTFOUND: return "no tensor or key of that name";
    case RLXQ_E_TAKEN: return "weight already taken";
    case RLXQ_E_SCRATCH: return "call needs more scratch than the no-allocation entry point holds";
    default: return "unknown status";
  }
}

const char* rlxq_last_error(const rlxq_ctx* ctx) { return ctx ? ctx->last_error.c_str() : ""; }

const char* rlxq_last_kernel(const rlxq_ctx* ctx) { return ctx ? ctx->last_kernel.c_str() : ""; }

int64_t rlxq_row_bytes(int scheme, int64_t k) {
  if (const int64_t sb = kquant_bytes(scheme); sb > 0) return (k <= 0 || k % 256) ? -1 : k / 256 * sb;
  int64_t bb = gguf_block_bytes(scheme);
  if (bb < 0 || k <= 0 || k % 32) return -1;
  return k / 32 * bb;
}

int rlxq_init(int device, rlxq_ctx** out) {
  if (!out) return RLXQ_E_NULL;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
    (void)hipGetLastError();
    return RLXQ_E_DEVICE;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return RLXQ_E_HIP;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return RLXQ_E_DEVICE;
  DeviceGuard g(device);
  if (!g.ok()) return RLXQ_E_HIP;
  rlxq_ctx* ctx = new (std::nothrow) rlxq_ctx();
  if (!ctx) return RLXQ_E_NOMEM;
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  ctx->max_lds = prop.sharedMemPerBlock;
  noalloc_setup(ctx);
  for (const Image& im : kImages) {
    if (im.end - im.begin <= 1) continue;  // component not built into this library
    hipModule_t m = nullptr;
    hipError_t e = hipModuleLoadData(&m, im.begin);
    if (e != hipSuccess) {
      std::fprintf(stderr, "rlxq: hipModuleLoadData(%s): %s\n", im.name, hip_msg(e).c_str());
      for (hipModule_t mm : ctx->modules) (void)hipModuleUnload(mm);
      delete ctx;
      return RLXQ_E_HIP;
    }
    ctx->modules.push_back(m);
  }
  *out = ctx;
  return RLXQ_OK;
}

int rlxq_destroy(rlxq_ctx* ctx) {
  if (!ctx) return RLXQ_E_NULL;
  {
    DeviceGuard g(ctx->device);
    if (!ctx->ws.empty()) (void)hipDeviceSynchronize();
    for (auto& kv : ctx->ws) {
      if (kv.second.p) (void)hipFree(kv.second.p);
      if (kv.second.counters) (void)hipFree(kv.second.counters);
      free_retired(kv.second);
    }
    for (hipModule_t m : ctx->modules) (void)hipModuleUnload(m);
  }
  delete ctx;
  return RLXQ_OK;
}

int rlxq_reserve_workspace(rlxq_ctx* ctx, void* stream, size_t bytes) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  DeviceGuard g(ctx->device);
  if (!g.ok()) return fail(ctx, RLXQ_E_HIP, "reserve_workspace: hipSetDevice");
  void* p = nullptr;
  int32_t* c = nullptr;
  const int rc = workspace(ctx, bytes, &p, stream);
  return rc ? rc : zeroed_counters(ctx, stream, &c);
}

int64_t rlxq_workspace_bytes(const rlxq_ctx* ctx, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  auto it = ctx->ws.find(stream);
  return it == ctx->ws.end() ? 0 : (int64_t)it->second.bytes;
}

int64_t rlxq_workspace_retired_bytes(const rlxq_ctx* ctx, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  auto it = ctx->ws.find(stream);
  if (it == ctx->ws.end()) return 0;
  int64_t t = 0;
  for (const rlxq_ctx::Retired& r : it->second.retired) t += (int64_t)r.bytes;
  return t;
}

int rlxq_release_stream(rlxq_ctx* ctx, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  auto it = ctx->ws.find(stream);
  if (it == ctx->ws.end()) return RLXQ_OK;
  DeviceGuard g(ctx->device);
  if (!g.ok()) return fail(ctx, RLXQ_E_HIP, "release_stream: hipSetDevice");
  // Work queued on the stream may still use its buffers.
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(ctx, RLXQ_E_HIP, "release_stream: sync: " + hip_msg(e));
  if (it->second.p) (void)hipFree(it->second.p);
  if (it->second.counters) (void)hipFree(it->second.counters);
  free_retired(it->second);
  ctx->ws.erase(it);
  return RLXQ_OK;
}

int rlxq_dequant_matmul(rlxq_ctx* ctx, int scheme, int group_size, const void* x, int x_dtype,
                        const void* w, const void* scales, const void* biases, int sb_dtype,
                        int64_t m, int64_t k, int64_t n, void* y, int y_dtype, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  ctx->last_error.clear();
  if (!x || !w || !y) return fail(ctx, RLXQ_E_NULL, "dequant_matmul: x, w and y must be non-null");
  if (m < 0 || k <= 0 || n < 0) return fail(ctx, RLXQ_E_SHAPE, "dequant_matmul: need m >= 0, k > 0, n >= 0");
  if (x_dtype != RLXQ_F32 && x_dtype != RLXQ_BF16) return fail(ctx, RLXQ_E_DTYPE, "dequant_matmul: x_dtype");
  if (y_dtype != RLXQ_F32 && y_dtype != RLXQ_BF16) return fail(ctx, RLXQ_E_DTYPE, "dequant_matmul: y_dtype");
  if (m == 0 || n == 0) return RLXQ_OK;
  DeviceGuard g(ctx->device);
  if (!g.ok()) return fail(ctx, RLXQ_E_HIP, "dequant_matmul: hipSetDevice");
  return gemv_dispatch(ctx, scheme, group_size, x, x_dtype, w, scales, biases, sb_dtype, m, k, n, y,
                       y_dtype, stream);
}

}  // extern "C"
