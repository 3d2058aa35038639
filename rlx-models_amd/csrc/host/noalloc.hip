// rlxq_dequant_matmul_noalloc: the dense DequantMatMul entry point for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// Its scratch (prepared activations, split-K partial sums) is one file-scope
// device array, `scratch`, of RLXQ_NOALLOC_SCRATCH_BYTES.  Each GPU holds its
// own copy, at its own address, until the process ends.  In host code the
// array's name is only a host-side handle: its device address on a device is
// taken once, with that device current, by hipGetSymbolAddress (from
// rlxq_init), kept per device, and only that address is ever handed to
// kernels.  Every call on one GPU shares that GPU's array, so calls that
// overlap on one GPU (two streams, two contexts, two threads) race on it.
// None of the dense path's kernels needs the scratch to start at zero: every
// byte they read there was written earlier in the same call.
//
// This file is compiled by hipcc (host code plus the device array) and linked
// into librlxq.so beside the g++ translation units.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "rlxq.h"
#include "rlxq_internal.hpp"

namespace {

static __device__ __align__(256) unsigned char scratch[RLXQ_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];        // device address of `scratch`, per device
hipError_t g_status[kMaxDevices];
bool g_done[kMaxDevices];

}  // namespace

namespace rlxq {

// Called by rlxq_init with `ctx->device` current: looks the array's address
// up once per device and records it (or the failure) in the context.
void noalloc_setup(rlxq_ctx* ctx) {
  const int dev = ctx->device;
  if (dev < 0 || dev >= kMaxDevices) {
    ctx->fixed_status = RLXQ_E_DEVICE;
    ctx->fixed_msg = "device index beyond the no-allocation table";
    return;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_done[dev]) {
    void* p = nullptr;
    g_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (g_status[dev] != hipSuccess) (void)hipGetLastError();
    g_ptr[dev] = g_status[dev] == hipSuccess ? p : nullptr;
    g_done[dev] = true;
  }
  if (g_status[dev] != hipSuccess || !g_ptr[dev]) {
    ctx->fixed_status = RLXQ_E_HIP;
    ctx->fixed_msg = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(g_status[dev]);
    return;
  }
  ctx->fixed_p = g_ptr[dev];
  ctx->fixed_bytes = RLXQ_NOALLOC_SCRATCH_BYTES;
  ctx->fixed_status = RLXQ_OK;
}

}  // namespace rlxq

extern "C" int rlxq_dequant_matmul_noalloc(rlxq_ctx* ctx, int scheme, int group_size, const void* x, int x_dtype,
                                           const void* w, const void* scales, const void* biases, int sb_dtype,
                                           int64_t m, int64_t k, int64_t n, void* y, int y_dtype, void* stream) {
  if (!ctx) return RLXQ_E_NULL;
  if (ctx->fixed_status != RLXQ_OK) {
    ctx->last_error = "dequant_matmul_noalloc: " + ctx->fixed_msg;
    return ctx->fixed_status;
  }
  // While set, the context's workspace() hands out ctx->fixed_p (never
  // allocating) and fails with RLXQ_E_SCRATCH past ctx->fixed_bytes.
  struct Fixed {
    rlxq_ctx* c;
    explicit Fixed(rlxq_ctx* c_) : c(c_) { c->fixed_active = true; }
    ~Fixed() { c->fixed_active = false; }
  } fixed(ctx);
  return rlxq_dequant_matmul(ctx, scheme, group_size, x, x_dtype, w, scales, biases, sb_dtype, m, k, n, y, y_dtype,
                             stream);
}
