// Internal declarations shared by the host-side translation units of librlxq.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "rlxq.h"

struct rlxq_ctx {
  int device = 0;
  std::vector<hipModule_t> modules;
  std::unordered_map<std::string, hipFunction_t> fn_cache;
  std::unordered_map<std::string, int> occ_cache;  // "kernel@lds" -> workgroups per CU
  std::string last_error;
  std::string last_kernel;
  int cu_count = 0;
  size_t max_lds = 65536;
  // Library-owned scratch (routing tables, quantised activations, split-K
  // partials), one buffer per stream so that calls on different streams can
  // overlap.  Grown on demand, by at least half its size each time, so the
  // buffers growth replaces add up to less than twice the live one.  A
  // replaced buffer moves to `retired`: if it was never handed out under
  // stream capture, with an event recorded behind the stream's queued work,
  // and it is freed once that event has completed (checked on later calls);
  // if a captured graph may name it (done == nullptr), it is kept until
  // rlxq_release_stream or rlxq_destroy.
  struct Retired {
    void* p;
    size_t bytes;
    hipEvent_t done;
  };
  struct Scratch {
    void* p = nullptr;
    size_t bytes = 0;
    bool captured = false;   // p was handed out while the stream was capturing
    std::vector<Retired> retired;
    // kCounterSlots int32 counters, zeroed when allocated; kernels that take
    // them leave them at zero (the fused MoE combine)
    int32_t* counters = nullptr;
  };
  static constexpr int64_t kCounterSlots = 16384;
  std::unordered_map<void*, Scratch> ws;
  // The no-allocation entry point's scratch: the device address of a static
  // device array (RLXQ_NOALLOC_SCRATCH_BYTES), looked up at init.  While
  // fixed_active, workspace() returns it instead of the per-stream buffers.
  void* fixed_p = nullptr;
  size_t fixed_bytes = 0;
  bool fixed_active = false;
  int fixed_status = RLXQ_E_HIP;
  std::string fixed_msg = "not set up";
};

#include "skinny_args.h"

namespace rlxq {

// Records `msg` as the context's last error and returns `code`.
int fail(rlxq_ctx* ctx, int code, const std::string& msg);

// Sets the context's device current for the lifetime of the guard.
class DeviceGuard {
 public:
  explicit DeviceGuard(int dev);
  ~DeviceGuard();
  bool ok() const { return ok_; }

 private:
  int prev_ = -1;
  bool ok_ = false;
};

// Looks a kernel up by name across the loaded code objects.
int get_fn(rlxq_ctx* ctx, const std::string& name, hipFunction_t* out);

// Looks up the no-allocation scratch of ctx->device (device current).
void noalloc_setup(rlxq_ctx* ctx);

// Workgroups of `threads` threads and `lds` bytes of LDS that one CU holds
// at once (cached per kernel and LDS size; at least 1).
int blocks_per_cu(rlxq_ctx* ctx, const std::string& name, hipFunction_t fn, int threads, size_t lds);

// Launches `fn` with the kernelParams array `args`.
int launch(rlxq_ctx* ctx, hipFunction_t fn, dim3 grid, dim3 block, size_t lds, void* stream,
           void** args, const char* what);

// Ensures at least `bytes` of context scratch for `stream`; returns its
// device pointer.
int workspace(rlxq_ctx* ctx, size_t bytes, void** out, void* stream);
// Frees the stream's retired buffers whose completion event has passed
// (reclaim), or all of them (free, after the stream has been synchronised).
void reclaim_retired(rlxq_ctx::Scratch& w);
void free_retired(rlxq_ctx::Scratch& w);
// The stream's zeroed counters (rlxq_ctx::kCounterSlots), allocated and
// cleared on the stream at first use (not under stream capture).
int zeroed_counters(rlxq_ctx* ctx, void* stream, int32_t** out);

bool is_gguf(int scheme);
bool is_mlx(int scheme);
// GGUF K-quant super-block bytes (256 weights): Q4_K 144, Q6_K 210, Q5_K
// 176, Q3_K 110, Q2_K 84, Q8_K 292; -1 for the other schemes.
int64_t kquant_bytes(int scheme);
// Slab dtype as the kernels read it (sb_bf16 field): 0 f32, 1 bf16, 2 bytes.
inline int sb_code(int sb_dtype) { return sb_dtype == RLXQ_BF16 ? 1 : (sb_dtype == RLXQ_U8 ? 2 : 0); }
int64_t gguf_block_bytes(int scheme);

// Validates a weight operand (scheme, alignment, MLX scale slabs) and returns
// the packed row stride in bytes.
int check_weights(rlxq_ctx* ctx, const char* what, int scheme, int group, const void* w, const void* scales,
                  const void* biases, int sb_dtype, int64_t k, int64_t* rb);
const char* scheme_name(int scheme);

// Entry points implemented in other translation units.
int gemv_dispatch(rlxq_ctx* ctx, int scheme, int group, const void* x, int x_dtype, const void* w,
                  const void* scales, const void* biases, int sb_dtype, int64_t m, int64_t k,
                  int64_t n, void* y, int y_dtype, void* stream);
bool skinny_applies(int scheme, int group, int sb_dtype, int64_t m, int64_t k);
// Order of the batched-decode activations within a 32-block: 1 the GGUF
// nibble-unpacking order, 2 MLX's 4-bit order, 0 natural (Q8_0, Q6_K, MLX
// 8-bit, MXFP4).
int sk_order(int scheme);
// MLX per-group scales and biases, or MXFP4's E8M0 scale bytes, for the
// batched-decode kernels (unused by the GGUF formats).
struct SkinnySb {
  const void* scales = nullptr;
  const void* biases = nullptr;
  int64_t group = 32;
  int32_t sb_bf16 = 0;
};
// Adds the [splits, M, N] f32 partial sums in a.part into a.y (y_ld, y_bf16)
// in slice order.
int splits_reduce(rlxq_ctx* ctx, rlxq_skinny_args& a, void* stream);
// x [m, k] -> prepared f16 activations (x16) and row factors (inv_s) at the
// start of the workspace; `extra` further bytes follow at *rest.  The
// fragment-major layout holds mp >= m rows (the rows past m zero); out_bf16
// stores bf16 instead of f16.  split: each row becomes two x16 rows, hi and
// lo (f32 activations keep ~22 significant bits), with a factor each: rows
// 2r, 2r + 1 (split 1), or 64-row blocks of 32 hi then 32 lo rows (split 2,
// row-major; m rounded up to 32, the extra rows zero).
int prep_x16(rlxq_ctx* ctx, const void* x, int x_dtype, int64_t m, int64_t k, int order, size_t extra,
             rlxq_x16_args& xa, char** rest, void* stream, bool frag_major = false, int64_t mp = 0,
             bool out_bf16 = false, int split = 0, int post_exp = 0);
// Exponent of the extra row factor the f16-MFMA kernels need for a scheme:
// -8 for MLX affine (their f16 weights are prescaled by 2^8), else 0.
int sk_post_exp(int scheme);
int skinny_dispatch(rlxq_ctx* ctx, int scheme, const void* x, int x_dtype, const void* w, int64_t rb, int64_t m,
                    int64_t k, int64_t n, void* y, int y_dtype, void* stream, const SkinnySb& sb = SkinnySb());
int i8b_dispatch(rlxq_ctx* ctx, int group, const void* x, int x_dtype, const void* w, const void* scales,
                 const void* zp, int sb_dtype, int64_t m, int64_t k, int64_t n, void* y, int y_dtype,
                 void* stream);

}  // namespace rlxq
