// Host-side session API: a C++ restatement of rlx-laguna's DeviceMatmul
// (crates/rlx-laguna/src/device_matmul.rs:82-296) over the rlxq C ABI.
//
// Host slices in, host f32 out.  Weights are uploaded once per distinct host
// pointer and byte length and stay resident, as the reference skips
// `set_param` when the weight pointer of a ShapeKey is unchanged (:41-62,
// :301-352).  Argument checks follow the reference's `bail!`s (:129-146,
// :177-196) and the scheme tag table (:64-76).
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <map>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "rlxq.h"

namespace rlxq {

class DeviceMatmul {
 public:
  static int try_new(int device, DeviceMatmul** out) {
    rlxq_ctx* ctx = nullptr;
    int rc = rlxq_init(device, &ctx);
    if (rc) return rc;
    auto* dm = new (std::nothrow) DeviceMatmul();
    if (!dm) {
      rlxq_destroy(ctx);
      return RLXQ_E_NOMEM;
    }
    dm->ctx_ = ctx;
    dm->device_ = device;
    int prev = -1;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device);
    hipError_t e = hipStreamCreate(&dm->stream_);
    if (prev >= 0) (void)hipSetDevice(prev);
    if (e != hipSuccess) {
      delete dm;
      return RLXQ_E_HIP;
    }
    *out = dm;
    return RLXQ_OK;
  }

  ~DeviceMatmul() {
    int prev = -1;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (auto& kv : resident_) (void)hipFree(kv.second);
    for (auto& kv : resident_gu_) (void)hipFree(kv.second);
    for (void* p : {x_dev_, y_dev_, idx_dev_, ids_dev_, mid_dev_}) (void)hipFree(p);
    if (stream_) (void)hipStreamDestroy(stream_);
    if (ctx_) rlxq_destroy(ctx_);
    if (prev >= 0) (void)hipSetDevice(prev);
  }

  const char* last_error() const { return err_.c_str(); }
  int64_t uploads() const { return uploads_; }

  // y[m*n] = x[m*k] . W^T (DeviceMatmul::matmul, device_matmul.rs:121-152).
  int matmul(const float* x, size_t x_len, const uint8_t* w, size_t w_len, size_t m, size_t k, size_t n,
             int scheme, float* y) {
    err_.clear();
    if (!x || !w || !y) return bail(RLXQ_E_NULL, "DeviceMatmul: null pointer");
    if (x_len != m * k) return bail(RLXQ_E_SHAPE, "DeviceMatmul x len " + std::to_string(x_len) + " != m*k=" + std::to_string(m * k));
    int rc = check_scheme(scheme);
    if (rc) return rc;
    if (w_len > UINT32_MAX) return bail(RLXQ_E_SHAPE, "DeviceMatmul: weight bytes too large");
    const int64_t rb = rlxq_row_bytes(scheme, (int64_t)k);
    if (rb < 0 || (uint64_t)rb * n != w_len)
      return bail(RLXQ_E_SHAPE, "DeviceMatmul: weight bytes " + std::to_string(w_len) + " != n * row_bytes(k)");
    if (m == 0 || n == 0) return RLXQ_OK;   // empty output
    Guard g(device_);
    void* wd = nullptr;
    if ((rc = resident(w, w_len, &wd))) return rc;
    if ((rc = ensure(&x_dev_, &x_cap_, x_len * 4)) || (rc = ensure(&y_dev_, &y_cap_, m * n * 4))) return rc;
    if ((rc = hip(hipMemcpyAsync(x_dev_, x, x_len * 4, hipMemcpyHostToDevice, stream_), "upload x"))) return rc;
    rc = rlxq_dequant_matmul(ctx_, scheme, 32, x_dev_, RLXQ_F32, wd, nullptr, nullptr, RLXQ_F32, (int64_t)m,
                             (int64_t)k, (int64_t)n, y_dev_, RLXQ_F32, stream_);
    if (rc) return bail(rc, rlxq_last_error(ctx_));
    if ((rc = hip(hipMemcpyAsync(y, y_dev_, m * n * 4, hipMemcpyDeviceToHost, stream_), "download y"))) return rc;
    return hip(hipStreamSynchronize(stream_), "sync");
  }

  // out[i] = x[i] . expert[expert_idx[i]]^T (DeviceMatmul::grouped_matmul,
  // device_matmul.rs:156-200).
  int grouped_matmul(const float* x, size_t x_len, const uint8_t* w, size_t w_len, const float* idx,
                     size_t idx_len, size_t m, size_t k, size_t n, size_t ne, int scheme, float* y) {
    err_.clear();
    if (!x || !w || !idx || !y) return bail(RLXQ_E_NULL, "DeviceMatmul grouped: null pointer");
    if (x_len != m * k) return bail(RLXQ_E_SHAPE, "DeviceMatmul grouped x len " + std::to_string(x_len) + " != m*k=" + std::to_string(m * k));
    if (idx_len != m) return bail(RLXQ_E_SHAPE, "DeviceMatmul grouped expert_idx len " + std::to_string(idx_len) + " != m=" + std::to_string(m));
    if (ne == 0) return bail(RLXQ_E_SHAPE, "DeviceMatmul grouped: num_experts == 0");
    int rc = check_scheme(scheme);
    if (rc) return rc;
    if (w_len > UINT32_MAX) return bail(RLXQ_E_SHAPE, "DeviceMatmul: weight bytes too large");
    const int64_t rb = rlxq_row_bytes(scheme, (int64_t)k);
    if (rb < 0 || (uint64_t)rb * n * ne != w_len)
      return bail(RLXQ_E_SHAPE, "DeviceMatmul grouped: weight bytes != num_experts * n * row_bytes(k)");
    if ((rc = check_idx(idx, m, ne, "DeviceMatmul grouped"))) return rc;
    if (m == 0 || n == 0) return RLXQ_OK;
    Guard g(device_);
    void* wd = nullptr;
    if ((rc = resident(w, w_len, &wd))) return rc;
    if ((rc = ensure(&x_dev_, &x_cap_, x_len * 4)) || (rc = ensure(&y_dev_, &y_cap_, m * n * 4)) ||
        (rc = ensure(&idx_dev_, &idx_cap_, m * 4)))
      return rc;
    if ((rc = hip(hipMemcpyAsync(x_dev_, x, x_len * 4, hipMemcpyHostToDevice, stream_), "upload x"))) return rc;
    if ((rc = hip(hipMemcpyAsync(idx_dev_, idx, m * 4, hipMemcpyHostToDevice, stream_), "upload idx"))) return rc;
    rc = rlxq_dequant_grouped_matmul(ctx_, scheme, 32, x_dev_, RLXQ_F32, wd, nullptr, nullptr, RLXQ_F32,
                                     (const float*)idx_dev_, (int64_t)m, (int64_t)k, (int64_t)n, (int64_t)ne,
                                     y_dev_, RLXQ_F32, stream_);
    if (rc) return bail(rc, rlxq_last_error(ctx_));
    if ((rc = hip(hipMemcpyAsync(y, y_dev_, m * n * 4, hipMemcpyDeviceToHost, stream_), "download y"))) return rc;
    return hip(hipStreamSynchronize(stream_), "sync");
  }

  // down(silu(gate(x)) * up(x)) per row, expert expert_idx[row] for all
  // three projections (DeviceMatmul::grouped_swiglu, device_matmul.rs:221-296;
  // its graph :383-426).  x [m, h], gate/up banks [E, inter, h], down bank
  // [E, h, inter], y [m, h].  Gate and up of one scheme are uploaded once into
  // a single gate|up bank (per expert: its inter gate rows, then its inter up
  // rows) and run as one fused launch with the SwiGLU in its epilogue;
  // different schemes run as two grouped launches and the SwiGLU kernel.
  int grouped_swiglu(const float* x, size_t x_len, const float* idx, size_t idx_len, const uint8_t* wg,
                     size_t wg_len, int gs, const uint8_t* wu, size_t wu_len, int us, const uint8_t* wd,
                     size_t wd_len, int ds, size_t m, size_t h, size_t inter, size_t ne, float* y) {
    err_.clear();
    if (!x || !idx || !wg || !wu || !wd || !y) return bail(RLXQ_E_NULL, "DeviceMatmul swiglu: null pointer");
    if (x_len != m * h) return bail(RLXQ_E_SHAPE, "DeviceMatmul swiglu x len " + std::to_string(x_len) + " != m*h=" + std::to_string(m * h));
    if (idx_len != m) return bail(RLXQ_E_SHAPE, "DeviceMatmul swiglu expert_idx len " + std::to_string(idx_len) + " != m=" + std::to_string(m));
    if (ne == 0) return bail(RLXQ_E_SHAPE, "DeviceMatmul swiglu: num_experts == 0");
    for (int s : {gs, us, ds})
      if (check_scheme(s)) return bail(RLXQ_E_SCHEME, "DeviceMatmul swiglu: unsupported scheme");
    const struct { const char* name; size_t len; int scheme; size_t rows, k; } ws[] = {
        {"gate", wg_len, gs, inter, h}, {"up", wu_len, us, inter, h}, {"down", wd_len, ds, h, inter}};
    for (const auto& w : ws) {
      if (w.len > UINT32_MAX) return bail(RLXQ_E_SHAPE, std::string("DeviceMatmul swiglu: ") + w.name + " weight bytes too large");
      const int64_t rb = rlxq_row_bytes(w.scheme, (int64_t)w.k);
      if (rb < 0 || (uint64_t)rb * w.rows * ne != w.len)
        return bail(RLXQ_E_SHAPE, std::string("DeviceMatmul swiglu: ") + w.name + " weight bytes != num_experts * rows * row_bytes");
    }
    int rc = check_idx(idx, m, ne, "DeviceMatmul swiglu");
    if (rc) return rc;
    if (m == 0) return RLXQ_OK;
    Guard g(device_);
    const size_t mid_bytes = m * inter * 4;
    if ((rc = ensure(&x_dev_, &x_cap_, x_len * 4)) || (rc = ensure(&y_dev_, &y_cap_, m * h * 4)) ||
        (rc = ensure(&idx_dev_, &idx_cap_, m * 4)) || (rc = ensure(&ids_dev_, &ids_cap_, m * 4)) ||
        (rc = ensure(&mid_dev_, &mid_cap_, (gs == us ? 1 : 3) * mid_bytes)))
      return rc;
    if ((rc = hip(hipMemcpyAsync(x_dev_, x, x_len * 4, hipMemcpyHostToDevice, stream_), "upload x"))) return rc;
    if ((rc = hip(hipMemcpyAsync(idx_dev_, idx, m * 4, hipMemcpyHostToDevice, stream_), "upload idx"))) return rc;
    float* mid = static_cast<float*>(mid_dev_);
    if (gs == us) {
      // int32 ids for the fused gate|up launch (top_k = 1, entry i reads row i)
      ids_host_.resize(m);
      for (size_t i = 0; i < m; i++) ids_host_[i] = (int32_t)idx[i];
      if ((rc = hip(hipMemcpyAsync(ids_dev_, ids_host_.data(), m * 4, hipMemcpyHostToDevice, stream_), "upload ids")))
        return rc;
      void* gu = nullptr;
      if ((rc = resident_pair(wg, wg_len, wu, wu_len, ne, &gu))) return rc;
      rc = rlxq_moe_grouped(ctx_, gs, RLXQ_MOE_EXPAND_SWIGLU, x_dev_, RLXQ_F32, gu,
                            static_cast<const int32_t*>(ids_dev_), nullptr, (int64_t)m, 1, (int64_t)h,
                            (int64_t)(2 * inter), (int64_t)ne, mid, RLXQ_F32, stream_);
      if (rc) return bail(rc, rlxq_last_error(ctx_));
    } else {
      // gate into gu[0 .. m*inter), up into gu[m*inter .. 2*m*inter): the
      // SwiGLU of one row of length m*inter is then the elementwise rule
      void *wgd = nullptr, *wud = nullptr;
      if ((rc = resident(wg, wg_len, &wgd)) || (rc = resident(wu, wu_len, &wud))) return rc;
      float* gu = mid + m * inter;
      const float* di = static_cast<const float*>(idx_dev_);
      if ((rc = rlxq_dequant_grouped_matmul(ctx_, gs, 32, x_dev_, RLXQ_F32, wgd, nullptr, nullptr, RLXQ_F32, di,
                                            (int64_t)m, (int64_t)h, (int64_t)inter, (int64_t)ne, gu, RLXQ_F32,
                                            stream_)) ||
          (rc = rlxq_dequant_grouped_matmul(ctx_, us, 32, x_dev_, RLXQ_F32, wud, nullptr, nullptr, RLXQ_F32, di,
                                            (int64_t)m, (int64_t)h, (int64_t)inter, (int64_t)ne, gu + m * inter,
                                            RLXQ_F32, stream_)) ||
          (rc = rlxq_swiglu(ctx_, gu, RLXQ_F32, 1, (int64_t)(m * inter), mid, RLXQ_F32, stream_)))
        return bail(rc, rlxq_last_error(ctx_));
    }
    void* wdd = nullptr;
    if ((rc = resident(wd, wd_len, &wdd))) return rc;
    rc = rlxq_dequant_grouped_matmul(ctx_, ds, 32, mid, RLXQ_F32, wdd, nullptr, nullptr, RLXQ_F32,
                                     static_cast<const float*>(idx_dev_), (int64_t)m, (int64_t)inter, (int64_t)h,
                                     (int64_t)ne, y_dev_, RLXQ_F32, stream_);
    if (rc) return bail(rc, rlxq_last_error(ctx_));
    if ((rc = hip(hipMemcpyAsync(y, y_dev_, m * h * 4, hipMemcpyDeviceToHost, stream_), "download y"))) return rc;
    return hip(hipStreamSynchronize(stream_), "sync");
  }

 private:
  struct Guard {
    int prev = -1;
    explicit Guard(int d) {
      (void)hipGetDevice(&prev);
      if (prev != d) (void)hipSetDevice(d);
    }
    ~Guard() {
      int cur = -1;
      (void)hipGetDevice(&cur);
      if (prev >= 0 && cur != prev) (void)hipSetDevice(prev);
    }
  };

  int bail(int code, const std::string& msg) {
    err_ = msg;
    return code;
  }

  int hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return RLXQ_OK;
    return bail(RLXQ_E_HIP, std::string("DeviceMatmul: ") + what + ": " + hipGetErrorString(e));
  }

  // The schemes whose packed bytes are self-describing (device_matmul.rs:64-76
  // lists the GGUF tags; anything else is "unsupported scheme").
  int check_scheme(int scheme) {
    if (rlxq_row_bytes(scheme, 256) > 0) return RLXQ_OK;   // the GGUF block and K-quant schemes
    return bail(RLXQ_E_SCHEME, "DeviceMatmul: unsupported scheme " + std::to_string(scheme));
  }

  // every expert index an integer in [0, ne)
  int check_idx(const float* idx, size_t m, size_t ne, const char* what) {
    for (size_t i = 0; i < m; i++) {
      const float e = idx[i];
      if (!(e >= 0.f) || e >= (float)ne || std::floor(e) != e)
        return bail(RLXQ_E_INDEX, std::string(what) + ": expert_idx[" + std::to_string(i) + "] out of range");
    }
    return RLXQ_OK;
  }

  int ensure(void** p, size_t* cap, size_t bytes) {
    if (bytes <= *cap) return RLXQ_OK;
    if (*p) {
      (void)hipStreamSynchronize(stream_);
      (void)hipFree(*p);
      *p = nullptr;
      *cap = 0;
    }
    size_t want = bytes < 256 ? 256 : bytes;
    if (hipMalloc(p, want) != hipSuccess) {
      *p = nullptr;
      return bail(RLXQ_E_NOMEM, "DeviceMatmul: hipMalloc failed");
    }
    *cap = want;
    return RLXQ_OK;
  }

  int resident(const uint8_t* w, size_t len, void** out) {
    auto key = std::make_pair(reinterpret_cast<uintptr_t>(w), len);
    auto it = resident_.find(key);
    if (it != resident_.end()) {
      *out = it->second;
      return RLXQ_OK;
    }
    void* d = nullptr;
    if (hipMalloc(&d, len ? len : 1) != hipSuccess) return bail(RLXQ_E_NOMEM, "DeviceMatmul: weight hipMalloc failed");
    int rc = hip(hipMemcpyAsync(d, w, len, hipMemcpyHostToDevice, stream_), "upload w");
    if (rc) {
      (void)hipFree(d);
      return rc;
    }
    resident_.emplace(key, d);
    uploads_++;
    *out = d;
    return RLXQ_OK;
  }

  // The gate|up bank of a (gate, up) pair of host stacks with ne slabs each:
  // slab e of the result is gate slab e followed by up slab e.
  int resident_pair(const uint8_t* wg, size_t g_len, const uint8_t* wu, size_t u_len, size_t ne, void** out) {
    auto key = std::make_tuple(reinterpret_cast<uintptr_t>(wg), g_len, reinterpret_cast<uintptr_t>(wu), u_len);
    auto it = resident_gu_.find(key);
    if (it != resident_gu_.end()) {
      *out = it->second;
      return RLXQ_OK;
    }
    const size_t slab = g_len / ne;   // gate and up slabs are the same size (same scheme and shape)
    void* d = nullptr;
    if (hipMalloc(&d, 2 * g_len ? 2 * g_len : 1) != hipSuccess)
      return bail(RLXQ_E_NOMEM, "DeviceMatmul: gate|up hipMalloc failed");
    int rc = hip(hipMemcpy2DAsync(d, 2 * slab, wg, slab, slab, ne, hipMemcpyHostToDevice, stream_), "upload gate");
    if (!rc)
      rc = hip(hipMemcpy2DAsync(static_cast<char*>(d) + slab, 2 * slab, wu, slab, slab, ne, hipMemcpyHostToDevice,
                                stream_),
               "upload up");
    if (rc) {
      (void)hipStreamSynchronize(stream_);
      (void)hipFree(d);
      return rc;
    }
    (void)u_len;
    resident_gu_.emplace(key, d);
    uploads_++;
    *out = d;
    return RLXQ_OK;
  }

  rlxq_ctx* ctx_ = nullptr;
  int device_ = 0;
  hipStream_t stream_ = nullptr;
  std::map<std::pair<uintptr_t, size_t>, void*> resident_;
  std::map<std::tuple<uintptr_t, size_t, uintptr_t, size_t>, void*> resident_gu_;
  void* x_dev_ = nullptr;
  void* y_dev_ = nullptr;
  void* idx_dev_ = nullptr;
  void* ids_dev_ = nullptr;
  void* mid_dev_ = nullptr;
  size_t x_cap_ = 0, y_cap_ = 0, idx_cap_ = 0, ids_cap_ = 0, mid_cap_ = 0;
  std::vector<int32_t> ids_host_;
  int64_t uploads_ = 0;
  std::string err_;
};

}  // namespace rlxq

struct rlxq_device_matmul {
  rlxq::DeviceMatmul* impl;
};

extern "C" {

int rlxq_dm_try_new(int device, rlxq_device_matmul** out) {
  if (!out) return RLXQ_E_NULL;
  *out = nullptr;
  rlxq::DeviceMatmul* impl = nullptr;
  int rc = rlxq::DeviceMatmul::try_new(device, &impl);
  if (rc) return rc;
  *out = new rlxq_device_matmul{impl};
  return RLXQ_OK;
}

void rlxq_dm_free(rlxq_device_matmul* dm) {
  if (!dm) return;
  delete dm->impl;
  delete dm;
}

const char* rlxq_dm_last_error(const rlxq_device_matmul* dm) { return dm ? dm->impl->last_error() : ""; }

int rlxq_dm_matmul(rlxq_device_matmul* dm, const float* x, size_t x_len, const uint8_t* w_bytes, size_t w_len,
                   size_t m, size_t k, size_t n, int scheme, float* y) {
  if (!dm) return RLXQ_E_NULL;
  return dm->impl->matmul(x, x_len, w_bytes, w_len, m, k, n, scheme, y);
}

int rlxq_dm_grouped_matmul(rlxq_device_matmul* dm, const float* x, size_t x_len, const uint8_t* w_bytes,
                           size_t w_len, const float* expert_idx, size_t idx_len, size_t m, size_t k, size_t n,
                           size_t num_experts, int scheme, float* y) {
  if (!dm) return RLXQ_E_NULL;
  return dm->impl->grouped_matmul(x, x_len, w_bytes, w_len, expert_idx, idx_len, m, k, n, num_experts, scheme, y);
}

int rlxq_dm_grouped_swiglu(rlxq_device_matmul* dm, const float* x, size_t x_len, const float* expert_idx,
                           size_t idx_len, const uint8_t* w_gate, size_t gate_len, int gate_scheme,
                           const uint8_t* w_up, size_t up_len, int up_scheme, const uint8_t* w_down,
                           size_t down_len, int down_scheme, size_t m, size_t h, size_t inter, size_t num_experts,
                           float* y) {
  if (!dm) return RLXQ_E_NULL;
  return dm->impl->grouped_swiglu(x, x_len, expert_idx, idx_len, w_gate, gate_len, gate_scheme, w_up, up_len,
                                  up_scheme, w_down, down_len, down_scheme, m, h, inter, num_experts, y);
}

int64_t rlxq_dm_upload_count(const rlxq_device_matmul* dm) { return dm ? dm->impl->uploads() : -1; }

}  // extern "C"
