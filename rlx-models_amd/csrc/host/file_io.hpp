// File -> host / device transfer shared by the checkpoint readers (GGUF,
// safetensors / MLX): positioned reads split over threads, and an upload
// through two pinned staging buffers, each copied to the device on the
// caller's stream while the other one is refilled.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>

namespace rlxq {

// pread until n bytes are read (false on an error or end of file).
bool pread_all(int fd, void* dst, uint64_t n, uint64_t off);
// pread_all split over up to 8 threads in parts of at least 4 MiB: one
// thread copying out of the page cache is slower than the copy to the device.
bool pread_par(int fd, uint8_t* dst, uint64_t n, uint64_t off);

class StagedUpload {
 public:
  static constexpr size_t kStageBytes = size_t(32) << 20;   // per staging buffer
  StagedUpload() = default;
  StagedUpload(const StagedUpload&) = delete;
  StagedUpload& operator=(const StagedUpload&) = delete;
  ~StagedUpload();
  // Bytes [off, off + len) of fd to device memory dst, copies queued on
  // stream; returns an rlxq status and sets *err on failure.  The buffers are
  // allocated on first use and kept until destruction.
  int run(int fd, uint64_t off, uint64_t len, void* dst, void* stream, std::string* err);

 private:
  void* stage_[2] = {nullptr, nullptr};
  hipEvent_t ev_[2] = {nullptr, nullptr};
  bool live_[2] = {false, false};
};

}  // namespace rlxq
