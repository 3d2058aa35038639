// File -> host / device transfer shared by the checkpoint readers.
#include "file_io.hpp"

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <thread>
#include <vector>

#include "rlxq.h"

namespace rlxq {

bool pread_all(int fd, void* dst, uint64_t n, uint64_t off) {
  uint8_t* d = static_cast<uint8_t*>(dst);
  while (n) {
    const size_t want = (size_t)std::min<uint64_t>(n, uint64_t(1) << 30);
    const ssize_t r = pread(fd, d, want, (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    d += r;
    off += (uint64_t)r;
    n -= (uint64_t)r;
  }
  return true;
}

bool pread_par(int fd, uint8_t* dst, uint64_t n, uint64_t off) {
  constexpr uint64_t kPart = uint64_t(4) << 20;
  const int parts = (int)std::min<uint64_t>(8, (n + kPart - 1) / kPart);
  if (parts <= 1) return pread_all(fd, dst, n, off);
  const uint64_t step = (n + parts - 1) / parts;
  std::atomic<bool> ok{true};
  std::vector<std::thread> th;
  uint64_t lo = step;   // part 0 runs on this thread
  try {
    for (; lo < n; lo += step) {
      const uint64_t len = std::min(step, n - lo);
      th.emplace_back([&ok, fd, dst, off, lo, len] {
        if (!pread_all(fd, dst + lo, len, off + lo)) ok = false;
      });
    }
  } catch (...) {   // no thread: read the remaining parts here
    if (!pread_all(fd, dst + lo, n - lo, off + lo)) ok = false;
  }
  if (!pread_all(fd, dst, std::min(step, n), off)) ok = false;
  for (auto& t : th) t.join();
  return ok;
}

StagedUpload::~StagedUpload() {
  for (int b = 0; b < 2; b++) {
    if (ev_[b]) {
      if (live_[b]) (void)hipEventSynchronize(ev_[b]);
      (void)hipEventDestroy(ev_[b]);
    }
    if (stage_[b]) (void)hipHostFree(stage_[b]);
  }
}

int StagedUpload::run(int fd, uint64_t off, uint64_t len, void* dst, void* stream, std::string* err) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int b = 0; b < 2; b++) {
    if (!stage_[b] && hipHostMalloc(&stage_[b], kStageBytes, hipHostMallocDefault) != hipSuccess) {
      stage_[b] = nullptr;
      *err = "pinned staging allocation failed";
      return RLXQ_E_NOMEM;
    }
    if (!ev_[b] && hipEventCreateWithFlags(&ev_[b], hipEventDisableTiming) != hipSuccess) {
      ev_[b] = nullptr;
      *err = "event creation failed";
      return RLXQ_E_HIP;
    }
  }
  uint8_t* d = static_cast<uint8_t*>(dst);
  int b = 0;
  for (uint64_t done = 0; done < len; done += kStageBytes, b ^= 1) {
    const uint64_t n = std::min<uint64_t>(kStageBytes, len - done);
    // the copy that last read this buffer must be finished before refilling it
    if (live_[b] && hipEventSynchronize(ev_[b]) != hipSuccess) {
      *err = "waiting for a staging copy failed";
      return RLXQ_E_HIP;
    }
    live_[b] = false;
    if (!pread_par(fd, static_cast<uint8_t*>(stage_[b]), n, off + done)) {
      *err = "read failed";
      return RLXQ_E_IO;
    }
    if (hipMemcpyAsync(d + done, stage_[b], n, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipEventRecord(ev_[b], s) != hipSuccess) {
      *err = "copy to the device failed";
      return RLXQ_E_HIP;
    }
    live_[b] = true;
  }
  return RLXQ_OK;
}

}  // namespace rlxq
