// Host<->device byte movement of the spyre backend.
//
// Reference: the reference's copies (torch_spyre/csrc/spyre_mem.cpp:281-438,
// 661-703) build and compile a DMA graph per call, convert every element on
// the host and accept `non_blocking` without acting on it.  Here a copy is
// a byte stream over the host link:
//   * pageable host memory goes through a per-device ring of pinned staging
//     buffers (4 x 16 MiB, hipHostMalloc): the host copies chunk i+1 into
//     one buffer (several threads) while the DMA engine moves chunk i out of
//     another, and an event per buffer stops the host from refilling a
//     buffer before its DMA has read it.  A host-to-device copy therefore
//     returns once its last chunk is staged (the source may be reused at
//     once); the device sees the data in stream order.  Device-to-host
//     copies keep several chunk DMAs in flight and drain them into the
//     destination as they land, and return when the data is there.
//   * pinned host memory (this backend's pinned allocator, or torch's) is
//     moved by one DMA straight from / to the user's buffer.  With
//     non_blocking=True nothing waits: the host storage is kept alive until
//     the copy's event has completed, and the caller synchronises before
//     touching the data (the torch contract for non-blocking copies).
#include <ATen/Parallel.h>
#include <ATen/detail/CUDAHooksInterface.h>

#include <algorithm>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <vector>

#include "spyre_ops_common.h"

namespace spyre {

namespace {

constexpr size_t kChunk = 16u << 20;     // bytes per staging buffer
constexpr int kSlots = 4;                 // staging buffers per device
constexpr size_t kParallelMin = 2u << 20;  // host copies split across threads above this
constexpr int64_t kPiece = 1 << 20;        // bytes per host thread task

void host_copy(void* dst, const void* src, size_t n) {
  if (n < kParallelMin) {
    std::memcpy(dst, src, n);
    return;
  }
  char* d = static_cast<char*>(dst);
  const char* s = static_cast<const char*>(src);
  at::parallel_for(0, static_cast<int64_t>(n), kPiece, [&](int64_t b, int64_t e) {
    std::memcpy(d + b, s + b, static_cast<size_t>(e - b));
  });
}

struct Slot {
  void* buf = nullptr;
  hipEvent_t ev = nullptr;
  bool pending = false;  // ev marks a DMA that uses buf
};

struct Engine {
  std::mutex mu;
  Slot slots[kSlots];
  int next = 0;
  bool ready = false;
  // Non-blocking pinned copies: (completion event, host storage kept alive).
  std::deque<std::pair<hipEvent_t, c10::Storage>> keep;

  void init(int dev) {
    if (ready) return;
    c10::DeviceGuard g(c10::Device(c10::DeviceType::PrivateUse1, static_cast<c10::DeviceIndex>(dev)));
    for (auto& s : slots) {
      SPYRE_HIP_CHECK(hipHostMalloc(&s.buf, kChunk, hipHostMallocDefault));
      SPYRE_HIP_CHECK(hipEventCreateWithFlags(&s.ev, hipEventDisableTiming));
    }
    ready = true;
  }
  Slot& take() {
    Slot& s = slots[next];
    next = (next + 1) % kSlots;
    if (s.pending) {
      SPYRE_HIP_CHECK(hipEventSynchronize(s.ev));
      s.pending = false;
    }
    return s;
  }
  // Drops keep-alive entries whose copies have completed (all when `all`,
  // after the stream has been synchronised).
  void reap(bool all) {
    while (!keep.empty()) {
      hipEvent_t ev = keep.front().first;
      if (!all) {
        const hipError_t q = hipEventQuery(ev);
        if (q == hipErrorNotReady) break;
        SPYRE_HIP_CHECK(q);
      }
      SPYRE_HIP_CHECK(hipEventDestroy(ev));
      keep.pop_front();
    }
  }
};

std::mutex g_engines_mu;
std::vector<std::unique_ptr<Engine>> g_engines;

Engine& engine(int dev) {
  std::lock_guard<std::mutex> lk(g_engines_mu);
  if (static_cast<int>(g_engines.size()) <= dev) g_engines.resize(dev + 1);
  if (!g_engines[dev]) g_engines[dev] = std::make_unique<Engine>();
  return *g_engines[dev];
}

void keep_alive(Engine& e, hipStream_t s, const c10::Storage& st) {
  hipEvent_t ev = nullptr;
  SPYRE_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  SPYRE_HIP_CHECK(hipEventRecord(ev, s));
  e.keep.emplace_back(ev, st);
}

}  // namespace

bool host_ptr_pinned(const void* p) {
  if (p == nullptr) return false;
  if (is_pinned_ptr(p)) return true;
  // torch's own pinned memory (pin_memory() on a ROCm build)
  const auto& hooks = at::detail::getCUDAHooks();
  return hooks.hasCUDA() && hooks.isPinnedPtr(p);
}

void h2d_bytes(int dev, void* dst, const at::Tensor& host, size_t n, bool non_blocking) {
  if (n == 0) return;
  hipStream_t s = stream(dev);
  Engine& e = engine(dev);
  std::lock_guard<std::mutex> lk(e.mu);
  e.reap(false);
  const char* src = static_cast<const char*>(host.data_ptr());
  if (host_ptr_pinned(src)) {
    SPYRE_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s));
    if (non_blocking)
      keep_alive(e, s, host.storage());
    else
      SPYRE_HIP_CHECK(hipStreamSynchronize(s));
    return;
  }
  e.init(dev);
  char* d = static_cast<char*>(dst);
  for (size_t off = 0; off < n; off += kChunk) {
    const size_t c = std::min(kChunk, n - off);
    Slot& sl = e.take();
    host_copy(sl.buf, src + off, c);
    SPYRE_HIP_CHECK(hipMemcpyAsync(d + off, sl.buf, c, hipMemcpyHostToDevice, s));
    SPYRE_HIP_CHECK(hipEventRecord(sl.ev, s));
    sl.pending = true;
  }
}

void d2h_bytes(int dev, const at::Tensor& host, const void* src, size_t n, bool non_blocking) {
  if (n == 0) return;
  hipStream_t s = stream(dev);
  Engine& e = engine(dev);
  std::lock_guard<std::mutex> lk(e.mu);
  e.reap(false);
  char* dst = static_cast<char*>(host.data_ptr());
  if (host_ptr_pinned(dst)) {
    SPYRE_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, s));
    if (non_blocking) {
      keep_alive(e, s, host.storage());
    } else {
      SPYRE_HIP_CHECK(hipStreamSynchronize(s));
      check_device_errors(dev);
    }
    return;
  }
  e.init(dev);
  const char* sp = static_cast<const char*>(src);
  const size_t nchunks = (n + kChunk - 1) / kChunk;
  std::vector<Slot*> used(nchunks, nullptr);
  auto issue = [&](size_t i) {
    const size_t off = i * kChunk, c = std::min(kChunk, n - off);
    Slot& sl = e.take();
    SPYRE_HIP_CHECK(hipMemcpyAsync(sl.buf, sp + off, c, hipMemcpyDeviceToHost, s));
    SPYRE_HIP_CHECK(hipEventRecord(sl.ev, s));
    sl.pending = true;
    used[i] = &sl;
  };
  const size_t ahead = std::min<size_t>(nchunks, kSlots);
  for (size_t i = 0; i < ahead; ++i) issue(i);
  for (size_t i = 0; i < nchunks; ++i) {
    Slot& sl = *used[i];
    SPYRE_HIP_CHECK(hipEventSynchronize(sl.ev));
    sl.pending = false;
    const size_t off = i * kChunk, c = std::min(kChunk, n - off);
    host_copy(dst + off, sl.buf, c);
    if (i + kSlots < nchunks) issue(i + kSlots);
  }
  check_device_errors(dev);
}

void release_copy_keepalive(int dev) {
  std::vector<Engine*> es;
  {
    std::lock_guard<std::mutex> lk(g_engines_mu);
    for (size_t d = 0; d < g_engines.size(); ++d)
      if (g_engines[d] && (dev < 0 || static_cast<int>(d) == dev)) es.push_back(g_engines[d].get());
  }
  for (Engine* e : es) {
    std::lock_guard<std::mutex> lk(e->mu);
    e->reap(true);
  }
}

}  // namespace spyre
