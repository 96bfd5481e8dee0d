// HIP runtime state, HBM caching allocator and pinned host allocator of the
// spyre backend.  See spyre_runtime.h.
#include "spyre_runtime.h"

#include <c10/core/CPUAllocator.h>
#include <c10/core/DeviceType.h>
#include <c10/util/Exception.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <map>
#include <mutex>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace spyre {

namespace {

constexpr int kMaxDevices = 64;

std::once_flag g_start_once;
std::atomic<bool> g_started{false};
int g_device_count = 0;

// Per-device lazily created state is published with a release store after
// its creation under the mutex and read with an acquire load, so a reader
// that sees the pointer also sees what it points to.
std::mutex g_stream_mu;
std::array<std::atomic<hipStream_t>, kMaxDevices> g_streams{};

std::array<std::atomic<uint64_t>, kMaxDevices> g_seeds{};
// Philox counter offset of each device's generator (blocks used so far).
std::array<std::atomic<uint64_t>, kMaxDevices> g_rng_offsets{};

// Per device: the host address of its error word and the device-side
// address kernels are given.
std::mutex g_err_mu;
std::array<std::atomic<int32_t*>, kMaxDevices> g_err_host{};
std::array<std::atomic<int32_t*>, kMaxDevices> g_err_dev{};

// Makes `device` current for a scope and restores the caller's device when
// the scope ends, also when a HIP check throws inside it.
class DeviceScope {
 public:
  explicit DeviceScope(int device) {
    SPYRE_HIP_CHECK(hipGetDevice(&prev_));
    if (prev_ != device) SPYRE_HIP_CHECK(hipSetDevice(device));
  }
  ~DeviceScope() { (void)hipSetDevice(prev_); }
  DeviceScope(const DeviceScope&) = delete;
  DeviceScope& operator=(const DeviceScope&) = delete;

 private:
  int prev_ = 0;
};

void do_start() {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    n = 0;
  }
  g_device_count = std::min(n, kMaxDevices);
  g_started = true;
}

}  // namespace

void start_runtime() { std::call_once(g_start_once, do_start); }

bool runtime_started() { return g_started.load(); }

int device_count() {
  start_runtime();
  return g_device_count;
}

int current_device() {
  int d = 0;
  SPYRE_HIP_CHECK(hipGetDevice(&d));
  return d;
}

void set_device(int device) {
  TORCH_CHECK(device >= 0 && device < device_count(), "spyre: invalid device index ", device,
              " (", device_count(), " device(s) visible)");
  int cur = -1;
  SPYRE_HIP_CHECK(hipGetDevice(&cur));
  if (cur != device) SPYRE_HIP_CHECK(hipSetDevice(device));
}

hipStream_t stream(int device) {
  if (device < 0) device = current_device();
  TORCH_CHECK(device < device_count(), "spyre: invalid device index ", device);
  hipStream_t s = g_streams[device].load(std::memory_order_acquire);
  if (s) return s;
  std::lock_guard<std::mutex> lk(g_stream_mu);
  s = g_streams[device].load(std::memory_order_relaxed);
  if (!s) {
    DeviceScope scope(device);
    SPYRE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    g_streams[device].store(s, std::memory_order_release);
  }
  return s;
}

void synchronize(int device) {
  if (device >= 0) {
    hipStream_t s = g_streams[device].load(std::memory_order_acquire);
    if (s) SPYRE_HIP_CHECK(hipStreamSynchronize(s));
    release_copy_keepalive(device);
    check_device_errors(device);
    return;
  }
  for (int d = 0; d < device_count(); ++d) {
    hipStream_t s = g_streams[d].load(std::memory_order_acquire);
    if (s) SPYRE_HIP_CHECK(hipStreamSynchronize(s));
  }
  release_copy_keepalive(-1);
  check_device_errors(-1);
}

int32_t* device_error_word(int device) {
  if (device < 0) device = current_device();
  TORCH_CHECK(device < device_count(), "spyre: invalid device index ", device);
  int32_t* dev = g_err_dev[device].load(std::memory_order_acquire);
  if (dev) return dev;
  std::lock_guard<std::mutex> lk(g_err_mu);
  dev = g_err_dev[device].load(std::memory_order_relaxed);
  if (!dev) {
    DeviceScope scope(device);
    void* h = nullptr;
    // fine-grained (coherent) so a kernel's store is visible to the host
    // once the kernel has completed
    SPYRE_HIP_CHECK(hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent));
    __atomic_store_n(static_cast<int32_t*>(h), 0, __ATOMIC_RELAXED);
    void* d = nullptr;
    SPYRE_HIP_CHECK(hipHostGetDevicePointer(&d, h, 0));
    dev = static_cast<int32_t*>(d);
    g_err_host[device].store(static_cast<int32_t*>(h), std::memory_order_release);
    g_err_dev[device].store(dev, std::memory_order_release);
  }
  return dev;
}

void check_device_errors(int device) {
  const int lo = device < 0 ? 0 : device;
  const int hi = device < 0 ? kMaxDevices : device + 1;
  for (int d = lo; d < hi; ++d) {
    int32_t* w = g_err_host[d].load(std::memory_order_acquire);
    if (w == nullptr || __atomic_load_n(w, __ATOMIC_ACQUIRE) == 0) continue;
    // read and clear in one step: two host threads never both report (or
    // both lose) the same error
    const int32_t code = __atomic_exchange_n(w, 0, __ATOMIC_ACQ_REL);
    if (code == 0) continue;
    if (code == 2)
      TORCH_CHECK_INDEX(false, "spyre: decode attention position outside the KV cache on "
                        "spyre:", d, " (code 2); the step wrote nothing");
    TORCH_CHECK_INDEX(false, "spyre: index out of range in a gather on spyre:", d,
                      " (index_select / embedding / an indexed load of a compiled kernel; "
                      "code ", code, "); the rows of out-of-range indices were zero-filled");
  }
}

bool has_sph(at::ScalarType t) {
  switch (t) {
    case at::kHalf:
    case at::kBFloat16:
    case at::kFloat:
    case at::kDouble:
    case at::kChar:
    case at::kByte:
    case at::kShort:
    case at::kInt:
    case at::kLong:
    case at::kBool:
      return true;
    default:
      return false;
  }
}

sph_dtype to_sph(at::ScalarType t) {
  switch (t) {
    case at::kHalf:
      return SPH_F16;
    case at::kBFloat16:
      return SPH_BF16;
    case at::kFloat:
      return SPH_F32;
    case at::kDouble:
      return SPH_F64;
    case at::kChar:
      return SPH_I8;
    case at::kByte:
      return SPH_U8;
    case at::kShort:
      return SPH_I16;
    case at::kInt:
      return SPH_I32;
    case at::kLong:
      return SPH_I64;
    case at::kBool:
      return SPH_BOOL;
    default:
      TORCH_CHECK(false, "spyre: dtype ", t, " is not supported by the MI355X kernels");
  }
}

int64_t stick_alloc_nbytes(c10::IntArrayRef sizes, int64_t elem_bytes) {
  constexpr int64_t kStick = 128;
  if (sizes.empty()) return kStick;
  const int64_t per_stick = std::max<int64_t>(1, kStick / elem_bytes);
  int64_t n = kStick * ((sizes.back() + per_stick - 1) / per_stick);
  for (size_t i = 0; i + 1 < sizes.size(); ++i) n *= sizes[i];
  return n;
}

void set_seed(int device, uint64_t seed) {
  if (device < 0) {
    for (auto& s : g_seeds) s = seed;
    for (auto& o : g_rng_offsets) o = 0;
  } else {
    TORCH_CHECK(device < kMaxDevices, "spyre: invalid device index ", device);
    g_seeds[device] = seed;
    g_rng_offsets[device] = 0;
  }
}

uint64_t rng_offset_advance(int device, uint64_t blocks) {
  TORCH_CHECK(device >= 0 && device < kMaxDevices, "spyre: invalid device index ", device);
  return g_rng_offsets[device].fetch_add(blocks);
}

uint64_t get_seed(int device) { return g_seeds[device < 0 ? 0 : device].load(); }

// ---------------------------------------------------------------------------
// HBM caching allocator
//
// Blocks are rounded (512 B below 1 MiB, 2 MiB above) and cached per device
// on free.  A freed block is handed out again only for work that is ordered
// after its last use: every spyre kernel and copy of a device runs on that
// device's single spyre stream, so stream order guarantees it.  On an
// out-of-memory error the cache is released and hipMalloc retried.
//
// Private pools (graph capture): while a pool is active on a device, that
// device's allocations are served from, and freed back to, the pool only,
// so the addresses a captured HIP graph uses are never handed to other work;
// blocks keep their pool when freed after the capture.  Releasing the pool
// (when its graph is destroyed) moves its free blocks to the general cache
// and redirects later frees of its blocks there as well.
// ---------------------------------------------------------------------------
namespace {

struct Block {
  void* ptr;
  size_t size;
  int device;
  int64_t pool;  // 0: general cache, else a private pool id
};

class CachingAllocator final : public c10::Allocator {
 public:
  at::DataPtr allocate(size_t nbytes) override {
    start_runtime();
    const int dev = current_device();
    const c10::Device device(c10::DeviceType::PrivateUse1, static_cast<c10::DeviceIndex>(dev));
    if (nbytes == 0) return {nullptr, nullptr, &noop_delete, device};
    const size_t size = round_size(nbytes);
    Block* b = nullptr;
    int64_t pool_id = 0;
    {
      std::lock_guard<std::mutex> lk(mu_);
      pool_id = active_pool_[dev];
      auto& pool = pool_id ? private_free_[pool_id] : free_[dev];
      // Best fit, without handing a block more than twice the request.
      auto it = pool.lower_bound(size);
      if (it != pool.end() && it->first <= 2 * size) {
        b = it->second;
        pool.erase(it);
      }
      stats_[dev].num_alloc_calls++;
    }
    if (!b) b = fresh_block(dev, size, pool_id);
    {
      std::lock_guard<std::mutex> lk(mu_);
      auto& st = stats_[dev];
      st.allocated += static_cast<int64_t>(b->size);
      st.peak_allocated = std::max(st.peak_allocated, st.allocated);
    }
    return {b->ptr, b, &release, device};
  }

  at::DeleterFnPtr raw_deleter() const override { return nullptr; }

  void copy_data(void* dest, const void* src, std::size_t count) const override {
    if (count == 0) return;
    hipStream_t s = stream(-1);
    SPYRE_HIP_CHECK(hipMemcpyAsync(dest, src, count, hipMemcpyDeviceToDevice, s));
  }

  MemoryStats stats(int dev) {
    std::lock_guard<std::mutex> lk(mu_);
    return stats_[dev];
  }

  void empty_cache() {
    synchronize(-1);
    std::lock_guard<std::mutex> lk(mu_);
    for (int d = 0; d < kMaxDevices; ++d) {
      for (auto& kv : free_[d]) {
        Block* b = kv.second;
        (void)hipFree(b->ptr);
        stats_[d].reserved -= static_cast<int64_t>(b->size);
        delete b;
      }
      free_[d].clear();
    }
  }

  static CachingAllocator& instance() {
    static CachingAllocator* inst = new CachingAllocator();  // never destroyed
    return *inst;
  }

  int64_t begin_pool(int dev) {
    std::lock_guard<std::mutex> lk(mu_);
    TORCH_CHECK(active_pool_[dev] == 0, "spyre: a private pool is already active on spyre:",
                dev);
    const int64_t id = ++next_pool_;
    live_pools_.insert(id);
    active_pool_[dev] = id;
    return id;
  }

  void end_pool(int dev) {
    std::lock_guard<std::mutex> lk(mu_);
    active_pool_[dev] = 0;
  }

  void release_pool(int64_t id) {
    std::lock_guard<std::mutex> lk(mu_);
    live_pools_.erase(id);
    for (int d = 0; d < kMaxDevices; ++d)
      if (active_pool_[d] == id) active_pool_[d] = 0;
    auto it = private_free_.find(id);
    if (it == private_free_.end()) return;
    for (auto& kv : it->second) {
      kv.second->pool = 0;
      free_[kv.second->device].emplace(kv.first, kv.second);
    }
    private_free_.erase(it);
  }

 private:
  static size_t round_size(size_t n) {
    constexpr size_t kSmall = 512, kLarge = size_t(2) << 20, kSplit = size_t(1) << 20;
    if (n < kSplit) return (n + kSmall - 1) / kSmall * kSmall;
    return (n + kLarge - 1) / kLarge * kLarge;
  }

  Block* fresh_block(int dev, size_t size, int64_t pool_id) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, size);
    if (e == hipErrorOutOfMemory) {
      (void)hipGetLastError();
      empty_cache();
      e = hipMalloc(&p, size);
    }
    if (e != hipSuccess) {
      (void)hipGetLastError();
      MemoryStats st = stats(dev);
      TORCH_CHECK(false, "spyre: out of device memory allocating ", size, " bytes on spyre:",
                  dev, " (allocated ", st.allocated, ", reserved ", st.reserved, "): ",
                  hipGetErrorString(e));
    }
    std::lock_guard<std::mutex> lk(mu_);
    stats_[dev].reserved += static_cast<int64_t>(size);
    stats_[dev].num_device_mallocs++;
    return new Block{p, size, dev, pool_id};
  }

  static void release(void* ctx) {
    Block* b = static_cast<Block*>(ctx);
    auto& self = instance();
    std::lock_guard<std::mutex> lk(self.mu_);
    self.stats_[b->device].allocated -= static_cast<int64_t>(b->size);
    if (b->pool != 0 && self.live_pools_.count(b->pool)) {
      self.private_free_[b->pool].emplace(b->size, b);
    } else {
      b->pool = 0;
      self.free_[b->device].emplace(b->size, b);
    }
  }

  static void noop_delete(void*) {}

  std::mutex mu_;
  std::array<std::multimap<size_t, Block*>, kMaxDevices> free_;
  std::array<MemoryStats, kMaxDevices> stats_{};
  std::array<int64_t, kMaxDevices> active_pool_{};
  std::unordered_map<int64_t, std::multimap<size_t, Block*>> private_free_;
  std::unordered_set<int64_t> live_pools_;
  int64_t next_pool_ = 0;
};

// Pinned host memory for copy staging (hipHostMalloc, never hipHostRegister).
class PinnedAllocator final : public c10::Allocator {
 public:
  at::DataPtr allocate(size_t nbytes) override {
    const c10::Device cpu(c10::DeviceType::CPU);
    if (nbytes == 0) return {nullptr, nullptr, &free_pinned, cpu};
    void* p = nullptr;
    SPYRE_HIP_CHECK(hipHostMalloc(&p, nbytes, hipHostMallocDefault));
    {
      std::lock_guard<std::mutex> lk(mu_);
      live_[reinterpret_cast<uintptr_t>(p)] = nbytes;
    }
    return {p, p, &free_pinned, cpu};
  }
  at::DeleterFnPtr raw_deleter() const override { return &free_pinned; }
  void copy_data(void* dest, const void* src, std::size_t count) const override {
    std::memcpy(dest, src, count);
  }
  // p inside a live block (views and offsets of pinned tensors count).
  bool owns(const void* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    std::lock_guard<std::mutex> lk(mu_);
    auto it = live_.upper_bound(a);
    if (it == live_.begin()) return false;
    --it;
    return a < it->first + it->second;
  }
  static PinnedAllocator& instance() {
    static PinnedAllocator* inst = new PinnedAllocator();
    return *inst;
  }

 private:
  static void free_pinned(void* p) {
    if (!p) return;
    {
      auto& self = instance();
      std::lock_guard<std::mutex> lk(self.mu_);
      self.live_.erase(reinterpret_cast<uintptr_t>(p));
    }
    (void)hipHostFree(p);
  }
  std::mutex mu_;
  std::map<uintptr_t, size_t> live_;  // block base -> bytes
};

}  // namespace

c10::Allocator* device_allocator() { return &CachingAllocator::instance(); }
c10::Allocator* pinned_allocator() { return &PinnedAllocator::instance(); }
bool is_pinned_ptr(const void* p) { return PinnedAllocator::instance().owns(p); }

MemoryStats memory_stats(int device) {
  if (device < 0) device = current_device();
  return CachingAllocator::instance().stats(device);
}

void empty_cache() { CachingAllocator::instance().empty_cache(); }

// ---------------------------------------------------------------------------
// HIP graphs of the spyre stream
// ---------------------------------------------------------------------------
Graph::~Graph() { reset(); }

void Graph::capture_begin() {
  TORCH_CHECK(!capturing_ && exec_ == nullptr, "spyre graph: already captured; reset() first");
  device_ = current_device();
  hipStream_t s = stream(device_);
  // Work queued before the capture must not be part of it (and must not be
  // waited on from inside it).
  synchronize(device_);
  pool_ = CachingAllocator::instance().begin_pool(device_);
  hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) {
    CachingAllocator::instance().end_pool(device_);
    CachingAllocator::instance().release_pool(pool_);
    pool_ = 0;
    SPYRE_HIP_CHECK(e);
  }
  capturing_ = true;
}

void Graph::capture_end() {
  TORCH_CHECK(capturing_, "spyre graph: capture_end without capture_begin");
  capturing_ = false;
  CachingAllocator::instance().end_pool(device_);
  hipGraph_t g = nullptr;
  SPYRE_HIP_CHECK(hipStreamEndCapture(stream(device_), &g));
  graph_ = g;
  hipGraphExec_t x = nullptr;
  SPYRE_HIP_CHECK(hipGraphInstantiate(&x, g, nullptr, nullptr, 0));
  exec_ = x;
}

void Graph::replay() {
  TORCH_CHECK(exec_ != nullptr, "spyre graph: nothing captured");
  SPYRE_HIP_CHECK(hipGraphLaunch(static_cast<hipGraphExec_t>(exec_), stream(device_)));
}

void Graph::reset() {
  if (capturing_) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(stream(device_), &g);
    if (g) (void)hipGraphDestroy(g);
    (void)hipGetLastError();
    CachingAllocator::instance().end_pool(device_);
    capturing_ = false;
  }
  if (exec_) {
    synchronize(device_);
    (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec_));
    exec_ = nullptr;
  }
  if (graph_) {
    (void)hipGraphDestroy(static_cast<hipGraph_t>(graph_));
    graph_ = nullptr;
  }
  if (pool_) {
    CachingAllocator::instance().release_pool(pool_);
    pool_ = 0;
  }
}

void free_runtime() {
  if (!runtime_started()) return;
  empty_cache();
  std::lock_guard<std::mutex> lk(g_stream_mu);
  for (int d = 0; d < kMaxDevices; ++d) {
    hipStream_t s = g_streams[d].exchange(nullptr, std::memory_order_acq_rel);
    if (s) (void)hipStreamDestroy(s);
  }
}

}  // namespace spyre

// Registered for the PrivateUse1 device type when the extension loads
// (reference: REGISTER_ALLOCATOR, torch_spyre/csrc/spyre_mem.cpp:554).
REGISTER_ALLOCATOR(c10::DeviceType::PrivateUse1, &spyre::CachingAllocator::instance());
