// Device runtime of the "spyre" PrivateUse1 backend on MI355X: HIP device
// selection, the per-device stream every spyre op is ordered on, the HBM
// caching allocator, and the mapping from torch dtypes to the kernel
// library's element types.
//
// Reference counterparts (torch-spyre tree): _startRuntime / GlobalRuntime
// (torch_spyre/csrc/module.cpp:40-59, module.h:27-53), SpyreAllocator
// (torch_spyre/csrc/spyre_mem.cpp:486-554) and the guard's device/stream
// state (torch_spyre/csrc/spyre_hooks.cpp:54-256).
#pragma once

#include <ATen/ATen.h>
#include <c10/core/Allocator.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>

#include "spyre_hip.h"

namespace spyre {

#define SPYRE_HIP_CHECK(expr)                                                   \
  do {                                                                          \
    hipError_t err_ = (expr);                                                   \
    TORCH_CHECK(err_ == hipSuccess, "spyre: HIP error ", static_cast<int>(err_), \
                " (", hipGetErrorString(err_), ") in ", #expr);                 \
  } while (0)

// Non-zero status of a C-ABI entry point -> RuntimeError with its message.
#define SPYRE_SPH_CHECK(expr)                                                   \
  do {                                                                          \
    int rc_ = (expr);                                                           \
    TORCH_CHECK(rc_ == 0, "spyre: ", #expr, " failed (status ", rc_, "): ",     \
                sph_last_error());                                              \
  } while (0)

// Runtime start (idempotent, thread-safe): probes the HIP devices.
void start_runtime();
// Releases cached device memory and the per-device streams.
void free_runtime();
bool runtime_started();

int device_count();
int current_device();
void set_device(int device);

// The stream all spyre work on `device` is ordered on (-1: current device).
// Created on first use with default priority.
hipStream_t stream(int device = -1);
// Blocks until all spyre work on `device` (-1: every device) has finished,
// then raises for any out-of-range index a kernel reported meanwhile.
void synchronize(int device = -1);

// Device error word of `device`: 4 bytes of pinned host memory mapped into
// the device's address space (the device-side address is returned).  A
// kernel that meets an index outside its table writes a nonzero code there,
// zero-fills what that index would have produced and carries on: there is
// no device trap and no fault.  The host reads the word at every point where
// it waits for the device (synchronize, blocking device-to-host copies,
// .item()) and raises; torch's CPU kernels raise at the call instead.
int32_t* device_error_word(int device);
// Raises c10::IndexError if a kernel on `device` (-1: every device) reported
// an out-of-range index since the last check; the report is cleared first.
// Call only after the device work in question has completed.
void check_device_errors(int device = -1);

// Kernel-library element type of a torch dtype; throws for unsupported ones.
sph_dtype to_sph(at::ScalarType t);
bool has_sph(at::ScalarType t);

// The HBM caching allocator registered for PrivateUse1.
c10::Allocator* device_allocator();
// Pinned host memory (hipHostMalloc) for staging copies.
c10::Allocator* pinned_allocator();
// True for any address inside a block of pinned_allocator().
bool is_pinned_ptr(const void* p);

// Host<->device byte copies on the spyre stream of `dev` (spyre_copy.cpp).
// `host` is a CPU tensor whose n bytes from data_ptr() are the host side.
// Pageable host memory is staged through pinned buffers (h2d returns once
// staged, d2h once the data is in `host`); pinned host memory is moved
// directly and, with non_blocking, without waiting (the host storage is
// kept alive until the copy completes).
bool host_ptr_pinned(const void* p);
void h2d_bytes(int dev, void* dst, const at::Tensor& host, size_t n, bool non_blocking);
void d2h_bytes(int dev, const at::Tensor& host, const void* src, size_t n, bool non_blocking);
// Releases the host storages held for completed non-blocking copies (-1:
// every device); called by synchronize().
void release_copy_keepalive(int dev);

struct MemoryStats {
  int64_t allocated = 0;      // bytes in live blocks
  int64_t reserved = 0;       // bytes obtained from hipMalloc and not freed
  int64_t peak_allocated = 0;
  int64_t num_alloc_calls = 0;
  int64_t num_device_mallocs = 0;
};
MemoryStats memory_stats(int device);
void empty_cache();

// A HIP graph captured from the spyre stream of the current device.
// Allocations made during the capture come from a private pool that stays
// reserved for the graph until reset() (or destruction), so replays read
// and write the same buffers the capture saw.  Work captured must be
// stream-ordered spyre work only (no host synchronisation, no memory set
// nodes); a replay is asynchronous like any other spyre op.
class Graph {
 public:
  Graph() = default;
  ~Graph();
  Graph(const Graph&) = delete;
  Graph& operator=(const Graph&) = delete;
  void capture_begin();
  void capture_end();
  void replay();
  void reset();
  int64_t pool() const { return pool_; }

 private:
  int device_ = 0;
  int64_t pool_ = 0;
  bool capturing_ = false;
  void* graph_ = nullptr;
  void* exec_ = nullptr;
};

// Bytes the reference's stick-granular sizing gives a tensor of `sizes`
// (torch_spyre/csrc/spyre_mem.cpp:598-611, with the stick count rounded up):
// 128 bytes per 128-byte stick of the last dim, times the other dims; 128
// bytes for a 0-d tensor.
int64_t stick_alloc_nbytes(c10::IntArrayRef sizes, int64_t elem_bytes);

// The device generator: Philox4x32-10 keyed by the seed, its counter offset
// advanced by the blocks each fill uses.  set_seed resets the offset.
void set_seed(int device, uint64_t seed);
uint64_t get_seed(int device);
// Returns the offset of the next fill on `device` and advances it by `blocks`.
uint64_t rng_offset_advance(int device, uint64_t blocks);

}  // namespace spyre
