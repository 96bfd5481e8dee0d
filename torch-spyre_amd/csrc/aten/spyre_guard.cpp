// Device guard and PrivateUse1 hooks of the spyre backend.
//
// Reference: SpyreGuardImpl / SpyreHooksInterface
// (torch_spyre/csrc/spyre_hooks.cpp:31-259) and the second guard of
// torch_spyre/csrc/spyre_mem.cpp:440-482.  Here exactly one guard is
// registered, it is backed by real HIP device/stream/event state (the
// reference's returns stream 0 and no-op events), and the hooks are handed
// to ATen through RegisterPrivateUse1HooksInterface (the reference keeps
// them in a private registry).
#include <ATen/detail/PrivateUse1HooksInterface.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>

#include "spyre_runtime.h"

namespace spyre {
namespace {

constexpr c10::DeviceType kDev = c10::DeviceType::PrivateUse1;

// Every spyre device has one stream (id 0): the stream spyre ops run on.
struct SpyreGuardImpl final : public c10::impl::DeviceGuardImplInterface {
  c10::DeviceType type() const override { return kDev; }

  c10::Device exchangeDevice(c10::Device d) const override {
    TORCH_INTERNAL_ASSERT(d.type() == kDev);
    const c10::Device old = getDevice();
    if (old.index() != d.index()) set_device(d.index());
    return old;
  }

  c10::Device getDevice() const override {
    // With no device visible (e.g. fake-tensor tracing on a host without a
    // GPU) the only meaningful index is 0; nothing is launched then.
    if (device_count() == 0) return c10::Device(kDev, 0);
    return c10::Device(kDev, static_cast<c10::DeviceIndex>(current_device()));
  }

  void setDevice(c10::Device d) const override {
    TORCH_INTERNAL_ASSERT(d.type() == kDev);
    set_device(d.index());
  }

  void uncheckedSetDevice(c10::Device d) const noexcept override {
    (void)hipSetDevice(d.index());
  }

  c10::Stream getStream(c10::Device d) const override {
    return c10::Stream(c10::Stream::UNSAFE, d, 0);
  }

  c10::Stream getDefaultStream(c10::Device d) const override { return getStream(d); }

  c10::Stream exchangeStream(c10::Stream s) const override { return s; }

  c10::DeviceIndex deviceCount() const noexcept override {
    int n = 0;
    try {
      n = device_count();
    } catch (...) {
      n = 0;
    }
    return static_cast<c10::DeviceIndex>(n);
  }

  void destroyEvent(void* event, const c10::DeviceIndex) const noexcept override {
    if (event) (void)hipEventDestroy(static_cast<hipEvent_t>(event));
  }

  void record(void** event, const c10::Stream& s, const c10::DeviceIndex device_index,
              const c10::EventFlag) const override {
    TORCH_CHECK(device_index == -1 || device_index == s.device_index(),
                "spyre: event device does not match the stream's device");
    const int dev = s.device_index();
    const int cur = current_device();
    if (cur != dev) set_device(dev);
    if (!*event) {
      hipEvent_t e = nullptr;
      SPYRE_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
      *event = e;
    }
    SPYRE_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(*event), stream(dev)));
    if (cur != dev) set_device(cur);
  }

  void block(void* event, const c10::Stream& s) const override {
    if (!event) return;
    SPYRE_HIP_CHECK(hipStreamWaitEvent(stream(s.device_index()), static_cast<hipEvent_t>(event), 0));
  }

  bool queryEvent(void* event) const override {
    if (!event) return true;
    hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
    if (e == hipErrorNotReady) {
      (void)hipGetLastError();
      return false;
    }
    SPYRE_HIP_CHECK(e);
    return true;
  }

  bool queryStream(const c10::Stream& s) const override {
    hipError_t e = hipStreamQuery(stream(s.device_index()));
    if (e == hipErrorNotReady) {
      (void)hipGetLastError();
      return false;
    }
    SPYRE_HIP_CHECK(e);
    return true;
  }

  void synchronizeStream(const c10::Stream& s) const override { synchronize(s.device_index()); }

  void synchronizeEvent(void* event) const override {
    if (event) SPYRE_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  }

  void synchronizeDevice(const c10::DeviceIndex device_index) const override {
    synchronize(device_index);
  }

  void recordDataPtrOnStream(const c10::DataPtr&, const c10::Stream&) const override {
    // One stream per device: stream order already protects cached blocks.
  }
};

C10_REGISTER_GUARD_IMPL(PrivateUse1, SpyreGuardImpl);

struct SpyreHooks final : public at::PrivateUse1HooksInterface {
  bool isBuilt() const override { return true; }
  bool isAvailable() const override { return device_count() > 0; }
  bool hasPrimaryContext(c10::DeviceIndex) const override { return runtime_started(); }
  void init() const override { start_runtime(); }

  at::Device getDeviceFromPtr(void* data) const override {
    hipPointerAttribute_t attr{};
    SPYRE_HIP_CHECK(hipPointerGetAttributes(&attr, data));
    return at::Device(kDev, static_cast<c10::DeviceIndex>(attr.device));
  }

  bool isPinnedPtr(const void* data) const override { return is_pinned_ptr(data); }

  c10::Allocator* getPinnedMemoryAllocator() const override { return pinned_allocator(); }

  void resizePrivateUse1Bytes(const c10::Storage& storage, size_t newsize) const override {
    // Grows or shrinks a storage by reallocating and copying the overlap.
    c10::StorageImpl* impl = storage.unsafeGetStorageImpl();
    TORCH_CHECK(impl->resizable(), "spyre: trying to resize a storage that is not resizable");
    const size_t old = impl->nbytes();
    at::DataPtr fresh = device_allocator()->allocate(newsize);
    const size_t n = std::min(old, newsize);
    if (n > 0 && impl->data()) {
      SPYRE_HIP_CHECK(hipMemcpyAsync(fresh.get(), impl->data(), n, hipMemcpyDeviceToDevice,
                                     stream(-1)));
    }
    impl->set_data_ptr_noswap(std::move(fresh));
    impl->set_nbytes(newsize);
  }
};

struct RegisterHooks {
  RegisterHooks() { at::RegisterPrivateUse1HooksInterface(new SpyreHooks()); }
};
RegisterHooks g_register_hooks;

}  // namespace
}  // namespace spyre
