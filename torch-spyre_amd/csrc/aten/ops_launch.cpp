// Compiled-kernel loader and launcher of the spyre backend (torch.compile
// path).
//
// Reference: launchKernel (torch_spyre/csrc/module.cpp:64-170), which
// deserialises a Spyre program from disk, patches its inputs and runs
// Load/Compile/Parse/Predict on every call.  Here the Inductor backend
// compiles each generated kernel once (hiprtc, gfx950 code object); the
// code object is loaded into each device on first use and every call is one
// hipModuleLaunchKernel on the device's spyre stream, after a host-side
// check that no argument is addressed beyond its storage.
#include <pybind11/pybind11.h>
#include <torch/extension.h>

#include <array>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "spyre_ops_common.h"

namespace spyre {

namespace {

struct LoadedKernel {
  std::string code;
  std::string name;
  std::mutex mu;
  std::array<hipModule_t, 64> module{};
  std::array<hipFunction_t, 64> fn{};
};

std::mutex g_kernels_mu;
std::vector<std::unique_ptr<LoadedKernel>> g_kernels;

hipFunction_t function_for(LoadedKernel& k, int dev) {
  TORCH_CHECK(dev >= 0 && dev < 64, "spyre: device index out of range");
  std::lock_guard<std::mutex> lk(k.mu);
  if (!k.fn[dev]) {
    const int cur = current_device();
    if (cur != dev) set_device(dev);
    hipModule_t m = nullptr;
    SPYRE_HIP_CHECK(hipModuleLoadData(&m, k.code.data()));
    hipFunction_t f = nullptr;
    SPYRE_HIP_CHECK(hipModuleGetFunction(&f, m, k.name.c_str()));
    k.module[dev] = m;
    k.fn[dev] = f;
    if (cur != dev) set_device(cur);
  }
  return k.fn[dev];
}

}  // namespace

int64_t load_kernel(const std::string& code_object, const std::string& name) {
  TORCH_CHECK(!code_object.empty(), "spyre: empty code object");
  auto k = std::make_unique<LoadedKernel>();
  k->code = code_object;
  k->name = name;
  std::lock_guard<std::mutex> lk(g_kernels_mu);
  g_kernels.push_back(std::move(k));
  return static_cast<int64_t>(g_kernels.size()) - 1;
}

void launch_kernel(int64_t handle, const std::vector<at::Tensor>& args, int64_t grid,
                   int64_t block, const std::vector<int64_t>& extents) {
  LoadedKernel* k = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_kernels_mu);
    TORCH_CHECK(handle >= 0 && handle < static_cast<int64_t>(g_kernels.size()),
                "spyre: unknown kernel handle ", handle);
    k = g_kernels[handle].get();
  }
  TORCH_CHECK(!args.empty(), "spyre: launch_kernel needs tensor arguments");
  TORCH_CHECK(extents.size() == args.size(), "spyre: one extent per argument expected");
  TORCH_CHECK(grid > 0 && grid < (int64_t(1) << 31) && block > 0 && block <= 1024,
              "spyre: bad launch shape ", grid, " x ", block);
  const int dev = args[0].get_device();
  std::vector<void*> ptrs(args.size());
  for (size_t i = 0; i < args.size(); ++i) {
    const at::Tensor& t = args[i];
    TORCH_CHECK(is_spyre(t) && t.get_device() == dev, "spyre: kernel argument ", i,
                " is not on spyre:", dev);
    if (extents[i] >= 0) {
      const int64_t one = 1;
      const int64_t n = extents[i];
      check_extent(t, t.data_ptr(), 1, &n, &one, t.element_size(), "compiled kernel");
    }
    ptrs[i] = t.data_ptr();
  }
  std::vector<void*> params(args.size());
  for (size_t i = 0; i < args.size(); ++i) params[i] = &ptrs[i];
  hipFunction_t f = function_for(*k, dev);
  c10::DeviceGuard guard(args[0].device());
  SPYRE_HIP_CHECK(hipModuleLaunchKernel(f, static_cast<unsigned>(grid), 1, 1,
                                        static_cast<unsigned>(block), 1, 1, 0, stream(dev),
                                        params.data(), nullptr));
}

}  // namespace spyre
