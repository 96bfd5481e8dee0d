// Compiled-kernel loader and launcher of the spyre backend (torch.compile
// path).
//
// Reference: launchKernel (torch_spyre/csrc/module.cpp:64-170, bound as
// launch_kernel(g2_path, args) at :176), which deserialises a Spyre program
// from disk, patches its inputs (the last argument is the output) and runs
// Load/Compile/Parse/Predict on every call.  Here the Inductor backend
// compiles each generated kernel once (hiprtc, gfx950 code object); the
// code object is loaded into each device on first use and every call is one
// hipModuleLaunchKernel on the device's spyre stream, after a host-side
// check that no argument is addressed beyond its storage.
//
// Three call forms:
//   launch_kernel(handle, args)                 launch shape stored at load
//   launch_kernel(path, args)                   the reference's form: `path`
//       is a gfx950 code object file and `path + ".launch"` its launch
//       description, one line "<kernel name> <grid> <block> <n> <extent>*n
//       [<error word>]"; the pair is read and registered on first use, then
//       cached by path
//   launch_kernel(handle, args, grid, block, extents)   explicit shape
// `args` are the kernel's parameters in order; the backend emits in-place
// buffers, then inputs, then outputs, so a kernel's single output is last as
// in the reference.  A kernel loaded with `error_word` (one that indexes
// indirectly) takes the device's error word as one more, last parameter,
// which the launcher appends.
#include <pybind11/pybind11.h>
#include <torch/extension.h>

#include <array>
#include <fstream>
#include <iterator>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "spyre_ops_common.h"

namespace spyre {

namespace {

struct LoadedKernel {
  std::string code;
  std::string name;
  // launch shape stored at load time (grid <= 0: none stored)
  int64_t grid = -1;
  int64_t block = -1;
  std::vector<int64_t> extents;
  bool error_word = false;
  std::mutex mu;
  std::array<hipModule_t, 64> module{};
  std::array<hipFunction_t, 64> fn{};
};

std::mutex g_kernels_mu;
std::vector<std::unique_ptr<LoadedKernel>> g_kernels;
std::unordered_map<std::string, int64_t> g_by_path;

void check_shape(int64_t grid, int64_t block) {
  TORCH_CHECK(grid > 0 && grid < (int64_t(1) << 31) && block > 0 && block <= 1024,
              "spyre: bad launch shape ", grid, " x ", block);
}

LoadedKernel* kernel_at(int64_t handle) {
  std::lock_guard<std::mutex> lk(g_kernels_mu);
  TORCH_CHECK(handle >= 0 && handle < static_cast<int64_t>(g_kernels.size()),
              "spyre: unknown kernel handle ", handle);
  return g_kernels[handle].get();
}

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

int64_t load_kernel(const std::string& code_object, const std::string& name, int64_t grid,
                    int64_t block, const std::vector<int64_t>& extents, bool error_word) {
  TORCH_CHECK(!code_object.empty(), "spyre: empty code object");
  TORCH_CHECK(!name.empty(), "spyre: empty kernel name");
  if (grid > 0 || block > 0) check_shape(grid, block);
  auto k = std::make_unique<LoadedKernel>();
  k->code = code_object;
  k->name = name;
  k->grid = grid;
  k->block = block;
  k->extents = extents;
  k->error_word = error_word;
  std::lock_guard<std::mutex> lk(g_kernels_mu);
  g_kernels.push_back(std::move(k));
  return static_cast<int64_t>(g_kernels.size()) - 1;
}

void launch_kernel(int64_t handle, const std::vector<at::Tensor>& args, int64_t grid,
                   int64_t block, const std::vector<int64_t>& extents) {
  LoadedKernel* k = kernel_at(handle);
  TORCH_CHECK(!args.empty(), "spyre: launch_kernel needs tensor arguments");
  TORCH_CHECK(extents.size() == args.size(), "spyre: one extent per argument expected (",
              extents.size(), " extents, ", args.size(), " arguments)");
  check_shape(grid, block);
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
  if (k->error_word) ptrs.push_back(device_error_word(dev));
  std::vector<void*> params(ptrs.size());
  for (size_t i = 0; i < ptrs.size(); ++i) params[i] = &ptrs[i];
  hipFunction_t f = function_for(*k, dev);
  c10::DeviceGuard guard(args[0].device());
  SPYRE_HIP_CHECK(hipModuleLaunchKernel(f, static_cast<unsigned>(grid), 1, 1,
                                        static_cast<unsigned>(block), 1, 1, 0, stream(dev),
                                        params.data(), nullptr));
}

void launch_kernel_stored(int64_t handle, const std::vector<at::Tensor>& args) {
  LoadedKernel* k = kernel_at(handle);
  TORCH_CHECK(k->grid > 0, "spyre: kernel ", handle,
              " was loaded without a launch shape; pass grid, block and extents");
  launch_kernel(handle, args, k->grid, k->block, k->extents);
}

int64_t load_kernel_file(const std::string& path) {
  {
    std::lock_guard<std::mutex> lk(g_kernels_mu);
    auto it = g_by_path.find(path);
    if (it != g_by_path.end()) return it->second;
  }
  std::ifstream co(path, std::ios::binary);
  TORCH_CHECK(co.good(), "spyre: cannot read code object ", path);
  std::string code((std::istreambuf_iterator<char>(co)), std::istreambuf_iterator<char>());
  std::ifstream meta(path + ".launch");
  TORCH_CHECK(meta.good(), "spyre: cannot read launch description ", path, ".launch");
  std::string name;
  int64_t grid = 0, block = 0, n = -1;
  meta >> name >> grid >> block >> n;
  TORCH_CHECK(!meta.fail() && n >= 0 && n <= 4096, "spyre: malformed launch description ", path,
              ".launch (expected \"<name> <grid> <block> <n> <extent>*n\")");
  std::vector<int64_t> extents(n);
  for (auto& e : extents) meta >> e;
  TORCH_CHECK(!meta.fail(), "spyre: launch description ", path, ".launch lists fewer than ", n,
              " extents");
  int64_t err_word = 0;
  if (!(meta >> err_word)) err_word = 0;  // optional last field
  TORCH_CHECK(grid > 0 && block > 0, "spyre: launch description ", path,
              ".launch has no launch shape");
  const int64_t h = load_kernel(code, name, grid, block, extents, err_word != 0);
  std::lock_guard<std::mutex> lk(g_kernels_mu);
  return g_by_path.emplace(path, h).first->second;
}

void launch_kernel_path(const std::string& path, const std::vector<at::Tensor>& args) {
  launch_kernel_stored(load_kernel_file(path), args);
}

}  // namespace spyre
