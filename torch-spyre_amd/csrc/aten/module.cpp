// torch_spyre._C: the Python face of the spyre backend's native runtime.
//
// Reference: PYBIND11_MODULE(_C) in torch_spyre/csrc/module.cpp:174-204
// (start_runtime, free_runtime, launch_kernel, SpyreTensorLayout with its
// StickFormat enum, three constructors, five fields and __str__).  Loading
// this module also registers the allocator, the device guard, the
// PrivateUse1 hooks and every eager ATen kernel (static registrations in the
// other translation units).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/extension.h>

#include "spyre_layout.h"
#include "spyre_runtime.h"

namespace py = pybind11;

namespace spyre {
// Compiled-kernel loader / launcher (ops_launch.cpp).
int64_t load_kernel(const std::string& code_object, const std::string& name, int64_t grid,
                    int64_t block, const std::vector<int64_t>& extents, bool error_word);
int64_t load_kernel_file(const std::string& path);
void launch_kernel(int64_t handle, const std::vector<at::Tensor>& args, int64_t grid,
                   int64_t block, const std::vector<int64_t>& extents);
void launch_kernel_stored(int64_t handle, const std::vector<at::Tensor>& args);
void launch_kernel_path(const std::string& path, const std::vector<at::Tensor>& args);
// Fused SwiGLU projection and RMSNorm-prologue GEMM (ops_gemm.cpp).
at::Tensor gemm_swiglu(const at::Tensor& x, const at::Tensor& w);
at::Tensor gemm_rmsnorm(const at::Tensor& x, const at::Tensor& norm_w, double eps,
                        const at::Tensor& w, bool swiglu);
// Fused attention (ops_attention.cpp).
at::Tensor attention_fwd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                         const c10::optional<at::Tensor>& mask, double scale, int64_t causal_q,
                         int64_t causal_off);
at::Tensor decode_attention_step(const at::Tensor& qkv, const at::Tensor& cos,
                                 const at::Tensor& sin, const at::Tensor& pos,
                                 at::Tensor& k_cache, at::Tensor& v_cache, int64_t n_heads,
                                 int64_t n_kv_heads, double scale, bool v_dim_major);
}  // namespace spyre

PYBIND11_MODULE(_C, m) {
  m.doc() = "torch_spyre native runtime for MI355X (gfx950)";

  m.def("start_runtime", &spyre::start_runtime, "Probes the HIP devices (idempotent).");
  m.def("free_runtime", &spyre::free_runtime,
        "Releases cached device memory and the spyre streams.");
  m.def("load_kernel", [](py::bytes code, const std::string& name, int64_t grid, int64_t block,
                          const std::vector<int64_t>& extents, bool error_word) {
    return spyre::load_kernel(std::string(code), name, grid, block, extents, error_word);
  }, py::arg("code_object"), py::arg("name"), py::arg("grid") = -1, py::arg("block") = -1,
        py::arg("extents") = std::vector<int64_t>{}, py::arg("error_word") = false,
        "Registers a gfx950 code object (loaded into each device on first launch), "
        "optionally with its launch shape and per-argument extents; error_word: the "
        "kernel takes the device error word as its last parameter.");
  m.def("load_kernel_file", &spyre::load_kernel_file, py::arg("path"),
        "Registers the code object at `path` with its launch description `path`.launch.");
  // The reference's form first: launch_kernel(path_or_handle, args), the
  // output last (torch_spyre/csrc/module.cpp:176).
  m.def("launch_kernel", &spyre::launch_kernel_path, py::arg("path"), py::arg("args"),
        "Launches the code object at `path` (launch description in `path`.launch) on the "
        "spyre stream of the arguments' device.");
  m.def("launch_kernel", &spyre::launch_kernel_stored, py::arg("handle"), py::arg("args"),
        "Launches a kernel loaded with its launch shape.");
  m.def("launch_kernel", &spyre::launch_kernel, py::arg("handle"), py::arg("args"),
        py::arg("grid"), py::arg("block"), py::arg("extents"),
        "Launches a loaded kernel on the spyre stream of the arguments' device; "
        "extents[i] >= 0 bounds the elements argument i may address.");

  m.def("attention_fwd", &spyre::attention_fwd, py::arg("q"), py::arg("k"), py::arg("v"),
        py::arg("mask"), py::arg("scale"), py::arg("causal_q") = 0, py::arg("causal_off") = 0,
        "softmax(scale * q k^T + mask) v on the spyre stream (q [B, mq, 128], k / v "
        "[B, sk, 128], mask [mq, sk] / [B or 1, mq, sk] or None; fp16 / bf16).");
  m.def("decode_attention_step", &spyre::decode_attention_step, py::arg("qkv"), py::arg("cos"),
        py::arg("sin"), py::arg("pos"), py::arg("k_cache"), py::arg("v_cache"),
        py::arg("n_heads"), py::arg("n_kv_heads"), py::arg("scale"),
        py::arg("v_dim_major") = false,
        "One decode step of grouped-query attention: RoPE of the step's queries and key at "
        "*pos, the key / value appended to the caches in place, attention over keys 0..pos "
        "(qkv [B, (H + 2 Hkv) * 128]) -> [B, H * 128].");
  m.def("gemm_swiglu", &spyre::gemm_swiglu, py::arg("x"), py::arg("w"),
        "silu(x w[:n]^T) * (x w[n:]^T) on the spyre stream (x [M, K], w [2n, K]).");
  m.def("gemm_rmsnorm", &spyre::gemm_rmsnorm, py::arg("x"), py::arg("norm_w"), py::arg("eps"),
        py::arg("w"), py::arg("swiglu") = false,
        "rms_norm(x) w^T, or with swiglu silu(gate) * up of the stacked weight, on the spyre "
        "stream (x [M, K], M <= 8 in one weight-stream kernel).");
  m.def("device_count", []() { return spyre::device_count(); });
  m.def("current_device", []() { return spyre::current_device(); });
  m.def("set_device", [](int d) { spyre::set_device(d); });
  m.def("synchronize", [](int d) {
    {
      py::gil_scoped_release nogil;
      spyre::synchronize(d);
    }
  }, py::arg("device") = -1);
  m.def("is_available", []() { return spyre::device_count() > 0; });
  m.def("manual_seed", [](uint64_t seed, int device) { spyre::set_seed(device, seed); },
        py::arg("seed"), py::arg("device") = -1);
  m.def("manual_seed_all", [](uint64_t seed) { spyre::set_seed(-1, seed); });
  m.def("initial_seed", [](int device) { return spyre::get_seed(device); },
        py::arg("device") = -1);
  m.def("_stream_handle", [](int device) {
    return reinterpret_cast<uintptr_t>(spyre::stream(device));
  }, py::arg("device") = -1, "hipStream_t (as an int) that spyre ops on `device` run on.");
  m.def("memory_allocated", [](int d) { return spyre::memory_stats(d).allocated; },
        py::arg("device") = -1);
  m.def("memory_reserved", [](int d) { return spyre::memory_stats(d).reserved; },
        py::arg("device") = -1);
  m.def("max_memory_allocated", [](int d) { return spyre::memory_stats(d).peak_allocated; },
        py::arg("device") = -1);
  m.def("memory_stats", [](int d) {
    auto s = spyre::memory_stats(d);
    py::dict r;
    r["allocated_bytes"] = s.allocated;
    r["reserved_bytes"] = s.reserved;
    r["peak_allocated_bytes"] = s.peak_allocated;
    r["num_alloc_calls"] = s.num_alloc_calls;
    r["num_device_mallocs"] = s.num_device_mallocs;
    return r;
  }, py::arg("device") = -1);
  m.def("empty_cache", &spyre::empty_cache);
  m.def("stick_alloc_nbytes", [](std::vector<int64_t> sizes, int64_t elem_bytes) {
    return spyre::stick_alloc_nbytes(sizes, elem_bytes);
  });
  m.def("get_device_properties", [](int d) {
    hipDeviceProp_t p{};
    SPYRE_HIP_CHECK(hipGetDeviceProperties(&p, d < 0 ? spyre::current_device() : d));
    py::dict r;
    r["name"] = std::string(p.name);
    r["gcnArchName"] = std::string(p.gcnArchName);
    r["multi_processor_count"] = p.multiProcessorCount;
    r["total_memory"] = static_cast<int64_t>(p.totalGlobalMem);
    r["max_shared_memory_per_block"] = static_cast<int64_t>(p.sharedMemPerBlock);
    r["clock_rate_khz"] = p.clockRate;
    r["warp_size"] = p.warpSize;
    return r;
  }, py::arg("device") = -1);

  py::class_<spyre::Graph>(m, "Graph", "HIP graph of the spyre stream (capture / replay).")
      .def(py::init<>())
      .def("capture_begin", &spyre::Graph::capture_begin)
      .def("capture_end", &spyre::Graph::capture_end)
      .def("replay", [](spyre::Graph& g) {
        py::gil_scoped_release nogil;
        g.replay();
      })
      .def("reset", &spyre::Graph::reset)
      .def("pool", &spyre::Graph::pool);

  using STL = spyre::SpyreTensorLayout;
  py::class_<STL> cls(m, "SpyreTensorLayout");
  py::enum_<STL::StickFormat>(cls, "StickFormat")
      .value("Dense", STL::Dense)
      .value("Sparse", STL::Sparse)
      .value("SparseMulti", STL::SparseMulti);
  cls.def_readwrite("device_size", &STL::device_size)
      .def_readwrite("device_strides", &STL::device_strides)
      .def_readwrite("dim_map", &STL::dim_map)
      .def_readwrite("num_stick_dims", &STL::num_stick_dims)
      .def_readwrite("format", &STL::format)
      .def("__str__", [](const STL& l) { return l.toString(); })
      .def("__repr__", [](const STL& l) { return l.toString(); })
      .def(py::init<std::vector<int64_t>, c10::ScalarType>())
      .def(py::init<std::vector<int64_t>, c10::ScalarType, std::vector<int32_t>,
                    STL::StickFormat>(),
           py::arg("host_size"), py::arg("dtype"), py::arg("dim_order"),
           py::arg("format") = STL::Dense)
      .def(py::init<std::vector<int64_t>, std::vector<int64_t>, std::vector<int32_t>, int32_t,
                    STL::StickFormat>());
}
