// Data-movement and miscellaneous ops of the spyre backend: cat, tril/triu,
// index_select (embedding), dropout, arange, cumsum and the random fills.
//
// Reference: generated cat (codegen/inputs/Metadata.yaml:45-47), tril
// (:322-324), embedding (:105-115); native_dropout stub
// (codegen/inputs/spyre_torch_ops.cpp:180-186); CPU fallbacks for ne / cumsum
// (:494-505).  Like the reference, cumsum, arange and the random fills run on
// the host and copy the result; everything else runs on the GPU.
#include <ATen/CPUGeneratorImpl.h>
#include <ATen/WrapDimUtils.h>
#include <ATen/native/Resize.h>
#include <torch/library.h>

#include <mutex>

#include "spyre_ops_common.h"

namespace spyre {
namespace {

at::Tensor& cat_out(const at::ITensorListRef& tensors, int64_t dim, at::Tensor& out) {
  std::vector<at::Tensor> ts;
  for (const at::Tensor& t : tensors) ts.push_back(t);
  TORCH_CHECK(!ts.empty(), "spyre: cat expects a non-empty list");
  // Legacy: 1-D empty tensors are skipped.
  const at::Tensor* ref = nullptr;
  for (const auto& t : ts)
    if (!(t.dim() == 1 && t.numel() == 0)) {
      ref = &t;
      break;
    }
  if (!ref) {
    at::native::resize_output(out, {0});
    return out;
  }
  const int64_t d = at::maybe_wrap_dim(dim, ref->dim());
  std::vector<int64_t> shape(ref->sizes().begin(), ref->sizes().end());
  int64_t total = 0;
  for (const auto& t : ts) {
    if (t.dim() == 1 && t.numel() == 0) continue;
    TORCH_CHECK(t.dim() == ref->dim(), "spyre: cat tensors must have the same rank");
    total += t.size(d);
  }
  shape[d] = total;
  at::native::resize_output(out, shape);
  int64_t off = 0;
  for (const auto& t : ts) {
    if (t.dim() == 1 && t.numel() == 0) continue;
    const int64_t len = t.size(d);
    if (len > 0) device_copy(out.narrow(d, off, len), is_spyre(t) ? t : t.to(out.device()));
    off += len;
  }
  return out;
}

template <int UPPER>
at::Tensor& tri_out(const at::Tensor& self, int64_t diagonal, at::Tensor& out) {
  TORCH_CHECK(self.dim() >= 2, "spyre: tril/triu need at least 2 dims");
  at::native::resize_output(out, self.sizes());
  if (self.numel() == 0) return out;
  at::Tensor x = contiguous_on_device(self);
  const bool direct = out.is_contiguous();
  at::Tensor y = direct ? out : empty_spyre(self.sizes(), out.scalar_type(), out.device());
  const int64_t rows = x.size(-2), cols = x.size(-1);
  const int64_t batch = x.numel() / (rows * cols);
  c10::DeviceGuard guard(self.device());
  SPYRE_SPH_CHECK(sph_tri(UPPER, diagonal, static_cast<int>(x.element_size()), x.data_ptr(),
                          y.data_ptr(), batch, rows, cols, stream(self.get_device())));
  if (!direct) device_copy(out, y);
  return out;
}

// Row gather along `dim` (embedding is index_select(weight, 0, ids)).  An
// index outside [0, size) zero-fills its row and is reported through the
// device error word, which raises IndexError at the next synchronisation
// (checking on the host at the call would cost a device-to-host round trip
// per call).
at::Tensor& index_select_out(const at::Tensor& self, int64_t dim, const at::Tensor& index,
                             at::Tensor& out) {
  TORCH_CHECK(index.dim() <= 1, "spyre: index_select expects a 0-D or 1-D index");
  TORCH_CHECK(index.scalar_type() == at::kLong || index.scalar_type() == at::kInt,
              "spyre: index_select expects int64 or int32 indices");
  const int64_t d = at::maybe_wrap_dim(dim, std::max<int64_t>(self.dim(), 1));
  at::Tensor idx = contiguous_on_device(is_spyre(index) ? index : index.to(self.device()))
                       .reshape({-1});
  const int64_t n = idx.numel();
  std::vector<int64_t> shape(self.sizes().begin(), self.sizes().end());
  if (self.dim() == 0) shape = {};
  else shape[d] = n;
  at::native::resize_output(out, shape);
  if (out.numel() == 0) return out;
  // Move `dim` to the front so every selected slice is one contiguous row.
  at::Tensor table = contiguous_on_device(d == 0 ? self : self.movedim(d, 0));
  const int64_t nrows = self.dim() == 0 ? 1 : table.size(0);
  const int64_t row_elems = nrows > 0 ? table.numel() / nrows : 0;
  const bool direct = d == 0 && out.is_contiguous();
  std::vector<int64_t> gshape(table.sizes().begin(), table.sizes().end());
  if (!gshape.empty()) gshape[0] = n;
  at::Tensor g = direct ? out : empty_spyre(gshape, self.scalar_type(), self.device());
  c10::DeviceGuard guard(self.device());
  SPYRE_SPH_CHECK(sph_gather_rows(table.data_ptr(), nrows, row_elems,
                                  static_cast<int>(table.element_size()), idx.data_ptr(),
                                  idx.scalar_type() == at::kLong ? 1 : 0, n, g.data_ptr(),
                                  device_error_word(self.get_device()),
                                  stream(self.get_device())));
  if (!direct) device_copy(out, d == 0 ? g : g.movedim(0, d));
  return out;
}

at::Tensor index_select(const at::Tensor& self, int64_t dim, const at::Tensor& index) {
  at::Tensor out = empty_spyre({0}, self.scalar_type(), self.device());
  return index_select_out(self, dim, index, out);
}

// Host-side generators of the random fills, seeded by torch.spyre.manual_seed.
std::mutex g_gen_mu;
at::Generator host_generator(int device) {
  static std::vector<std::pair<uint64_t, at::Generator>> gens(64);
  std::lock_guard<std::mutex> lk(g_gen_mu);
  const uint64_t seed = get_seed(device);
  auto& slot = gens[device];
  if (!slot.second.defined() || slot.first != seed) {
    slot = {seed, at::make_generator<at::CPUGeneratorImpl>(seed)};
  }
  return slot.second;
}

at::Generator pick_gen(const std::optional<at::Generator>& g, int device) {
  if (g.has_value() && g->defined() && g->device().is_cpu()) return *g;
  return host_generator(device);
}

std::tuple<at::Tensor, at::Tensor> native_dropout(const at::Tensor& input, double p,
                                                  std::optional<bool> train) {
  at::Tensor mask = empty_spyre(input.sizes(), at::kBool, input.device());
  if (!train.value_or(true) || p == 0.0) {
    mask.fill_(true);
    return {input.clone(), mask};
  }
  TORCH_CHECK(p > 0.0 && p <= 1.0, "spyre: dropout probability must be in [0, 1]");
  at::Tensor keep_cpu = at::empty(input.sizes(), input.options().device(at::kCPU).dtype(at::kFloat));
  keep_cpu.uniform_(0.0, 1.0, pick_gen(std::nullopt, input.get_device()));
  mask.copy_(keep_cpu.ge(p));
  at::Tensor out = at::where(mask, input, at::zeros({}, input.options()));
  // p == 1 drops everything: scale 0 (as torch), not 0 * inf
  return {out.mul(p == 1.0 ? 0.0 : 1.0 / (1.0 - p)), mask};
}

at::Tensor& arange_out(const at::Scalar& start, const at::Scalar& end, const at::Scalar& step,
                       at::Tensor& out) {
  at::Tensor host = at::arange(start, end, step, out.options().device(at::kCPU));
  at::native::resize_output(out, host.sizes());
  out.copy_(host);
  return out;
}

at::Tensor& cumsum_out(const at::Tensor& self, int64_t dim, std::optional<at::ScalarType> dtype,
                       at::Tensor& out) {
  at::Tensor host = at::cumsum(self.to(at::kCPU), dim, dtype);
  at::native::resize_output(out, host.sizes());
  out.copy_(host);
  return out;
}

at::Tensor& normal_(at::Tensor& self, double mean, double std,
                    std::optional<at::Generator> gen) {
  at::Tensor host = at::empty(self.sizes(), self.options().device(at::kCPU));
  host.normal_(mean, std, pick_gen(gen, self.get_device()));
  self.copy_(host);
  return self;
}

at::Tensor& uniform_(at::Tensor& self, double from, double to,
                     std::optional<at::Generator> gen) {
  at::Tensor host = at::empty(self.sizes(), self.options().device(at::kCPU));
  host.uniform_(from, to, pick_gen(gen, self.get_device()));
  self.copy_(host);
  return self;
}

at::Tensor& random_from_(at::Tensor& self, int64_t from, std::optional<int64_t> to,
                         std::optional<at::Generator> gen) {
  at::Tensor host = at::empty(self.sizes(), self.options().device(at::kCPU));
  host.random_(from, to, pick_gen(gen, self.get_device()));
  self.copy_(host);
  return self;
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("cat.out", TORCH_FN(cat_out));
  m.impl("tril.out", TORCH_FN(tri_out<0>));
  m.impl("triu.out", TORCH_FN(tri_out<1>));
  m.impl("index_select", TORCH_FN(index_select));
  m.impl("index_select.out", TORCH_FN(index_select_out));
  m.impl("native_dropout", TORCH_FN(native_dropout));
  m.impl("arange.start_out", TORCH_FN(arange_out));
  m.impl("cumsum.out", TORCH_FN(cumsum_out));
  m.impl("normal_", TORCH_FN(normal_));
  m.impl("uniform_", TORCH_FN(uniform_));
  m.impl("random_.from", TORCH_FN(random_from_));
}

}  // namespace spyre
