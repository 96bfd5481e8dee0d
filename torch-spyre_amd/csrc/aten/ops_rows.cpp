// Reductions, softmax and normalisation ops of the spyre backend.
//
// Reference: eager ReduceSum / mean (codegen/inputs/Metadata.yaml:299-302,
// codegen/inputs/spyre_torch_ops.cpp:456-490), _softmax
// (Metadata.yaml:275-277), the native_layer_norm stub that returns its input
// (spyre_torch_ops.cpp:188-194) and the 5-launch RMSNorm composite
// (pow/mean/add/rsqrt/mul).  Here softmax, LayerNorm and RMSNorm are each one
// wavefront-reduction kernel (sph_softmax_rows / sph_layernorm /
// sph_rmsnorm) and reductions one sph_reduce launch, all accumulating in fp32.
#include <ATen/WrapDimUtils.h>
#include <ATen/native/Resize.h>
#include <torch/library.h>

#include <cmath>
#include <limits>

#include "spyre_ops_common.h"

namespace spyre {
namespace {

// ---------------------------------------------------------------------------
// Reductions
// ---------------------------------------------------------------------------

// Reduces `self` over `dims` (empty = all) into `out`, whose shape is the
// reduced shape (keepdim or not).
void reduce_into(int op, const at::Tensor& self, at::IntArrayRef dims_in, bool keepdim,
                 const at::Tensor& out) {
  at::Tensor x = self.dim() == 0 ? self.reshape({1}) : self;
  const int nd = static_cast<int>(x.dim());
  TORCH_CHECK(nd <= SPH_MAX_DIMS, "spyre: reductions support at most ", SPH_MAX_DIMS, " dims");
  uint32_t mask = 0;
  if (dims_in.empty()) {
    mask = (nd >= 32) ? 0xffffffffu : ((1u << nd) - 1u);
  } else {
    for (int64_t d : dims_in) mask |= 1u << at::maybe_wrap_dim(d, std::max<int64_t>(nd, 1));
  }
  if (x.numel() == 0 && out.numel() == 0) return;
  sph_operand in{}, o{};
  in.data = x.data_ptr();
  in.dtype = to_sph(x.scalar_type());
  o.data = out.data_ptr();
  o.dtype = to_sph(out.scalar_type());
  std::vector<int64_t> sizes(x.sizes().begin(), x.sizes().end());
  // Output strides per input dim: reduced dims get 0; the others take the
  // output's strides in order (keepdim keeps size-1 dims in place).
  int od = 0;
  const bool kd = keepdim || self.dim() == 0 || out.dim() == nd;
  for (int d = 0; d < nd; ++d) {
    in.strides[d] = x.stride(d);
    if (mask & (1u << d)) {
      o.strides[d] = 0;
      if (kd) ++od;
    } else {
      o.strides[d] = out.dim() > 0 ? out.stride(od) : 0;
      ++od;
    }
  }
  check_extent(x, in.data, nd, sizes.data(), in.strides, x.element_size(), "reduce input");
  std::vector<int64_t> osizes(sizes);
  for (int d = 0; d < nd; ++d)
    if (mask & (1u << d)) osizes[d] = 1;
  check_extent(out, o.data, nd, osizes.data(), o.strides, out.element_size(), "reduce output");
  SPYRE_SPH_CHECK(sph_reduce(op, &in, &o, nd, sizes.data(), mask, stream(self.get_device())));
}

std::vector<int64_t> reduced_shape(const at::Tensor& self, at::IntArrayRef dims, bool keepdim) {
  const int64_t nd = self.dim();
  std::vector<bool> red(nd, dims.empty());
  for (int64_t d : dims) red[at::maybe_wrap_dim(d, std::max<int64_t>(nd, 1))] = true;
  std::vector<int64_t> shape;
  for (int64_t d = 0; d < nd; ++d) {
    if (!red[d])
      shape.push_back(self.size(d));
    else if (keepdim)
      shape.push_back(1);
  }
  return shape;
}

at::Tensor& sum_out(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                    std::optional<at::ScalarType> dtype, at::Tensor& out) {
  const auto dims = dim.value_or(at::IntArrayRef{});
  at::native::resize_output(out, reduced_shape(self, dims, keepdim));
  reduce_into(SPH_RED_SUM, self, dims, keepdim, out);
  return out;
}

at::Tensor& mean_out(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                     std::optional<at::ScalarType> dtype, at::Tensor& out) {
  const auto dims = dim.value_or(at::IntArrayRef{});
  at::native::resize_output(out, reduced_shape(self, dims, keepdim));
  reduce_into(SPH_RED_MEAN, self, dims, keepdim, out);
  return out;
}

template <int OP>
at::Tensor& minmax_out(const at::Tensor& self, at::IntArrayRef dim, bool keepdim,
                       at::Tensor& out) {
  at::native::resize_output(out, reduced_shape(self, dim, keepdim));
  reduce_into(OP, self, dim, keepdim, out);
  return out;
}

template <int OP>
at::Tensor& arg_out(const at::Tensor& self, std::optional<int64_t> dim, bool keepdim,
                    at::Tensor& out) {
  if (!dim.has_value()) {
    at::Tensor flat = contiguous_on_device(self).reshape({-1});
    at::native::resize_output(out, keepdim ? std::vector<int64_t>(self.dim(), 1)
                                           : std::vector<int64_t>{});
    reduce_into(OP, flat, {0}, false, out.reshape({}));
    return out;
  }
  const int64_t d = at::maybe_wrap_dim(*dim, std::max<int64_t>(self.dim(), 1));
  at::native::resize_output(out, reduced_shape(self, {d}, keepdim));
  reduce_into(OP, self, {d}, keepdim, out);
  return out;
}

std::tuple<at::Tensor&, at::Tensor&> max_dim_out(const at::Tensor& self, int64_t dim,
                                                 bool keepdim, at::Tensor& values,
                                                 at::Tensor& indices) {
  const int64_t d = at::maybe_wrap_dim(dim, std::max<int64_t>(self.dim(), 1));
  const auto shape = reduced_shape(self, {d}, keepdim);
  at::native::resize_output(values, shape);
  at::native::resize_output(indices, shape);
  reduce_into(SPH_RED_MAX, self, {d}, keepdim, values);
  reduce_into(SPH_RED_ARGMAX, self, {d}, keepdim, indices);
  return {values, indices};
}

std::tuple<at::Tensor&, at::Tensor&> min_dim_out(const at::Tensor& self, int64_t dim,
                                                 bool keepdim, at::Tensor& values,
                                                 at::Tensor& indices) {
  const int64_t d = at::maybe_wrap_dim(dim, std::max<int64_t>(self.dim(), 1));
  const auto shape = reduced_shape(self, {d}, keepdim);
  at::native::resize_output(values, shape);
  at::native::resize_output(indices, shape);
  reduce_into(SPH_RED_MIN, self, {d}, keepdim, values);
  reduce_into(SPH_RED_ARGMIN, self, {d}, keepdim, indices);
  return {values, indices};
}

template <int OP>
at::Tensor full_minmax(const at::Tensor& self) {
  TORCH_CHECK(self.numel() > 0, "spyre: max()/min() of an empty tensor");
  at::Tensor out = empty_spyre({}, self.scalar_type(), self.device());
  reduce_into(OP, self, {}, false, out);
  return out;
}

template <int OP>
at::Tensor& anyall_out(const at::Tensor& self, at::Tensor& out) {
  at::native::resize_output(out, {});
  reduce_into(OP, self, {}, false, out);
  return out;
}

template <int OP>
at::Tensor& anyall_dims_out(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                            at::Tensor& out) {
  const auto dims = dim.value_or(at::IntArrayRef{});
  at::native::resize_output(out, reduced_shape(self, dims, keepdim));
  reduce_into(OP, self, dims, keepdim, out);
  return out;
}

// ---------------------------------------------------------------------------
// Softmax
// ---------------------------------------------------------------------------
void softmax_into(const at::Tensor& self, int64_t dim, int flags, const at::Tensor& out) {
  if (self.numel() == 0) return;
  if (self.dim() == 0) {
    out.fill_((flags & SPH_SOFTMAX_LOG) ? 0.0 : 1.0);
    return;
  }
  const int64_t d = at::maybe_wrap_dim(dim, self.dim());
  const bool last = d == self.dim() - 1;
  at::Tensor x = last ? contiguous_on_device(self) : contiguous_on_device(self.transpose(d, -1));
  const int64_t cols = x.size(-1);
  const int64_t rows = x.numel() / cols;
  const bool direct = last && out.is_contiguous();
  at::Tensor y = direct ? out : empty_spyre(x.sizes(), out.scalar_type(), out.device());
  c10::DeviceGuard guard(self.device());
  SPYRE_SPH_CHECK(sph_softmax_rows(to_sph(x.scalar_type()), to_sph(y.scalar_type()),
                                   x.data_ptr(), cols, y.data_ptr(), cols, rows, cols, 1.0f,
                                   flags, 1, 0, stream(self.get_device())));
  if (!direct) device_copy(out, last ? y : y.transpose(d, -1));
}

at::Tensor& softmax_out(const at::Tensor& self, int64_t dim, bool half_to_float,
                        at::Tensor& out) {
  at::native::resize_output(out, self.sizes());
  softmax_into(self, dim, 0, out);
  return out;
}

at::Tensor& log_softmax_out(const at::Tensor& self, int64_t dim, bool half_to_float,
                            at::Tensor& out) {
  at::native::resize_output(out, self.sizes());
  softmax_into(self, dim, SPH_SOFTMAX_LOG, out);
  return out;
}

// ---------------------------------------------------------------------------
// LayerNorm / RMSNorm
// ---------------------------------------------------------------------------

// Weight / bias in a dtype the kernels accept (fp32 or the activation dtype).
at::Tensor norm_param(const std::optional<at::Tensor>& p, at::ScalarType act, int64_t cols,
                      at::ScalarType& wdt) {
  if (!p.has_value() || !p->defined()) return at::Tensor();
  at::Tensor w = p->reshape({cols});
  if (w.scalar_type() != act && w.scalar_type() != at::kFloat) w = w.to(at::kFloat);
  w = contiguous_on_device(w);
  wdt = w.scalar_type();
  return w;
}

std::vector<int64_t> stat_shape(const at::Tensor& x, size_t nnorm) {
  std::vector<int64_t> s(x.sizes().begin(), x.sizes().end() - nnorm);
  for (size_t i = 0; i < nnorm; ++i) s.push_back(1);
  return s;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> native_layer_norm(
    const at::Tensor& input, c10::SymIntArrayRef normalized_shape,
    const std::optional<at::Tensor>& weight, const std::optional<at::Tensor>& bias,
    double eps) {
  const auto ns = c10::asIntArrayRefUnchecked(normalized_shape);
  int64_t cols = 1;
  for (int64_t s : ns) cols *= s;
  at::Tensor x = contiguous_on_device(input);
  const int64_t rows = cols > 0 ? x.numel() / cols : 0;
  const auto act = x.scalar_type();
  at::ScalarType wdt = act;
  at::Tensor w = norm_param(weight, act, cols, wdt);
  at::ScalarType bdt = wdt;
  at::Tensor b = norm_param(bias, act, cols, bdt);
  if (w.defined() && b.defined() && wdt != bdt) {
    w = w.to(at::kFloat);
    b = b.to(at::kFloat);
    wdt = at::kFloat;
  } else if (!w.defined() && b.defined()) {
    wdt = bdt;
  }
  at::Tensor y = empty_spyre(x.sizes(), act, x.device());
  at::Tensor mean = empty_spyre({rows}, at::kFloat, x.device());
  at::Tensor rstd = empty_spyre({rows}, at::kFloat, x.device());
  c10::DeviceGuard guard(x.device());
  if (rows > 0)
    SPYRE_SPH_CHECK(sph_layernorm(to_sph(act), to_sph(wdt), x.data_ptr(), nullptr,
                                  w.defined() ? w.data_ptr() : nullptr,
                                  b.defined() ? b.data_ptr() : nullptr, y.data_ptr(), nullptr,
                                  mean.data_ptr<float>(), rstd.data_ptr<float>(), rows, cols,
                                  static_cast<float>(eps), stream(x.get_device())));
  // Saved statistics in the activation dtype with the kept dims, as torch's
  // CPU kernel returns them.
  const auto ss = stat_shape(x, ns.size());
  return {y, mean.to(act).view(ss), rstd.to(act).view(ss)};
}

std::tuple<at::Tensor, at::Tensor> fused_rms_norm(const at::Tensor& input,
                                                  at::IntArrayRef normalized_shape,
                                                  const std::optional<at::Tensor>& weight,
                                                  std::optional<double> eps) {
  int64_t cols = 1;
  for (int64_t s : normalized_shape) cols *= s;
  at::Tensor x = contiguous_on_device(input);
  const int64_t rows = cols > 0 ? x.numel() / cols : 0;
  const auto act = x.scalar_type();
  at::ScalarType wdt = act;
  at::Tensor w = norm_param(weight, act, cols, wdt);
  // torch's default eps: machine epsilon of the accumulation type
  const double e = eps.has_value() ? *eps
                                   : (act == at::kDouble ? std::numeric_limits<double>::epsilon()
                                                         : std::numeric_limits<float>::epsilon());
  at::Tensor y = empty_spyre(x.sizes(), act, x.device());
  at::Tensor rstd = empty_spyre({rows}, at::kFloat, x.device());
  c10::DeviceGuard guard(x.device());
  if (rows > 0)
    SPYRE_SPH_CHECK(sph_rmsnorm(to_sph(act), to_sph(wdt), x.data_ptr(), nullptr,
                                w.defined() ? w.data_ptr() : nullptr, y.data_ptr(), nullptr,
                                rstd.data_ptr<float>(), rows, cols, static_cast<float>(e),
                                stream(x.get_device())));
  return {y, rstd.view(stat_shape(x, normalized_shape.size()))};
}

at::Tensor rms_norm(const at::Tensor& input, c10::SymIntArrayRef normalized_shape,
                    const std::optional<at::Tensor>& weight, std::optional<double> eps) {
  return std::get<0>(
      fused_rms_norm(input, c10::asIntArrayRefUnchecked(normalized_shape), weight, eps));
}

// ---------------------------------------------------------------------------
// Vector norm (reference: linalg_vector_norm, a base-template op of
// codegen/inputs/Metadata.yaml:139): |x| reduced in fp32 by the device
// reductions - ord 2 as the square root of one sum-of-squares reduction,
// ord 1 a sum of |x|, +-inf a max / min of |x|, 0 the count of non-zeros,
// any other ord (sum |x|^ord)^(1/ord) - then cast to the result dtype.
// ---------------------------------------------------------------------------
at::Tensor& linalg_vector_norm_out(const at::Tensor& self, const at::Scalar& ord,
                                   at::OptionalIntArrayRef dim, bool keepdim,
                                   std::optional<at::ScalarType> dtype, at::Tensor& out) {
  TORCH_CHECK(at::isFloatingType(self.scalar_type()),
              "spyre: linalg.vector_norm expects a floating-point input, got ",
              self.scalar_type());
  const double p = ord.toDouble();
  const auto dims = dim.value_or(at::IntArrayRef{});
  const auto shape = reduced_shape(self, dims, keepdim);
  at::native::resize_output(out, shape);
  if (self.numel() == 0) {
    TORCH_CHECK(p >= 0.0 && !std::isinf(p),
                "linalg.vector_norm cannot compute the ", ord, " norm on an empty tensor "
                "because the operation does not have an identity");
  }
  at::Tensor acc = empty_spyre(shape, at::kFloat, self.device());
  c10::DeviceGuard guard(self.device());
  if (p == 2.0) {
    reduce_into(SPH_RED_SUMSQ, self, dims, keepdim, acc);
    acc.sqrt_();
  } else if (p == 0.0) {
    reduce_into(SPH_RED_SUM, self.ne(0).to(at::kFloat), dims, keepdim, acc);
  } else if (std::isinf(p)) {
    reduce_into(p > 0 ? SPH_RED_MAX : SPH_RED_MIN, self.abs().to(at::kFloat), dims, keepdim,
                acc);
  } else if (p == 1.0) {
    reduce_into(SPH_RED_SUM, self.abs().to(at::kFloat), dims, keepdim, acc);
  } else {
    reduce_into(SPH_RED_SUM, self.abs().to(at::kFloat).pow(p), dims, keepdim, acc);
    acc.pow_(1.0 / p);
  }
  out.copy_(acc);
  return out;
}

at::Tensor linalg_vector_norm(const at::Tensor& self, const at::Scalar& ord,
                              at::OptionalIntArrayRef dim, bool keepdim,
                              std::optional<at::ScalarType> dtype) {
  const at::ScalarType odt = dtype.value_or(self.scalar_type());
  at::Tensor out = empty_spyre({0}, odt, self.device());
  linalg_vector_norm_out(self, ord, dim, keepdim, dtype, out);
  return out;
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("linalg_vector_norm", TORCH_FN(linalg_vector_norm));
  m.impl("linalg_vector_norm.out", TORCH_FN(linalg_vector_norm_out));
  m.impl("sum.IntList_out", TORCH_FN(sum_out));
  m.impl("mean.out", TORCH_FN(mean_out));
  m.impl("amax.out", TORCH_FN(minmax_out<SPH_RED_MAX>));
  m.impl("amin.out", TORCH_FN(minmax_out<SPH_RED_MIN>));
  m.impl("argmax.out", TORCH_FN(arg_out<SPH_RED_ARGMAX>));
  m.impl("argmin.out", TORCH_FN(arg_out<SPH_RED_ARGMIN>));
  m.impl("max.dim_max", TORCH_FN(max_dim_out));
  m.impl("min.dim_min", TORCH_FN(min_dim_out));
  m.impl("max", TORCH_FN(full_minmax<SPH_RED_MAX>));
  m.impl("min", TORCH_FN(full_minmax<SPH_RED_MIN>));
  m.impl("any.all_out", TORCH_FN(anyall_out<SPH_RED_ANY>));
  m.impl("all.all_out", TORCH_FN(anyall_out<SPH_RED_ALL>));
  m.impl("any.dims_out", TORCH_FN(anyall_dims_out<SPH_RED_ANY>));
  m.impl("all.dims_out", TORCH_FN(anyall_dims_out<SPH_RED_ALL>));
  m.impl("_softmax.out", TORCH_FN(softmax_out));
  m.impl("_log_softmax.out", TORCH_FN(log_softmax_out));
  m.impl("native_layer_norm", TORCH_FN(native_layer_norm));
  m.impl("_fused_rms_norm", TORCH_FN(fused_rms_norm));
  m.impl("rms_norm", TORCH_FN(rms_norm));
}

}  // namespace spyre
