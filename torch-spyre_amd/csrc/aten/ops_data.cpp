// Data-movement and miscellaneous ops of the spyre backend: cat, tril/triu,
// index_select (embedding), dropout, arange, cumsum and the random fills.
//
// Reference: generated cat (codegen/inputs/Metadata.yaml:45-47), tril
// (:322-324), embedding (:105-115); native_dropout stub
// (codegen/inputs/spyre_torch_ops.cpp:180-186); CPU fallbacks for ne / cumsum
// (:494-505).  Here all of them run on the GPU: cumsum as a device scan,
// arange as a device fill, the random fills and dropout from the device's
// Philox generator (seeded by torch.spyre.manual_seed).
#include <ATen/CPUGeneratorImpl.h>
#include <ATen/WrapDimUtils.h>
#include <ATen/native/Resize.h>
#include <torch/library.h>

#include <algorithm>
#include <cmath>
#include <limits>
#include <mutex>
#include <utility>

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

// (seed, counter offset) of the next random fill of `blocks` Philox blocks
// on `device`: the device generator's, advanced past this fill.  With an
// explicit CPU generator the fill is keyed by one 64-bit draw of it at
// offset 0 instead, so it is reproducible from that generator.
std::pair<uint64_t, uint64_t> philox_state(const std::optional<at::Generator>& gen, int device,
                                           int64_t blocks) {
  if (gen.has_value() && gen->defined()) {
    TORCH_CHECK(gen->device().is_cpu(),
                "spyre: random fills take a CPU generator or none (the device's own)");
    at::Generator g = *gen;
    auto* impl = at::check_generator<at::CPUGeneratorImpl>(g);
    std::lock_guard<std::mutex> lk(g.mutex());
    return {impl->random64(), 0};
  }
  return {get_seed(device), rng_offset_advance(device, static_cast<uint64_t>(blocks))};
}

// Runs `fill(ptr)` on a contiguous image of `self` and copies it in when
// `self` is not contiguous itself.
template <typename F>
at::Tensor& fill_contiguous(at::Tensor& self, F&& fill) {
  if (self.numel() == 0) return self;
  c10::DeviceGuard guard(self.device());
  if (self.is_contiguous()) {
    fill(self);
  } else {
    at::Tensor tmp = empty_spyre(self.sizes(), self.scalar_type(), self.device());
    fill(tmp);
    device_copy(self, tmp);
  }
  return self;
}

at::Tensor& random_fill(at::Tensor& self, int kind, double a, double b, int64_t ifrom,
                        uint64_t irange, const std::optional<at::Generator>& gen) {
  const sph_dtype dt = to_sph(self.scalar_type());
  const int64_t blocks = sph_random_blocks(kind, dt, self.numel(), irange);
  const auto [seed, offset] = philox_state(gen, self.get_device(), blocks);
  return fill_contiguous(self, [&](at::Tensor& t) {
    SPYRE_SPH_CHECK(sph_random_fill(kind, dt, t.data_ptr(), t.numel(), seed, offset, a, b, ifrom,
                                    irange, stream(t.get_device())));
  });
}

std::tuple<at::Tensor, at::Tensor> native_dropout(const at::Tensor& input, double p,
                                                  std::optional<bool> train) {
  at::Tensor mask = empty_spyre(input.sizes(), at::kBool, input.device());
  if (!train.value_or(true) || p == 0.0) {
    mask.fill_(true);
    return {input.clone(), mask};
  }
  TORCH_CHECK(p > 0.0 && p <= 1.0, "spyre: dropout probability must be in [0, 1]");
  const at::ScalarType st = input.scalar_type();
  TORCH_CHECK(st == at::kHalf || st == at::kBFloat16 || st == at::kFloat,
              "spyre: dropout supports float16, bfloat16 and float32");
  at::Tensor x = contiguous_on_device(input);
  at::Tensor y = empty_spyre(input.sizes(), st, input.device());
  const int64_t n = x.numel();
  if (n == 0) return {y, mask};
  // p == 1 drops everything: scale 0 (as torch), not 0 * inf
  const float scale = p == 1.0 ? 0.0f : static_cast<float>(1.0 / (1.0 - p));
  const auto [seed, offset] = philox_state(std::nullopt, input.get_device(), (n + 3) / 4);
  c10::DeviceGuard guard(input.device());
  SPYRE_SPH_CHECK(sph_dropout(to_sph(st), x.data_ptr(), y.data_ptr(),
                              static_cast<uint8_t*>(mask.data_ptr()), n, static_cast<float>(p),
                              scale, seed, offset, stream(input.get_device())));
  return {y, mask};
}

at::ScalarType cumsum_type(const at::Tensor& self, std::optional<at::ScalarType> dtype);

// Output length of arange as torch computes it: integer arithmetic for
// int64 outputs, double otherwise.
int64_t arange_size(const at::Scalar& start, const at::Scalar& end, const at::Scalar& step,
                    at::ScalarType dt) {
  if (dt == at::kLong) {
    const int64_t xs = start.to<int64_t>(), xe = end.to<int64_t>(), st = step.to<int64_t>();
    TORCH_CHECK(st != 0, "step must be nonzero");
    TORCH_CHECK((st > 0 && xe >= xs) || (st < 0 && xe <= xs),
                "upper bound and larger bound inconsistent with step sign");
    const int64_t sgn = (st > 0) - (st < 0);
    return (xe - xs + st - sgn) / st;
  }
  const double xs = start.to<double>(), xe = end.to<double>(), st = step.to<double>();
  TORCH_CHECK(st > 0 || st < 0, "step must be nonzero");
  TORCH_CHECK(std::isfinite(xs) && std::isfinite(xe), "unsupported range: ", xs, " -> ", xe);
  TORCH_CHECK((st > 0 && xe >= xs) || (st < 0 && xe <= xs),
              "upper bound and larger bound inconsistent with step sign");
  const double size_d = std::ceil((xe - xs) / st);
  TORCH_CHECK(size_d >= 0 && size_d <= static_cast<double>(std::numeric_limits<int64_t>::max()),
              "invalid size, possible overflow?");
  return static_cast<int64_t>(size_d);
}

at::Tensor& arange_out(const at::Scalar& start, const at::Scalar& end, const at::Scalar& step,
                       at::Tensor& out) {
  const at::ScalarType dt = out.scalar_type();
  TORCH_CHECK(dt != at::kBool, "spyre: arange does not produce bool");
  const int64_t n = arange_size(start, end, step, dt);
  if (out.numel() != n) at::native::resize_output(out, {n});
  const bool integral = at::isIntegralType(dt, /*includeBool=*/false);
  return fill_contiguous(out, [&](at::Tensor& t) {
    SPYRE_SPH_CHECK(sph_arange(to_sph(dt), integral ? 0.0 : start.to<double>(),
                               integral ? 0.0 : step.to<double>(),
                               integral ? start.to<int64_t>() : 0,
                               integral ? step.to<int64_t>() : 0, n, t.data_ptr(),
                               stream(t.get_device())));
  });
}

at::Tensor& cumsum_out(const at::Tensor& self, int64_t dim, std::optional<at::ScalarType> dtype,
                       at::Tensor& out) {
  // result dtype as torch: the requested one, int64 for integral (and bool)
  // inputs, else the input's; the input is converted to it first
  const at::ScalarType rt = cumsum_type(self, dtype);
  TORCH_CHECK(out.scalar_type() == rt, "spyre: cumsum out dtype ", out.scalar_type(),
              " does not match the result dtype ", rt);
  TORCH_CHECK(rt != at::kBool, "spyre: cumsum does not accumulate in bool");
  at::native::resize_output(out, self.sizes());
  if (self.numel() == 0) return out;
  if (self.dim() == 0) {
    device_copy(out, self);
    return out;
  }
  const int64_t d = at::maybe_wrap_dim(dim, self.dim());
  at::Tensor x = contiguous_on_device(self.scalar_type() == rt ? self : self.to(rt));
  int64_t outer = 1, inner = 1;
  for (int64_t i = 0; i < d; ++i) outer *= x.size(i);
  for (int64_t i = d + 1; i < x.dim(); ++i) inner *= x.size(i);
  const int64_t len = x.size(d);
  return fill_contiguous(out, [&](at::Tensor& t) {
    SPYRE_SPH_CHECK(sph_cumsum(to_sph(rt), x.data_ptr(), t.data_ptr(), outer, len, inner,
                               stream(t.get_device())));
  });
}

at::ScalarType cumsum_type(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
  return dtype.has_value() ? *dtype
         : at::isIntegralType(self.scalar_type(), /*includeBool=*/true) ? at::kLong
                                                                         : self.scalar_type();
}

at::Tensor cumsum(const at::Tensor& self, int64_t dim, std::optional<at::ScalarType> dtype) {
  at::Tensor out = empty_spyre(self.sizes(), cumsum_type(self, dtype), self.device());
  return cumsum_out(self, dim, dtype, out);
}

at::Tensor& cumsum_(at::Tensor& self, int64_t dim, std::optional<at::ScalarType> dtype) {
  TORCH_CHECK(!dtype.has_value() || *dtype == self.scalar_type(),
              "spyre: in-place cumsum keeps the tensor's dtype");
  TORCH_CHECK(cumsum_type(self, std::nullopt) == self.scalar_type(),
              "spyre: in-place cumsum of ", self.scalar_type(), " would change its dtype");
  return cumsum_out(self, dim, dtype, self);
}

at::Tensor& normal_(at::Tensor& self, double mean, double std,
                    std::optional<at::Generator> gen) {
  TORCH_CHECK(std >= 0.0, "normal expects std >= 0.0, but found std ", std);
  TORCH_CHECK(at::isFloatingType(self.scalar_type()), "spyre: normal_ needs a float tensor");
  return random_fill(self, SPH_RNG_NORMAL, mean, std, 0, 0, gen);
}

at::Tensor& uniform_(at::Tensor& self, double from, double to,
                     std::optional<at::Generator> gen) {
  TORCH_CHECK(from <= to, "uniform_ expects to return a [from, to) range, but found from=", from,
              " > to=", to);
  TORCH_CHECK(at::isFloatingType(self.scalar_type()), "spyre: uniform_ needs a float tensor");
  return random_fill(self, SPH_RNG_UNIFORM, from, to, 0, 0, gen);
}

// random_(from, to): integers in [from, to), or [from, the dtype's largest
// exactly representable integer] when `to` is None (2^mantissa bits for
// floating types), as torch's random_.
at::Tensor& random_from_(at::Tensor& self, int64_t from, std::optional<int64_t> to,
                         std::optional<at::Generator> gen) {
  const at::ScalarType dt = self.scalar_type();
  uint64_t range = 0;
  if (to.has_value()) {
    TORCH_CHECK(from < *to, "random_ expects 'from' to be less than 'to', but got from=", from,
                " >= to=", *to);
    range = static_cast<uint64_t>(*to) - static_cast<uint64_t>(from);
  } else {
    int64_t to_inc = 0;
    switch (dt) {
      case at::kHalf: to_inc = int64_t(1) << 11; break;
      case at::kBFloat16: to_inc = int64_t(1) << 8; break;
      case at::kFloat: to_inc = int64_t(1) << 24; break;
      case at::kDouble: to_inc = int64_t(1) << 53; break;
      case at::kBool: to_inc = 1; break;
      case at::kByte: to_inc = 255; break;
      case at::kChar: to_inc = 127; break;
      case at::kShort: to_inc = 32767; break;
      case at::kInt: to_inc = 2147483647; break;
      case at::kLong: to_inc = std::numeric_limits<int64_t>::max(); break;
      default: TORCH_CHECK(false, "spyre: random_ does not support ", dt);
    }
    TORCH_CHECK(from <= to_inc, "random_ expects 'from' casted to dtype to be less than or equal "
                "to 'to_inc' casted to dtype");
    range = static_cast<uint64_t>(to_inc) - static_cast<uint64_t>(from) + 1;
    if (range == 0) range = ~uint64_t(0);  // the full 64-bit range (from = int64 min)
  }
  return random_fill(self, SPH_RNG_INT, 0.0, 0.0, from, range, gen);
}

at::Tensor& random_(at::Tensor& self, std::optional<at::Generator> gen) {
  return random_from_(self, 0, std::nullopt, gen);
}

at::Tensor& random_to_(at::Tensor& self, int64_t to, std::optional<at::Generator> gen) {
  return random_from_(self, 0, to, gen);
}

// Advanced indexing, self[indices] (reference: the `index` Gather of
// codegen/inputs/Metadata.yaml:158).  Boolean masks become the long
// indices of their true elements; negative indices wrap; an index outside
// its dimension raises IndexError.  The index tensors broadcast to one shape
// B; the indexed dimensions (moved to the front when they are not adjacent,
// as torch orders the result) are flattened into one, whose flat index
// sum_k idx_k * prod(later indexed sizes) is gathered with one
// index_select: result = sizes before + B + sizes after.
at::Tensor index_tensor(const at::Tensor& self,
                        const c10::List<std::optional<at::Tensor>>& indices) {
  TORCH_CHECK(static_cast<int64_t>(indices.size()) <= self.dim(),
              "too many indices for tensor of dimension ", self.dim(), " (got ",
              indices.size(), ")");
  std::vector<int64_t> dims;
  std::vector<at::Tensor> idx;
  int64_t d = 0;
  for (size_t i = 0; i < indices.size(); ++i) {
    const std::optional<at::Tensor> o = indices.get(i);
    if (!o.has_value() || !o->defined()) {
      ++d;
      continue;
    }
    const at::Tensor& t = *o;
    if (t.scalar_type() == at::kBool || t.scalar_type() == at::kByte) {
      // a mask over the next t.dim() dimensions: the coordinates of its
      // true elements, found on the host (their count sets the shape)
      for (int64_t k = 0; k < t.dim(); ++k)
        TORCH_CHECK_INDEX(d + k < self.dim() && t.size(k) == self.size(d + k),
                          "The shape of the mask ", t.sizes(), " at index ", k,
                          " does not match the shape of the indexed tensor ", self.sizes());
      const at::Tensor nz = t.cpu().to(at::kBool).nonzero();  // [count, t.dim()]
      for (int64_t k = 0; k < t.dim(); ++k) {
        dims.push_back(d + k);
        idx.push_back(nz.select(1, k).contiguous().to(self.device()));
      }
      d += t.dim();
    } else {
      TORCH_CHECK_INDEX(at::isIntegralType(t.scalar_type(), false),
                        "tensors used as indices must be long, int, byte or bool tensors");
      dims.push_back(d);
      idx.push_back(t.to(self.device(), at::kLong));
      ++d;
    }
  }
  TORCH_CHECK(!dims.empty(), "spyre: index with no index tensor");
  TORCH_CHECK(d <= self.dim(), "too many indices for tensor of dimension ", self.dim());
  // broadcast shape of the index tensors
  std::vector<at::Tensor> bt = at::broadcast_tensors(idx);
  const auto bshape = bt[0].sizes().vec();
  bool adjacent = true;
  for (size_t k = 1; k < dims.size(); ++k) adjacent = adjacent && dims[k] == dims[k - 1] + 1;
  // self with the indexed dims together (in order) starting at `first`
  at::Tensor x = self;
  int64_t first = dims[0];
  if (!adjacent) {
    std::vector<int64_t> perm(dims.begin(), dims.end());
    for (int64_t k = 0; k < self.dim(); ++k)
      if (std::find(dims.begin(), dims.end(), k) == dims.end()) perm.push_back(k);
    x = self.permute(perm);
    first = 0;
  }
  const int64_t nk = static_cast<int64_t>(dims.size());
  // flat index over the indexed block, each index wrapped and checked
  at::Tensor flat;
  int64_t span = 1;
  for (int64_t k = nk - 1; k >= 0; --k) {
    const int64_t size = x.size(first + k);
    at::Tensor ik = bt[k];
    if (ik.numel() > 0) {
      const int64_t lo = ik.amin().item<int64_t>(), hi = ik.amax().item<int64_t>();
      TORCH_CHECK_INDEX(lo >= -size && hi < size, "index ", lo < -size ? lo : hi,
                        " is out of bounds for dimension ", dims[k], " with size ", size);
      if (lo < 0) ik = at::where(ik.lt(0), ik.add(size), ik);
    }
    at::Tensor term = span == 1 ? ik : ik.mul(span);
    flat = flat.defined() ? flat.add(term) : term;
    span *= size;
  }
  std::vector<int64_t> xs(x.sizes().begin(), x.sizes().begin() + first);
  xs.push_back(span);
  xs.insert(xs.end(), x.sizes().begin() + first + nk, x.sizes().end());
  at::Tensor g = x.reshape(xs).index_select(first, flat.reshape({-1}));
  std::vector<int64_t> rs(x.sizes().begin(), x.sizes().begin() + first);
  rs.insert(rs.end(), bshape.begin(), bshape.end());
  rs.insert(rs.end(), x.sizes().begin() + first + nk, x.sizes().end());
  return g.reshape(rs);
}

at::Tensor& index_tensor_out(const at::Tensor& self,
                             const c10::List<std::optional<at::Tensor>>& indices,
                             at::Tensor& out) {
  at::Tensor r = index_tensor(self, indices);
  at::native::resize_output(out, r.sizes());
  out.copy_(r);
  return out;
}

// native_dropout_backward (reference: codegen/inputs/Metadata.yaml:93):
// grad * mask * scale, evaluated left to right in grad's dtype as torch's
// CPU kernel does.
at::Tensor native_dropout_backward(const at::Tensor& grad, const at::Tensor& mask,
                                   double scale) {
  TORCH_CHECK(grad.sizes() == mask.sizes(), "spyre: dropout backward: grad ", grad.sizes(),
              " and mask ", mask.sizes(), " differ in shape");
  return grad.mul(mask.to(grad.scalar_type())).mul_(scale);
}

// upsample_nearest2d (reference: codegen/inputs/Metadata.yaml:331): two
// row gathers (index_select over H, then over W) with torch's nearest
// index: the identity when the size is unchanged, o >> 1 when doubled,
// else min(floor(o * s), in - 1) with s = 1 / scale (a given scale > 0)
// or in / out in float.
std::vector<int64_t> nearest_indices(int64_t in, int64_t out, std::optional<double> scale) {
  std::vector<int64_t> idx(static_cast<size_t>(out));
  const float s = (scale.has_value() && *scale > 0.0) ? static_cast<float>(1.0 / *scale)
                                                      : static_cast<float>(in) / out;
  for (int64_t o = 0; o < out; ++o) {
    if (out == in) idx[o] = o;
    else if (out == 2 * in) idx[o] = o >> 1;
    else idx[o] = std::min(static_cast<int64_t>(std::floor(o * s)), in - 1);
  }
  return idx;
}

at::Tensor& upsample_nearest2d_out(const at::Tensor& self, c10::SymIntArrayRef output_size,
                                   std::optional<double> scales_h,
                                   std::optional<double> scales_w, at::Tensor& out) {
  const auto os = c10::asIntArrayRefUnchecked(output_size);
  TORCH_CHECK(os.size() == 2, "spyre: upsample_nearest2d expects two output sizes");
  TORCH_CHECK(self.dim() == 4, "spyre: upsample_nearest2d expects a 4-D input, got ",
              self.dim(), " dims");
  const int64_t ih = self.size(2), iw = self.size(3), oh = os[0], ow = os[1];
  TORCH_CHECK(ih > 0 && iw > 0 && oh > 0 && ow > 0,
              "spyre: upsample_nearest2d: input and output sizes must be positive");
  auto dev = [&](const std::vector<int64_t>& v) {
    return at::tensor(v, at::TensorOptions().dtype(at::kLong)).to(self.device());
  };
  at::Tensor y = self.index_select(2, dev(nearest_indices(ih, oh, scales_h)))
                     .index_select(3, dev(nearest_indices(iw, ow, scales_w)));
  at::native::resize_output(out, y.sizes());
  out.copy_(y);
  return out;
}

at::Tensor upsample_nearest2d(const at::Tensor& self, c10::SymIntArrayRef output_size,
                              std::optional<double> scales_h, std::optional<double> scales_w) {
  at::Tensor out = empty_spyre({0}, self.scalar_type(), self.device());
  return upsample_nearest2d_out(self, output_size, scales_h, scales_w, out);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("cat.out", TORCH_FN(cat_out));
  m.impl("tril.out", TORCH_FN(tri_out<0>));
  m.impl("triu.out", TORCH_FN(tri_out<1>));
  m.impl("index.Tensor", TORCH_FN(index_tensor));
  m.impl("index.Tensor_out", TORCH_FN(index_tensor_out));
  m.impl("index_select", TORCH_FN(index_select));
  m.impl("index_select.out", TORCH_FN(index_select_out));
  m.impl("native_dropout", TORCH_FN(native_dropout));
  m.impl("native_dropout_backward", TORCH_FN(native_dropout_backward));
  m.impl("upsample_nearest2d", TORCH_FN(upsample_nearest2d));
  m.impl("upsample_nearest2d.out", TORCH_FN(upsample_nearest2d_out));
  m.impl("arange.start_out", TORCH_FN(arange_out));
  m.impl("cumsum.out", TORCH_FN(cumsum_out));
  m.impl("cumsum", TORCH_FN(cumsum));
  m.impl("cumsum_", TORCH_FN(cumsum_));
  m.impl("normal_", TORCH_FN(normal_));
  m.impl("uniform_", TORCH_FN(uniform_));
  m.impl("random_.from", TORCH_FN(random_from_));
  m.impl("random_", TORCH_FN(random_));
  m.impl("random_.to", TORCH_FN(random_to_));
}

}  // namespace spyre
