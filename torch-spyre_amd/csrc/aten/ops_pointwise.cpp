// Eager elementwise ops of the spyre backend on the kernel library's strided
// pointwise engine (sph_pointwise).
//
// Reference: the generated base/list_inp eager ops of
// codegen/inputs/Metadata.yaml (add :18-20, sub :296-298, mul :185-187,
// div :84-86, exp, gelu :125-132, silu :269-271, rsqrt :251-253,
// pow :236-238, eq/ge/..., where) rendered by codegen/templates/base.jinja2:
// 16-241, and the clone of codegen/inputs/spyre_torch_ops.cpp:507-583.
//
// Broadcasting, type promotion and output allocation come from torch's
// TensorIterator (the same metadata logic torch's CPU kernels use); the
// arithmetic is one kernel launch per op.  Structured ops are registered by
// their .out overload: torch's generic functional / in-place wrappers call
// it.  Values follow torch's CPU semantics: fp16/bf16 inputs are computed
// in fp32 and rounded once; integer add/sub/mul/compare stay exact.
#include <ATen/MemoryOverlap.h>
#include <ATen/native/Resize.h>
#include <torch/library.h>

#include <cmath>
#include <limits>

#include "spyre_ops_common.h"

namespace spyre {

void check_extent(const at::Tensor& t, const void* ptr, int ndim, const int64_t* sizes,
                  const int64_t* strides, int64_t elem_bytes, const char* what) {
  int64_t lo = 0, hi = 0;
  for (int d = 0; d < ndim; ++d) {
    if (sizes[d] == 0) return;  // nothing addressed
    const int64_t span = (sizes[d] - 1) * strides[d];
    if (span < 0) lo += span;
    else hi += span;
  }
  const c10::Storage& st = t.storage();
  const auto* base = static_cast<const char*>(st.data());
  const auto* p = static_cast<const char*>(ptr);
  const auto* first = p + lo * elem_bytes;
  const auto* last = p + (hi + 1) * elem_bytes;
  TORCH_CHECK(base != nullptr && first >= base && last <= base + st.nbytes(), "spyre: ", what,
              ": operand addresses bytes [", static_cast<const void*>(first), ", ",
              static_cast<const void*>(last), ") outside its storage [",
              static_cast<const void*>(base), ", +", st.nbytes(), ")");
}

void check_matrix_extent(const at::Tensor& t, const void* ptr, int64_t rows, int64_t cols,
                         int64_t ld, int trans, int64_t batch, int64_t batch_stride,
                         const char* what) {
  const int64_t sizes[3] = {batch, rows, cols};
  const int64_t strides[3] = {batch_stride, trans ? 1 : ld, trans ? ld : 1};
  check_extent(t, ptr, 3, sizes, strides, t.element_size(), what);
}

// ---------------------------------------------------------------------------
// TensorIterator -> sph_pointwise
// ---------------------------------------------------------------------------
void launch_iter(int op, const at::TensorIteratorBase& iter, double alpha, double beta) {
  if (iter.numel() == 0) return;
  TORCH_CHECK(iter.noutputs() == 1, "spyre: pointwise kernels have one output");
  const int nt = iter.ntensors();
  int nd = iter.ndim();
  TORCH_CHECK(nd <= SPH_MAX_DIMS, "spyre: elementwise op over more than ", SPH_MAX_DIMS,
              " non-collapsible dims");
  bool all_same = true;
  for (int i = 1; i < nt; ++i) all_same = all_same && iter.dtype(i) == iter.dtype(0);
  std::vector<sph_operand> ops(nt);
  int64_t sizes[SPH_MAX_DIMS] = {1};
  for (int d = 0; d < nd; ++d) sizes[nd - 1 - d] = iter.shape()[d];
  for (int i = 0; i < nt; ++i) {
    const at::ScalarType dt = iter.dtype(i);
    const int64_t isz = static_cast<int64_t>(iter.element_size(i));
    if (has_sph(dt)) {
      ops[i].dtype = to_sph(dt);
    } else {
      TORCH_CHECK(op == SPH_PW_COPY && all_same, "spyre: dtype ", dt,
                  " is only supported by same-dtype copies");
      ops[i].dtype = isz == 1 ? SPH_U8 : isz == 2 ? SPH_I16 : isz == 4 ? SPH_I32 : SPH_I64;
      TORCH_CHECK(isz == 1 || isz == 2 || isz == 4 || isz == 8, "spyre: unsupported dtype ", dt);
    }
    ops[i].data = iter.data_ptr(i);
    const auto st = iter.strides(i);
    for (int d = 0; d < nd; ++d) ops[i].strides[nd - 1 - d] = st[d] / isz;
    check_extent(iter.tensor(i), ops[i].data, nd, sizes, ops[i].strides, isz, "pointwise");
  }
  if (nd == 0) {
    nd = 1;
    sizes[0] = 1;
    for (auto& o : ops) o.strides[0] = 0;
  }
  const int dev = iter.device(0).index();
  SPYRE_SPH_CHECK(sph_pointwise(op, nt - 1, ops.data(), nd, sizes, alpha, beta, stream(dev)));
}

namespace {

// A same-dtype copy into a dense destination whose source is contiguous
// along another dimension than the destination (a transposed view made
// contiguous, a head split or merge): one tiled transpose, coalesced on both
// sides.  Other copies (and small transposes) take the elementwise engine.
bool transpose_copy(const at::Tensor& dst, const at::Tensor& src) {
  if (src.scalar_type() != dst.scalar_type() || !src.sizes().equals(dst.sizes()) ||
      !is_spyre(src) || src.get_device() != dst.get_device() ||
      !dst.is_non_overlapping_and_dense())
    return false;
  int u = -1, v = -1;
  for (int64_t d = 0; d < dst.dim(); ++d) {
    if (dst.size(d) == 1) continue;
    if (dst.stride(d) == 1 && u < 0) u = static_cast<int>(d);
    if (src.stride(d) == 1 && v < 0) v = static_cast<int>(d);
  }
  if (u < 0 || v < 0 || u == v || dst.size(u) < 16 || dst.size(v) < 16) return false;
  int64_t bs[4], bsrc[4], bdst[4];
  int nb = 0;
  for (int64_t d = 0; d < dst.dim(); ++d) {
    if (d == u || d == v || dst.size(d) == 1) continue;
    if (nb == 4) return false;
    bs[nb] = dst.size(d);
    bsrc[nb] = src.stride(d);
    bdst[nb] = dst.stride(d);
    ++nb;
  }
  // (get_overlap_status answers TooHard for any source that is not dense,
  // such as a column slice of a wider matrix: a source in other storage
  // cannot overlap the destination)
  if (src.storage().is_alias_of(dst.storage()) &&
      at::get_overlap_status(dst, src) != at::MemOverlapStatus::No)
    return false;
  c10::DeviceGuard guard(dst.device());
  SPYRE_SPH_CHECK(sph_transpose_copy(static_cast<int>(dst.element_size()), src.data_ptr(),
                                     dst.data_ptr(), dst.size(u), dst.size(v), src.stride(u),
                                     dst.stride(v), nb, bs, bsrc, bdst, stream(dst.get_device())));
  return true;
}

}  // namespace

void device_copy(const at::Tensor& dst, const at::Tensor& src) {
  if (dst.numel() == 0) return;
  if (transpose_copy(dst, src)) return;
  auto iter = at::TensorIteratorConfig()
                  .add_output(dst)
                  .add_const_input(src)
                  .resize_outputs(false)
                  .check_all_same_dtype(false)
                  .set_check_mem_overlap(true)
                  .build();
  launch_iter(SPH_PW_COPY, iter);
}

at::Tensor contiguous_on_device(const at::Tensor& t) {
  if (t.is_contiguous()) return t;
  at::Tensor out = empty_spyre(t.sizes(), t.scalar_type(), t.device());
  device_copy(out, t);
  return out;
}

namespace {

// A CPU 0-d operand moved to the device (broadcast with stride 0).
at::Tensor on_device(const at::Tensor& t, const at::Tensor& like) {
  if (!t.defined() || is_spyre(t)) return t;
  TORCH_CHECK(t.dim() == 0, "spyre: expected a spyre tensor, got a ", t.device(),
              " tensor of ", t.dim(), " dims");
  at::Tensor d = empty_spyre({}, t.scalar_type(), like.device());
  d.copy_(t);
  return d;
}

at::Tensor& unary_out(int op, const at::Tensor& self, at::Tensor& out, double alpha = 0.0,
                      double beta = 0.0) {
  auto iter = at::TensorIteratorConfig()
                  .add_output(out)
                  .add_const_input(self)
                  .check_all_same_dtype(false)
                  .build();
  launch_iter(op, iter, alpha, beta);
  return out;
}

// out = op(a, b) with a, b broadcast.  A CPU 0-d operand (a wrapped Python
// number) that the caller did not turn into a scalar op is moved to the
// device first.
at::Tensor& binary_out(int op, const at::Tensor& a, const at::Tensor& b, at::Tensor& out,
                       double alpha = 1.0) {
  at::Tensor da = on_device(a, is_spyre(a) ? a : b);
  at::Tensor db = on_device(b, is_spyre(b) ? b : a);
  auto iter = at::TensorIteratorConfig()
                  .add_output(out)
                  .add_const_input(da)
                  .add_const_input(db)
                  .check_all_same_dtype(false)
                  .build();
  launch_iter(op, iter, alpha, 0.0);
  return out;
}

double scalar_of(const at::Tensor& t) { return t.item<double>(); }

// --- arithmetic -------------------------------------------------------------
at::Tensor& add_out(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha,
                    at::Tensor& out) {
  const double a = alpha.toDouble();
  if (is_cpu_scalar(other) && is_spyre(self))
    return unary_out(SPH_PW_ADD_SCALAR, self, out, a * scalar_of(other));
  return binary_out(SPH_PW_ADD, self, other, out, a);
}

at::Tensor& sub_out(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha,
                    at::Tensor& out) {
  const double a = alpha.toDouble();
  if (is_cpu_scalar(other) && is_spyre(self))
    return unary_out(SPH_PW_ADD_SCALAR, self, out, -a * scalar_of(other));
  return binary_out(SPH_PW_SUB, self, other, out, a);
}

at::Tensor& mul_out(const at::Tensor& self, const at::Tensor& other, at::Tensor& out) {
  if (is_cpu_scalar(other) && is_spyre(self))
    return unary_out(SPH_PW_MUL_SCALAR, self, out, scalar_of(other));
  if (is_cpu_scalar(self) && is_spyre(other))
    return unary_out(SPH_PW_MUL_SCALAR, other, out, scalar_of(self));
  return binary_out(SPH_PW_MUL, self, other, out);
}

at::Tensor& div_out(const at::Tensor& self, const at::Tensor& other, at::Tensor& out) {
  if (is_cpu_scalar(other) && is_spyre(self))
    return unary_out(SPH_PW_DIV_SCALAR, self, out, scalar_of(other));
  return binary_out(SPH_PW_DIV, self, other, out);
}

at::Tensor rsub_tensor(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha) {
  // other - alpha * self
  const auto dt = at::result_type(self, other);
  at::Tensor out = empty_spyre(at::infer_size(self.sizes(), other.sizes()), dt,
                               is_spyre(self) ? self.device() : other.device());
  if (is_cpu_scalar(other) && is_spyre(self)) {
    // alpha * self then rsub by the scalar: out = s - alpha*self
    unary_out(SPH_PW_MUL_SCALAR, self, out, alpha.toDouble());
    return unary_out(SPH_PW_RSUB_SCALAR, out, out, scalar_of(other));
  }
  return binary_out(SPH_PW_SUB, other, self, out, alpha.toDouble());
}

at::Tensor& maximum_out(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  return binary_out(SPH_PW_MAXIMUM, a, b, out);
}
at::Tensor& minimum_out(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  return binary_out(SPH_PW_MINIMUM, a, b, out);
}

at::Tensor& pow_ts_out(const at::Tensor& self, const at::Scalar& e, at::Tensor& out) {
  return unary_out(SPH_PW_POW_SCALAR, self, out, e.toDouble());
}
at::Tensor& pow_tt_out(const at::Tensor& self, const at::Tensor& e, at::Tensor& out) {
  if (is_cpu_scalar(e) && is_spyre(self))
    return unary_out(SPH_PW_POW_SCALAR, self, out, scalar_of(e));
  return binary_out(SPH_PW_POW, self, e, out);
}
at::Tensor& pow_st_out(const at::Scalar& base, const at::Tensor& e, at::Tensor& out) {
  return unary_out(SPH_PW_RPOW_SCALAR, e, out, base.toDouble());
}

at::Tensor& lerp_out(const at::Tensor& self, const at::Tensor& end, const at::Scalar& w,
                     at::Tensor& out) {
  return binary_out(SPH_PW_LERP, self, end, out, w.toDouble());
}

at::Tensor& addcmul_out(const at::Tensor& self, const at::Tensor& t1, const at::Tensor& t2,
                        const at::Scalar& value, at::Tensor& out) {
  const at::Tensor s0 = on_device(self, out), s1 = on_device(t1, out), s2 = on_device(t2, out);
  auto iter = at::TensorIteratorConfig()
                  .add_output(out)
                  .add_const_input(s0)
                  .add_const_input(s1)
                  .add_const_input(s2)
                  .check_all_same_dtype(false)
                  .build();
  launch_iter(SPH_PW_ADDCMUL, iter, value.toDouble());
  return out;
}

// --- comparisons -----------------------------------------------------------
template <int OP, int SOP>
at::Tensor& cmp_tensor_out(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  if (is_cpu_scalar(b) && is_spyre(a)) return unary_out(SOP, a, out, scalar_of(b));
  return binary_out(OP, a, b, out);
}
template <int SOP>
at::Tensor& cmp_scalar_out(const at::Tensor& a, const at::Scalar& s, at::Tensor& out) {
  return unary_out(SOP, a, out, s.toDouble());
}

at::Tensor& logical_and_out(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  return binary_out(SPH_PW_LOGICAL_AND, a, b, out);
}
at::Tensor& logical_or_out(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  return binary_out(SPH_PW_LOGICAL_OR, a, b, out);
}

at::Tensor isnan(const at::Tensor& self) {
  at::Tensor out = empty_spyre(self.sizes(), at::kBool, self.device());
  return binary_out(SPH_PW_NE, self, self, out);
}

// --- unary -----------------------------------------------------------------
template <int OP>
at::Tensor& unary_op_out(const at::Tensor& self, at::Tensor& out) {
  return unary_out(OP, self, out);
}

at::Tensor& gelu_out(const at::Tensor& self, c10::string_view approximate, at::Tensor& out) {
  return unary_out(approximate == "tanh" ? SPH_PW_GELU_TANH : SPH_PW_GELU, self, out);
}

at::Tensor relu(const at::Tensor& self) {
  at::Tensor out = empty_spyre(self.sizes(), self.scalar_type(), self.device());
  return unary_out(SPH_PW_RELU, self, out);
}
at::Tensor& relu_(at::Tensor& self) { return unary_out(SPH_PW_RELU, self, self); }

at::Tensor& leaky_relu_out(const at::Tensor& self, const at::Scalar& slope, at::Tensor& out) {
  return unary_out(SPH_PW_LEAKY_RELU, self, out, slope.toDouble());
}

at::Tensor& clamp_out(const at::Tensor& self, const std::optional<at::Scalar>& lo,
                      const std::optional<at::Scalar>& hi, at::Tensor& out) {
  const double inf = std::numeric_limits<double>::infinity();
  return unary_out(SPH_PW_CLAMP, self, out, lo ? lo->toDouble() : -inf,
                   hi ? hi->toDouble() : inf);
}
at::Tensor& clamp_min_out(const at::Tensor& self, const at::Scalar& lo, at::Tensor& out) {
  return unary_out(SPH_PW_CLAMP, self, out, lo.toDouble(), std::numeric_limits<double>::infinity());
}
at::Tensor& clamp_max_out(const at::Tensor& self, const at::Scalar& hi, at::Tensor& out) {
  return unary_out(SPH_PW_CLAMP, self, out, -std::numeric_limits<double>::infinity(), hi.toDouble());
}
at::Tensor hardtanh(const at::Tensor& self, const at::Scalar& lo, const at::Scalar& hi) {
  at::Tensor out = empty_spyre(self.sizes(), self.scalar_type(), self.device());
  return unary_out(SPH_PW_CLAMP, self, out, lo.toDouble(), hi.toDouble());
}

// --- selection -------------------------------------------------------------
at::Tensor& where_out(const at::Tensor& cond, const at::Tensor& self, const at::Tensor& other,
                      at::Tensor& out) {
  const at::Tensor& like = is_spyre(self) ? self : is_spyre(other) ? other : cond;
  const at::Tensor c0 = on_device(cond, like), a0 = on_device(self, like),
                   b0 = on_device(other, like);
  auto iter = at::TensorIteratorConfig()
                  .add_output(out)
                  .add_const_input(c0)
                  .add_const_input(a0)
                  .add_const_input(b0)
                  .check_all_same_dtype(false)
                  .build();
  launch_iter(SPH_PW_WHERE, iter);
  return out;
}

at::Tensor where_self(const at::Tensor& cond, const at::Tensor& self, const at::Tensor& other) {
  const auto dt = at::result_type(self, other);
  const auto shape = at::infer_size(at::infer_size(cond.sizes(), self.sizes()), other.sizes());
  const at::Tensor& like = is_spyre(self) ? self : is_spyre(other) ? other : cond;
  at::Tensor out = empty_spyre(shape, dt, like.device());
  return where_out(cond, self, other, out);
}

at::Tensor& masked_fill_scalar_(at::Tensor& self, const at::Tensor& mask, const at::Scalar& v) {
  const at::Tensor val = on_device(at::scalar_tensor(v, self.options().device(at::kCPU)), self);
  auto iter = at::TensorIteratorConfig()
                  .add_output(self)
                  .add_const_input(mask)
                  .add_const_input(val)
                  .add_const_input(self)
                  .check_all_same_dtype(false)
                  .resize_outputs(false)
                  .set_check_mem_overlap(false)
                  .build();
  launch_iter(SPH_PW_WHERE, iter);
  return self;
}

at::Tensor& masked_fill_tensor_(at::Tensor& self, const at::Tensor& mask, const at::Tensor& v) {
  TORCH_CHECK(v.dim() == 0, "spyre: masked_fill_ only supports a 0-dimension value tensor");
  return masked_fill_scalar_(self, mask, v.item());
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("add.out", TORCH_FN(add_out));
  m.impl("sub.out", TORCH_FN(sub_out));
  m.impl("mul.out", TORCH_FN(mul_out));
  m.impl("div.out", TORCH_FN(div_out));
  m.impl("rsub.Tensor", TORCH_FN(rsub_tensor));
  m.impl("maximum.out", TORCH_FN(maximum_out));
  m.impl("minimum.out", TORCH_FN(minimum_out));
  m.impl("pow.Tensor_Scalar_out", TORCH_FN(pow_ts_out));
  m.impl("pow.Tensor_Tensor_out", TORCH_FN(pow_tt_out));
  m.impl("pow.Scalar_out", TORCH_FN(pow_st_out));
  m.impl("lerp.Scalar_out", TORCH_FN(lerp_out));
  m.impl("addcmul.out", TORCH_FN(addcmul_out));

  m.impl("eq.Tensor_out", TORCH_FN((cmp_tensor_out<SPH_PW_EQ, SPH_PW_EQ_SCALAR>)));
  m.impl("ne.Tensor_out", TORCH_FN((cmp_tensor_out<SPH_PW_NE, SPH_PW_NE_SCALAR>)));
  m.impl("lt.Tensor_out", TORCH_FN((cmp_tensor_out<SPH_PW_LT, SPH_PW_LT_SCALAR>)));
  m.impl("le.Tensor_out", TORCH_FN((cmp_tensor_out<SPH_PW_LE, SPH_PW_LE_SCALAR>)));
  m.impl("gt.Tensor_out", TORCH_FN((cmp_tensor_out<SPH_PW_GT, SPH_PW_GT_SCALAR>)));
  m.impl("ge.Tensor_out", TORCH_FN((cmp_tensor_out<SPH_PW_GE, SPH_PW_GE_SCALAR>)));
  m.impl("eq.Scalar_out", TORCH_FN(cmp_scalar_out<SPH_PW_EQ_SCALAR>));
  m.impl("ne.Scalar_out", TORCH_FN(cmp_scalar_out<SPH_PW_NE_SCALAR>));
  m.impl("lt.Scalar_out", TORCH_FN(cmp_scalar_out<SPH_PW_LT_SCALAR>));
  m.impl("le.Scalar_out", TORCH_FN(cmp_scalar_out<SPH_PW_LE_SCALAR>));
  m.impl("gt.Scalar_out", TORCH_FN(cmp_scalar_out<SPH_PW_GT_SCALAR>));
  m.impl("ge.Scalar_out", TORCH_FN(cmp_scalar_out<SPH_PW_GE_SCALAR>));
  m.impl("logical_and.out", TORCH_FN(logical_and_out));
  m.impl("logical_or.out", TORCH_FN(logical_or_out));
  m.impl("isnan", TORCH_FN(isnan));

  m.impl("neg.out", TORCH_FN(unary_op_out<SPH_PW_NEG>));
  m.impl("abs.out", TORCH_FN(unary_op_out<SPH_PW_ABS>));
  m.impl("exp.out", TORCH_FN(unary_op_out<SPH_PW_EXP>));
  m.impl("log.out", TORCH_FN(unary_op_out<SPH_PW_LOG>));
  m.impl("sqrt.out", TORCH_FN(unary_op_out<SPH_PW_SQRT>));
  m.impl("rsqrt.out", TORCH_FN(unary_op_out<SPH_PW_RSQRT>));
  m.impl("reciprocal.out", TORCH_FN(unary_op_out<SPH_PW_RECIPROCAL>));
  m.impl("sigmoid.out", TORCH_FN(unary_op_out<SPH_PW_SIGMOID>));
  m.impl("tanh.out", TORCH_FN(unary_op_out<SPH_PW_TANH>));
  m.impl("silu.out", TORCH_FN(unary_op_out<SPH_PW_SILU>));
  m.impl("sin.out", TORCH_FN(unary_op_out<SPH_PW_SIN>));
  m.impl("cos.out", TORCH_FN(unary_op_out<SPH_PW_COS>));
  m.impl("erf.out", TORCH_FN(unary_op_out<SPH_PW_ERF>));
  m.impl("log1p.out", TORCH_FN(unary_op_out<SPH_PW_LOG1P>));
  m.impl("expm1.out", TORCH_FN(unary_op_out<SPH_PW_EXPM1>));
  m.impl("mish.out", TORCH_FN(unary_op_out<SPH_PW_MISH>));
  m.impl("logical_not.out", TORCH_FN(unary_op_out<SPH_PW_LOGICAL_NOT>));
  m.impl("bitwise_not.out", TORCH_FN(unary_op_out<SPH_PW_BITWISE_NOT>));
  m.impl("sign.out", TORCH_FN(unary_op_out<SPH_PW_SIGN>));
  m.impl("floor.out", TORCH_FN(unary_op_out<SPH_PW_FLOOR>));
  m.impl("ceil.out", TORCH_FN(unary_op_out<SPH_PW_CEIL>));
  m.impl("round.out", TORCH_FN(unary_op_out<SPH_PW_ROUND>));
  m.impl("trunc.out", TORCH_FN(unary_op_out<SPH_PW_TRUNC>));
  m.impl("gelu.out", TORCH_FN(gelu_out));
  m.impl("relu", TORCH_FN(relu));
  m.impl("relu_", TORCH_FN(relu_));
  m.impl("leaky_relu.out", TORCH_FN(leaky_relu_out));
  m.impl("clamp.out", TORCH_FN(clamp_out));
  m.impl("clamp_min.out", TORCH_FN(clamp_min_out));
  m.impl("clamp_max.out", TORCH_FN(clamp_max_out));
  m.impl("hardtanh", TORCH_FN(hardtanh));

  m.impl("where.self_out", TORCH_FN(where_out));
  m.impl("where.self", TORCH_FN(where_self));
  m.impl("masked_fill_.Scalar", TORCH_FN(masked_fill_scalar_));
  m.impl("masked_fill_.Tensor", TORCH_FN(masked_fill_tensor_));
}

}  // namespace spyre
