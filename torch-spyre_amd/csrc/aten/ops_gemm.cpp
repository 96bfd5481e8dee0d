// Matrix products of the spyre backend on the MFMA GEMM (sph_gemm /
// sph_gemm_strided_batched): mm, bmm, addmm, baddbmm.  matmul and linear are
// torch composites that reach these.
//
// Reference: spyre__mm_default (codegen/inputs/spyre_torch_ops.cpp:214-293),
// spyre__bmm_default (:297-377), spyre__addmm_* (:381-452, which ignores
// beta; here beta follows torch: D = beta*self + alpha*(A@B), self ignored
// when beta == 0).  The reference's "tall operands" transpose trick
// (:218-219, :290) is unnecessary: the kernel reads either operand
// transposed through its strides.
#include <ATen/native/Resize.h>
#include <torch/library.h>

#include "spyre_ops_common.h"

namespace spyre {
namespace {

// A [rows, cols] matrix view as the kernel addresses it: row-major with
// leading dim `ld` (trans = 0) or transposed / column-major (trans = 1).
struct MatView {
  at::Tensor keep;  // owns a contiguous copy when one was needed
  const void* ptr = nullptr;
  int trans = 0;
  int64_t ld = 0;
};

MatView mat_view(const at::Tensor& t) {
  const int64_t r = t.size(0), c = t.size(1);
  const int64_t s0 = t.stride(0), s1 = t.stride(1);
  MatView v;
  if (c == 1 || s1 == 1) {
    if (r == 1 || s0 >= std::max<int64_t>(c, 1)) {
      v.ptr = t.data_ptr();
      v.trans = 0;
      v.ld = r == 1 ? std::max<int64_t>(c, 1) : s0;
      return v;
    }
  }
  if (r == 1 || s0 == 1) {
    if (c == 1 || s1 >= std::max<int64_t>(r, 1)) {
      v.ptr = t.data_ptr();
      v.trans = 1;
      v.ld = c == 1 ? std::max<int64_t>(r, 1) : s1;
      return v;
    }
  }
  v.keep = contiguous_on_device(t);
  v.ptr = v.keep.data_ptr();
  v.trans = 0;
  v.ld = std::max<int64_t>(c, 1);
  return v;
}

void check_gemm_dtype(const at::Tensor& a, const at::Tensor& b, const char* what) {
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "spyre: ", what,
              ": operands must have the same dtype, got ", a.scalar_type(), " and ",
              b.scalar_type());
  TORCH_CHECK(a.scalar_type() == at::kHalf || a.scalar_type() == at::kBFloat16, "spyre: ", what,
              " runs on the fp16/bf16 MFMA units; got ", a.scalar_type());
}

// D = alpha * A @ B + beta * C for 2-D operands; C (optional) broadcast to
// D's shape.  D must be row-major-addressable; otherwise a contiguous result
// is computed and copied.
void gemm2d(const at::Tensor& a, const at::Tensor& b, const at::Tensor& d, float alpha,
            float beta, const at::Tensor& c) {
  const int64_t m = a.size(0), k = a.size(1), n = b.size(1);
  if (d.numel() == 0) return;
  const bool d_ok = d.stride(1) == 1 && (m == 1 || d.stride(0) >= n);
  at::Tensor dd = d_ok ? d : empty_spyre({m, n}, d.scalar_type(), d.device());
  MatView va = mat_view(a), vb = mat_view(b);
  const void* cp = nullptr;
  int64_t ldc_r = 0, ldc_c = 0;
  at::Tensor ce;
  if (c.defined() && beta != 0.f) {
    ce = c.expand({m, n});
    if (ce.scalar_type() != d.scalar_type()) ce = ce.to(d.scalar_type());
    cp = ce.data_ptr();
    ldc_r = ce.stride(0);
    ldc_c = ce.stride(1);
  }
  check_matrix_extent(va.keep.defined() ? va.keep : a, va.ptr, m, k, va.ld, va.trans, 1, 0,
                      "mm operand A");
  check_matrix_extent(vb.keep.defined() ? vb.keep : b, vb.ptr, k, n, vb.ld, vb.trans, 1, 0,
                      "mm operand B");
  check_matrix_extent(dd, dd.data_ptr(), m, n, m == 1 ? n : dd.stride(0), 0, 1, 0, "mm output");
  if (cp) {
    const int64_t cs[2] = {m, n}, cst[2] = {ldc_r, ldc_c};
    check_extent(ce, cp, 2, cs, cst, ce.element_size(), "addmm input");
  }
  c10::DeviceGuard guard(d.device());
  // workspace for a split-K last round of tiles, when the shape has one
  const int64_t nws = sph_gemm_workspace_bytes(1, m, n, k);
  at::Tensor ws = nws > 0 ? empty_spyre({nws}, at::kByte, d.device()) : at::Tensor();
  SPYRE_SPH_CHECK(sph_gemm_ex(to_sph(d.scalar_type()), va.trans, vb.trans, 1, m, n, k, alpha,
                              va.ptr, va.ld, 0, vb.ptr, vb.ld, 0, cp ? beta : 0.f, cp, ldc_r,
                              ldc_c, 0, dd.data_ptr(), m == 1 ? n : dd.stride(0), 0,
                              SPH_EPI_NONE, ws.defined() ? ws.data_ptr() : nullptr,
                              ws.defined() ? nws : 0, stream(d.get_device())));
  if (!d_ok) device_copy(d, dd);
}

// Batched form over dim 0; operands whose batch slices are not uniformly
// strided row/column-major matrices are made contiguous first.
void gemm3d(const at::Tensor& a_in, const at::Tensor& b_in, const at::Tensor& d, float alpha,
            float beta, const at::Tensor& c) {
  const int64_t bs = a_in.size(0), m = a_in.size(1), k = a_in.size(2), n = b_in.size(2);
  if (d.numel() == 0) return;
  auto norm = [](const at::Tensor& t, MatView& v, int64_t& bstride) -> at::Tensor {
    at::Tensor s = t;
    v = mat_view(t.select(0, 0));
    if (v.keep.defined()) {
      s = contiguous_on_device(t);
      v = mat_view(s.select(0, 0));
    }
    bstride = t.size(0) == 1 ? 0 : s.stride(0);
    return s;
  };
  MatView va, vb;
  int64_t sa = 0, sb = 0;
  at::Tensor a = norm(a_in, va, sa);
  at::Tensor b = norm(b_in, vb, sb);
  const bool d_ok = d.is_contiguous();
  at::Tensor dd = d_ok ? d : empty_spyre({bs, m, n}, d.scalar_type(), d.device());
  const void* cp = nullptr;
  int64_t ldc_r = 0, ldc_c = 0, sc = 0;
  at::Tensor ce;
  if (c.defined() && beta != 0.f) {
    ce = c.expand({bs, m, n});
    if (ce.scalar_type() != d.scalar_type()) ce = ce.to(d.scalar_type());
    cp = ce.data_ptr();
    sc = ce.stride(0);
    ldc_r = ce.stride(1);
    ldc_c = ce.stride(2);
  }
  check_matrix_extent(a, va.ptr, m, k, va.ld, va.trans, bs, sa, "bmm operand A");
  check_matrix_extent(b, vb.ptr, k, n, vb.ld, vb.trans, bs, sb, "bmm operand B");
  check_matrix_extent(dd, dd.data_ptr(), m, n, n, 0, bs, m * n, "bmm output");
  if (cp) {
    const int64_t cs[3] = {bs, m, n}, cst[3] = {sc, ldc_r, ldc_c};
    check_extent(ce, cp, 3, cs, cst, ce.element_size(), "baddbmm input");
  }
  c10::DeviceGuard guard(d.device());
  SPYRE_SPH_CHECK(sph_gemm_strided_batched(
      to_sph(d.scalar_type()), va.trans, vb.trans, bs, m, n, k, alpha, va.ptr, va.ld, sa, vb.ptr,
      vb.ld, sb, cp ? beta : 0.f, cp, ldc_r, ldc_c, sc, dd.data_ptr(), n, m * n, SPH_EPI_NONE,
      stream(d.get_device())));
  if (!d_ok) device_copy(d, dd);
}

at::Tensor& mm_out(const at::Tensor& self, const at::Tensor& mat2, at::Tensor& out) {
  TORCH_CHECK(self.dim() == 2 && mat2.dim() == 2, "spyre: mm expects 2-D operands");
  TORCH_CHECK(self.size(1) == mat2.size(0), "spyre: mm shapes cannot be multiplied (",
              self.size(0), "x", self.size(1), " and ", mat2.size(0), "x", mat2.size(1), ")");
  check_gemm_dtype(self, mat2, "mm");
  at::native::resize_output(out, {self.size(0), mat2.size(1)});
  gemm2d(self, mat2, out, 1.f, 0.f, at::Tensor());
  return out;
}

at::Tensor& bmm_out(const at::Tensor& self, const at::Tensor& mat2, at::Tensor& out) {
  TORCH_CHECK(self.dim() == 3 && mat2.dim() == 3, "spyre: bmm expects 3-D operands");
  TORCH_CHECK(self.size(0) == mat2.size(0) && self.size(2) == mat2.size(1),
              "spyre: bmm shapes cannot be multiplied");
  check_gemm_dtype(self, mat2, "bmm");
  at::native::resize_output(out, {self.size(0), self.size(1), mat2.size(2)});
  gemm3d(self, mat2, out, 1.f, 0.f, at::Tensor());
  return out;
}

at::Tensor& addmm_out(const at::Tensor& self, const at::Tensor& mat1, const at::Tensor& mat2,
                      const at::Scalar& beta, const at::Scalar& alpha, at::Tensor& out) {
  TORCH_CHECK(mat1.dim() == 2 && mat2.dim() == 2, "spyre: addmm expects 2-D matrices");
  TORCH_CHECK(mat1.size(1) == mat2.size(0), "spyre: addmm shapes cannot be multiplied");
  check_gemm_dtype(mat1, mat2, "addmm");
  at::native::resize_output(out, {mat1.size(0), mat2.size(1)});
  gemm2d(mat1, mat2, out, static_cast<float>(alpha.toDouble()),
         static_cast<float>(beta.toDouble()), self);
  return out;
}

at::Tensor& baddbmm_out(const at::Tensor& self, const at::Tensor& b1, const at::Tensor& b2,
                        const at::Scalar& beta, const at::Scalar& alpha, at::Tensor& out) {
  TORCH_CHECK(b1.dim() == 3 && b2.dim() == 3, "spyre: baddbmm expects 3-D operands");
  check_gemm_dtype(b1, b2, "baddbmm");
  at::native::resize_output(out, {b1.size(0), b1.size(1), b2.size(2)});
  gemm3d(b1, b2, out, static_cast<float>(alpha.toDouble()), static_cast<float>(beta.toDouble()),
         self);
  return out;
}

}  // namespace

// silu(x w[:n]^T) * (x w[n:]^T) for x [M, K], w [2n, K] on spyre: one fused
// GEMM (sph_gemm_swiglu) when the shape fits it, else the three device ops
// (mm, silu, mul) with the rounding the unfused program has.
at::Tensor gemm_swiglu(const at::Tensor& x_in, const at::Tensor& w_in) {
  TORCH_CHECK(is_spyre(x_in) && is_spyre(w_in), "spyre swiglu_mm: spyre tensors expected");
  TORCH_CHECK(x_in.dim() == 2 && w_in.dim() == 2 && x_in.size(1) == w_in.size(1) &&
                  w_in.size(0) % 2 == 0,
              "spyre swiglu_mm: x [M, K] and w [2n, K] expected");
  check_gemm_dtype(x_in, w_in, "swiglu_mm");
  const int64_t m = x_in.size(0), k = x_in.size(1), n = w_in.size(0) / 2;
  at::Tensor out = empty_spyre({m, n}, x_in.scalar_type(), x_in.device());
  if (out.numel() == 0) return out;
  at::Tensor x = x_in.stride(1) == 1 ? x_in : contiguous_on_device(x_in);
  at::Tensor w = w_in.stride(1) == 1 ? w_in : contiguous_on_device(w_in);
  c10::DeviceGuard guard(out.device());
  const bool fits = ((m % 256 == 0 && n % 128 == 0 && k % 64 == 0) ||
                     (m <= 8 && k >= 64 && k % 8 == 0 && k <= 8192)) && k > 0 &&
                    x.stride(0) % 8 == 0 && w.stride(0) % 8 == 0 &&
                    reinterpret_cast<uintptr_t>(x.data_ptr()) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(w.data_ptr()) % 16 == 0;
  if (fits) {
    check_matrix_extent(x, x.data_ptr(), m, k, x.stride(0), 0, 1, 0, "swiglu_mm x");
    check_matrix_extent(w, w.data_ptr(), 2 * n, k, w.stride(0), 0, 1, 0, "swiglu_mm w");
    const int64_t nws = sph_gemm_swiglu_workspace_bytes(m, n, k);
    at::Tensor ws = nws > 0 ? empty_spyre({nws}, at::kByte, out.device()) : at::Tensor();
    const int rc = sph_gemm_swiglu(to_sph(out.scalar_type()), m, n, k, x.data_ptr(), x.stride(0),
                                   w.data_ptr(), w.stride(0), out.data_ptr(), n,
                                   ws.defined() ? ws.data_ptr() : nullptr, ws.defined() ? nws : 0,
                                   stream(out.get_device()));
    if (rc == 0) return out;
    TORCH_CHECK(rc == SPH_ERR_UNSUPPORTED || rc == SPH_ERR_TOO_LARGE, "spyre: sph_gemm_swiglu failed (status ",
                rc, "): ", sph_last_error());
  }
  at::Tensor gu = at::mm(x, w.t());
  out.copy_(at::silu(gu.narrow(1, 0, n)) * gu.narrow(1, n, n));
  return out;
}

// rms_norm(x) w^T (swiglu: silu(gate) * up of the stacked [2n, K] weight)
// for decode rows (M <= 8) in one weight-stream launch (sph_gemm_rmsnorm);
// other shapes run the norm and the product as separate spyre ops.
at::Tensor gemm_rmsnorm(const at::Tensor& x_in, const at::Tensor& norm_w_in, double eps,
                        const at::Tensor& w_in, bool swiglu) {
  TORCH_CHECK(is_spyre(x_in) && is_spyre(norm_w_in) && is_spyre(w_in),
              "spyre rms_norm_mm: spyre tensors expected");
  TORCH_CHECK(x_in.dim() == 2 && w_in.dim() == 2 && norm_w_in.dim() == 1 &&
                  x_in.size(1) == w_in.size(1) && norm_w_in.size(0) == x_in.size(1) &&
                  (!swiglu || w_in.size(0) % 2 == 0),
              "spyre rms_norm_mm: x [M, K], norm_w [K] and w [N, K] (swiglu: [2n, K]) expected");
  check_gemm_dtype(x_in, w_in, "rms_norm_mm");
  TORCH_CHECK(norm_w_in.scalar_type() == x_in.scalar_type(),
              "spyre rms_norm_mm: norm weight dtype must match x");
  const int64_t m = x_in.size(0), k = x_in.size(1);
  const int64_t n = swiglu ? w_in.size(0) / 2 : w_in.size(0);
  at::Tensor out = empty_spyre({m, n}, x_in.scalar_type(), x_in.device());
  if (out.numel() == 0) return out;
  at::Tensor x = x_in.stride(1) == 1 ? x_in : contiguous_on_device(x_in);
  at::Tensor w = w_in.stride(1) == 1 ? w_in : contiguous_on_device(w_in);
  at::Tensor nw = contiguous_on_device(norm_w_in);
  auto al = [](const at::Tensor& t) {
    return reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
  };
  const bool fits = m <= 8 && k >= 64 && k % 8 == 0 && k <= 8192 && x.stride(0) % 8 == 0 &&
                    w.stride(0) % 8 == 0 && al(x) && al(w) && al(nw);
  c10::DeviceGuard guard(out.device());
  if (fits) {
    check_matrix_extent(x, x.data_ptr(), m, k, x.stride(0), 0, 1, 0, "rms_norm_mm x");
    check_matrix_extent(w, w.data_ptr(), swiglu ? 2 * n : n, k, w.stride(0), 0, 1, 0,
                        "rms_norm_mm w");
    SPYRE_SPH_CHECK(sph_gemm_rmsnorm(to_sph(out.scalar_type()), m, n, k, x.data_ptr(),
                                     x.stride(0), nw.data_ptr(), static_cast<float>(eps),
                                     w.data_ptr(), w.stride(0), out.data_ptr(), n, swiglu ? 1 : 0,
                                     stream(out.get_device())));
    return out;
  }
  at::Tensor xn = at::rms_norm(x, {k}, nw, eps);
  if (!swiglu) return at::mm(xn, w.t());
  return gemm_swiglu(xn, w);
}

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("mm.out", TORCH_FN(mm_out));
  m.impl("bmm.out", TORCH_FN(bmm_out));
  m.impl("addmm.out", TORCH_FN(addmm_out));
  m.impl("baddbmm.out", TORCH_FN(baddbmm_out));
}

}  // namespace spyre
