// Helpers shared by the eager ATen kernels of the spyre backend: launching
// the kernel library's strided pointwise engine over a TensorIterator, and
// small argument utilities.
#pragma once

#include <ATen/ATen.h>
#include <ATen/TensorIterator.h>

#include "spyre_runtime.h"

namespace spyre {

inline bool is_spyre(const at::Tensor& t) { return t.device().is_privateuseone(); }

// Runs sph_pointwise(op) over a built TensorIterator (outputs first, then
// inputs), on the stream of the iterator's device.  Dims are passed
// outermost-first; operands of dtypes the kernels do not know are accepted
// for COPY when every operand has that dtype (bits moved as integers of the
// same width).
void launch_iter(int op, const at::TensorIteratorBase& iter, double alpha = 0.0,
                 double beta = 0.0);

// dst = src (broadcast to dst's shape, dtype converted), both on the same
// spyre device.
void device_copy(const at::Tensor& dst, const at::Tensor& src);

// A contiguous spyre tensor with the data of `t` (t itself if contiguous).
at::Tensor contiguous_on_device(const at::Tensor& t);

// Value of a 0-d CPU tensor (a wrapped Python number) as a double.
inline bool is_cpu_scalar(const at::Tensor& t) { return t.dim() == 0 && t.device().is_cpu(); }

// Host-side guard run before every launch: the bytes a kernel addresses
// through (ptr, sizes, element strides) must lie inside `t`'s storage.
// Throws instead of letting a wrong stride reach the GPU.
void check_extent(const at::Tensor& t, const void* ptr, int ndim, const int64_t* sizes,
                  const int64_t* strides, int64_t elem_bytes, const char* what);

// Same for a row-major / transposed matrix of `rows` x `cols` with leading
// dim `ld` (trans: element (i, j) at i + j*ld).
void check_matrix_extent(const at::Tensor& t, const void* ptr, int64_t rows, int64_t cols,
                         int64_t ld, int trans, int64_t batch, int64_t batch_stride,
                         const char* what);

// Allocates an uninitialised spyre tensor (contiguous).
at::Tensor empty_spyre(at::IntArrayRef sizes, at::ScalarType dtype, c10::Device device);

}  // namespace spyre
