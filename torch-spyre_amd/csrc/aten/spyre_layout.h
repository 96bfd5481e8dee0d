// SpyreTensorLayout: the generic stick (tiled) layout descriptor.
//
// Same class, constructors, fields and string form as the reference
// (torch_spyre/csrc/spyre_tensor_impl.h:29-93, spyre_tensor_impl.cpp:29-111,
// pybind in torch_spyre/csrc/module.cpp:180-203), because user code and the
// reference's tests (tests/tensor/test_tensor_layout.py) read these fields.
//
// The layout: a 128-byte "stick" holds E = 128 / elem_bytes consecutive
// elements of the stick dimension (the last entry of dim_order).  The device
// tensor has dims [ceil(S / E), the other host dims in dim_order order, E],
// row-major; dim_map names the host dim behind each device dim, so the stick
// dim appears twice (outermost and innermost).  With the stick dim = K this
// is the K-panel layout of a GEMM operand: the [rows x E] slice of one K
// panel is a contiguous block, fed by whole-stick (128-byte) loads.
#pragma once

#include <c10/core/ScalarType.h>

#include <cstdint>
#include <string>
#include <vector>

namespace spyre {

class SpyreTensorLayout {
 public:
  enum StickFormat { Dense = 0, Sparse, SparseMulti };

  std::vector<int64_t> device_size;
  std::vector<int64_t> device_strides;
  std::vector<int32_t> dim_map;
  int32_t num_stick_dims = 1;
  StickFormat format = Dense;

  // Generic stick layout: dim_order = [0, 1, ..., n-1].
  SpyreTensorLayout(std::vector<int64_t> host_size, c10::ScalarType dtype);
  // dim_order lists the host dims in decreasing-stride order; its last entry
  // is the stick dim.
  SpyreTensorLayout(std::vector<int64_t> host_size, c10::ScalarType dtype,
                    std::vector<int32_t> dim_order, StickFormat format = Dense);
  // Explicit fields.
  SpyreTensorLayout(std::vector<int64_t> device_size, std::vector<int64_t> device_strides,
                    std::vector<int32_t> dim_map, int32_t num_stick_dims, StickFormat format);

  // Elements per stick for a dtype.
  static int64_t elems_per_stick(c10::ScalarType dtype);
  // Bytes of the device tensor (= device_size[0] * device_strides[0] * elem).
  int64_t nbytes(c10::ScalarType dtype) const;

  std::string toString() const;

 private:
  void init(const std::vector<int64_t>& host_size, c10::ScalarType dtype,
            const std::vector<int32_t>& dim_order, StickFormat format);
};

}  // namespace spyre
