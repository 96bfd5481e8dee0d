#include "spyre_layout.h"

#include <c10/util/Exception.h>

#include <numeric>
#include <sstream>

namespace spyre {

namespace {
constexpr int64_t kStickBytes = 128;

template <typename T>
void join(std::ostringstream& os, const std::vector<T>& v) {
  for (size_t i = 0; i < v.size(); ++i) os << (i ? ", " : "") << v[i];
}
}  // namespace

int64_t SpyreTensorLayout::elems_per_stick(c10::ScalarType dtype) {
  return kStickBytes / static_cast<int64_t>(c10::elementSize(dtype));
}

SpyreTensorLayout::SpyreTensorLayout(std::vector<int64_t> host_size, c10::ScalarType dtype) {
  std::vector<int32_t> order(host_size.size());
  std::iota(order.begin(), order.end(), 0);
  init(host_size, dtype, order, Dense);
}

SpyreTensorLayout::SpyreTensorLayout(std::vector<int64_t> host_size, c10::ScalarType dtype,
                                     std::vector<int32_t> dim_order, StickFormat fmt) {
  init(host_size, dtype, dim_order, fmt);
}

SpyreTensorLayout::SpyreTensorLayout(std::vector<int64_t> dsize, std::vector<int64_t> dstrides,
                                     std::vector<int32_t> dmap, int32_t nstick, StickFormat fmt)
    : device_size(std::move(dsize)),
      device_strides(std::move(dstrides)),
      dim_map(std::move(dmap)),
      num_stick_dims(nstick),
      format(fmt) {}

void SpyreTensorLayout::init(const std::vector<int64_t>& host_size, c10::ScalarType dtype,
                             const std::vector<int32_t>& dim_order, StickFormat fmt) {
  const int n = static_cast<int>(host_size.size());
  TORCH_CHECK(n >= 1, "SpyreTensorLayout: needs at least one host dimension");
  TORCH_CHECK(static_cast<int>(dim_order.size()) == n,
              "SpyreTensorLayout: dim_order must name every host dimension");
  std::vector<bool> seen(n, false);
  for (int32_t d : dim_order) {
    TORCH_CHECK(d >= 0 && d < n && !seen[d], "SpyreTensorLayout: dim_order must be a permutation");
    seen[d] = true;
  }
  const int64_t e = elems_per_stick(dtype);
  const int nd = n + 1;
  const int32_t stick = dim_order[n - 1];
  device_size.assign(nd, 0);
  device_strides.assign(nd, 0);
  dim_map.assign(nd, 0);
  format = fmt;
  num_stick_dims = 1;
  // outermost: number of sticks along the stick dim; innermost: the stick
  dim_map[0] = stick;
  device_size[0] = (host_size[stick] + e - 1) / e;
  dim_map[nd - 1] = stick;
  device_size[nd - 1] = e;
  for (int i = 1; i < nd - 1; ++i) {
    dim_map[i] = dim_order[i - 1];
    device_size[i] = host_size[dim_order[i - 1]];
  }
  int64_t s = 1;
  for (int i = nd - 1; i >= 0; --i) {
    device_strides[i] = s;
    s *= device_size[i];
  }
}

int64_t SpyreTensorLayout::nbytes(c10::ScalarType dtype) const {
  if (device_size.empty()) return 0;
  return device_size[0] * device_strides[0] * static_cast<int64_t>(c10::elementSize(dtype));
}

std::string SpyreTensorLayout::toString() const {
  std::ostringstream os;
  os << "SpyreTensorLayout(device_size=[";
  join(os, device_size);
  os << "], device_strides=[";
  join(os, device_strides);
  os << "], dim_map =[";
  join(os, dim_map);
  os << "], num_stick_dims=" << num_stick_dims << ", format=\""
     << (format == Dense ? "Dense" : format == Sparse ? "Sparse" : "SparseMulti") << "\")";
  return os.str();
}

}  // namespace spyre
