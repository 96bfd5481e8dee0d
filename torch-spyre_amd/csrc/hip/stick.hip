// Stick (tiled) layout conversion on the GPU: a bit-exact permutation between
// a strided host-order tensor and SpyreTensorLayout's generic stick format.
//
// Device dims (ndim + 1 of them), row-major:
//   [ceil(S / E), size[dim_order[0]], ..., size[dim_order[ndim-2]], E]
// where S = size[dim_order[ndim-1]] is the stick dim and E = 128 / elem_bytes.
// Device element (s, i_0, ..., i_{ndim-2}, e) is host element with
// stick-dim index s*E + e and dim dim_order[j] index i_j; padding elements
// (s*E + e >= S) are zero.  One thread moves one element; each 128-byte
// stick is written (pack) or read (unpack) by 128/elem_bytes consecutive
// threads, so the device side is fully coalesced.
#include "sph_common.h"

namespace sph {
namespace {

struct StickArgs {
  int ndim;                          // host dims
  int64_t dev_size[SPH_MAX_DIMS + 1];
  int64_t host_stride_of_dev[SPH_MAX_DIMS + 1];  // host stride for device dims 1..ndim-1
  int64_t stick_host_stride;
  int64_t stick_size;                // S
  int64_t elems_per_stick;           // E
  int64_t total;                     // prod(dev_size)
};

int build_args(int ndim, const int64_t* host_sizes, const int64_t* host_strides,
               const int32_t* dim_order, int elem_bytes, StickArgs& a) {
  SPH_REQUIRE(ndim >= 1 && ndim <= SPH_MAX_DIMS, SPH_ERR_INVALID_ARG, "stick: ndim must be 1..8");
  SPH_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
              SPH_ERR_INVALID_ARG, "stick: elem_bytes must be 1, 2, 4 or 8");
  unsigned seen = 0;
  for (int i = 0; i < ndim; ++i) {
    SPH_REQUIRE(dim_order[i] >= 0 && dim_order[i] < ndim && !(seen & (1u << dim_order[i])),
                SPH_ERR_INVALID_ARG, "stick: dim_order is not a permutation");
    seen |= 1u << dim_order[i];
    SPH_REQUIRE(host_sizes[i] >= 0, SPH_ERR_INVALID_ARG, "stick: negative size");
  }
  a.ndim = ndim;
  a.elems_per_stick = 128 / elem_bytes;
  const int sd = dim_order[ndim - 1];
  a.stick_size = host_sizes[sd];
  a.stick_host_stride = host_strides ? host_strides[sd] : 0;
  a.dev_size[0] = ceil_div(a.stick_size, a.elems_per_stick);
  for (int j = 0; j < ndim - 1; ++j) {
    a.dev_size[j + 1] = host_sizes[dim_order[j]];
    a.host_stride_of_dev[j + 1] = host_strides ? host_strides[dim_order[j]] : 0;
  }
  a.dev_size[ndim] = a.elems_per_stick;
  a.total = 1;
  for (int j = 0; j <= ndim; ++j) a.total *= a.dev_size[j];
  return SPH_OK;
}

// Host offset of device element `lin`, or -1 for a padding element.
__device__ inline int64_t host_off(const StickArgs& a, int64_t lin) {
  int64_t rem = lin;
  const int64_t e = rem % a.elems_per_stick;
  rem /= a.elems_per_stick;
  int64_t off = 0;
  for (int j = a.ndim - 1; j >= 1; --j) {
    const int64_t c = rem % a.dev_size[j];
    rem /= a.dev_size[j];
    off += c * a.host_stride_of_dev[j];
  }
  const int64_t s = rem;  // stick index
  const int64_t si = s * a.elems_per_stick + e;
  if (si >= a.stick_size) return -1;
  return off + si * a.stick_host_stride;
}

template <typename V>
__global__ void __launch_bounds__(256) stick_pack_kernel(const V* __restrict__ src,
                                                         V* __restrict__ dst, const StickArgs a) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < a.total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t h = host_off(a, i);
    dst[i] = (h >= 0) ? src[h] : V{};
  }
}

template <typename V>
__global__ void __launch_bounds__(256) stick_unpack_kernel(const V* __restrict__ src,
                                                           V* __restrict__ dst, const StickArgs a) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < a.total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t h = host_off(a, i);
    if (h >= 0) dst[h] = src[i];
  }
}

template <bool PACK>
int run(const void* src, void* dst, const StickArgs& a, int elem_bytes, hipStream_t st) {
  if (a.total == 0) return SPH_OK;
  int64_t g = (a.total + 255) / 256;
  if (g > 65536) g = 65536;
  const unsigned grid = static_cast<unsigned>(g);
#define SPH_STICK_RUN(V)                                                                    \
  if (PACK)                                                                                 \
    stick_pack_kernel<V><<<grid, 256, 0, st>>>(static_cast<const V*>(src), static_cast<V*>(dst), a); \
  else                                                                                      \
    stick_unpack_kernel<V><<<grid, 256, 0, st>>>(static_cast<const V*>(src), static_cast<V*>(dst), a);
  switch (elem_bytes) {
    case 1: SPH_STICK_RUN(uint8_t) break;
    case 2: SPH_STICK_RUN(uint16_t) break;
    case 4: SPH_STICK_RUN(uint32_t) break;
    default: SPH_STICK_RUN(uint64_t) break;
  }
#undef SPH_STICK_RUN
  return check_launch(PACK ? "sph_stick_pack" : "sph_stick_unpack");
}

}  // namespace
}  // namespace sph

using namespace sph;

extern "C" int64_t sph_stick_nbytes(int ndim, const int64_t* host_sizes, const int32_t* dim_order,
                                    int elem_bytes) {
  StickArgs a{};
  if (build_args(ndim, host_sizes, nullptr, dim_order, elem_bytes, a) != SPH_OK) return -1;
  return a.total * elem_bytes;
}

extern "C" int sph_stick_pack(const void* src, void* dst, int ndim, const int64_t* host_sizes,
                              const int64_t* host_strides, const int32_t* dim_order,
                              int elem_bytes, sph_stream_t stream) {
  StickArgs a{};
  if (int e = build_args(ndim, host_sizes, host_strides, dim_order, elem_bytes, a)) return e;
  return run<true>(src, dst, a, elem_bytes, as_stream(stream));
}

extern "C" int sph_stick_unpack(const void* src, void* dst, int ndim, const int64_t* host_sizes,
                                const int64_t* host_strides, const int32_t* dim_order,
                                int elem_bytes, sph_stream_t stream) {
  StickArgs a{};
  if (int e = build_args(ndim, host_sizes, host_strides, dim_order, elem_bytes, a)) return e;
  return run<false>(src, dst, a, elem_bytes, as_stream(stream));
}
