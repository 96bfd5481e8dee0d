/*
 * CPU restatement of the reference's stick-layout arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: this file is the checker the parity tests, the
 * smoke check and bench.py's cpu_baseline leg compare the HIP path against.
 * No product code links or calls it.
 *
 * Functions and the reference code they restate (torch-spyre tree):
 *   orc_stl_init        SpyreTensorLayout::init(host_size, dtype, dim_order)
 *                       torch_spyre/csrc/spyre_tensor_impl.cpp:40-74
 *   orc_alloc_nbytes    spyre_empty_strided sizing, spyre_mem.cpp:598-611 with
 *                       get_device_shape :99-126, stick count rounded UP
 *                       (the reference's padding branch keeps 1 stick for any
 *                       non-multiple size; orc_alloc_nbytes_reference keeps
 *                       that rule so the deviation is visible in tests)
 *   orc_stick_pack /    the permutation the DMA stick conversion performs,
 *   orc_stick_unpack    spyre_mem.cpp:190-244, in SpyreTensorLayout's generic
 *                       stick order (device dims [ceil(S/E), dims in
 *                       dim_order[:-1], E]), padding zeroed.
 */
#include <stdint.h>
#include <string.h>

#define ORC_STICK_BYTES 128
#define ORC_MAX_DIMS 8

/* device_size / device_strides / dim_map each get ndim + 1 entries. */
int orc_stl_init(int ndim, const int64_t* host_size, int elem_bytes, const int32_t* dim_order,
                 int64_t* device_size, int64_t* device_strides, int32_t* dim_map) {
  if (ndim < 1 || ndim > ORC_MAX_DIMS || elem_bytes <= 0) return -1;
  const int dev = ndim + 1;
  const int64_t e = ORC_STICK_BYTES / elem_bytes;
  const int32_t stick_dim = dim_order[ndim - 1];
  dim_map[0] = stick_dim;
  dim_map[dev - 1] = stick_dim;
  device_size[0] = (host_size[stick_dim] + e - 1) / e;
  device_size[dev - 1] = e;
  for (int i = 1; i < dev - 1; ++i) {
    dim_map[i] = dim_order[i - 1];
    device_size[i] = host_size[dim_order[i - 1]];
  }
  int64_t stride = 1;
  for (int i = dev - 1; i >= 0; --i) {
    device_strides[i] = stride;
    stride *= device_size[i];
  }
  return 0;
}

/* Bytes of device memory for a row-major host tensor: 128 bytes per stick,
 * stick dim = last dim, 0-d tensors take one stick. */
int64_t orc_alloc_nbytes(int ndim, const int64_t* host_size, int elem_bytes) {
  const int64_t e = ORC_STICK_BYTES / elem_bytes;
  if (ndim == 0) return ORC_STICK_BYTES;
  int64_t sticks = (host_size[ndim - 1] + e - 1) / e;
  for (int i = 0; i < ndim - 1; ++i) sticks *= host_size[i];
  return sticks * ORC_STICK_BYTES;
}

/* The reference's rule as written: a stick dim that is not a multiple of the
 * stick size gets exactly one stick, whatever its length. */
int64_t orc_alloc_nbytes_reference(int ndim, const int64_t* host_size, int elem_bytes) {
  const int64_t e = ORC_STICK_BYTES / elem_bytes;
  if (ndim == 0) return ORC_STICK_BYTES;
  const int64_t s = host_size[ndim - 1];
  int64_t sticks = (s % e != 0) ? 1 : s / e;
  for (int i = 0; i < ndim - 1; ++i) sticks *= host_size[i];
  return sticks * ORC_STICK_BYTES;
}

/* Host element offset (in elements) of device element `lin`, -1 = padding. */
static int64_t host_offset(int ndim, const int64_t* host_size, const int64_t* host_strides,
                           const int32_t* dim_order, int64_t e, int64_t lin) {
  int64_t rem = lin;
  const int64_t ei = rem % e;
  rem /= e;
  int64_t off = 0;
  for (int j = ndim - 2; j >= 0; --j) {
    const int64_t sz = host_size[dim_order[j]];
    const int64_t c = rem % sz;
    rem /= sz;
    off += c * host_strides[dim_order[j]];
  }
  const int32_t sd = dim_order[ndim - 1];
  const int64_t si = rem * e + ei;
  if (si >= host_size[sd]) return -1;
  return off + si * host_strides[sd];
}

static int64_t device_elems(int ndim, const int64_t* host_size, const int32_t* dim_order,
                            int64_t e) {
  int64_t n = (host_size[dim_order[ndim - 1]] + e - 1) / e * e;
  for (int j = 0; j < ndim - 1; ++j) n *= host_size[dim_order[j]];
  return n;
}

int orc_stick_pack(const void* src, void* dst, int ndim, const int64_t* host_size,
                   const int64_t* host_strides, const int32_t* dim_order, int elem_bytes) {
  if (ndim < 1 || ndim > ORC_MAX_DIMS) return -1;
  const int64_t e = ORC_STICK_BYTES / elem_bytes;
  const int64_t n = device_elems(ndim, host_size, dim_order, e);
  const uint8_t* s = (const uint8_t*)src;
  uint8_t* d = (uint8_t*)dst;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t h = host_offset(ndim, host_size, host_strides, dim_order, e, i);
    if (h < 0)
      memset(d + i * elem_bytes, 0, (size_t)elem_bytes);
    else
      memcpy(d + i * elem_bytes, s + h * elem_bytes, (size_t)elem_bytes);
  }
  return 0;
}

int orc_stick_unpack(const void* src, void* dst, int ndim, const int64_t* host_size,
                     const int64_t* host_strides, const int32_t* dim_order, int elem_bytes) {
  if (ndim < 1 || ndim > ORC_MAX_DIMS) return -1;
  const int64_t e = ORC_STICK_BYTES / elem_bytes;
  const int64_t n = device_elems(ndim, host_size, dim_order, e);
  const uint8_t* s = (const uint8_t*)src;
  uint8_t* d = (uint8_t*)dst;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t h = host_offset(ndim, host_size, host_strides, dim_order, e, i);
    if (h >= 0) memcpy(d + h * elem_bytes, s + i * elem_bytes, (size_t)elem_bytes);
  }
  return 0;
}
