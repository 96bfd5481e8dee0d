// Tensor creation, metadata and copy kernels of the spyre backend.
//
// Reference: torch_spyre/csrc/spyre_mem.cpp:557-711 (empty, empty_strided,
// as_strided, set_, _copy_from) and codegen/inputs/spyre_torch_ops.cpp
// (view :52-55, _local_scalar_dense :58-68, fill_ :394-403).
//
// Device tensors are plain strided tensors whose storage is MI355X HBM, so
// every PyTorch view (transposes included) works; their storage is sized
// with the reference's 128-byte stick rule.  Host<->device copies move the
// bytes on the device's spyre stream (spyre_copy.cpp); any dtype
// conversion, broadcast or stride change happens either on the host side of
// the copy (torch's own CPU copy) or on the device in the strided copy
// kernel, so copies are bit-exact.  Differences from the reference, on
// purpose: 0-d tensors stay 0-d; device-to-device copies move data (the
// reference copies host-side handles); dtype changes are allowed in copies.
#include <ATen/EmptyTensor.h>
#include <ATen/native/Resize.h>
#include <ATen/ops/_reshape_alias_native.h>
#include <ATen/ops/as_strided_native.h>
#include <ATen/ops/view_native.h>
#include <c10/core/TensorImpl.h>
#include <torch/library.h>

#include <cstring>

#include "spyre_ops_common.h"

namespace spyre {

namespace {

constexpr c10::DispatchKeySet kSpyreKeys(c10::DispatchKey::PrivateUse1);

c10::Device resolve_device(std::optional<c10::Device> d) {
  start_runtime();
  if (!d.has_value()) return c10::Device(c10::DeviceType::PrivateUse1, current_device());
  TORCH_CHECK(d->is_privateuseone(), "spyre: expected a spyre device, got ", *d);
  if (!d->has_index())
    return c10::Device(c10::DeviceType::PrivateUse1, current_device());
  return *d;
}

// Storage of a new tensor: the reference's stick-granular size, or the bytes
// the strides address if those are more (non-contiguous empty_strided).
at::Tensor make_tensor(at::IntArrayRef size, at::IntArrayRef stride, at::ScalarType dtype,
                       c10::Device device) {
  at::detail::check_size_nonnegative(size);
  const int64_t isz = static_cast<int64_t>(c10::elementSize(dtype));
  int64_t nbytes = stick_alloc_nbytes(size, isz);
  const int64_t need =
      static_cast<int64_t>(at::detail::computeStorageNbytes(size, stride, isz));
  if (need > nbytes) nbytes = need;
  c10::DeviceGuard guard(device);
  c10::Allocator* alloc = device_allocator();
  auto storage = c10::make_intrusive<c10::StorageImpl>(c10::StorageImpl::use_byte_size_t(),
                                                       nbytes, alloc->allocate(nbytes), alloc,
                                                       /*resizable=*/true);
  auto t = at::detail::make_tensor<c10::TensorImpl>(c10::Storage(std::move(storage)), kSpyreKeys,
                                                   c10::scalarTypeToTypeMeta(dtype));
  t.unsafeGetTensorImpl()->set_sizes_and_strides(size, stride);
  return t;
}

}  // namespace

at::Tensor empty_spyre(at::IntArrayRef sizes, at::ScalarType dtype, c10::Device device) {
  return make_tensor(sizes, c10::contiguous_strides(sizes), dtype, device);
}

at::Tensor spyre_empty_strided(c10::IntArrayRef size, c10::IntArrayRef stride,
                               std::optional<c10::ScalarType> dtype_opt,
                               std::optional<c10::Layout> layout_opt,
                               std::optional<c10::Device> device_opt,
                               std::optional<bool> pin_memory_opt) {
  TORCH_CHECK(c10::layout_or_default(layout_opt) == c10::Layout::Strided,
              "spyre: only strided tensors are supported");
  TORCH_CHECK(!c10::pinned_memory_or_default(pin_memory_opt),
              "spyre: pinned memory is a property of CPU tensors");
  return make_tensor(size, stride, c10::dtype_or_default(dtype_opt), resolve_device(device_opt));
}

at::Tensor spyre_empty(c10::IntArrayRef size, std::optional<c10::ScalarType> dtype_opt,
                       std::optional<c10::Layout> layout_opt,
                       std::optional<c10::Device> device_opt, std::optional<bool> pin_memory_opt,
                       std::optional<c10::MemoryFormat> memory_format_opt) {
  auto t = spyre_empty_strided(size, c10::contiguous_strides(size), dtype_opt, layout_opt,
                               device_opt, pin_memory_opt);
  const auto mf = memory_format_opt.value_or(c10::MemoryFormat::Contiguous);
  if (mf != c10::MemoryFormat::Contiguous && mf != c10::MemoryFormat::Preserve)
    t.unsafeGetTensorImpl()->empty_tensor_restride(mf);
  return t;
}

at::Tensor spyre_as_strided(const at::Tensor& self, c10::IntArrayRef size,
                            c10::IntArrayRef stride, std::optional<int64_t> storage_offset) {
  return at::native::as_strided_tensorimpl(self, size, stride, storage_offset);
}

at::Tensor spyre_view(const at::Tensor& self, c10::IntArrayRef size) {
  return at::native::view(self, size);
}

at::Tensor spyre_reshape_alias(const at::Tensor& self, c10::IntArrayRef size,
                               c10::IntArrayRef stride) {
  return at::native::_reshape_alias(self, size, stride);
}

at::Tensor& spyre_set_storage(at::Tensor& result, c10::Storage storage, int64_t storage_offset,
                              c10::IntArrayRef size, c10::IntArrayRef stride) {
  at::native::checkSetStorage(result, storage, storage_offset, size, stride);
  result.unsafeGetTensorImpl()->set_storage_offset(storage_offset);
  at::OptionalIntArrayRef st =
      stride.data() != nullptr ? at::OptionalIntArrayRef(stride) : std::nullopt;
  at::native::resize_impl_cpu_(result.unsafeGetTensorImpl(), size, st,
                               /*resize_storage=*/false);
  return result;
}

at::Tensor& spyre_set_storage_only(at::Tensor& result, c10::Storage storage) {
  const int64_t isz = static_cast<int64_t>(result.element_size());
  const int64_t n = static_cast<int64_t>(storage.nbytes()) / isz;
  return spyre_set_storage(result, std::move(storage), 0, {n}, {});
}

const at::Tensor& spyre_resize_(const at::Tensor& self, c10::IntArrayRef size,
                                std::optional<c10::MemoryFormat> memory_format) {
  auto* impl = self.unsafeGetTensorImpl();
  impl->set_sizes_contiguous(size);
  const int64_t isz = static_cast<int64_t>(self.element_size());
  const size_t need = static_cast<size_t>((self.storage_offset() + self.numel()) * isz);
  const c10::Storage& st = impl->unsafe_storage();
  if (need > st.nbytes()) {
    c10::StorageImpl* s = st.unsafeGetStorageImpl();
    TORCH_CHECK(s->resizable(), "spyre: trying to resize a storage that is not resizable");
    c10::DeviceGuard guard(self.device());
    at::DataPtr fresh = device_allocator()->allocate(need);
    if (st.nbytes() > 0 && s->data())
      SPYRE_HIP_CHECK(hipMemcpyAsync(fresh.get(), s->data(), st.nbytes(),
                                     hipMemcpyDeviceToDevice, stream(self.get_device())));
    s->set_data_ptr_noswap(std::move(fresh));
    s->set_nbytes(need);
  }
  if (memory_format.has_value() && *memory_format != c10::MemoryFormat::Preserve)
    impl->empty_tensor_restride(*memory_format);
  return self;
}

// ---------------------------------------------------------------------------
// Copies
// ---------------------------------------------------------------------------
namespace {

// A CPU tensor whose bytes are exactly the image of `like` (same dtype,
// sizes and strides, dense): `t` itself when it already is one.
bool same_image(const at::Tensor& t, const at::Tensor& like) {
  return t.scalar_type() == like.scalar_type() && t.sizes().equals(like.sizes()) &&
         t.strides().equals(like.strides()) && t.is_non_overlapping_and_dense();
}

// dst (spyre) = src (CPU), any shapes broadcastable, any dtypes.
void copy_h2d(const at::Tensor& src, const at::Tensor& dst, bool non_blocking) {
  c10::DeviceGuard guard(dst.device());
  const int dev = dst.get_device();
  const bool dense = dst.is_non_overlapping_and_dense();
  const size_t nbytes = static_cast<size_t>(dst.numel()) * dst.element_size();
  // Host image of dst's values in dst's dtype (the source itself when its
  // bytes already are that image); dense, so it moves as one byte stream.
  at::Tensor host;
  if (dense && same_image(src, dst)) {
    host = src;
  } else {
    host = dense ? at::empty_strided(dst.sizes(), dst.strides(), dst.options().device(at::kCPU))
                 : at::empty(dst.sizes(), dst.options().device(at::kCPU));
    host.copy_(src);
  }
  if (dense) {
    h2d_bytes(dev, dst.data_ptr(), host, nbytes, non_blocking);
    return;
  }
  at::Tensor staging = empty_spyre(dst.sizes(), dst.scalar_type(), dst.device());
  h2d_bytes(dev, staging.data_ptr(), host, nbytes, non_blocking && host.is_same(src));
  device_copy(dst, staging);
}

// dst (CPU) = src (spyre).
void copy_d2h(const at::Tensor& src, const at::Tensor& dst, bool non_blocking) {
  c10::DeviceGuard guard(src.device());
  const int dev = src.get_device();
  at::Tensor dsrc = src.is_non_overlapping_and_dense() ? src : contiguous_on_device(src);
  const size_t nbytes = static_cast<size_t>(dsrc.numel()) * dsrc.element_size();
  if (same_image(dst, dsrc)) {
    d2h_bytes(dev, dst, dsrc.data_ptr(), nbytes, non_blocking);
    return;
  }
  at::Tensor host = at::empty_strided(dsrc.sizes(), dsrc.strides(),
                                      dsrc.options().device(at::kCPU));
  d2h_bytes(dev, host, dsrc.data_ptr(), nbytes, false);
  dst.copy_(host);
}

void copy_d2d(const at::Tensor& src, const at::Tensor& dst) {
  if (src.get_device() != dst.get_device()) {
    // Peer copy through a dense image of the source.
    at::Tensor dsrc = contiguous_on_device(src);
    at::Tensor img = empty_spyre(dsrc.sizes(), dsrc.scalar_type(), dst.device());
    const size_t nbytes = static_cast<size_t>(dsrc.numel()) * dsrc.element_size();
    synchronize(src.get_device());
    SPYRE_HIP_CHECK(hipMemcpyPeerAsync(img.data_ptr(), dst.get_device(), dsrc.data_ptr(),
                                       src.get_device(), nbytes, stream(dst.get_device())));
    c10::DeviceGuard guard(dst.device());
    device_copy(dst, img);
    return;
  }
  c10::DeviceGuard guard(dst.device());
  const bool same_layout = src.scalar_type() == dst.scalar_type() &&
                           src.sizes().equals(dst.sizes()) &&
                           src.strides().equals(dst.strides()) &&
                           dst.is_non_overlapping_and_dense();
  if (same_layout) {
    if (src.data_ptr() == dst.data_ptr()) return;
    const size_t nbytes = static_cast<size_t>(dst.numel()) * dst.element_size();
    SPYRE_HIP_CHECK(hipMemcpyAsync(dst.data_ptr(), src.data_ptr(), nbytes,
                                   hipMemcpyDeviceToDevice, stream(dst.get_device())));
    return;
  }
  if ((has_sph(src.scalar_type()) && has_sph(dst.scalar_type())) ||
      src.scalar_type() == dst.scalar_type()) {
    device_copy(dst, src);
    return;
  }
  // dtype pair the kernels cannot convert (e.g. float8): convert on the host.
  at::Tensor host = src.to(at::kCPU).to(dst.scalar_type());
  copy_h2d(host, dst, false);
}

}  // namespace

// non_blocking: a copy between a spyre tensor and pinned host memory
// returns without waiting for the DMA (synchronise before touching the host
// side); copies with pageable memory behave as if blocking, except that a
// host-to-device copy returns once its data is staged.
at::Tensor spyre_copy_from(const at::Tensor& self, const at::Tensor& dst, bool non_blocking) {
  if (dst.numel() == 0) return dst;
  if (self.is_cpu() && is_spyre(dst)) {
    copy_h2d(self, dst, non_blocking);
  } else if (is_spyre(self) && dst.is_cpu()) {
    copy_d2h(self, dst, non_blocking);
  } else if (is_spyre(self) && is_spyre(dst)) {
    copy_d2d(self, dst);
  } else {
    TORCH_CHECK(false, "spyre: copy between ", self.device(), " and ", dst.device(),
                " is not supported");
  }
  return dst;
}

at::Tensor spyre_copy_from_and_resize(const at::Tensor& self, const at::Tensor& dst) {
  spyre_resize_(dst, self.sizes(), std::nullopt);
  return spyre_copy_from(self, dst, false);
}

// .item(): one element to the host (reference: spyre___local_scalar_dense,
// codegen/inputs/spyre_torch_ops.cpp:58-68, which rejects device tensors).
c10::Scalar spyre_local_scalar_dense(const at::Tensor& self) {
  TORCH_CHECK(self.numel() == 1, "spyre: a Tensor with ", self.numel(),
              " elements cannot be converted to Scalar");
  c10::DeviceGuard guard(self.device());
  at::Tensor host = at::empty({}, self.options().device(at::kCPU));
  hipStream_t s = stream(self.get_device());
  SPYRE_HIP_CHECK(hipMemcpyAsync(host.data_ptr(), self.data_ptr(), self.element_size(),
                                 hipMemcpyDeviceToHost, s));
  SPYRE_HIP_CHECK(hipStreamSynchronize(s));
  check_device_errors(self.get_device());
  return host.item();
}

// fill_: the value is converted to the tensor's dtype by torch on the host
// (so rounding is torch's own), then its bit pattern is broadcast on the
// device (reference: spyre__fill_Scalar fills on the CPU and copies,
// codegen/inputs/spyre_torch_ops.cpp:394-403).
at::Tensor& spyre_fill_(at::Tensor& self, const c10::Scalar& value) {
  if (self.numel() == 0) return self;
  c10::DeviceGuard guard(self.device());
  at::Tensor v = at::scalar_tensor(value, self.options().device(at::kCPU));
  const int64_t isz = self.element_size();
  double bits = 0.0;
  sph_dtype as = SPH_I64;
  if (isz == 8) {
    // 8-byte types: the value itself (exact for float64; int64 exact below 2^53)
    as = self.scalar_type() == at::kDouble ? SPH_F64 : SPH_I64;
    TORCH_CHECK(as == SPH_F64 || self.scalar_type() == at::kLong,
                "spyre: fill_ of dtype ", self.scalar_type(), " is not supported");
    bits = as == SPH_F64 ? v.item<double>() : static_cast<double>(v.item<int64_t>());
  } else {
    uint32_t u = 0;
    std::memcpy(&u, v.data_ptr(), isz);
    bits = static_cast<double>(u);
    as = isz == 1 ? SPH_U8 : isz == 2 ? SPH_I16 : SPH_I32;
    if (isz == 2) bits = static_cast<double>(static_cast<int16_t>(u));
    if (isz == 4) bits = static_cast<double>(static_cast<int32_t>(u));
  }
  sph_operand out{};
  out.data = self.data_ptr();
  out.dtype = as;
  const int nd = static_cast<int>(self.dim());
  TORCH_CHECK(nd <= SPH_MAX_DIMS, "spyre: fill_ supports at most 8 dims");
  std::vector<int64_t> sizes(self.sizes().begin(), self.sizes().end());
  for (int d = 0; d < nd; ++d) out.strides[d] = self.stride(d);
  SPYRE_SPH_CHECK(sph_pointwise(SPH_PW_FILL, 0, &out, nd, sizes.data(), bits, 0.0,
                                stream(self.get_device())));
  return self;
}

at::Tensor& spyre_fill_tensor_(at::Tensor& self, const at::Tensor& value) {
  TORCH_CHECK(value.dim() == 0, "spyre: fill_ only supports 0-dimension value tensors");
  return spyre_fill_(self, value.item());
}

at::Tensor& spyre_zero_(at::Tensor& self) { return spyre_fill_(self, 0); }

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("empty.memory_format", TORCH_FN(spyre_empty));
  m.impl("empty_strided", TORCH_FN(spyre_empty_strided));
  m.impl("as_strided", TORCH_FN(spyre_as_strided));
  m.impl("view", TORCH_FN(spyre_view));
  m.impl("_reshape_alias", TORCH_FN(spyre_reshape_alias));
  m.impl("set_.source_Storage_storage_offset", TORCH_FN(spyre_set_storage));
  m.impl("set_.source_Storage", TORCH_FN(spyre_set_storage_only));
  m.impl("resize_", TORCH_FN(spyre_resize_));
  m.impl("_copy_from", TORCH_FN(spyre_copy_from));
  m.impl("_copy_from_and_resize", TORCH_FN(spyre_copy_from_and_resize));
  m.impl("_local_scalar_dense", TORCH_FN(spyre_local_scalar_dense));
  m.impl("fill_.Scalar", TORCH_FN(spyre_fill_));
  m.impl("fill_.Tensor", TORCH_FN(spyre_fill_tensor_));
  m.impl("zero_", TORCH_FN(spyre_zero_));
}

}  // namespace spyre
