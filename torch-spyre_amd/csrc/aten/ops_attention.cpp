// Fused attention of the spyre backend: softmax(scale * q k^T + mask) v in
// one kernel (sph_attention_fwd), without the [mq, sk] score matrix.
//
// Reference: the reference computes attention as three eager ops,
// spyre__bmm_default (codegen/inputs/spyre_torch_ops.cpp:297-377) for the
// scores, the generated add and _softmax (codegen/inputs/Metadata.yaml:
// 275-277) and spyre__bmm_default again for P v.  The compile backend
// substitutes this entry for that chain when its shapes fit (head dim 128,
// query rows a multiple of 128, or at most 16 per batch entry for a decode
// step (sph_attention_decode), fp16/bf16); called directly it accepts the
// same shapes and raises otherwise.
#include <torch/extension.h>

#include "spyre_ops_common.h"

namespace spyre {

namespace {

// t with unit innermost stride and a 16-byte multiple row stride (copied
// when needed).
at::Tensor rows_aligned(const at::Tensor& t) {
  const int64_t eb = t.element_size();
  if (t.stride(-1) == 1 && (t.dim() < 2 || (t.stride(-2) * eb) % 16 == 0) &&
      reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0 &&
      (t.dim() < 3 || t.size(0) == 1 || (t.stride(0) * eb) % 16 == 0))
    return t;
  return contiguous_on_device(t);
}

}  // namespace

at::Tensor attention_fwd(const at::Tensor& q_in, const at::Tensor& k_in, const at::Tensor& v_in,
                         const c10::optional<at::Tensor>& mask_in, double scale,
                         int64_t causal_q, int64_t causal_off) {
  TORCH_CHECK(is_spyre(q_in) && is_spyre(k_in) && is_spyre(v_in),
              "spyre attention: q, k, v must be spyre tensors");
  TORCH_CHECK(q_in.dim() == 3 && k_in.dim() == 3 && v_in.dim() == 3,
              "spyre attention: q, k, v must be [batch, rows, head_dim]");
  const int64_t B = q_in.size(0), mq = q_in.size(1), d = q_in.size(2), sk = k_in.size(1);
  TORCH_CHECK(k_in.size(0) == B && v_in.size(0) == B && k_in.size(2) == d && v_in.size(1) == sk &&
                  v_in.size(2) == d,
              "spyre attention: k / v shapes do not match q");
  const at::ScalarType dt = q_in.scalar_type();
  TORCH_CHECK(dt == at::kHalf || dt == at::kBFloat16, "spyre attention: dtype must be fp16 or bf16");
  TORCH_CHECK(k_in.scalar_type() == dt && v_in.scalar_type() == dt,
              "spyre attention: q, k, v dtypes differ");
  // Decode shapes (at most 16 query rows per batch entry) take V in either
  // layout: key-major, or dim-major as a KV cache kept for P V stores it.
  const bool decode = mq <= 16 && mq > 0;
  const bool v_dim_major = decode && v_in.stride(1) == 1 && v_in.stride(2) != 1 &&
                           (v_in.stride(2) * v_in.element_size()) % 16 == 0 &&
                           reinterpret_cast<uintptr_t>(v_in.data_ptr()) % 16 == 0 &&
                           (B == 1 || (v_in.stride(0) * v_in.element_size()) % 16 == 0);
  at::Tensor q = rows_aligned(q_in), k = rows_aligned(k_in);
  at::Tensor v = v_dim_major ? v_in : rows_aligned(v_in);
  at::Tensor out = empty_spyre({B, mq, d}, dt, q.device());
  if (out.numel() == 0) return out;

  const void* mp = nullptr;
  int64_t ldm = 0, sm = 0;
  at::Tensor mask, ws;
  if (mask_in.has_value() && mask_in->defined()) {
    at::Tensor m = *mask_in;
    TORCH_CHECK(is_spyre(m) && m.scalar_type() == dt,
                "spyre attention: the mask must be a spyre tensor of the q dtype");
    TORCH_CHECK((m.dim() == 2 || (m.dim() == 3 && (m.size(0) == B || m.size(0) == 1))) &&
                    m.size(-2) == mq && m.size(-1) == sk,
                "spyre attention: the mask must be [rows, keys] or [batch or 1, rows, keys]");
    // (a row stride of 0, one mask row for every query row, is kept)
    if (m.stride(-1) != 1 || (m.stride(-2) != 0 && m.stride(-2) < sk) || (m.stride(-2) % 8) != 0 ||
        reinterpret_cast<uintptr_t>(m.data_ptr()) % 16 != 0 ||
        (m.dim() == 3 && m.size(0) > 1 && m.stride(0) % 8 != 0)) {
      // Copied into rows padded to a multiple of 8 elements (16 bytes), the
      // kernel's mask row alignment, whatever the key count.
      const int64_t sk8 = (sk + 7) / 8 * 8;
      std::vector<int64_t> shp(m.sizes().begin(), m.sizes().end());
      shp.back() = sk8;
      at::Tensor padded = empty_spyre(shp, dt, q_in.device());
      padded.narrow(-1, 0, sk).copy_(m);
      m = padded.narrow(-1, 0, sk);
    }
    mask = m;
    mp = m.data_ptr();
    ldm = m.stride(-2);
    sm = (m.dim() == 3 && m.size(0) > 1) ? m.stride(0) : 0;
    const int64_t mb = (m.dim() == 3 && m.size(0) > 1) ? B : 1;
    const int64_t ms[3] = {mb, mq, sk}, mst[3] = {sm, ldm, 1};
    check_extent(m, mp, 3, ms, mst, m.element_size(), "attention mask");
  }
  // mask-block classes (prefill with a mask) or the key-split partials (decode)
  if (decode || mp != nullptr) {
    const int64_t nws = sph_attention_workspace_bytes(B, mq, sk, sm);
    if (nws > 0) ws = empty_spyre({nws}, at::kByte, q.device());
  }
  const int64_t qs[3] = {B, mq, d}, qst[3] = {B == 1 ? 0 : q.stride(0), q.stride(1), 1};
  const int64_t ks[3] = {B, sk, d}, kst[3] = {B == 1 ? 0 : k.stride(0), k.stride(1), 1};
  const int64_t vst[3] = {B == 1 ? 0 : v.stride(0), v.stride(1), v.stride(2)};
  check_extent(q, q.data_ptr(), 3, qs, qst, q.element_size(), "attention q");
  check_extent(k, k.data_ptr(), 3, ks, kst, k.element_size(), "attention k");
  check_extent(v, v.data_ptr(), 3, ks, vst, v.element_size(), "attention v");
  c10::DeviceGuard guard(q.device());
  if (decode) {
    SPYRE_SPH_CHECK(sph_attention_decode(
        to_sph(dt), B, mq, sk, d, q.data_ptr(), q.stride(1), qst[0], k.data_ptr(), k.stride(1),
        kst[0], v.data_ptr(), v.stride(1), v.stride(2), vst[0], mp, ldm, sm, causal_q, causal_off,
        static_cast<float>(scale), out.data_ptr(), d, mq * d,
        ws.defined() ? ws.data_ptr() : nullptr, ws.defined() ? ws.numel() : 0,
        stream(q.get_device())));
    return out;
  }
  SPYRE_SPH_CHECK(sph_attention_fwd(
      to_sph(dt), B, mq, sk, d, q.data_ptr(), q.stride(1), qst[0], k.data_ptr(), k.stride(1),
      kst[0], v.data_ptr(), v.stride(1), vst[0], mp, ldm, sm, causal_q, causal_off,
      static_cast<float>(scale), out.data_ptr(), d, mq * d, ws.defined() ? ws.data_ptr() : nullptr,
      ws.defined() ? ws.numel() : 0, stream(q.get_device())));
  return out;
}

}  // namespace spyre
