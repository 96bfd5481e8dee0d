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

namespace spyre {

// One decode step of attention with its KV-cache append
// (sph_decode_attention_step): qkv [B, (H + 2 Hkv) * 128] the step's
// projection rows, cos / sin [max_len, 128] RoPE tables, pos a one-element
// int64 spyre tensor holding the step's position, k_cache [B, Hkv, max_len,
// 128] and v_cache [B, Hkv, max_len, 128], or with v_dim_major the
// transposed buffer [B, Hkv, 128, max_len], updated in place; returns
// [B, H * 128].  A position outside the caches raises at the next
// synchronisation, as an out-of-range gather does.
at::Tensor decode_attention_step(const at::Tensor& qkv_in, const at::Tensor& cos_in,
                                 const at::Tensor& sin_in, const at::Tensor& pos,
                                 at::Tensor& k_cache, at::Tensor& v_cache, int64_t n_heads,
                                 int64_t n_kv_heads, double scale, bool v_dim_major) {
  TORCH_CHECK(is_spyre(qkv_in) && is_spyre(cos_in) && is_spyre(sin_in) && is_spyre(pos) &&
                  is_spyre(k_cache) && is_spyre(v_cache),
              "spyre decode_attention: every argument must be a spyre tensor");
  const at::ScalarType dt = qkv_in.scalar_type();
  TORCH_CHECK(dt == at::kHalf || dt == at::kBFloat16,
              "spyre decode_attention: dtype must be fp16 or bf16");
  TORCH_CHECK(cos_in.scalar_type() == dt && sin_in.scalar_type() == dt &&
                  k_cache.scalar_type() == dt && v_cache.scalar_type() == dt,
              "spyre decode_attention: qkv, tables and caches must share one dtype");
  TORCH_CHECK(pos.scalar_type() == at::kLong && pos.numel() == 1,
              "spyre decode_attention: pos must be a one-element int64 tensor");
  TORCH_CHECK(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
              "spyre decode_attention: n_heads must be a multiple of n_kv_heads");
  constexpr int64_t D = 128;
  TORCH_CHECK(qkv_in.dim() == 2 && qkv_in.size(1) == (n_heads + 2 * n_kv_heads) * D,
              "spyre decode_attention: qkv must be [batch, (n_heads + 2 n_kv_heads) * 128]");
  const int64_t B = qkv_in.size(0);
  TORCH_CHECK(k_cache.dim() == 4 && k_cache.size(0) == B && k_cache.size(1) == n_kv_heads &&
                  k_cache.size(3) == D && k_cache.stride(3) == 1,
              "spyre decode_attention: k_cache must be [batch, n_kv_heads, max_len, 128] with "
              "unit dim stride");
  const int64_t L = k_cache.size(2);
  TORCH_CHECK(v_cache.dim() == 4 && v_cache.size(0) == B && v_cache.size(1) == n_kv_heads,
              "spyre decode_attention: v_cache must be [batch, n_kv_heads, ...]");
  TORCH_CHECK(v_dim_major ? (v_cache.size(2) == D && v_cache.size(3) == L && v_cache.stride(3) == 1)
                          : (v_cache.size(2) == L && v_cache.size(3) == D && v_cache.stride(3) == 1),
              "spyre decode_attention: v_cache must be [batch, n_kv_heads, max_len, 128], or "
              "with v_dim_major [batch, n_kv_heads, 128, max_len], with unit last stride");
  TORCH_CHECK(cos_in.dim() == 2 && cos_in.size(0) >= L && cos_in.size(1) == D &&
                  sin_in.sizes() == cos_in.sizes(),
              "spyre decode_attention: cos / sin must be [>= max_len, 128]");
  at::Tensor qkv = qkv_in.stride(1) == 1 && (qkv_in.stride(0) % 8 == 0 || B == 1)
                       ? qkv_in
                       : contiguous_on_device(qkv_in);
  at::Tensor cs = cos_in.stride(1) == 1 ? cos_in : contiguous_on_device(cos_in);
  at::Tensor sn = sin_in.strides() == cs.strides() ? sin_in : contiguous_on_device(sin_in);
  if (sn.strides() != cs.strides()) cs = contiguous_on_device(cs);
  at::Tensor out = empty_spyre({B, n_heads * D}, dt, qkv.device());
  if (B == 0) return out;
  const int64_t v_ks = v_dim_major ? 1 : v_cache.stride(2);
  const int64_t v_ds = v_dim_major ? v_cache.stride(2) : 1;
  const int64_t ks[4] = {B, n_kv_heads, L, D};
  const int64_t kst[4] = {k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), 1};
  const int64_t vst[4] = {v_cache.stride(0), v_cache.stride(1), v_ks, v_ds};
  check_extent(k_cache, k_cache.data_ptr(), 4, ks, kst, k_cache.element_size(), "k_cache");
  check_extent(v_cache, v_cache.data_ptr(), 4, ks, vst, v_cache.element_size(), "v_cache");
  const int64_t qs[2] = {B, qkv.size(1)}, qst[2] = {qkv.stride(0), 1};
  check_extent(qkv, qkv.data_ptr(), 2, qs, qst, qkv.element_size(), "qkv");
  const int64_t ts[2] = {L, D}, tst[2] = {cs.stride(0), 1};
  check_extent(cs, cs.data_ptr(), 2, ts, tst, cs.element_size(), "cos");
  check_extent(sn, sn.data_ptr(), 2, ts, tst, sn.element_size(), "sin");
  const int64_t nws = sph_decode_attention_step_workspace_bytes(B, n_heads, n_kv_heads, L);
  at::Tensor ws = empty_spyre({nws}, at::kByte, qkv.device());
  c10::DeviceGuard guard(qkv.device());
  const int dev = qkv.get_device();
  SPYRE_SPH_CHECK(sph_decode_attention_step(
      to_sph(dt), B, n_heads, n_kv_heads, D, qkv.data_ptr(), qkv.stride(0), cs.data_ptr(),
      sn.data_ptr(), cs.stride(0), pos.data_ptr<int64_t>(), device_error_word(dev),
      k_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
      v_cache.data_ptr(), v_cache.stride(0), v_cache.stride(1), v_ks, v_ds, L,
      static_cast<float>(scale), out.data_ptr(), out.stride(0), ws.data_ptr(), nws, stream(dev)));
  return out;
}

}  // namespace spyre
