"""The `torch.ops.spyre.*` custom operators.

Reference: torch_spyre/_inductor/customops.py:22-154 (op names, schemas,
which ops are spyre-only, and the descriptors their fake implementations
attach).  The reference leaves `swap`, `slice`, `exx2`, `layernormscale` and
`layernormnorm` without an eager body (the first two return uninitialised
memory, the last three `pass`); here every op computes its result on the
device with the spyre eager kernels, so each can be called eagerly, inside a
compiled graph (as an extern call) and compared with a CPU formula.  The
bodies (`*_impl`) are compositions of tensor ops, registered for the spyre
device only, as in the reference:

  compact(x)          1-D dense copy of x  (= slice(swap(x)))
  swap(x)             1-D x laid out SPARSE: element i at storage i*S,
                      S = elements per 128-byte stick (64 for fp16)
  slice(x)            1-D dense copy of a (sparse) x
  layer_norm(x, [N], w, b, eps)
                      F.layer_norm over the last dim (the fused HIP kernel)
  exx2(x, scale, zero_mean)
                      per row of the last dim, a SPARSE_MULTI stick holding
                      m1 = scale*sum(x) (0 when zero_mean) at slot 0 and
                      m2 = scale*sum(x*x) at slot 1; the returned tensor
                      views slot 0 (shape x.shape[:-1], stride S)
  layernormscale(s, eps)
                      rstd = 1/sqrt(max(m2 - m1*m1, 0) + eps) from exx2's
                      sticks, SPARSE (one stick per row)
  layernormnorm(x, mean, rstd, w, b)
                      (x - mean) * rstd * w + b with mean/rstd broadcast
                      along the last dim

With scale = 1/N, layernormnorm(x, exx2(x), layernormscale(exx2(x), eps),
w, b) is F.layer_norm(x, [N], w, b, eps), and with zero_mean it is RMSNorm
(the decomposition the reference uses for layer_norm,
decompositions.py:28-36).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import Unsupported
from .stickify import (SpyreDCI, StickFormat, elems_per_stick, spyre_reduction_result_shape,
                       tensor_get_dci)


def _require_1d(name: str, t: torch.Tensor) -> None:
    if t.dim() != 1:
        raise Unsupported(f"{name} only implemented for 1-D tensors")


def _sparse_like(t: torch.Tensor, size, fmt: StickFormat, slots: int = 1) -> torch.Tensor:
    """A tensor of `size` with one stick per innermost element, backed by a
    buffer that also holds `slots` values per stick."""
    eps = elems_per_stick(t.dtype)
    dci = SpyreDCI(list(range(len(size))), format=fmt)
    strides = dci.spyre_strides(size, t.dtype)
    rows = 1
    for s in size:
        rows *= int(s)
    base = t.new_empty((max(rows, 1) * eps,))
    assert slots <= eps
    out = base.as_strided(tuple(size), tuple(strides), 0)
    out.spyre_dci = dci
    return out


def _slot(t: torch.Tensor, k: int) -> torch.Tensor:
    return t.as_strided(t.size(), t.stride(), t.storage_offset() + k)


# ---- compact / swap / slice -------------------------------------------------

@torch.library.custom_op("spyre::compact", mutates_args=())
def compact(input: torch.Tensor) -> torch.Tensor:
    _require_1d("compact", input)
    return input.clone(memory_format=torch.contiguous_format)


@compact.register_fake
def _(input):
    _require_1d("compact", input)
    out = input.new_empty(input.size())
    out.spyre_dci = SpyreDCI([0], format=StickFormat.DENSE)
    return out


def swap_impl(input: torch.Tensor) -> torch.Tensor:
    _require_1d("swap", input)
    out = _sparse_like(input, list(input.size()), StickFormat.SPARSE)
    out.copy_(input)
    return out


@torch.library.custom_op("spyre::swap", mutates_args=(), device_types="spyre")
def swap(input: torch.Tensor) -> torch.Tensor:
    return swap_impl(input)


@swap.register_fake
def _(input):
    _require_1d("swap", input)
    out = input.new_empty_strided(input.size(), (elems_per_stick(input.dtype),))
    out.spyre_dci = SpyreDCI([0], format=StickFormat.SPARSE)
    return out


@torch.library.custom_op("spyre::slice", mutates_args=(), device_types="spyre")
def slice(input: torch.Tensor) -> torch.Tensor:  # noqa: A001 - reference op name
    _require_1d("slice", input)
    return input.clone(memory_format=torch.contiguous_format)


@slice.register_fake
def _(input):
    _require_1d("slice", input)
    out = input.new_empty(input.size())
    out.spyre_dci = SpyreDCI([0], format=StickFormat.DENSE)
    return out


# ---- layer norm and its statistics ops --------------------------------------

@torch.library.custom_op("spyre::layer_norm", mutates_args=())
def layer_norm(x: torch.Tensor, normalized_shape: list[int], weight: Optional[torch.Tensor] = None,
               bias: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    if len(normalized_shape) != 1:
        raise Unsupported(f"spyre.layernorm: unsupported reduction shape {normalized_shape}")
    return torch.native_layer_norm(x, normalized_shape, weight, bias, eps)[0]


@layer_norm.register_fake
def _(x, normalized_shape, weight=None, bias=None, eps=1e-5):
    if len(normalized_shape) != 1:
        raise Unsupported(f"spyre.layernorm: unsupported reduction shape {normalized_shape}")
    out = x.new_empty(x.size())
    out.spyre_dci = tensor_get_dci(x)
    return out


def _stats_size(x: torch.Tensor):
    size, dci = spyre_reduction_result_shape(x, [x.dim() - 1], False)
    if not dci.format == StickFormat.SPARSE:
        raise Unsupported(f"exx2 reduces the stick dimension only, got {tensor_get_dci(x)}")
    return size


def exx2_impl(x: torch.Tensor, exx2Scale: float, useZeroMean: bool) -> torch.Tensor:
    size = _stats_size(x)
    out = _sparse_like(x, size, StickFormat.SPARSE_MULTI, slots=2)
    xf = x.float()
    m2 = (xf * xf).sum(-1) * exx2Scale
    if useZeroMean:
        m1 = torch.zeros_like(m2)
    else:
        m1 = xf.sum(-1) * exx2Scale
    out.copy_(m1)
    _slot(out, 1).copy_(m2)
    return out


@torch.library.custom_op("spyre::exx2", mutates_args=(), device_types="spyre")
def exx2(x: torch.Tensor, exx2Scale: float, useZeroMean: bool) -> torch.Tensor:
    return exx2_impl(x, exx2Scale, useZeroMean)


@exx2.register_fake
def _(x, exx2Scale, useZeroMean):
    size = _stats_size(x)
    out = x.new_empty_strided(size, SpyreDCI(list(range(len(size))), format=StickFormat.SPARSE_MULTI)
                              .spyre_strides(size, x.dtype))
    out.spyre_dci = SpyreDCI(list(range(len(size))), format=StickFormat.SPARSE_MULTI)
    return out


def _check_stats(name: str, s: torch.Tensor) -> None:
    # statistics sticks: one stick per row (innermost stride = one stick)
    if s.dim() and s.stride(-1) != elems_per_stick(s.dtype):
        raise Unsupported(f"{name}: Unexpected format {tensor_get_dci(s).format}")


def layernormscale_impl(x: torch.Tensor, eps: float) -> torch.Tensor:
    _check_stats("layernormscale", x)
    m1 = x.float()
    m2 = _slot(x, 1).float()
    var = torch.clamp_min(m2 - m1 * m1, 0.0)
    out = _sparse_like(x, list(x.size()), StickFormat.SPARSE)
    out.copy_(torch.rsqrt(var + eps))
    return out


@torch.library.custom_op("spyre::layernormscale", mutates_args=(), device_types="spyre")
def layernormscale(x: torch.Tensor, eps: float) -> torch.Tensor:
    return layernormscale_impl(x, eps)


@layernormscale.register_fake
def _(x, eps):
    _check_stats("layernormscale", x)
    size = list(x.size())
    dci = SpyreDCI(list(range(len(size))), format=StickFormat.SPARSE)
    out = x.new_empty_strided(size, dci.spyre_strides(size, x.dtype))
    out.spyre_dci = dci
    return out


def layernormnorm_impl(x: torch.Tensor, mean: torch.Tensor, norm_mean: torch.Tensor,
                       weight: Optional[torch.Tensor], bias: Optional[torch.Tensor]) -> torch.Tensor:
    y = (x.float() - mean.float().unsqueeze(-1)) * norm_mean.float().unsqueeze(-1)
    if weight is not None:
        y = y * weight.float()
    if bias is not None:
        y = y + bias.float()
    return y.to(x.dtype)


@torch.library.custom_op("spyre::layernormnorm", mutates_args=(), device_types="spyre")
def layernormnorm(x: torch.Tensor, mean: torch.Tensor, norm_mean: torch.Tensor,
                  weight: Optional[torch.Tensor], bias: Optional[torch.Tensor]) -> torch.Tensor:
    return layernormnorm_impl(x, mean, norm_mean, weight, bias)


@layernormnorm.register_fake
def _(x, mean, norm_mean, weight, bias):
    out = x.new_empty(x.size())
    out.spyre_dci = tensor_get_dci(x)
    return out


# ---- fused attention --------------------------------------------------------

@torch.library.custom_op("spyre::attention", mutates_args=())
def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor],
              scale: float) -> torch.Tensor:
    """softmax(scale * q k^T + mask, -1) v for q [B, mq, d], k / v [B, sk, d],
    mask broadcastable to [B, mq, sk] or None; softmax in fp32, its result
    rounded to the input dtype before the second product.  This is the
    chain the reference runs as spyre__bmm_default
    (codegen/inputs/spyre_torch_ops.cpp:297-377), add + _softmax
    (codegen/inputs/Metadata.yaml:275-277) and bmm again; on other devices
    it runs as that chain, on spyre as one fused kernel."""
    s = torch.bmm(q, k.transpose(1, 2)) * scale
    if mask is not None:
        s = s + mask
    p = torch.softmax(s.float(), dim=-1).to(q.dtype)
    return torch.bmm(p, v)


@attention.register_kernel("spyre")
def _(q, k, v, mask, scale):
    from torch_spyre import _C

    return _C.attention_fwd(q, k, v, mask, float(scale))


@attention.register_fake
def _(q, k, v, mask, scale):
    return q.new_empty((q.shape[0], q.shape[1], v.shape[2]))


# ---- fused SwiGLU projection ------------------------------------------------

@torch.library.custom_op("spyre::swiglu_mm", mutates_args=())
def swiglu_mm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """silu(x w[:n]^T) * (x w[n:]^T) for x [M, K] and the stacked gate / up
    weight w [2n, K]: the gate and up projections of a SwiGLU MLP with the
    activation product.  On other devices it runs as the unfused chain the
    reference would run (spyre__mm_default, spyre_torch_ops.cpp:214-293, then
    the generated silu and mul ops); on spyre as one GEMM whose epilogue
    forms silu(gate) * up from the fp32 sums."""
    n = w.shape[0] // 2
    gu = torch.mm(x, w.t())
    return torch.nn.functional.silu(gu[:, :n]) * gu[:, n:]


@swiglu_mm.register_kernel("spyre")
def _(x, w):
    from torch_spyre import _C

    return _C.gemm_swiglu(x, w)


@swiglu_mm.register_fake
def _(x, w):
    return x.new_empty((x.shape[0], w.shape[0] // 2))


# ---- transposing copy --------------------------------------------------------

@torch.library.custom_op("spyre::transpose_copy", mutates_args=())
def transpose_copy(x: torch.Tensor, dims: list[int]) -> torch.Tensor:
    """x.permute(dims).contiguous(): the reference's transpose data op
    (torch_spyre/_inductor/codegen/data_ops.py:16-630, "restickify") as a
    copy.  On spyre the copy runs as one LDS-tiled transpose
    (sph_transpose_copy) whenever the permutation moves the contiguous
    dimension; elsewhere it is the plain permute and copy."""
    return x.permute(dims).contiguous()


@transpose_copy.register_fake
def _(x, dims):
    return x.new_empty([x.shape[d] for d in dims])


# ---- RMSNorm folded into the decode projections ----------------------------

@torch.library.custom_op("spyre::rms_norm_mm", mutates_args=())
def rms_norm_mm(x: torch.Tensor, norm_w: torch.Tensor, eps: float, w: torch.Tensor,
                swiglu: bool) -> torch.Tensor:
    """rms_norm(x, norm_w, eps) @ w.T for x [M, K] and an nn.Linear weight w
    [N, K]; with swiglu, w stacks the gate and up rows [2n, K] and the
    result is silu(gate) * up.  The reference runs the norm as its composite
    ops (pow / mean / add / rsqrt / mul, Metadata.yaml:236-253) and the
    product as spyre__mm_default (spyre_torch_ops.cpp:214-293); on other
    devices this is that chain, on spyre (decode rows, M <= 8) one
    weight-stream kernel with the norm as its prologue (sph_gemm_rmsnorm)."""
    xn = torch.nn.functional.rms_norm(x, (x.shape[-1],), norm_w, eps)
    if not swiglu:
        return torch.mm(xn, w.t())
    n = w.shape[0] // 2
    gu = torch.mm(xn, w.t())
    return torch.nn.functional.silu(gu[:, :n]) * gu[:, n:]


@rms_norm_mm.register_kernel("spyre")
def _(x, norm_w, eps, w, swiglu):
    from torch_spyre import _C

    return _C.gemm_rmsnorm(x, norm_w, float(eps), w, bool(swiglu))


@rms_norm_mm.register_fake
def _(x, norm_w, eps, w, swiglu):
    return x.new_empty((x.shape[0], w.shape[0] // 2 if swiglu else w.shape[0]))


# ---- decode-step attention with its KV-cache append ------------------------

@torch.library.custom_op("spyre::decode_attention", mutates_args=("k_cache", "v_cache"))
def decode_attention(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     pos: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     n_heads: int, n_kv_heads: int, scale: float,
                     v_dim_major: bool) -> torch.Tensor:
    """One decode step of grouped-query attention for qkv [B, (H + 2 Hkv) *
    D] (the step's query heads, then its keys, then its values): RoPE
    (rotate-half, tables cos / sin [max_len, D]) of the queries and keys at
    position pos (a one-element int64 tensor), the keys and values written
    into k_cache [B, Hkv, max_len, D] and v_cache ([B, Hkv, max_len, D], or
    [B, Hkv, D, max_len] with v_dim_major) at pos, then softmax(scale q
    K[0..pos]^T) V[0..pos] per query head (head j reads KV head j // (H /
    Hkv)); returns [B, H * D].  On other devices it runs as the op-by-op
    chain (pointwise RoPE, index_copy_, bmm -> masked softmax -> bmm) the
    reference would run (codegen/inputs/spyre_torch_ops.cpp:297-377,
    Metadata.yaml:275-277); on spyre as one kernel
    (sph_decode_attention_step)."""
    B = qkv.shape[0]
    D = k_cache.shape[-1]
    H, Hkv = n_heads, n_kv_heads
    L = k_cache.shape[2]
    q = qkv[:, :H * D].reshape(B, H, D)
    k = qkv[:, H * D:(H + Hkv) * D].reshape(B, Hkv, D)
    v = qkv[:, (H + Hkv) * D:].reshape(B, Hkv, D)
    c, s = cos.index_select(0, pos), sin.index_select(0, pos)  # [1, D]

    def rope(x):
        half = D // 2
        rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
        return x * c + rot * s

    q, k = rope(q), rope(k)
    k_cache.index_copy_(2, pos, k.unsqueeze(2))
    if v_dim_major:
        v_cache.index_copy_(3, pos, v.unsqueeze(3))
        vv = v_cache.transpose(2, 3)
    else:
        v_cache.index_copy_(2, pos, v.unsqueeze(2))
        vv = v_cache
    keys = torch.arange(L, device=qkv.device)
    mask = torch.where(keys <= pos, 0.0, float("-inf")).to(qkv.dtype)
    qg = q.reshape(B * Hkv, H // Hkv, D)
    sc = torch.bmm(qg, k_cache.reshape(B * Hkv, L, D).transpose(1, 2)) * scale + mask
    p = torch.softmax(sc.float(), dim=-1).to(qkv.dtype)
    o = torch.bmm(p, vv.reshape(B * Hkv, L, D).contiguous())
    return o.reshape(B, H * D)


@decode_attention.register_kernel("spyre")
def _(qkv, cos, sin, pos, k_cache, v_cache, n_heads, n_kv_heads, scale, v_dim_major):
    from torch_spyre import _C

    return _C.decode_attention_step(qkv, cos, sin, pos, k_cache, v_cache, int(n_heads),
                                    int(n_kv_heads), float(scale), bool(v_dim_major))


@decode_attention.register_fake
def _(qkv, cos, sin, pos, k_cache, v_cache, n_heads, n_kv_heads, scale, v_dim_major):
    return qkv.new_empty((qkv.shape[0], n_heads * k_cache.shape[-1]))
