"""numpy restatements of the floating-point ops on the torch_spyre hot path.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference checks every device result against PyTorch's CPU op on the same
inputs (tests/_inductor/utils_inductor.py:186-198 compare_with_cpu,
tests/test_ops.py:40-43); BASELINE fixes that oracle as "CPU fp32 math cast to
fp16".  These functions restate each op from its mathematical definition in
float32 (float64 where noted) so they can be pinned independently of torch:
tests/test_oracle.py checks them against torch's CPU kernels, closed forms and
the reference tests' known answers.

Inputs are numpy arrays (any float dtype; fp16 inputs are widened exactly);
outputs are float32 unless stated.  Callers round to fp16 with .astype.
"""

from __future__ import annotations

import numpy as np
from scipy.special import erf as _erf


def _f32(x):
    return np.asarray(x).astype(np.float32)


def softmax(x, axis=-1, scale=1.0, causal_q_len=0, causal_offset=0, log=False):
    """softmax / log_softmax over `axis` of scale*x.

    Reference op: aten::_softmax as generated for spyre (codegen/inputs/
    Metadata.yaml:275-277) and its compiled decomposition amax -> sub -> exp
    -> sum -> div (torch_spyre/_inductor/choices.py:58-83).  With
    causal_q_len > 0 (last axis only, x viewed as rows), column c of row r is
    masked (-inf) when c > r % causal_q_len + causal_offset."""
    a = _f32(x) * np.float32(scale)
    if causal_q_len:
        assert axis in (-1, a.ndim - 1)
        rows = a.reshape(-1, a.shape[-1])
        r = np.arange(rows.shape[0])[:, None] % causal_q_len
        c = np.arange(rows.shape[1])[None, :]
        rows = np.where(c > r + causal_offset, np.float32(-np.inf), rows)
        a = rows.reshape(a.shape)
    m = np.max(a, axis=axis, keepdims=True)
    with np.errstate(invalid="ignore"):
        z = a - m
        e = np.exp(z)
        s = np.sum(e, axis=axis, keepdims=True, dtype=np.float64).astype(np.float32)
        if log:
            return (z - np.log(s)).astype(np.float32)
        return (e / s).astype(np.float32)


def _round_to(x, dtype):
    """float32 values rounded to `dtype` (a numpy dtype, or "bfloat16":
    round to nearest even on the upper 16 bits of the float32 pattern)."""
    x = np.asarray(x, dtype=np.float32)
    if isinstance(dtype, str) and dtype == "bfloat16":
        b = x.view(np.uint32).astype(np.uint64)
        r = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
        out = r.astype(np.uint32).view(np.float32)
        return np.where(np.isnan(x), x, out)
    return x.astype(dtype).astype(np.float32)


def rmsnorm(x, weight=None, eps=1e-5, residual=None, act_dtype=np.float16):
    """Returns (y, h): h = round_to(act_dtype)(x + residual) (or x), and
    y = h * rsqrt(mean(h^2) + eps) * weight over the last axis.

    Reference op: the eager composite pow -> mean -> add -> rsqrt -> mul
    (codegen/inputs/Metadata.yaml:236-238,251-253; spyre_torch_ops.cpp:
    456-474); torch.nn.functional.rms_norm is the CPU comparator."""
    h = _f32(x)
    if residual is not None:
        h = _round_to(h + _f32(residual), act_dtype)
    ms = np.mean(h.astype(np.float64) ** 2, axis=-1, keepdims=True)
    r = (1.0 / np.sqrt(ms + eps)).astype(np.float32)
    y = h * r
    if weight is not None:
        y = y * _f32(weight)
    return y.astype(np.float32), h


def rmsnorm_linear(x, norm_w, w, eps=1e-5, act_dtype=np.float16, swiglu=False):
    """rms_norm(x, norm_w) @ w.T with the norm folded into the product (the
    decode-step kernel, no reference counterpart: the reference runs the
    norm's composite and spyre__mm_default, spyre_torch_ops.cpp:214-293):
    x * norm_w is rounded to act_dtype (None: not rounded), the float32 sums
    are scaled by each row's rsqrt(mean(x^2) + eps).  swiglu: w stacks gate
    and up rows [2n, K] and the result is silu(gate) * up.  Float32 result,
    not rounded."""
    h = _f32(x)
    ms = np.mean(h.astype(np.float64) ** 2, axis=-1, keepdims=True)
    rs = (1.0 / np.sqrt(ms + eps)).astype(np.float32)
    xw = h * _f32(norm_w)
    if act_dtype is not None:
        xw = _round_to(xw, act_dtype)
    y = np.matmul(xw, _f32(w).T) * rs
    if swiglu:
        n = y.shape[-1] // 2
        y = silu(y[..., :n]) * y[..., n:]
    return y.astype(np.float32)


def layernorm(x, weight=None, bias=None, eps=1e-5, residual=None, act_dtype=np.float16):
    """Returns (y, h, mean, rstd) of LayerNorm over the last axis (biased
    variance), h as in rmsnorm.

    Reference op: the compiled chain exx2 -> layernormscale -> layernormnorm
    (torch_spyre/_inductor/decompositions.py:26-36, customops.py:102-154:
    E[x], E[x^2] with scale 1/N, rstd = 1/sqrt(var + eps), (x - mean) * rstd
    * w + b).  The eager spyre op is a stub returning its input
    (spyre_torch_ops.cpp:188-194), so torch.nn.functional.layer_norm on CPU
    is the comparator."""
    h = _f32(x)
    if residual is not None:
        h = _round_to(h + _f32(residual), act_dtype)
    h64 = h.astype(np.float64)
    mean = np.mean(h64, axis=-1, keepdims=True)
    var = np.mean((h64 - mean) ** 2, axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    y = (h64 - mean) * rstd
    if weight is not None:
        y = y * _f32(weight)
    if bias is not None:
        y = y + _f32(bias)
    return (y.astype(np.float32), h, mean[..., 0].astype(np.float32),
            rstd[..., 0].astype(np.float32))


def gelu(x):
    """GELU, erf form: 0.5 x (1 + erf(x / sqrt 2)).  Reference op: generated
    gelu with approximate forced to "none" (codegen/inputs/Metadata.yaml:
    125-132)."""
    a = _f32(x).astype(np.float64)
    return (0.5 * a * (1.0 + _erf(a / np.sqrt(2.0)))).astype(np.float32)


def attention(q, k, v, scale, mask=None, causal_q_len=0, causal_offset=0):
    """softmax(scale * q k^T + mask) v per leading batch index (fp32 scores
    and probabilities, float64 row sums).  The chain the reference runs for
    attention: spyre__bmm_default (codegen/inputs/spyre_torch_ops.cpp:
    297-377) for the scores, the generated add and _softmax
    (Metadata.yaml:275-277), bmm again for P v.  q [..., mq, d], k / v
    [..., sk, d], mask broadcastable to [..., mq, sk]; causal as in
    `softmax` (row r keeps columns c <= r % causal_q_len + causal_offset)."""
    s = np.matmul(_f32(q), np.swapaxes(_f32(k), -1, -2)) * np.float32(scale)
    if mask is not None:
        s = s + _f32(mask)
    p = softmax(s, axis=-1, causal_q_len=causal_q_len, causal_offset=causal_offset)
    return np.matmul(p, _f32(v)).astype(np.float32)


def gelu_affine_rowsum(x, s, b):
    """y = gelu(x * s + b) (s, b broadcast over rows), r = sum_c y (fp32 y).
    The fused chain of config 3 (gelu followed by ReduceSum,
    Metadata.yaml:125-132, 299-302)."""
    y = gelu(_f32(x) * _f32(s) + _f32(b))
    r = np.sum(y.astype(np.float64), axis=-1).astype(np.float32)
    return y, r


def silu(x):
    a = _f32(x).astype(np.float64)
    return (a / (1.0 + np.exp(-a))).astype(np.float32)


def gemm(a, b, alpha=1.0, beta=0.0, c=None, epilogue="none", acc=np.float32):
    """D = epi(alpha * a @ b + beta * c), fp32 (or `acc`) accumulation.

    Reference ops: spyre__mm_default / spyre__bmm_default / spyre__addmm_*
    (codegen/inputs/spyre_torch_ops.cpp:214-452).  The reference's addmm
    ignores beta (:389-390); this oracle (and the build) use torch's
    beta * self + alpha * (a @ b)."""
    d = np.matmul(np.asarray(a).astype(acc), np.asarray(b).astype(acc)).astype(np.float32)
    d = d * np.float32(alpha)
    if c is not None and beta != 0.0:
        d = d + np.float32(beta) * _f32(c)
    if epilogue == "relu":
        d = np.maximum(d, 0)
    elif epilogue == "gelu":
        d = gelu(d)
    elif epilogue == "silu":
        d = silu(d)
    return d.astype(np.float32)


def rope(x, positions, theta=1e4):
    """Rotary embedding, rotate-half convention, on x[tokens, heads, d]:
    inv_freq_i = theta^(-2i/d), angle = pos * inv_freq (fp32), then
    [x1 cos - x2 sin, x2 cos + x1 sin] in float64."""
    a = _f32(x).astype(np.float64)
    d = a.shape[-1]
    half = d // 2
    inv = (1.0 / (np.float32(theta) ** (np.arange(0, d, 2, dtype=np.float32) / np.float32(d))))
    ang = (np.asarray(positions, dtype=np.float32)[:, None] * inv[None, :].astype(np.float32))
    cos = np.cos(ang.astype(np.float64))[:, None, :]
    sin = np.sin(ang.astype(np.float64))[:, None, :]
    x1, x2 = a[..., :half], a[..., half:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1).astype(np.float32)
