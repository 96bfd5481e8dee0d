"""Decompositions of the spyre custom operators, and the `F.layer_norm`
route to `spyre::layer_norm`.

Reference: torch_spyre/_inductor/decompositions.py:21-58.  `compact` is
slice(swap(x)) as in the reference.  `layer_norm` decomposes into aten's
native_layer_norm rather than into exx2 -> layernormscale -> layernormnorm
(three kernels and a variance formed as E[x^2] - E[x]^2 in the activation
dtype): Inductor turns the aten form into one fused Welford row kernel, with
any residual add or other producer fused into it.

The `F.layer_norm` replacement routes spyre tensors normalised over one
dimension to `spyre::layer_norm` (the reference's condition) when no
argument requires grad: the custom op has no autograd formula, so training
graphs keep torch's differentiable layer norm.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch
import torch.nn.functional as F

_orig_layer_norm = F.layer_norm
_registered = False


def compact_decomp(x: torch.Tensor) -> torch.Tensor:
    return torch.ops.spyre.slice(torch.ops.spyre.swap(x))


def layernorm_decomp(input: torch.Tensor, normalized_shape: list, weight: Optional[torch.Tensor] = None,
                     bias: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    return torch.ops.aten.native_layer_norm.default(input, normalized_shape, weight, bias, eps)[0]


def spyre_layer_norm(input: torch.Tensor, normalized_shape: Sequence[int],
                     weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                     eps: float = 1e-5) -> torch.Tensor:
    if (isinstance(input, torch.Tensor) and input.device.type == "spyre"
            and len(normalized_shape) == 1
            and not (torch.is_grad_enabled() and any(
                t is not None and t.requires_grad for t in (input, weight, bias)))):
        return torch.ops.spyre.layer_norm(input, list(normalized_shape), weight, bias, eps)
    return _orig_layer_norm(input, normalized_shape, weight, bias, eps)


def register() -> None:
    global _registered
    if _registered:
        return
    from torch._inductor.decomposition import register_decomposition

    register_decomposition([torch.ops.spyre.compact])(compact_decomp)
    register_decomposition([torch.ops.spyre.layer_norm])(layernorm_decomp)
    F.layer_norm = spyre_layer_norm
    _registered = True
