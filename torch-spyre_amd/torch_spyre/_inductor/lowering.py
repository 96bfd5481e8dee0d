"""Inductor lowerings of the spyre custom operators.

Reference: torch_spyre/_inductor/lowering.py:25-153.  `swap` and `slice` are
copies between the dense and the one-element-per-stick layout; they lower to
pointwise nodes, so `compact` (= slice(swap(x))) fuses into a single copy
kernel, and a `swap` result that leaves the graph is written with the
stick stride its fake implementation declares.  The reference's global
`aten.mm` lowering is not reproduced: matrix products stay extern calls to
the MFMA GEMM for every device.  `exx2`, `layernormscale` and
`layernormnorm` have no lowering: inside a compiled graph they run as extern
calls of their eager implementations, while `spyre::layer_norm` is
decomposed into aten's layer norm, which Inductor fuses into one kernel.
"""

from __future__ import annotations

import torch
from torch._inductor import lowering as L
from torch._inductor.ir import Pointwise


def _copy_lowering(x):
    return Pointwise.create(
        device=x.get_device(),
        dtype=x.get_dtype(),
        inner_fn=x.make_loader(),
        ranges=x.get_size(),
    )


def register() -> None:
    spyre = torch.ops.spyre
    for op in (spyre.swap.default, spyre.slice.default):
        if op not in L.lowerings:
            L.register_lowering(op, type_promotion_kind=None)(_copy_lowering)
