"""Kernel descriptions the spyre Inductor backend writes into generated
wrapper code (reference: torch_spyre/_inductor/runtime/__init__.py:20-45,
same class names).

A KernelSpec here carries the HIP source of one generated kernel (one of the
hand-written templates in ../include/spyre_inductor_rt.h, instantiated with
the fused loop body), its launch shape, and per argument the number of
elements it may address, which the launcher checks against each tensor's
storage before every launch.
"""

from __future__ import annotations

import dataclasses
from typing import Optional, Union

import torch


@dataclasses.dataclass
class TensorArg:
    is_input: bool
    arg_index: int
    dtype: torch.dtype
    # Elements addressed from the tensor's data pointer (max offset + 1);
    # None when it cannot be bounded at compile time (masked / indirect).
    extent: Optional[int] = None


@dataclasses.dataclass
class ConstantArg:
    value: Union[bool, float, int]
    dtype: torch.dtype


@dataclasses.dataclass
class KernelSpec:
    op: str                      # template: "pointwise" or "reduction"
    is_reduction: bool
    dimensions: list[int]        # [xnumel] or [xnumel, rnumel]
    args: list[TensorArg]        # kernel parameter order
    grid: int
    block: int
    source: str                  # HIP C++ of the kernel `symbol`
    op_info: dict = dataclasses.field(default_factory=dict)
    # the kernel takes the device error word as a last parameter (indirect
    # indexing: out-of-range indices are reported there, see launch_kernel)
    error_word: bool = False
    # the kernel's extern "C" name; generated kernels are named for their
    # kind and a hash of their source (spyre_pw_<hash> / spyre_red_<hash>),
    # so each shows up under its own name in a profiler's kernel trace
    symbol: str = "spyre_kernel"


@dataclasses.dataclass
class UnimplementedOp:
    op: str
