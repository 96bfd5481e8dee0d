"""Stick-layout descriptors of spyre tensors (the DCI algebra).

Reference: torch_spyre/_inductor/stickify.py:30-245.  A spyre tensor is
described by a SpyreDCI: the order of its dimensions from the largest stride
to the smallest (`dim_order`, PyTorch convention), how many trailing entries
of that order form the 128-byte "stick" (`num_stick_dims`, always 1) and
whether each stick is filled (DENSE), holds one element (SPARSE, the result
of a reduction over the stick dimension) or a few per-row statistics
(SPARSE_MULTI, the result of `spyre::exx2`).  The functions here are the
shape / descriptor rules of matmul, reduction and broadcasting pointwise
results; they are pure functions of sizes, dim orders and formats.

On MI355X the HBM layout of DENSE tensors is PyTorch's row-major one (a
128-byte stick is one full cache line of the innermost dimension, so the
generic descriptor needs no padding or retiling).  The sparse formats keep
the reference's physical meaning -- one stick per value, i.e. an innermost
stride of `elems_per_stick(dtype)` -- and only the spyre custom ops that the
reference defines with sparse results produce them.

Where the reference's rules are index-inconsistent this module follows the
meaning instead (each case is exercised by tests on tiny shapes):
  * reducing a non-identity dim_order removes the entry whose VALUE is the
    reduced dim (the reference removes the entry at that POSITION; both
    agree for the generic order);
  * a reduction over non-stick dims keeps the input's format (the
    reference returns DENSE even for a SPARSE input);
  * broadcasting aligns dims from the right before asking whether the other
    operand is broadcast along an operand's stick dim (the reference indexes
    the result's dims with the operand's dim number).
"""

from __future__ import annotations

import dataclasses
import enum
from typing import Sequence, Tuple, Union

import torch

from . import Unsupported

BYTES_IN_STICK = 128


def elems_per_stick(dtype: torch.dtype) -> int:
    """Elements of `dtype` in one 128-byte stick (64 for fp16/bf16)."""
    return BYTES_IN_STICK // dtype.itemsize


class StickFormat(enum.Enum):
    DENSE = 1
    SPARSE = 2
    SPARSE_MULTI = 3


@dataclasses.dataclass
class SpyreDCI:
    """Descriptor of a tensor's stick layout.

    dim_order[0] is the dimension with the largest stride, dim_order[-1]
    the one with the smallest; dim_order[-num_stick_dims:] are the stick
    dimensions (reference: SpyreDCI, stickify.py:42-110).
    """

    dim_order: list
    num_stick_dims: int = 1
    format: StickFormat = StickFormat.DENSE

    def __post_init__(self):
        if self.num_stick_dims != 1:
            raise Unsupported(f"{self.num_stick_dims} stick dimensions (only 1 is supported)")
        self.dim_order = [int(d) for d in self.dim_order]

    @staticmethod
    def generic_stick_dci(t: torch.Tensor) -> "SpyreDCI":
        """Row-major order with the innermost dimension as the stick."""
        return SpyreDCI(list(range(t.dim())))

    def get_stick_dims(self) -> list:
        return self.dim_order[len(self.dim_order) - self.num_stick_dims:]

    def is_stick_dim(self, dim: Union[int, Sequence[int]]) -> bool:
        sticks = self.get_stick_dims()
        if isinstance(dim, int):
            return dim in sticks
        return any(d in sticks for d in dim)

    def is_stick_reduction(self, axis: Sequence[int]) -> bool:
        """True if `axis` reduces the stick dim; mixing stick and non-stick
        dims in one reduction is unsupported (reference :80-92)."""
        sticks = self.get_stick_dims()
        hits = [d in sticks for d in axis]
        if any(hits) and not all(hits):
            raise Unsupported(f"reduction on both stick and non-stick dimensions {list(axis)}")
        return any(hits)

    def spyre_strides(self, size: Sequence[int], dtype: torch.dtype) -> list:
        """Element strides of a tensor of `size` in this layout: row-major
        along dim_order; sparse formats give every innermost element a
        stick of its own (reference :94-101)."""
        if len(size) != len(self.dim_order):
            raise ValueError(f"size {list(size)} does not match dim_order {self.dim_order}")
        step = 1 if self.format == StickFormat.DENSE else elems_per_stick(dtype)
        strides = [0] * len(size)
        for d in reversed(self.dim_order):
            strides[d] = step
            step = step * size[d]
        return strides

    def spyre_layout(self, device: torch.device, size: Sequence, dtype: torch.dtype):
        return SpyreFixedLayout(device, dtype, list(size), self.spyre_strides(size, dtype), self)

    @staticmethod
    def from_tensor(t: torch.Tensor) -> "SpyreDCI":
        """Descriptor implied by a tensor's strides: dims ordered by
        decreasing stride (ties keep the logical order) and SPARSE when the
        innermost stride is one stick."""
        n = t.dim()
        order = sorted(range(n), key=lambda d: (-t.stride(d), d))
        eps = elems_per_stick(t.dtype)
        sparse = n > 0 and eps > 1 and t.stride(order[-1]) == eps
        return SpyreDCI(order, format=StickFormat.SPARSE if sparse else StickFormat.DENSE)


def _fixed_layout_base():
    from torch._inductor.ir import FixedLayout
    return FixedLayout


class SpyreFixedLayout(_fixed_layout_base()):
    """An Inductor FixedLayout that carries the SpyreDCI it was derived
    from (reference: stickify.py:113-140)."""

    def __init__(self, device, dtype, size, stride, dci: SpyreDCI) -> None:
        super().__init__(device, dtype, size, stride)
        self.dci = dci

    def __str__(self) -> str:
        idx = "" if self.device.index is None else f":{self.device.index}"
        return (f"{type(self).__name__}('{self.device.type}{idx}', {self.dtype}, "
                f"size={self.size}, stride={self.stride}, dci={self.dci})")

    __repr__ = __str__

    def get_allocation_size(self):
        return self.size


def tensor_get_dci(self: torch.Tensor) -> SpyreDCI:
    """`Tensor.get_dci()`: the descriptor attached by a spyre op, else the
    one the tensor's strides imply (the generic stick layout for a
    contiguous tensor)."""
    dci = getattr(self, "spyre_dci", None)
    if not isinstance(dci, SpyreDCI):
        dci = SpyreDCI.from_tensor(self)
        try:
            self.spyre_dci = dci
        except Exception:  # pragma: no cover - tensors that refuse attributes
            pass
    return dci


def install_spyre_tensors() -> None:
    """Adds `torch.Tensor.get_dci` (reference: tensors.py:30-45).  Unlike the
    reference no fake-tensor or Inductor internals are patched: descriptors
    that are not attached by a spyre op are recovered from strides."""
    if getattr(torch.Tensor, "get_dci", None) is not tensor_get_dci:
        torch.Tensor.get_dci = tensor_get_dci


def spyre_matmul_result_shape(x: torch.Tensor, y: torch.Tensor) -> Tuple[list, SpyreDCI]:
    """[M,K] @ [K,N] -> ([M,N], x's dim order); both operands DENSE with the
    same dim order (reference :143-154)."""
    xd, yd = tensor_get_dci(x), tensor_get_dci(y)
    if xd.format != StickFormat.DENSE or yd.format != StickFormat.DENSE:
        raise Unsupported(f"matmul on non-dense tensors {xd} {yd}")
    if xd.dim_order != yd.dim_order:
        raise Unsupported(f"matmul stick dimensions mismatch {xd} {yd}")
    return [x.size(0), y.size(1)], SpyreDCI(list(xd.dim_order))


def spyre_reduction_result_shape(x: torch.Tensor, axis: Union[int, Sequence[int]],
                                 keepdims: bool = False) -> Tuple[list, SpyreDCI]:
    """Size and descriptor of a reduction of `x` over `axis` (reference
    :157-188).  Reducing the stick dim gives a SPARSE result."""
    n = x.dim()
    axes = [axis] if isinstance(axis, int) else list(axis)
    axes = sorted({(a + n if a < 0 else a) if n else 0 for a in axes})
    dci = tensor_get_dci(x)
    stick = dci.is_stick_reduction(axes)
    fmt = StickFormat.SPARSE if stick else dci.format
    size = list(x.size())
    if keepdims:
        for a in axes:
            if n:
                size[a] = 1
        return size, SpyreDCI(list(dci.dim_order), format=fmt)
    res_size = [s for d, s in enumerate(size) if d not in axes]
    res_order = [o - sum(1 for a in axes if a < o) for o in dci.dim_order if o not in axes]
    return res_size, SpyreDCI(res_order, format=fmt)


def spyre_pointwise_result_shape(x: torch.Tensor, y: torch.Tensor) -> Tuple[list, SpyreDCI]:
    """Broadcast size and descriptor of a binary pointwise op (reference
    :191-245): equal formats pass through; a DENSE operand combined with a
    sparse one is allowed only when the sparse operand is broadcast along the
    DENSE operand's stick dim (the result is DENSE)."""
    xs, ys = list(x.size()), list(y.size())
    n = max(len(xs), len(ys))
    res = [1] * n
    x_b, y_b = [False] * n, [False] * n
    for i in range(1, n + 1):
        a = xs[-i] if i <= len(xs) else None
        b = ys[-i] if i <= len(ys) else None
        if a is None:
            res[-i], x_b[-i] = b, True
        elif b is None:
            res[-i], y_b[-i] = a, True
        elif a == b:
            res[-i] = a
        elif b == 1:
            res[-i], y_b[-i] = a, True
        elif a == 1:
            res[-i], x_b[-i] = b, True
        else:
            raise RuntimeError("Shape mismatch: objects cannot be broadcast to a single shape")
    xd, yd = tensor_get_dci(x), tensor_get_dci(y)

    def stick_of(dci: SpyreDCI, rank: int) -> int:
        # the operand's stick dim as a (negative) index into the result
        return dci.get_stick_dims()[0] - rank

    if xd.format == yd.format:
        fmt = xd.format
    elif xd.format == StickFormat.DENSE and xd.dim_order and y_b[stick_of(xd, len(xs))]:
        fmt = StickFormat.DENSE
    elif yd.format == StickFormat.DENSE and yd.dim_order and x_b[stick_of(yd, len(ys))]:
        fmt = StickFormat.DENSE
    else:
        raise Unsupported(f"binop with incompatible DCIs: {xd} {yd} {x_b} {y_b}")
    return res, SpyreDCI(list(range(n)), format=fmt)
