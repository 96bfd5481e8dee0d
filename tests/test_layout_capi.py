"""torch_spyre._C.SpyreTensorLayout (CPU: the class is pure host arithmetic).

The golden vectors are the reference's own (tests/tensor/test_tensor_layout.py
:28-94); the closed form is also checked against the oracle's independent C
restatement (oracle/layout.c) on a sweep of shapes, dtypes and dim orders, and
the stick allocation rule against the oracle's sizing.
"""

import itertools

import pytest
import torch

import torch_spyre  # noqa: F401
from torch_spyre._C import SpyreTensorLayout as STL

from oracle import layout as L

from helpers import golden


def _check(stl, size, strides, dmap, fmt=STL.StickFormat.Dense):
    assert stl.device_size == size
    assert stl.device_strides == strides
    assert stl.dim_map == dmap
    assert stl.format == fmt
    assert stl.num_stick_dims == 1


def test_backend_registered():
    assert torch._C._get_privateuse1_backend_name() == "spyre"


def test_layout_golden():
    for c in golden("spyre_tensor_layout")["cases"]:
        stl = (STL(c["host_size"], torch.float16) if c["dim_order"] is None
               else STL(c["host_size"], torch.float16, c["dim_order"]))
        _check(stl, c["device_size"], c["device_strides"], c["dim_map"])


def test_explicit_and_sparse_constructors():
    x = STL([512, 256], torch.float16)
    y = STL([4, 512, 64], [32768, 64, 1], [1, 0, 1], 1, STL.StickFormat.Dense)
    for f in ("format", "num_stick_dims", "dim_map", "device_strides", "device_size"):
        assert getattr(x, f) == getattr(y, f)
    s = STL([4, 512, 64], [32768, 64, 1], [1, 0, 1], 1, STL.StickFormat.Sparse)
    assert s.format == STL.StickFormat.Sparse


def test_str_golden():
    g = golden("spyre_tensor_layout")["str"]
    assert str(STL(g["host_size"], torch.float16)) == g["text"]


@pytest.mark.parametrize("dtype,eb", [(torch.float16, 2), (torch.float32, 4), (torch.int8, 1),
                                      (torch.bfloat16, 2), (torch.int64, 8)])
def test_matches_oracle_restatement(dtype, eb):
    for shape in ([1], [63], [65], [3, 7], [130, 5], [2, 3, 129], [4, 1, 5, 300]):
        for order in itertools.permutations(range(len(shape))):
            stl = STL(list(shape), dtype, list(order))
            ds, dst, dm = L.stl_init(list(shape), eb, list(order))
            assert (stl.device_size, stl.device_strides, stl.dim_map) == (ds, dst, dm), \
                (shape, order, dtype)


def test_rejects_bad_dim_order():
    with pytest.raises(RuntimeError):
        STL([4, 5], torch.float16, [0, 0])


def test_stick_alloc_rule_matches_oracle():
    from torch_spyre import _C

    for shape in ([2], [128], [129], [512, 4096], [3, 65], [2, 3, 1]):
        for eb in (1, 2, 4):
            assert _C.stick_alloc_nbytes(shape, eb) == L.alloc_nbytes(shape, eb)
    assert _C.stick_alloc_nbytes([], 2) == 128
