"""ctypes front end of oracle/layout.c (stick-layout arithmetic).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

  stl_init            SpyreTensorLayout::init, torch_spyre/csrc/spyre_tensor_impl.cpp:40-74
  stl_to_string       SpyreTensorLayout::toString, spyre_tensor_impl.cpp:76-111
  alloc_nbytes        spyre_empty_strided sizing, torch_spyre/csrc/spyre_mem.cpp:598-611
                      (stick count rounded up; alloc_nbytes_reference keeps the
                      reference's one-stick padding rule, spyre_mem.cpp:109-118)
  stick_pack/unpack   the DMA stick permutation (spyre_mem.cpp:190-244) in the
                      generic stick order of SpyreTensorLayout
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

STICK_BYTES = 128


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            from . import build as _b

            _b.build()
        lib = ctypes.CDLL(_LIB_PATH)
        i64p = ctypes.POINTER(ctypes.c_int64)
        i32p = ctypes.POINTER(ctypes.c_int32)
        lib.orc_stl_init.argtypes = [ctypes.c_int, i64p, ctypes.c_int, i32p, i64p, i64p, i32p]
        lib.orc_stl_init.restype = ctypes.c_int
        lib.orc_alloc_nbytes.argtypes = [ctypes.c_int, i64p, ctypes.c_int]
        lib.orc_alloc_nbytes.restype = ctypes.c_int64
        lib.orc_alloc_nbytes_reference.argtypes = [ctypes.c_int, i64p, ctypes.c_int]
        lib.orc_alloc_nbytes_reference.restype = ctypes.c_int64
        for fn in (lib.orc_stick_pack, lib.orc_stick_unpack):
            fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, i64p, i64p, i32p,
                           ctypes.c_int]
            fn.restype = ctypes.c_int
        _lib = lib
    return _lib


def _i64(seq):
    return (ctypes.c_int64 * max(1, len(seq)))(*seq)


def _i32(seq):
    return (ctypes.c_int32 * max(1, len(seq)))(*seq)


def stl_init(host_size, elem_bytes, dim_order=None):
    """Returns (device_size, device_strides, dim_map) as lists."""
    n = len(host_size)
    if dim_order is None:
        dim_order = list(range(n))
    ds, dst, dm = _i64([0] * (n + 1)), _i64([0] * (n + 1)), _i32([0] * (n + 1))
    rc = _load().orc_stl_init(n, _i64(host_size), elem_bytes, _i32(dim_order), ds, dst, dm)
    if rc != 0:
        raise ValueError("orc_stl_init failed")
    return list(ds[: n + 1]), list(dst[: n + 1]), list(dm[: n + 1])


def stl_to_string(device_size, device_strides, dim_map, num_stick_dims=1, fmt="Dense"):
    """Text form of SpyreTensorLayout (spyre_tensor_impl.cpp:76-111)."""
    j = lambda xs: ", ".join(str(int(x)) for x in xs)  # noqa: E731
    return (f"SpyreTensorLayout(device_size=[{j(device_size)}], "
            f"device_strides=[{j(device_strides)}], dim_map =[{j(dim_map)}], "
            f"num_stick_dims={num_stick_dims}, format=\"{fmt}\")")


def alloc_nbytes(host_size, elem_bytes):
    return int(_load().orc_alloc_nbytes(len(host_size), _i64(host_size), elem_bytes))


def alloc_nbytes_reference(host_size, elem_bytes):
    return int(_load().orc_alloc_nbytes_reference(len(host_size), _i64(host_size), elem_bytes))


def stick_nbytes(host_size, elem_bytes, dim_order=None):
    ds, _, _ = stl_init(host_size, elem_bytes, dim_order)
    n = 1
    for d in ds:
        n *= d
    return n * elem_bytes


def stick_pack(host: np.ndarray, dim_order=None) -> np.ndarray:
    """Host-order array -> flat uint8 array in the stick layout."""
    n = host.ndim
    if dim_order is None:
        dim_order = list(range(n))
    eb = host.dtype.itemsize
    out = np.zeros(stick_nbytes(list(host.shape), eb, dim_order), dtype=np.uint8)
    strides = [s // eb for s in host.strides]
    rc = _load().orc_stick_pack(host.ctypes.data, out.ctypes.data, n, _i64(list(host.shape)),
                                _i64(strides), _i32(dim_order), eb)
    if rc != 0:
        raise ValueError("orc_stick_pack failed")
    return out


def stick_unpack(dev: np.ndarray, shape, dtype, dim_order=None) -> np.ndarray:
    """Flat stick-layout bytes -> contiguous host-order array."""
    n = len(shape)
    if dim_order is None:
        dim_order = list(range(n))
    out = np.zeros(shape, dtype=dtype)
    eb = out.dtype.itemsize
    strides = [s // eb for s in out.strides]
    dev = np.ascontiguousarray(dev)
    rc = _load().orc_stick_unpack(dev.ctypes.data, out.ctypes.data, n, _i64(list(shape)),
                                  _i64(strides), _i32(dim_order), eb)
    if rc != 0:
        raise ValueError("orc_stick_unpack failed")
    return out
