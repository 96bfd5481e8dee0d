"""ctypes binding of the C-ABI kernel library (include/spyre_hip.h).

This is the thinnest host-side caller of the boundary: the compiled-kernel
runners, the benchmarks and the C-ABI parity tests use it; the eager ATen
kernels call the same entry points from C++ (torch_spyre/_C).  Loading fails
loudly when the library has not been built: there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libspyre_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "spyre_hip.h")

# sph_dtype codes
F16, BF16, F32, F64, I8, U8, I16, I32, I64, BOOL = range(10)
MAX_DIMS = 8

# epilogues / flags (mirrors of the header's enums)
EPI_NONE, EPI_RELU, EPI_GELU, EPI_SILU = 0, 1, 2, 3
SOFTMAX_LOG, SOFTMAX_CAUSAL = 1, 2

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_f32 = ctypes.c_float
c_f64 = ctypes.c_double
vp = ctypes.c_void_p


class Operand(ctypes.Structure):
    _fields_ = [("data", vp), ("dtype", ctypes.c_int32), ("pad_", ctypes.c_int32),
                ("strides", c_i64 * MAX_DIMS)]


_SIGS = {
    "sph_last_error": ([], ctypes.c_char_p),
    "sph_abi_version": ([], c_int),
    "sph_softmax_rows": ([c_int, c_int, vp, c_i64, vp, c_i64, c_i64, c_i64, c_f32, c_int,
                          c_i64, c_i64, vp], c_int),
    "sph_softmax_rows_f16": ([vp, vp, c_i64, c_i64, vp], c_int),
    "sph_rmsnorm": ([c_int, c_int, vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_f32, vp], c_int),
    "sph_layernorm": ([c_int, c_int, vp, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_f32,
                       vp], c_int),
    "sph_rmsnorm_f16": ([vp, vp, vp, vp, vp, c_i64, c_i64, c_f32, vp], c_int),
    "sph_layernorm_f16": ([vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_f32, vp], c_int),
    "sph_gelu_affine_rowsum": ([c_int, vp, vp, vp, c_f32, c_f32, vp, vp, c_i64, c_i64, vp],
                               c_int),
    "sph_gelu_affine_rowsum_f16": ([vp, vp, vp, vp, vp, c_i64, c_i64, vp], c_int),
    "sph_gemm": ([c_int, c_int, c_int, c_i64, c_i64, c_i64, c_f32, vp, c_i64, vp, c_i64,
                  c_f32, vp, c_i64, c_i64, vp, c_i64, c_int, vp], c_int),
    "sph_gemm_strided_batched": ([c_int, c_int, c_int, c_i64, c_i64, c_i64, c_i64, c_f32, vp,
                                  c_i64, c_i64, vp, c_i64, c_i64, c_f32, vp, c_i64, c_i64,
                                  c_i64, vp, c_i64, c_i64, c_int, vp], c_int),
    "sph_gemm_swiglu": ([c_int, c_i64, c_i64, c_i64, vp, c_i64, vp, c_i64, vp, c_i64, vp, c_i64,
                         vp], c_int),
    "sph_gemm_swiglu_workspace_bytes": ([c_i64, c_i64, c_i64], c_i64),
    "sph_gemm_ex": ([c_int, c_int, c_int, c_i64, c_i64, c_i64, c_i64, c_f32, vp, c_i64, c_i64, vp,
                     c_i64, c_i64, c_f32, vp, c_i64, c_i64, c_i64, vp, c_i64, c_i64, c_int, vp,
                     c_i64, vp], c_int),
    "sph_gemm_workspace_bytes": ([c_i64, c_i64, c_i64, c_i64], c_i64),
    "sph_gemm_rmsnorm": ([c_int, c_i64, c_i64, c_i64, vp, c_i64, vp, c_f32, vp, c_i64, vp, c_i64,
                          c_int, vp], c_int),
    "sph_gemm_f16": ([c_i64, c_i64, c_i64, vp, vp, vp, vp], c_int),
    "sph_bmm_f16": ([c_i64, c_i64, c_i64, c_i64, vp, vp, vp, vp], c_int),
    "sph_attention_fwd": ([c_int, c_i64, c_i64, c_i64, c_i64, vp, c_i64, c_i64, vp, c_i64,
                           c_i64, vp, c_i64, c_i64, vp, c_i64, c_i64, c_i64, c_i64, c_f32, vp,
                           c_i64, c_i64, vp, c_i64, vp], c_int),
    "sph_attention_workspace_bytes": ([c_i64, c_i64, c_i64, c_i64], c_i64),
    "sph_attention_decode": ([c_int, c_i64, c_i64, c_i64, c_i64, vp, c_i64, c_i64, vp, c_i64,
                              c_i64, vp, c_i64, c_i64, c_i64, vp, c_i64, c_i64, c_i64, c_i64,
                              c_f32, vp, c_i64, c_i64, vp, c_i64, vp], c_int),
    "sph_attention_decode_workspace_bytes": ([c_i64, c_i64, c_i64], c_i64),
    "sph_decode_attention_step": ([c_int, c_i64, c_i64, c_i64, c_i64, vp, c_i64, vp, vp, c_i64,
                                   vp, vp, vp, c_i64, c_i64, c_i64, vp, c_i64, c_i64, c_i64,
                                   c_i64, c_i64, c_f32, vp, c_i64, vp, c_i64, vp], c_int),
    "sph_decode_attention_step_workspace_bytes": ([c_i64, c_i64, c_i64, c_i64], c_i64),
    "sph_attention_fwd_noalloc": ([c_int, c_i64, c_i64, c_i64, c_i64, vp, c_i64, c_i64, vp,
                                   c_i64, c_i64, vp, c_i64, c_i64, vp, c_i64, c_i64, c_i64, c_i64,
                                   c_f32, vp, c_i64, c_i64, vp], c_int),
    "sph_attention_fwd_noalloc_max_bytes": ([], c_i64),
    "sph_arange": ([c_int, c_f64, c_f64, c_i64, c_i64, c_i64, vp, vp], c_int),
    "sph_cumsum": ([c_int, vp, vp, c_i64, c_i64, c_i64, vp], c_int),
    "sph_random_fill": ([c_int, c_int, vp, c_i64, ctypes.c_uint64, ctypes.c_uint64, c_f64, c_f64,
                         c_i64, ctypes.c_uint64, vp], c_int),
    "sph_random_blocks": ([c_int, c_int, c_i64, ctypes.c_uint64], c_i64),
    "sph_transpose_copy": ([c_int, vp, vp, c_i64, c_i64, c_i64, c_i64, c_int, vp, vp, vp, vp],
                           c_int),
    "sph_dropout": ([c_int, vp, vp, vp, c_i64, c_f32, c_f32, ctypes.c_uint64, ctypes.c_uint64,
                     vp], c_int),
    "sph_pointwise": ([c_int, c_int, ctypes.POINTER(Operand), c_int, ctypes.POINTER(c_i64),
                       c_f64, c_f64, vp], c_int),
    "sph_reduce": ([c_int, ctypes.POINTER(Operand), ctypes.POINTER(Operand), c_int,
                    ctypes.POINTER(c_i64), ctypes.c_uint32, vp], c_int),
    "sph_gather_rows": ([vp, c_i64, c_i64, c_int, vp, c_int, c_i64, vp, vp, vp], c_int),
    "sph_tri": ([c_int, c_i64, c_int, vp, vp, c_i64, c_i64, c_i64, vp], c_int),
    "sph_rope": ([c_int, vp, vp, vp, c_i64, c_i64, c_i64, c_f32, vp], c_int),
    "sph_stick_nbytes": ([c_int, ctypes.POINTER(c_i64), ctypes.POINTER(ctypes.c_int32), c_int],
                         c_i64),
    "sph_stick_pack": ([vp, vp, c_int, ctypes.POINTER(c_i64), ctypes.POINTER(c_i64),
                        ctypes.POINTER(ctypes.c_int32), c_int, vp], c_int),
    "sph_stick_unpack": ([vp, vp, c_int, ctypes.POINTER(c_i64), ctypes.POINTER(c_i64),
                          ctypes.POINTER(ctypes.c_int32), c_int, vp], c_int),
}

_lib = None


def lib():
    """The loaded kernel library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"torch_spyre: kernel library {LIB_PATH} is missing; build it with "
                "`python torch-spyre_amd/build.py` (there is no non-HIP fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def header_functions() -> list[str]:
    """Names of every function declared in include/spyre_hip.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sph_[a-z0-9_]+)\s*\(", text)))


class SpyreKernelError(RuntimeError):
    pass


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().sph_last_error().decode(errors="replace")
        raise SpyreKernelError(f"{what} failed (status {rc}): {msg}")


def call(name: str, *args) -> None:
    """Calls entry point `name` and raises on a non-zero status."""
    check(getattr(lib(), name)(*args), name)


def torch_dtype_code(dtype) -> int:
    import torch

    table = {
        torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32, torch.float64: F64,
        torch.int8: I8, torch.uint8: U8, torch.int16: I16, torch.int32: I32,
        torch.int64: I64, torch.bool: BOOL,
    }
    try:
        return table[dtype]
    except KeyError:
        raise TypeError(f"torch_spyre: dtype {dtype} is not supported by the kernel library")


def i64_array(vals):
    vals = list(vals)
    return (c_i64 * max(1, len(vals)))(*vals)


def i32_array(vals):
    vals = list(vals)
    return (ctypes.c_int32 * max(1, len(vals)))(*vals)


def operand(ptr: int, dtype_code: int, strides) -> Operand:
    op = Operand()
    op.data = ptr
    op.dtype = dtype_code
    st = list(strides) + [0] * (MAX_DIMS - len(strides))
    for i in range(MAX_DIMS):
        op.strides[i] = st[i]
    return op
