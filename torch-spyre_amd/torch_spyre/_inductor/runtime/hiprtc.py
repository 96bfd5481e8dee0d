"""Compiles generated HIP kernel sources to gfx950 code objects with hiprtc.

The reference hands each generated SuperDSC program to an external compiler
(`dxp_standalone`, torch_spyre/_inductor/runtime/async_compile.py:41-88) at
compile time.  Here hiprtc (the HIP runtime compiler shipped with the
PyTorch-ROCm wheel, the same ROCm release as the HIP runtime the process
uses) compiles the kernel in-process in well under a second; code objects
are cached on disk under Inductor's cache directory, keyed by a hash of the
source, the options and the runtime header.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
INCLUDE_DIR = os.path.join(os.path.dirname(_HERE), "include")
OFFLOAD_ARCH = os.environ.get("SPYRE_OFFLOAD_ARCH", "gfx950")
# Packed-fp32 VALU forms are kept out of generated kernels, as out of the
# library's own.
OPTIONS = [f"--offload-arch={OFFLOAD_ARCH}", "-O3", "-std=c++17", f"-I{INCLUDE_DIR}",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

_lib = None
_lock = threading.Lock()


def _load():
    global _lib
    if _lib is None:
        import torch

        cands = [os.path.join(os.path.dirname(torch.__file__), "lib", "libhiprtc.so"),
                 "/opt/rocm/lib/libhiprtc.so"]
        for c in cands:
            if os.path.exists(c):
                lib = ctypes.CDLL(c)
                break
        else:
            raise RuntimeError("torch_spyre: libhiprtc.so not found; the compile backend "
                               "needs hiprtc")
        vp = ctypes.c_void_p
        lib.hiprtcCreateProgram.argtypes = [ctypes.POINTER(vp), ctypes.c_char_p, ctypes.c_char_p,
                                            ctypes.c_int, vp, vp]
        lib.hiprtcCompileProgram.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
        lib.hiprtcGetProgramLogSize.argtypes = [vp, ctypes.POINTER(ctypes.c_size_t)]
        lib.hiprtcGetProgramLog.argtypes = [vp, ctypes.c_char_p]
        lib.hiprtcGetCodeSize.argtypes = [vp, ctypes.POINTER(ctypes.c_size_t)]
        lib.hiprtcGetCode.argtypes = [vp, ctypes.c_char_p]
        lib.hiprtcDestroyProgram.argtypes = [ctypes.POINTER(vp)]
        _lib = lib
    return _lib


def _header_digest() -> str:
    h = hashlib.sha256()
    for f in sorted(os.listdir(INCLUDE_DIR)):
        with open(os.path.join(INCLUDE_DIR, f), "rb") as fh:
            h.update(f.encode() + fh.read())
    return h.hexdigest()


def _cache_dir() -> str:
    from torch._inductor.runtime.runtime_utils import cache_dir

    d = os.path.join(cache_dir(), "spyre-hip", OFFLOAD_ARCH)
    os.makedirs(d, exist_ok=True)
    return d


class HipCompileError(RuntimeError):
    pass


def compile_source(source: str, name: str = "spyre_kernel.hip") -> bytes:
    """Returns the gfx950 code object of `source` (cached on disk)."""
    key = hashlib.sha256((source + "\0" + " ".join(OPTIONS) + "\0" + _header_digest())
                         .encode()).hexdigest()
    path = os.path.join(_cache_dir(), key + ".co")
    if os.path.exists(path):
        with open(path, "rb") as f:
            return f.read()
    lib = _load()
    with _lock:
        prog = ctypes.c_void_p()
        rc = lib.hiprtcCreateProgram(ctypes.byref(prog), source.encode(), name.encode(), 0,
                                     None, None)
        if rc != 0:
            raise HipCompileError(f"hiprtcCreateProgram failed ({rc})")
        try:
            opts = [o.encode() for o in OPTIONS]
            arr = (ctypes.c_char_p * len(opts))(*opts)
            rc = lib.hiprtcCompileProgram(prog, len(opts), arr)
            n = ctypes.c_size_t()
            lib.hiprtcGetProgramLogSize(prog, ctypes.byref(n))
            log = ctypes.create_string_buffer(max(1, n.value))
            lib.hiprtcGetProgramLog(prog, log)
            if rc != 0:
                raise HipCompileError(
                    f"hiprtc failed to compile {name} ({rc}):\n"
                    f"{log.value.decode(errors='replace')}\n--- source ---\n{source}")
            lib.hiprtcGetCodeSize(prog, ctypes.byref(n))
            code = ctypes.create_string_buffer(n.value)
            lib.hiprtcGetCode(prog, code)
            blob = code.raw[: n.value]
        finally:
            lib.hiprtcDestroyProgram(ctypes.byref(prog))
    tmp = f"{path}.{os.getpid()}.tmp"
    with open(tmp, "wb") as f:
        f.write(blob)
    os.replace(tmp, path)
    return blob


def write_launchable(code: bytes, launch_line: str) -> str:
    """Writes a code object and its launch description (`<path>.launch`)
    under the cache directory, named by their content; returns the path that
    torch_spyre._C.launch_kernel(path, args) takes."""
    key = hashlib.sha256(code + b"\0" + launch_line.encode()).hexdigest()
    d = os.path.join(_cache_dir(), "launch")
    os.makedirs(d, exist_ok=True)
    path = os.path.join(d, key + ".co")
    if not (os.path.exists(path) and os.path.exists(path + ".launch")):
        for p, blob in ((path, code), (path + ".launch", launch_line.encode())):
            tmp = f"{p}.{os.getpid()}.tmp"
            with open(tmp, "wb") as f:
                f.write(blob)
            os.replace(tmp, p)
    return path
