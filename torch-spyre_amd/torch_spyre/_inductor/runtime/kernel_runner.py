"""Runners the generated wrapper code calls: `kernel.run(*buffers)`
(reference: torch_spyre/_inductor/runtime/kernel_runner.py:19-40).

A runner holds a hiprtc code object loaded into torch_spyre._C and launches
it with torch_spyre._C.launch_kernel on the spyre stream of the arguments'
device; no compilation happens per call (the reference reloads and
recompiles its program on every call, torch_spyre/csrc/module.cpp:64-170).
"""

from __future__ import annotations

from typing import Optional

from . import KernelSpec

# the symbol of a kernel whose KernelSpec names none
KERNEL_SYMBOL = "spyre_kernel"


def launch_extents(spec: KernelSpec) -> list[int]:
    return [a.extent if a.extent is not None else -1 for a in spec.args]


def launch_description(spec: KernelSpec) -> str:
    """The `.launch` line torch_spyre._C.launch_kernel(path, args) reads:
    "<kernel name> <grid> <block> <n> <extent>*n <error word>"."""
    ext = launch_extents(spec)
    return " ".join([spec.symbol or KERNEL_SYMBOL, str(spec.grid), str(spec.block), str(len(ext)),
                     *map(str, ext), str(int(spec.error_word))]) + "\n"


class SpyreUnimplementedRunner:
    def __init__(self, name: str, op: str):
        self.kernel_name = name
        self.op = op

    def run(self, *args, **kwargs):
        raise RuntimeError(
            f"Invoked {self.kernel_name} which contains unimplemented operation {self.op}")


class SpyreHipKernelRunner:
    """`path` (optional) is the kernel's code object on disk with its launch
    description beside it (`path`.launch), for callers that launch by path
    as the reference's runner does: torch_spyre._C.launch_kernel(path, args)."""

    def __init__(self, name: str, spec: KernelSpec, code_object: bytes,
                 path: Optional[str] = None):
        from torch_spyre import _C

        self.kernel_name = name
        self.spec = spec
        self.path = path
        # extents[i] bounds argument i (-1 = not checked)
        self.extents = launch_extents(spec)
        self.handle = _C.load_kernel(code_object, spec.symbol or KERNEL_SYMBOL, spec.grid, spec.block,
                                     self.extents, spec.error_word)

    def run(self, *args, **kwargs):
        from torch_spyre import _C

        # the reference's two-argument form (torch_spyre/csrc/module.cpp:176)
        _C.launch_kernel(self.handle, list(args))
