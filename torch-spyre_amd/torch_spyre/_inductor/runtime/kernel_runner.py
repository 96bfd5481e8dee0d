"""Runners the generated wrapper code calls: `kernel.run(*buffers)`
(reference: torch_spyre/_inductor/runtime/kernel_runner.py:19-40).

A runner holds a hiprtc code object loaded into torch_spyre._C and launches
it with torch_spyre._C.launch_kernel on the spyre stream of the arguments'
device; no compilation happens per call (the reference reloads and
recompiles its program on every call, torch_spyre/csrc/module.cpp:64-170).
"""

from __future__ import annotations

from . import KernelSpec


class SpyreUnimplementedRunner:
    def __init__(self, name: str, op: str):
        self.kernel_name = name
        self.op = op

    def run(self, *args, **kwargs):
        raise RuntimeError(
            f"Invoked {self.kernel_name} which contains unimplemented operation {self.op}")


class SpyreHipKernelRunner:
    def __init__(self, name: str, spec: KernelSpec, code_object: bytes):
        from torch_spyre import _C

        self.kernel_name = name
        self.spec = spec
        self.handle = _C.load_kernel(code_object, "spyre_kernel")
        # extents[i] bounds argument i (-1 = not checked)
        self.extents = [a.extent if a.extent is not None else -1 for a in spec.args]

    def run(self, *args, **kwargs):
        from torch_spyre import _C

        _C.launch_kernel(self.handle, list(args), self.spec.grid, self.spec.block, self.extents)
