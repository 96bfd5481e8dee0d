"""Compile step of generated kernels (reference: SpyreAsyncCompile,
torch_spyre/_inductor/runtime/async_compile.py:41-88, which writes sdsc.json
and runs dxp_standalone).  Here the KernelSpec's HIP source is compiled by
hiprtc for gfx950 (cached on disk) and loaded into the runtime."""

from __future__ import annotations

from typing import Any, Union

from . import KernelSpec, UnimplementedOp
from .hiprtc import compile_source, write_launchable
from .kernel_runner import SpyreHipKernelRunner, SpyreUnimplementedRunner, launch_description


class SpyreAsyncCompile:
    def __init__(self) -> None:
        pass

    def hip(self, kernel_name: str, ks: Union[KernelSpec, UnimplementedOp]):
        if isinstance(ks, UnimplementedOp):
            return SpyreUnimplementedRunner(kernel_name, ks.op)
        code = compile_source(ks.source, f"{kernel_name}.hip")
        path = write_launchable(code, launch_description(ks))
        return SpyreHipKernelRunner(kernel_name, ks, code, path)

    # Name kept from the reference's wrapper code.
    sdsc = hip

    def wait(self, scope: dict[str, Any]) -> None:
        pass
