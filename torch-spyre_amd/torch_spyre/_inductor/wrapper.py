"""Python wrapper codegen for the spyre device (reference:
SpyrePythonWrapperCodegen, torch_spyre/_inductor/wrapper.py:29-99).  The
generated module imports the spyre kernel runtime and defines
`async_compile` as SpyreAsyncCompile, whose `.hip(...)` compiles each
KernelSpec; buffers are allocated with empty_strided on the spyre device as
for any other device."""

from __future__ import annotations

from torch._inductor.codegen.wrapper import PythonWrapperCodegen


class SpyrePythonWrapperCodegen(PythonWrapperCodegen):
    @staticmethod
    def create(is_subgraph, subgraph_name, parent_wrapper, partition_signatures=None):
        if is_subgraph:
            return super(SpyrePythonWrapperCodegen, SpyrePythonWrapperCodegen).create(
                is_subgraph, subgraph_name, parent_wrapper, partition_signatures)
        return SpyrePythonWrapperCodegen()

    def write_header(self) -> None:
        super().write_header()
        self.imports.splice(
            """
            from torch_spyre._inductor.runtime import KernelSpec, TensorArg, UnimplementedOp
            from torch_spyre._inductor.runtime.async_compile import SpyreAsyncCompile
            """,
            strip=True,
        )
        self.header.writeline("async_compile = SpyreAsyncCompile()")
