"""Graph-pass hook of the spyre backend.

Reference: torch_spyre/_inductor/passes/__init__.py:26-49, which installs a
pre-grad list containing RemoveElementTypeConversions (every
`convert_element_type` deleted, "all device ops are fp16") into Inductor's
global config.  Here the passes run through the per-device custom pass of
`register_backend_for_device`, i.e. only on post-grad graphs that hold spyre
tensors, and no conversion is removed: kernels upcast to fp32 internally, so
the conversions Inductor sees are the ones the program asked for.  The list
holds the attention fusion (bmm -> softmax -> bmm as one fused kernel,
fuse_attention.py), the SwiGLU projection fusion (x W^T -> silu(gate) *
up as one GEMM, fuse_swiglu.py), for decode steps RMSNorm folded into the
projections that read it and residual adds into the projections that feed
them (fuse_decode_norm.py), and transposing copies as one tiled transpose
(fuse_transpose.py); a pass is any callable taking the GraphModule.
"""

from __future__ import annotations

import os
from typing import Any, Callable, List, Optional

import torch
from torch._inductor.custom_graph_pass import CustomGraphModulePass, get_hash_for_files

from .fuse_attention import fuse_attention
from .fuse_decode_norm import fuse_decode_norm, fuse_residual
from .fuse_swiglu import fuse_swiglu
from .fuse_transpose import fuse_transpose

custom_post_passes: List[Callable[[torch.fx.GraphModule], None]] = [
    fuse_attention, fuse_swiglu, fuse_decode_norm, fuse_residual, fuse_transpose]


class CustomPostPasses(CustomGraphModulePass):
    def __call__(self, gm: torch.fx.GraphModule) -> None:
        for p in custom_post_passes:
            p(gm)

    def uuid(self) -> Optional[Any]:
        # Inductor keys its compiled-graph cache on this value: it covers
        # every source of the backend (passes, scheduling, the kernel
        # generator, lowerings, the device runtime header), so a cached
        # graph is never reused after any of them changes.
        inductor_dir = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
        files = {__file__}
        for root, _, names in os.walk(inductor_dir):
            for n in names:
                if n.endswith((".py", ".h")):
                    files.add(os.path.join(root, n))
        for p in custom_post_passes:
            f = getattr(p, "file", None)
            if callable(f):
                files.add(f())
        names = tuple(getattr(p, "__module__", "") + "." + getattr(p, "__qualname__", repr(p))
                      for p in custom_post_passes)
        return (get_hash_for_files(tuple(sorted(files))), names)
