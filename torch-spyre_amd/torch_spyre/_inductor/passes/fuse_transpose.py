"""Post-grad pass: a contiguous copy of a permuted tensor that moves its
innermost dimension becomes one `torch.ops.spyre.transpose_copy` call.

Reference: the reference lowers such copies (`x.t().contiguous()`,
`transpose(x, 0, 2).contiguous()`) to its "transpose"/"restickify" data ops
(torch_spyre/_inductor/codegen/data_ops.py:16-630, classified by
spyre_kernel.py:301-311).  Inductor would otherwise emit an elementwise copy
that reads (or writes) one element per 64-byte run; the custom op runs an
LDS-tiled transpose (sph_transpose_copy) whose reads and writes are both
coalesced.  Only `clone(permute(x, dims), contiguous)` with dims[-1] not the
last dimension and a static shape is replaced; a permutation that keeps the
innermost dimension is already a coalesced copy and stays with Inductor.
"""

from __future__ import annotations

import torch

from .fuse_attention import _is, _val

aten = torch.ops.aten


def fuse_transpose(gm: torch.fx.GraphModule) -> int:
    g = gm.graph
    n = 0
    for node in list(g.nodes):
        if not _is(node, aten.clone.default):
            continue
        mf = node.kwargs.get("memory_format", None)
        if mf not in (None, torch.contiguous_format):
            continue
        perm = node.args[0]
        if not _is(perm, aten.permute.default):
            continue
        x, dims = perm.args
        xv, ov = _val(x), _val(node)
        if xv is None or ov is None or not isinstance(dims, (list, tuple)):
            continue
        nd = len(dims)
        dims = [d % nd for d in dims]
        if nd < 2 or dims[-1] == nd - 1 or not all(isinstance(s, int) for s in xv.shape):
            continue
        with g.inserting_before(node):
            new = g.call_function(torch.ops.spyre.transpose_copy.default, (x, list(dims)))
        new.meta.update(node.meta)
        node.replace_all_uses_with(new)
        g.erase_node(node)
        if not perm.users:
            g.erase_node(perm)
        n += 1
    if n:
        g.lint()
        gm.recompile()
    return n


def _file() -> str:
    return __file__


fuse_transpose.file = _file  # the pass hook hashes this file into its cache key
