"""Post-grad pass: a contiguous copy of a permuted tensor that moves its
innermost dimension becomes one `torch.ops.spyre.transpose_copy` call.

Reference: the reference lowers such copies (`x.t().contiguous()`,
`transpose(x, 0, 2).contiguous()`) to its "transpose"/"restickify" data ops
(torch_spyre/_inductor/codegen/data_ops.py:16-630, classified by
spyre_kernel.py:301-311).  Inductor would otherwise emit an elementwise copy
that reads (or writes) one element per 64-byte run; the custom op runs an
LDS-tiled transpose (sph_transpose_copy) whose reads and writes are both
coalesced.  Replaced, for a chain of permutes of x whose composed dims move
the innermost dimension (dims[-1] not x's last) and a static shape:
  * `clone(permute(...), contiguous)` -> `transpose_copy(x, dims)`;
  * the source of `copy(dst, permute(...))` (a permuted tensor written into
    a view, e.g. a transposed slice of a KV cache) -> `transpose_copy(x,
    dims)`, so the copy that remains moves rows along the same dimension on
    both sides.
A permutation that keeps the innermost dimension is already a coalesced copy
and stays with Inductor.
"""

from __future__ import annotations

import torch

from .fuse_attention import _is, _val

aten = torch.ops.aten


def _permute_chain(node):
    """(x, dims) with node == x.permute(dims) for a chain of permutes, or None."""
    dims = None
    while _is(node, aten.permute.default):
        x, d = node.args
        if not isinstance(d, (list, tuple)):
            return None
        nd = len(d)
        d = [i % nd for i in d]
        dims = d if dims is None else [d[i] for i in dims]
        node = x
    return None if dims is None else (node, dims)


def _moves_innermost(x, dims) -> bool:
    xv = _val(x)
    nd = len(dims)
    return (xv is not None and nd >= 2 and dims[-1] != nd - 1 and xv.dim() == nd and
            all(isinstance(s, int) for s in xv.shape))


def _drop_dead_permutes(g, node) -> None:
    while _is(node, aten.permute.default) and not node.users:
        x = node.args[0]
        g.erase_node(node)
        node = x


def fuse_transpose(gm: torch.fx.GraphModule) -> int:
    g = gm.graph
    n = 0
    for node in list(g.nodes):
        if _is(node, aten.clone.default):
            # A clone without a memory format preserves the permuted strides
            # (preserve_format): only a clone whose result is contiguous is a
            # transposing copy.
            mf = node.kwargs.get("memory_format", None)
            out = _val(node)
            if mf not in (None, torch.contiguous_format) or out is None:
                continue
            if mf is None and not out.is_contiguous():
                continue
            chain = _permute_chain(node.args[0])
            if chain is None or not _moves_innermost(*chain):
                continue
            src = node.args[0]
            with g.inserting_before(node):
                new = g.call_function(torch.ops.spyre.transpose_copy.default,
                                      (chain[0], list(chain[1])))
            new.meta.update(node.meta)
            node.replace_all_uses_with(new)
            g.erase_node(node)
            _drop_dead_permutes(g, src)
            n += 1
        elif _is(node, aten.copy.default) and len(node.args) >= 2:
            src = node.args[1]
            chain = _permute_chain(src)
            if chain is None or not _moves_innermost(*chain) or _val(src) is None:
                continue
            with g.inserting_before(node):
                new = g.call_function(torch.ops.spyre.transpose_copy.default,
                                      (chain[0], list(chain[1])))
            new.meta["val"] = _val(src).contiguous()
            node.replace_input_with(src, new)
            _drop_dead_permutes(g, src)
            n += 1
    if n:
        g.lint()
        gm.recompile()
    return n


def _file() -> str:
    return __file__


fuse_transpose.file = _file  # the pass hook hashes this file into its cache key
