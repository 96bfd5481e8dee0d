"""Post-grad pass: the gate/up projection of a SwiGLU MLP and its
activation product become one `torch.ops.spyre.swiglu_mm` call.

Reference: the reference runs x W^T (spyre__mm_default,
codegen/inputs/spyre_torch_ops.cpp:214-293) and the generated silu and mul
ops separately and forbids fusion (torch_spyre/_inductor/choices.py:58-83).
Here, on spyre graphs, the chain

    gu = mm(x, permute(w, [1, 0]))          # w [2n, K], gate rows first
    v  = reshape(gu, [..., 2n])             # optional
    g  = convert(slice(v, -1, 0, n), f32)
    s  = convert(mul(g, sigmoid(g)), f16)   # silu, as Inductor decomposes it
    y  = mul(s, slice(v, -1, n, 2n))        # either operand order

is replaced by swiglu_mm(x, w) (reshaped like y) when a fused kernel takes
the shape (fp16 / bf16; M % 256 == 0, n % 128 == 0, K % 64 == 0 for the
tiled GEMM of prefill, or M <= 8 with K % 8 == 0 and 64 <= K <= 8192 for
the weight-stream kernel of decode) and no intermediate is used elsewhere:
the [M, 2n] projection is then never written to HBM.
"""

from __future__ import annotations

from typing import Optional

import torch

from .fuse_attention import _is, _only_users, _val

aten = torch.ops.aten
prims = torch.ops.prims

ROW_BLOCK, COL_BLOCK, K_BLOCK = 256, 128, 64  # tiled GEMM (prefill)
STREAM_ROWS, STREAM_K = 8, 8192               # weight-stream kernel (decode)
_BIG = 2 ** 62


def _last(dim, ndim) -> bool:
    return dim in (-1, ndim - 1)


def _slice(node, v, ndim) -> Optional[tuple]:
    """(start, end) of slice(v, last dim, start, end) or None."""
    if not _is(node, aten.slice.Tensor) or node.args[0] is not v:
        return None
    args = list(node.args) + [None] * (5 - len(node.args))
    dim, start, end, step = args[1], args[2], args[3], args[4]
    if not _last(dim if dim is not None else 0, ndim) or (step not in (None, 1)):
        return None
    return (start or 0, end if end is not None else _BIG)


def _match(y: torch.fx.Node) -> Optional[tuple]:
    a, b = y.args[0], y.args[1]
    for s16, up in ((a, b), (b, a)):
        if not _is(s16, prims.convert_element_type.default):
            continue
        silu = s16.args[0]
        if not _is(silu, aten.mul.Tensor):
            continue
        p, q = silu.args
        g, sg = (p, q) if _is(q, aten.sigmoid.default) else (q, p)
        if not (_is(sg, aten.sigmoid.default) and sg.args[0] is g and
                _is(g, prims.convert_element_type.default) and g.args[1] == torch.float32):
            continue
        gate = g.args[0]
        if not (_is(gate, aten.slice.Tensor) and _is(up, aten.slice.Tensor)):
            continue
        v = gate.args[0]
        if up.args[0] is not v:
            continue
        vv = _val(v)
        if vv is None:
            continue
        ndim = vv.dim()
        gs, us = _slice(gate, v, ndim), _slice(up, v, ndim)
        if gs is None or us is None:
            continue
        two_n = vv.shape[-1]
        if not isinstance(two_n, int) or two_n % 2:
            continue
        n = two_n // 2
        if gs != (0, n) or us[0] != n or min(us[1], two_n) != two_n:
            continue
        mm, view = (v.args[0], v) if _is(v, aten.reshape.default) or _is(v, aten.view.default) else (v, None)
        if not _is(mm, aten.mm.default):
            continue
        x, wt = mm.args
        if not (_is(wt, aten.permute.default) and list(wt.args[1]) == [1, 0]):
            continue
        w = wt.args[0]
        chain = [y, s16, silu, sg, g, gate, up] + ([view] if view is not None else []) + [mm]
        inside = set(chain)
        if not all(_only_users(nd, inside) for nd in chain[1:]):
            continue
        xv, wv, yv = _val(x), _val(w), _val(y)
        if xv is None or wv is None or yv is None:
            continue
        dt = xv.dtype
        if dt not in (torch.float16, torch.bfloat16) or wv.dtype != dt or s16.args[1] != dt:
            continue
        if xv.dim() != 2 or wv.dim() != 2 or yv.dtype != dt:
            continue
        M, K = xv.shape
        if not all(isinstance(t, int) for t in (M, K)) or tuple(wv.shape) != (2 * n, K):
            continue
        tiles = M % ROW_BLOCK == 0 and n % COL_BLOCK == 0 and K % K_BLOCK == 0
        stream = M <= STREAM_ROWS and K % 8 == 0 and 64 <= K <= STREAM_K
        if not (tiles or stream):
            continue
        return x, w, chain
    return None


def fuse_swiglu(gm: torch.fx.GraphModule) -> int:
    """Rewrites every matching chain in `gm`; returns how many."""
    g = gm.graph
    count = 0
    for node in list(g.nodes):
        if not _is(node, aten.mul.Tensor) or node.graph is not g:
            continue
        m = _match(node)
        if m is None:
            continue
        x, w, chain = m
        out_shape = list(_val(node).shape)
        with g.inserting_before(node):
            new = g.call_function(torch.ops.spyre.swiglu_mm.default, (x, w))
            new.meta["val"] = torch.ops.spyre.swiglu_mm.default(_val(x), _val(w))
            res = new
            if len(out_shape) != 2:
                res = g.call_function(aten.reshape.default, (new, out_shape))
                res.meta["val"] = _val(node).new_empty(out_shape)
        node.replace_all_uses_with(res)
        for n in chain:
            if not n.users:
                g.erase_node(n)
        count += 1
    if count:
        g.lint()
        gm.recompile()
    return count


def _file() -> str:
    return __file__


fuse_swiglu.file = _file  # the pass hook hashes this file into its cache key
