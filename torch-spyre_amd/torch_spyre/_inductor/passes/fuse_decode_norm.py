"""Post-grad passes for decode-shaped graphs (at most 8 token rows): an
RMSNorm becomes the prologue of the projections that read it, and a
residual add becomes the epilogue of the projection that feeds it.

Reference: the reference runs RMSNorm as its composite ops (pow / mean /
add / rsqrt / mul, codegen/Metadata.yaml:236-253), each projection as
spyre__mm_default (codegen/inputs/spyre_torch_ops.cpp:214-293) and the
residual add as a generated pointwise op, and forbids fusion across them
(torch_spyre/_inductor/choices.py:58-83).  In a decode step every one of
those is a separate launch over a few KB of activations, so here:

fuse_decode_norm rewrites

    c = convert(h, f32)                     # h [..., K] fp16 / bf16
    r = rsqrt(add(mean(pow(c, 2), [-1], keepdim), eps))
    y = convert(mul(mul(c, r), w), dtype)   # w [K]; either operand order
    x = reshape(y, [M, K])                  # optional
    mm(x, permute(W, [1, 0]))  /  spyre.swiglu_mm(x, W)

into spyre.rms_norm_mm(reshape(h, [M, K]), w, eps, W, swiglu) for every
projection reading y (all of y's readers must be such projections), when
M <= 8, K % 8 == 0 and 64 <= K <= 8192: the weight-stream kernel stages
x * w into LDS and scales its sums by the rows' 1 / rms(x).

fuse_residual rewrites

    add(h, reshape(mm(x, permute(W, [1, 0])), shape))   # either order

into reshape(addmm(reshape(h, [M, N]), x, permute(W, [1, 0])), shape) for
M <= 8 and h of the add's own shape and dtype: the GEMM's epilogue adds the
residual to its float32 sums.
"""

from __future__ import annotations

from typing import Optional

import torch

from .fuse_attention import _is, _only_users, _val

aten = torch.ops.aten
prims = torch.ops.prims

MAX_ROWS, MAX_K = 8, 8192
_HALF = (torch.float16, torch.bfloat16)


def _strip_reshape(n):
    if _is(n, aten.reshape.default) or _is(n, aten.view.default):
        return n.args[0], n
    return n, None


def _scalar(n) -> Optional[float]:
    return float(n) if isinstance(n, (int, float)) and not isinstance(n, bool) else None


def _norm_chain(y: torch.fx.Node) -> Optional[tuple]:
    """(h, w, eps, nodes) of the RMSNorm chain producing y, or None."""
    if not (_is(y, prims.convert_element_type.default) and y.args[1] in _HALF):
        return None
    m1 = y.args[0]
    if not _is(m1, aten.mul.Tensor):
        return None
    for m, w in ((m1.args[0], m1.args[1]), (m1.args[1], m1.args[0])):
        if not _is(m, aten.mul.Tensor):
            continue
        for c, r in ((m.args[0], m.args[1]), (m.args[1], m.args[0])):
            if not (_is(r, aten.rsqrt.default) and
                    _is(c, prims.convert_element_type.default) and c.args[1] == torch.float32):
                continue
            a = r.args[0]
            if not _is(a, aten.add.Scalar) and not _is(a, aten.add.Tensor):
                continue
            mn, eps = a.args[0], _scalar(a.args[1])
            if eps is None or not _is(mn, aten.mean.dim):
                continue
            p = mn.args[0]
            keep = (mn.args[2] if len(mn.args) > 2 else mn.kwargs.get("keepdim", False))
            if not (_is(p, aten.pow.Tensor_Scalar) and p.args[0] is c and p.args[1] == 2 and keep):
                continue
            h = c.args[0]
            hv, wv = _val(h), _val(w)
            if hv is None or wv is None or hv.dim() < 1:
                continue
            if list(mn.args[1]) not in ([-1], [hv.dim() - 1]):
                continue
            if hv.dtype != y.args[1] or wv.dtype != hv.dtype or wv.dim() != 1:
                continue
            if wv.shape[0] != hv.shape[-1]:
                continue
            return h, w, eps, [y, m1, m, r, a, mn, p, c]
    return None


def _projection(u: torch.fx.Node, x: torch.fx.Node) -> Optional[tuple]:
    """(weight, swiglu) when u projects x by an nn.Linear weight."""
    if _is(u, aten.mm.default) and u.args[0] is x:
        wt = u.args[1]
        if _is(wt, aten.permute.default) and list(wt.args[1]) == [1, 0]:
            return wt.args[0], False, wt
        return None
    if _is(u, torch.ops.spyre.swiglu_mm.default) and u.args[0] is x:
        return u.args[1], True, None
    return None


def fuse_decode_norm(gm: torch.fx.GraphModule) -> int:
    """Folds every matching RMSNorm into its projections; returns how many
    projections were rewritten."""
    g = gm.graph
    count = 0
    for y in list(g.nodes):
        if y.graph is not g or not _is(y, prims.convert_element_type.default):
            continue
        chain = _norm_chain(y)
        if chain is None:
            continue
        h, w, eps, nodes = chain
        if not all(_only_users(nd, set(nodes)) for nd in nodes[1:]):
            continue
        hv = _val(h)
        K = hv.shape[-1]
        M = 1
        for d in hv.shape[:-1]:
            M *= d
        if not (isinstance(K, int) and isinstance(M, int)):
            continue
        if not (1 <= M <= MAX_ROWS and K % 8 == 0 and 64 <= K <= MAX_K):
            continue
        # y feeds the projections directly or through one reshape to [M, K]
        readers = list(y.users)
        view = None
        if len(readers) == 1:
            base, v2 = _strip_reshape(readers[0])
            if v2 is not None and base is y:
                view = v2
        x = view if view is not None else y
        if _val(x) is None or list(_val(x).shape) != [M, K]:
            continue
        projs = [_projection(u, x) for u in x.users]
        if not projs or any(pr is None for pr in projs):
            continue
        if any(_val(W) is None or _val(W).dim() != 2 or _val(W).shape[1] != K or
               _val(W).dtype != hv.dtype for W, _, _ in projs):
            continue
        with g.inserting_before(y):
            h2 = h
            if hv.dim() != 2:
                h2 = g.call_function(aten.reshape.default, (h, [M, K]))
                h2.meta["val"] = hv.reshape(M, K)
        for u, (W, swiglu, wt) in zip(list(x.users), projs):
            with g.inserting_before(u):
                new = g.call_function(torch.ops.spyre.rms_norm_mm.default,
                                      (h2, w, eps, W, swiglu))
                new.meta["val"] = torch.ops.spyre.rms_norm_mm.default(_val(h2), _val(w), eps,
                                                                      _val(W), swiglu)
            u.replace_all_uses_with(new)
            g.erase_node(u)
            if wt is not None and not wt.users:
                g.erase_node(wt)
            count += 1
        for nd in ([view] if view is not None else []) + nodes:
            if not nd.users:
                g.erase_node(nd)
    if count:
        g.lint()
        gm.recompile()
    return count


def _residual_match(add: torch.fx.Node) -> Optional[tuple]:
    if len(add.args) != 2 or add.kwargs.get("alpha", 1) != 1:
        return None
    av = _val(add)
    if av is None or av.dtype not in _HALF:
        return None
    for h, v in ((add.args[0], add.args[1]), (add.args[1], add.args[0])):
        mm, view = _strip_reshape(v)
        if not _is(mm, aten.mm.default):
            continue
        x, wt = mm.args
        if not (_is(wt, aten.permute.default) and list(wt.args[1]) == [1, 0]):
            continue
        hv, mv = _val(h), _val(mm)
        if hv is None or mv is None or tuple(hv.shape) != tuple(av.shape):
            continue
        if hv.dtype != av.dtype or mv.dtype != av.dtype:
            continue
        M, N = mv.shape
        if not (isinstance(M, int) and 1 <= M <= MAX_ROWS) or hv.numel() != M * N:
            continue
        inside = {add} | ({view} if view is not None else set())
        if not _only_users(mm, inside if view is None else {view}):
            continue
        if view is not None and not _only_users(view, {add}):
            continue
        return h, x, wt, mm, view
    return None


def fuse_residual(gm: torch.fx.GraphModule) -> int:
    """Folds every matching residual add into its projection's epilogue;
    returns how many."""
    g = gm.graph
    count = 0
    for add in list(g.nodes):
        if add.graph is not g or not _is(add, aten.add.Tensor):
            continue
        m = _residual_match(add)
        if m is None:
            continue
        h, x, wt, mm, view = m
        hv, mv = _val(h), _val(mm)
        shape = list(_val(add).shape)
        with g.inserting_before(add):
            c = h
            if hv.dim() != 2 or tuple(hv.shape) != tuple(mv.shape):
                c = g.call_function(aten.reshape.default, (h, list(mv.shape)))
                c.meta["val"] = hv.reshape(mv.shape)
            new = g.call_function(aten.addmm.default, (c, x, wt))
            new.meta["val"] = mv.new_empty(mv.shape)
            res = new
            if shape != list(mv.shape):
                res = g.call_function(aten.reshape.default, (new, shape))
                res.meta["val"] = _val(add).new_empty(shape)
        add.replace_all_uses_with(res)
        g.erase_node(add)
        if view is not None:
            g.erase_node(view)
        g.erase_node(mm)
        count += 1
    if count:
        g.lint()
        gm.recompile()
    return count


def _file() -> str:
    return __file__


fuse_decode_norm.file = _file  # the pass hook hashes this file into its cache key
fuse_residual.file = _file
