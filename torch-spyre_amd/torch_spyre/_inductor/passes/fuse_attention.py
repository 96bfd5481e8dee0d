"""Post-grad pass: bmm -> scale -> (+ mask) -> softmax -> bmm becomes one
`torch.ops.spyre.attention` call.

Reference: the reference has no fused attention; it runs the chain as
separate ops (spyre__bmm_default, codegen/inputs/spyre_torch_ops.cpp:297-377;
add and _softmax, codegen/inputs/Metadata.yaml:275-277) and forbids fusion
in its scheduler (torch_spyre/_inductor/choices.py:58-83).  Here the chain
is replaced, on spyre graphs only, when the fused kernel takes its shapes:
fp16 / bf16, head dim 128, query rows a multiple of 128, and a mask (if
any) of the same dtype shaped [mq, sk] or [B or 1, mq, sk], or one mask row
[sk] / [1, sk] broadcast over the rows (expanded to [mq, sk] as a view).  The fused op
computes the same function (fp32 scores and softmax, probabilities rounded
to the input dtype before the second product).

After Inductor's decompositions the softmax of a half-precision tensor
reads
    x32 = convert_element_type(pre, f32); m = amax(x32, [-1], True)
    e = exp(sub(x32, m)); p = div(e, sum(e, [-1], True))
    p16 = convert_element_type(p, f16)
which is what the matcher walks, backwards from the second bmm.  Without a
mask Inductor moves a scalar scale into the exponent instead
(softmax(x * c) = exp((x * sign - max) * |c|) / sum, x upcast first):
    X = mul(convert_element_type(bmm, f32), sign); m = amax(X, [-1], True)
    e = exp(mul(sub(X, m), |c|)); ...
which is matched too.
"""

from __future__ import annotations

import math
import numbers
from typing import Optional

import torch

aten = torch.ops.aten
prims = torch.ops.prims

HEAD_DIM = 128
ROW_BLOCK = 128


def _val(n):
    return n.meta.get("val") if isinstance(n, torch.fx.Node) else None


def _is(n, target) -> bool:
    return isinstance(n, torch.fx.Node) and n.op == "call_function" and n.target == target


def _only_users(n, users) -> bool:
    return set(n.users) <= set(users)


def _last_dim(dims, ndim) -> bool:
    return list(dims) in ([-1], [ndim - 1])


def _match(bmm2: torch.fx.Node) -> Optional[tuple]:
    """(q, k, v, mask, scale, nodes of the chain) or None."""
    p16, v = bmm2.args
    if not _is(p16, prims.convert_element_type.default) or len(p16.users) != 1:
        return None
    div = p16.args[0]
    if not _is(div, aten.div.Tensor):
        return None
    e, den = div.args
    if not (_is(e, aten.exp.default) and _is(den, aten.sum.dim_IntList) and den.args[0] is e):
        return None
    sub = e.args[0]
    inner_scale = None  # the exponent-scaled form: exp(mul(sub, c))
    expmul = None
    if _is(sub, aten.mul.Tensor) and isinstance(sub.args[1], numbers.Real) and \
            not isinstance(sub.args[1], bool) and float(sub.args[1]) > 0:
        expmul, inner_scale, sub = sub, float(sub.args[1]), sub.args[0]
    if not _is(sub, aten.sub.Tensor):
        return None
    xs, mx = sub.args
    if not (_is(mx, aten.amax.default) and mx.args[0] is xs):
        return None
    ndim = 3
    if not (_last_dim(mx.args[1], ndim) and _last_dim(den.args[1], ndim)):
        return None
    if not (len(mx.args) > 2 and mx.args[2] and len(den.args) > 2 and den.args[2]):
        return None
    if inner_scale is not None:
        return _match_exp_scaled(bmm2, p16, div, den, e, expmul, sub, mx, xs, inner_scale, v)
    x32 = xs
    if not _is(x32, prims.convert_element_type.default):
        return None
    pre = x32.args[0]
    mask = None
    if _is(pre, aten.add.Tensor):
        a, b = pre.args
        if _is(a, aten.mul.Tensor) or _is(a, aten.div.Tensor):
            scaled, mask = a, b
        elif _is(b, aten.mul.Tensor) or _is(b, aten.div.Tensor):
            scaled, mask = b, a
        else:
            return None
        if not isinstance(mask, torch.fx.Node):
            return None
    else:
        scaled = pre
    if not (_is(scaled, aten.mul.Tensor) or _is(scaled, aten.div.Tensor)):
        return None
    bmm1, c = scaled.args
    if not isinstance(c, numbers.Real) or isinstance(c, bool):
        return None
    scale = float(c) if scaled.target == aten.mul.Tensor else 1.0 / float(c)
    if not _is(bmm1, aten.bmm.default):
        return None
    chain = [p16, div, den, e, sub, mx, x32, pre, scaled]
    if mask is None:
        chain.remove(pre)
    if _val(x32) is None or _val(x32).dtype != torch.float32:
        return None
    if mask is not None and (_val(pre) is None or _val(pre).dtype != p16.args[1]):
        return None
    return _finish(bmm2, bmm1, chain, v, mask, scale)


def _match_exp_scaled(bmm2, p16, div, den, e, expmul, sub, mx, xs, c, v) -> Optional[tuple]:
    """exp(mul(sub(X, amax(X)), c)), X = mul(convert(bmm, f32), sign) or
    convert(bmm, f32): softmax(bmm * sign * c) without a mask."""
    chain = [p16, div, den, e, expmul, sub, mx, xs]
    sign = 1.0
    x32 = xs
    if _is(xs, aten.mul.Tensor):
        sg = xs.args[1]
        if not isinstance(sg, numbers.Real) or isinstance(sg, bool) or float(sg) not in (1.0, -1.0):
            return None
        sign, x32 = float(sg), xs.args[0]
        chain.append(x32)
    if not _is(x32, prims.convert_element_type.default) or x32.args[1] != torch.float32:
        return None
    bmm1 = x32.args[0]
    if not _is(bmm1, aten.bmm.default):
        return None
    return _finish(bmm2, bmm1, chain, v, None, sign * c)


def _finish(bmm2, bmm1, chain, v, mask, scale) -> Optional[tuple]:
    """Operand, use and shape checks shared by both forms."""
    p16 = chain[0]
    if not _is(bmm1, aten.bmm.default):
        return None
    # The kernel folds the scale into exp2 after taking the row max, which
    # holds for positive finite scales only (a negative sign form or a
    # multiplication by a negative constant stays on the unfused chain).
    if not (math.isfinite(scale) and scale > 0):
        return None
    q, kt = bmm1.args
    if not (_is(kt, aten.permute.default) and list(kt.args[1]) == [0, 2, 1]):
        return None
    k = kt.args[0]
    chain = chain + [bmm1]
    # every intermediate feeds only the chain
    inside = set(chain) | {bmm2}
    for n in chain:
        if not _only_users(n, inside):
            return None
    # shapes and dtypes the fused kernel takes
    qv, kv, vv, ov = _val(q), _val(k), _val(v), _val(bmm2)
    if any(t is None for t in (qv, kv, vv, ov)):
        return None
    dt = qv.dtype
    if dt not in (torch.float16, torch.bfloat16) or kv.dtype != dt or vv.dtype != dt:
        return None
    if p16.args[1] != dt:
        return None
    if qv.dim() != 3 or kv.dim() != 3 or vv.dim() != 3:
        return None
    B, mq, d = qv.shape
    sk = kv.shape[1]
    if not all(isinstance(x, int) for x in (B, mq, d, sk)):
        return None  # dynamic shapes stay unfused
    # Decode shapes (a few rows per KV head) stay on the unfused chain: the
    # fused decode kernel (sph_attention_decode) measured slower than it in
    # the c5 decode step (4.77 against 4.65 ms per step).
    if d != HEAD_DIM or mq % ROW_BLOCK or tuple(kv.shape) != (B, sk, d) or \
            tuple(vv.shape) != (B, sk, d):
        return None
    expand = None
    if mask is not None:
        mv = _val(mask)
        if mv is None or mv.dtype != dt:
            return None
        shp = tuple(mv.shape)
        if shp in ((sk,), (1, sk)):
            expand = [mq, sk]
        elif not (shp == (mq, sk) or (len(shp) == 3 and shp[0] in (1, B) and shp[1:] == (mq, sk))):
            return None
    return q, k, v, mask, scale, chain, expand


def fuse_attention(gm: torch.fx.GraphModule) -> int:
    """Rewrites every matching chain in `gm`; returns how many."""
    g = gm.graph
    n_fused = 0
    for node in list(g.nodes):
        if not _is(node, aten.bmm.default):
            continue
        m = _match(node)
        if m is None:
            continue
        q, k, v, mask, scale, chain, expand = m
        with g.inserting_before(node):
            if expand is not None:  # one mask row for every query row
                mask = g.call_function(aten.expand.default, (mask, expand))
                mask.meta["val"] = _val(m[3]).expand(expand)
            new = g.call_function(torch.ops.spyre.attention.default, (q, k, v, mask, scale))
        new.meta.update(node.meta)
        node.replace_all_uses_with(new)
        g.erase_node(node)
        for n in chain:  # producers after consumers
            if not n.users:
                g.erase_node(n)
        n_fused += 1
    if n_fused:
        g.lint()
        gm.recompile()
    return n_fused


def _file() -> str:
    return __file__


fuse_attention.file = _file  # the pass hook hashes this file into its cache key
