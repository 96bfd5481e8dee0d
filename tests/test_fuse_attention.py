"""The attention fusion pass of the spyre compile backend, on the CPU host.

bmm(q, k^T) * scale (+ mask) -> softmax -> bmm(., v) is rewritten into one
torch.ops.spyre.attention call when the fused kernel takes the shapes.  The
pass is exercised here on CPU graphs (installed as Inductor's post-grad
custom pass for the test), where the op runs as the reference chain, so the
compiled result must equal eager exactly; on fake spyre tensors the
generated wrapper must call the fused op and emit no softmax kernel.  The
kernel's numerics against the oracle are GPU tests (test_kernels_gpu.py,
test_compile_gpu.py).
"""

import math

import pytest
import torch

import torch_spyre  # noqa: F401
from torch_spyre._inductor import customops  # noqa: F401
from torch_spyre._inductor.passes.fuse_attention import fuse_attention
from torch_spyre.examples import decoder as D

from test_compile_codegen import _compile, _kernels, fake_device  # noqa: F401


def _run(fn, *args):
    """torch.compile(fn) on CPU with the pass installed: (outputs, fused count)."""
    import torch._inductor.config as cfg

    counts = []
    torch._dynamo.reset()
    with cfg.patch({"post_grad_custom_post_pass": lambda g: counts.append(fuse_attention(g.owning_module)),
                    "fx_graph_cache": False}):
        out = torch.compile(fn)(*args)
    return out, sum(counts)


def _chain(q, k, v, mask=None, scale=1 / math.sqrt(128), div=False):
    s = torch.bmm(q, k.transpose(1, 2))
    s = s / (1 / scale) if div else s * scale
    if mask is not None:
        s = s + mask
    return torch.bmm(torch.softmax(s, dim=-1), v)


def _qkv(b, mq, sk, d=128, dtype=torch.float16, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=g).to(dtype) for s in ((b, mq, d), (b, sk, d), (b, sk, d))]


def _causal(mq, sk, dtype=torch.float16):
    return torch.full((mq, sk), float("-inf")).triu(1).to(dtype)  # row r keeps keys <= r


@pytest.mark.parametrize("variant", ["mask2d", "mask3d", "mask_b1", "nomask", "div", "bf16",
                                     "mask_first"])
def test_chain_is_fused_and_unchanged(variant):
    dtype = torch.bfloat16 if variant == "bf16" else torch.float16
    q, k, v = _qkv(2, 256, 192, dtype=dtype)
    mask = _causal(256, 192, dtype)
    if variant == "mask3d":
        mask = torch.stack([mask, mask.flip(1)])
    elif variant == "mask_b1":
        mask = mask[None]
    elif variant == "nomask":
        mask = None
    if variant == "mask_first":
        def fn(q, k, v, m):
            return torch.bmm(torch.softmax(m + torch.bmm(q, k.transpose(1, 2)) * 0.25, -1), v)
    else:
        def fn(q, k, v, m):
            return _chain(q, k, v, m, div=variant == "div")
    out, n = _run(fn, q, k, v, mask)
    assert n == 1
    if variant == "div":  # the op multiplies by 1/c where the program divided by c
        torch.testing.assert_close(out, fn(q, k, v, mask), rtol=2e-3, atol=2e-3)
    else:
        assert torch.equal(out, fn(q, k, v, mask))


@pytest.mark.parametrize("case", ["head64", "rows_off_block", "fp32", "scores_escape",
                                  "probs_escape", "mask_cols_off"])
def test_unfit_chains_stay_unfused(case):
    d, mq, dtype = 128, 256, torch.float16
    if case == "head64":
        d = 64
    elif case == "rows_off_block":
        mq = 200
    elif case == "fp32":
        dtype = torch.float32
    q, k, v = _qkv(2, mq, 128, d=d, dtype=dtype)
    mask = torch.zeros(mq, 128, dtype=dtype)

    def fn(q, k, v, m):
        s = torch.bmm(q, k.transpose(1, 2)) * 0.1 + m
        p = torch.softmax(s, -1)
        o = torch.bmm(p, v)
        if case == "scores_escape":
            return o, s
        if case == "probs_escape":
            return o, p
        return o

    if case == "mask_cols_off":
        mask = torch.zeros(mq, 1, dtype=dtype)  # [mq, 1]: broadcast keys, not a kernel layout
    _, n = _run(fn, q, k, v, mask)
    assert n == 0


def test_decoder_attention_is_fused():
    # the decoder's grouped-query attention (query heads stacked along the
    # rows, causal mask repeated per head) is the pattern the pass targets
    cfg = D.DecoderConfig(hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=256,
                          vocab=64, n_layers=1)
    S = 64
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, S, 4, 128, generator=g).half()
    k = torch.randn(1, 2, S, 128, generator=g).half()
    v = torch.randn(1, 2, S, 128, generator=g).half()
    mask = D.causal_mask(cfg, S, "cpu")
    out, n = _run(lambda q, k, v, m: D._attention(q, k, v, cfg, m), q, k, v, mask)
    assert n == 1
    assert torch.equal(out, D._attention(q, k, v, cfg, mask))


def test_spyre_wrapper_calls_fused_attention(fake_device):
    code = _compile(lambda q, k, v, m: _chain(q, k, v, m),
                    [((8, 512, 128), torch.float16), ((8, 256, 128), torch.float16),
                     ((8, 256, 128), torch.float16), ((512, 256), torch.float16)])
    assert "torch.ops.spyre.attention.default(" in code
    assert "extern_kernels.bmm(" not in code
    assert not any("softmax" in k or "amax" in k for k in _kernels(code)), _kernels(code)


@pytest.mark.parametrize("mask_kind", ["row", "row2d", "full", "none"])
@pytest.mark.parametrize("mq", [4, 16, 256])
def test_row_broadcast_masks_fuse_and_decode_shapes_do_not(mask_kind, mq):
    # one mask row shared by every query row ([sk] or [1, sk], expanded as a
    # view) is fused; decode shapes (a few rows per KV head) stay on the
    # unfused chain, which measured faster there than the fused decode kernel
    sk = 96
    q, k, v = _qkv(3, mq, sk, seed=4)
    row = torch.zeros(sk, dtype=torch.float16)
    row[80:] = float("-inf")
    mask = {"row": row, "row2d": row[None], "full": row.expand(mq, sk).contiguous(),
            "none": None}[mask_kind]
    if mask is None:
        out, n = _run(lambda q, k, v: _chain(q, k, v), q, k, v)
        ref = _chain(q, k, v)
    else:
        out, n = _run(lambda q, k, v, m: _chain(q, k, v, m), q, k, v, mask)
        ref = _chain(q, k, v, mask)
    assert n == (1 if mq % 128 == 0 else 0)
    if n:
        assert torch.equal(out, ref)  # the fused op runs the same chain on CPU
    else:
        torch.testing.assert_close(out, ref, rtol=1e-2, atol=1e-2)  # Inductor's own kernels


@pytest.mark.parametrize("sk", [77, 130])
def test_masks_with_any_key_count_fuse(sk):
    # the op pads mask rows to the kernel's 16-byte row alignment, so a key
    # count off a multiple of 8 is fused like any other
    q, k, v = _qkv(2, 128, sk, seed=5)
    mask = _causal(128, sk)
    out, n = _run(lambda q, k, v, m: _chain(q, k, v, m), q, k, v, mask)
    assert n == 1
    # (Inductor pads the stride of the 77- or 130-wide probability buffer,
    # which moves CPU BLAS to another blocking: equal to rounding, not bits)
    torch.testing.assert_close(out, _chain(q, k, v, mask), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("form", ["neg_mul", "neg_div", "neg_nomask", "zero", "inf"])
def test_nonpositive_or_infinite_scales_stay_unfused(form):
    # the kernel folds a positive finite scale into exp2 after the row max;
    # every other scale keeps the unfused chain (and its result)
    q, k, v = _qkv(2, 128, 64, seed=6)
    mask = None if form == "neg_nomask" else _causal(128, 64)
    scale = {"neg_mul": -0.125, "neg_div": -0.125, "neg_nomask": -0.125, "zero": 0.0,
             "inf": float("inf")}[form]
    if mask is None:
        out, n = _run(lambda q, k, v: _chain(q, k, v, None, scale=scale), q, k, v)
        ref = _chain(q, k, v, None, scale=scale)
    else:
        out, n = _run(lambda q, k, v, m: _chain(q, k, v, m, scale=scale, div=form == "neg_div"),
                      q, k, v, mask)
        ref = _chain(q, k, v, mask, scale=scale, div=form == "neg_div")
    assert n == 0
    torch.testing.assert_close(out, ref, rtol=1e-2, atol=1e-2, equal_nan=True)
