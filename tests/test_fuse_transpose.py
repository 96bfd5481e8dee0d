"""The transposing-copy pass of the spyre compile backend, on the CPU host.

`clone(permute(x, dims))` that moves the innermost dimension is rewritten
into one torch.ops.spyre.transpose_copy call (an LDS-tiled transpose on the
device, sph_transpose_copy).  Exercised on CPU graphs, where the op is the
plain permute and copy, so the compiled result must equal eager exactly; on
fake spyre tensors the generated wrapper must call the op.  The reference's
cases (tests/_inductor/test_inductor_ops.py:198-218: x.t().contiguous() at
1088 x 320, transpose(x, 0|1, 2).contiguous() at 512 x 256 x 128) run on the
GPU in test_compiled_ops_gpu.py.
"""

import pytest
import torch

import torch_spyre  # noqa: F401
from torch_spyre._inductor import customops  # noqa: F401
from torch_spyre._inductor.passes.fuse_transpose import fuse_transpose

from test_compile_codegen import _compile, fake_device  # noqa: F401


def _run(fn, *args):
    import torch._inductor.config as cfg

    counts = []
    torch._dynamo.reset()
    with cfg.patch({"post_grad_custom_post_pass": lambda g: counts.append(fuse_transpose(g.owning_module)),
                    "fx_graph_cache": False}):
        out = torch.compile(fn)(*args)
    return out, sum(counts)


@pytest.mark.parametrize("case", ["t2d", "t02", "t12", "perm3"])
def test_transposing_copies_fused(case):
    g = torch.Generator().manual_seed(0xAFFE)
    if case == "t2d":
        x = torch.randn(88, 40, generator=g).half()
        fn = lambda x: x.t().contiguous()  # noqa: E731
    elif case == "t02":
        x = torch.randn(16, 8, 24, generator=g)
        fn = lambda x: torch.transpose(x, 0, 2).contiguous()  # noqa: E731
    elif case == "t12":
        x = torch.randn(16, 8, 24, generator=g)
        fn = lambda x: torch.transpose(x, 1, 2).contiguous()  # noqa: E731
    else:
        x = torch.randn(4, 6, 8, 10, generator=g)
        fn = lambda x: x.permute(0, 3, 1, 2).contiguous()  # noqa: E731
    out, n = _run(fn, x)
    assert n == 1
    assert torch.equal(out, fn(x)) and out.is_contiguous()


def test_innermost_kept_stays_with_inductor():
    x = torch.randn(6, 8, 10)
    fn = lambda x: x.permute(1, 0, 2).contiguous()  # noqa: E731
    out, n = _run(fn, x)
    assert n == 0
    assert torch.equal(out, fn(x))


def test_clone_preserving_strides_is_left_alone():
    # clone() without a memory format keeps the permuted strides: it is not
    # a transposing copy, and the result's strides stay eager's
    x = torch.randn(88, 40).half()
    fn = lambda x: x.t().clone() * 2  # noqa: E731
    out, n = _run(fn, x)
    assert n == 0
    assert torch.equal(out, fn(x)) and out.stride() == fn(x).stride()
    fn = lambda x: x.t().clone()  # noqa: E731
    out, n = _run(fn, x)
    assert n == 0
    assert torch.equal(out, fn(x)) and out.stride() == fn(x).stride()


def test_spyre_wrapper_calls_transpose_copy(fake_device):
    code = _compile(lambda x: x.t().contiguous(), [((1088, 320), torch.float16)])
    assert "torch.ops.spyre.transpose_copy.default(" in code


def test_permute_chain_composes():
    # two permutes whose composition moves the innermost dimension
    x = torch.randn(2, 6, 4, 8)
    fn = lambda x: x.permute(0, 2, 1, 3).permute(0, 1, 3, 2).contiguous()  # noqa: E731
    out, n = _run(fn, x)
    assert n == 1
    assert torch.equal(out, fn(x))


def test_copy_of_transposed_tensor_into_a_slice():
    # the decoder's prefill writes V transposed into a slice of a dim-major
    # cache: cache[:, :, :, :S].copy_(v.transpose(1, 2).transpose(2, 3))
    g = torch.Generator().manual_seed(7)
    B, S, H, D, L = 2, 40, 3, 16, 48
    v = torch.randn(B, S, H, D, generator=g).half()

    def fn(v, cache):
        cache[:, :, :, :S].copy_(v.transpose(1, 2).transpose(2, 3))
        return cache.sum()

    cache = torch.zeros(B, H, D, L).half()
    want_cache = cache.clone()
    want = fn(v, want_cache)
    out, n = _run(fn, v, cache)
    assert n == 1
    assert torch.equal(cache, want_cache) and torch.equal(out, want)


def test_copy_keeping_innermost_is_left_alone():
    v = torch.randn(2, 40, 3, 16)

    def fn(v, cache):
        cache[:, :, :40].copy_(v.transpose(1, 2))
        return cache.sum()

    cache = torch.zeros(2, 3, 48, 16)
    out, n = _run(fn, v, cache)
    assert n == 0
