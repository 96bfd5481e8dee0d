"""The SwiGLU projection fusion pass of the spyre compile backend, on the
CPU host.

x W^T -> silu(gate) * up (W the stacked [2n, K] gate / up weight) is
rewritten into one torch.ops.spyre.swiglu_mm call when the fused GEMM takes
the shape.  On CPU graphs (the pass installed as Inductor's post-grad
custom pass for the test) the op runs as the unfused chain, so the compiled
result must equal eager exactly; on fake spyre tensors the wrapper must
call the fused op.  The kernel's numerics against the oracle are GPU tests
(test_kernels_gpu.py::test_gemm_swiglu, test_decoder_gpu.py).
"""

import pytest
import torch
import torch.nn.functional as F

import torch_spyre  # noqa: F401
from torch_spyre._inductor import customops  # noqa: F401
from torch_spyre._inductor.passes.fuse_swiglu import fuse_swiglu
from torch_spyre.examples import decoder as D

from test_compile_codegen import _compile, fake_device  # noqa: F401


def _run(fn, *args):
    import torch._inductor.config as cfg

    counts = []
    torch._dynamo.reset()
    with cfg.patch({"post_grad_custom_post_pass": lambda g: counts.append(fuse_swiglu(g.owning_module)),
                    "fx_graph_cache": False}):
        out = torch.compile(fn)(*args)
    return out, sum(counts)


def _inputs(m, n, k, dtype=torch.float16, lead=()):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(*lead, m, k, generator=g).to(dtype)
    w = (torch.randn(2 * n, k, generator=g) * 0.05).to(dtype)
    return x, w


def _swiglu(x, w, order="gu"):
    n = w.shape[0] // 2
    gu = F.linear(x, w)
    g, u = gu[..., :n], gu[..., n:]
    return F.silu(g) * u if order == "gu" else u * F.silu(g)


@pytest.mark.parametrize("variant", ["2d", "3d", "swapped", "bf16", "decode"])
def test_swiglu_is_fused_and_unchanged(variant):
    dtype = torch.bfloat16 if variant == "bf16" else torch.float16
    lead = (1,) if variant == "3d" else ()
    m, n = (4, 200) if variant == "decode" else (256, 128)  # decode: weight-stream shape
    x, w = _inputs(m, n, 64, dtype, lead)
    order = "ug" if variant == "swapped" else "gu"
    out, n = _run(lambda x, w: _swiglu(x, w, order), x, w)
    assert n == 1
    assert torch.equal(out, _swiglu(x, w, order))


@pytest.mark.parametrize("case", ["rows", "cols", "k", "fp32", "gu_escapes", "uneven_split"])
def test_unfit_swiglu_stays_unfused(case):
    m, n, k, dtype = 256, 128, 64, torch.float16
    if case == "rows":
        m = 200  # neither whole 256-row tiles nor a decode shape
    elif case == "cols":
        n = 96
    elif case == "k":
        k = 40
    elif case == "fp32":
        dtype = torch.float32
    x, w = _inputs(m, n, k, dtype)

    def fn(x, w):
        nn = w.shape[0] // 2
        gu = F.linear(x, w)
        if case == "uneven_split":
            return F.silu(gu[..., :nn - 64]) * gu[..., nn - 64:2 * nn - 128]
        y = F.silu(gu[..., :nn]) * gu[..., nn:]
        return (y, gu) if case == "gu_escapes" else y

    _, cnt = _run(fn, x, w)
    assert cnt == 0


def test_decoder_mlp_is_fused():
    cfg = D.DecoderConfig(hidden=256, n_heads=2, n_kv_heads=1, head_dim=128, intermediate=128,
                          vocab=64, n_layers=1)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 256, 256, generator=g).half()
    w = {"wgu": (torch.randn(256, 256, generator=g) * 0.05).half(),
         "wd": (torch.randn(256, 128, generator=g) * 0.05).half()}
    out, n = _run(lambda x, wgu, wd: D._mlp(x, {"wgu": wgu, "wd": wd}, cfg), x, w["wgu"], w["wd"])
    assert n == 1
    assert torch.equal(out, D._mlp(x, w, cfg))


def test_spyre_wrapper_calls_fused_swiglu(fake_device):
    code = _compile(lambda x, w: _swiglu(x, w),
                    [((512, 256), torch.float16), ((512, 256), torch.float16)])
    assert "torch.ops.spyre.swiglu_mm.default(" in code
    assert "extern_kernels.mm(" not in code
