"""The decode-step folds of the spyre compile backend, on the CPU host:
RMSNorm into the projections that read it (spyre.rms_norm_mm) and residual
adds into the projections that feed them (addmm), for at most 8 token rows.

On CPU graphs (the passes installed as Inductor's post-grad custom pass for
the test) rms_norm_mm runs as the composite it replaces, so a folded norm
changes nothing; addmm on the CPU adds the residual to its own sums, so the
folded residual may differ from the eager rounding by an fp16 unit.  On
fake spyre tensors the wrapper must call the fused op.  The kernel's
numerics are GPU tests (test_kernels_gpu.py::test_gemm_rmsnorm,
test_decoder_gpu.py against the oracle's compiled-program model).
"""

import pytest
import torch
import torch.nn.functional as F

import torch_spyre  # noqa: F401
from torch_spyre._inductor import customops  # noqa: F401
from torch_spyre._inductor.passes.fuse_decode_norm import fuse_decode_norm, fuse_residual
from torch_spyre._inductor.passes.fuse_swiglu import fuse_swiglu
from torch_spyre.examples import decoder as D

from test_compile_codegen import _compile, fake_device  # noqa: F401


def _run(fn, *args, passes=(fuse_decode_norm, fuse_residual)):
    import torch._inductor.config as cfg

    counts = {p.__name__: 0 for p in passes}

    def hook(g):
        for p in passes:
            counts[p.__name__] += p(g.owning_module)

    torch._dynamo.reset()
    with cfg.patch({"post_grad_custom_post_pass": hook, "fx_graph_cache": False}):
        out = torch.compile(fn, dynamic=False)(*args)
    return out, counts


def _t(*shape, seed=0, scale=1.0, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _norm_proj(h, nw, w):
    return F.linear(F.rms_norm(h, (h.shape[-1],), nw, 1e-5), w)


@pytest.mark.parametrize("variant", ["2d", "3d", "bf16", "m1", "k8192", "two_readers"])
def test_norm_folds_into_projection(variant):
    dtype = torch.bfloat16 if variant == "bf16" else torch.float16
    m, k = (1, 256) if variant == "m1" else (4, 8192 if variant == "k8192" else 256)
    lead = (m, 1) if variant == "3d" else (m,)
    h = _t(*lead, k, seed=1, scale=3.0, dtype=dtype)
    nw = _t(k, seed=2, scale=0.1, dtype=dtype) + 1
    w = _t(96, k, seed=3, scale=0.05, dtype=dtype)
    w2 = _t(40, k, seed=4, scale=0.05, dtype=dtype)
    if variant == "two_readers":
        def fn(h, nw, w, w2):
            x = F.rms_norm(h, (k,), nw, 1e-5)
            return F.linear(x, w), F.linear(x, w2)
        out, n = _run(fn, h, nw, w, w2)
        assert n["fuse_decode_norm"] == 2
        for a, b in zip(out, fn(h, nw, w, w2)):
            assert torch.equal(a, b)
        return
    out, n = _run(_norm_proj, h, nw, w)
    assert n["fuse_decode_norm"] == 1
    assert torch.equal(out, _norm_proj(h, nw, w))


@pytest.mark.parametrize("case", ["rows", "k_align", "k_small", "k_large", "fp32", "escapes",
                                  "not_linear"])
def test_unfit_norm_stays_unfused(case):
    m, k, dtype = 4, 256, torch.float16
    if case == "rows":
        m = 9
    elif case == "k_align":
        k = 260
    elif case == "k_small":
        k = 56
    elif case == "k_large":
        k = 8200
    elif case == "fp32":
        dtype = torch.float32
    h = _t(m, k, seed=1, dtype=dtype)
    nw = _t(k, seed=2, dtype=dtype)
    w = _t(64, k, seed=3, scale=0.05, dtype=dtype)

    def fn(h, nw, w):
        x = F.rms_norm(h, (k,), nw, 1e-5)
        if case == "escapes":
            return F.linear(x, w), x
        if case == "not_linear":
            return x @ w[:, :k].T.contiguous() + 1, x.sum()
        return F.linear(x, w)

    _, n = _run(fn, h, nw, w)
    assert n["fuse_decode_norm"] == 0


def test_residual_folds_into_projection():
    a = _t(4, 1, 512, seed=5)
    h = _t(4, 1, 256, seed=6, scale=2.0)
    w = _t(256, 512, seed=7, scale=0.05)

    def fn(h, a, w):
        return h + F.linear(a, w)

    out, n = _run(fn, h, a, w)
    assert n["fuse_residual"] == 1
    want = (h.float() + a.float() @ w.float().T)
    torch.testing.assert_close(out.float(), want, rtol=2e-3, atol=2e-3)
    # M > 8 rows: unchanged
    _, n = _run(fn, _t(16, 1, 256, seed=6), _t(16, 1, 512, seed=5), w)
    assert n["fuse_residual"] == 0
    # the projection also used elsewhere: unchanged
    _, n = _run(lambda h, a, w: (lambda p: (h + p, p.sum()))(F.linear(a, w)), h, a, w)
    assert n["fuse_residual"] == 0


def test_decode_step_folds_every_norm_and_residual():
    cfg = D.DecoderConfig(hidden=256, n_heads=2, n_kv_heads=1, head_dim=128, intermediate=256,
                          vocab=64, n_layers=2)
    params = D.init_params(cfg, "cpu", seed=3)
    B, S = 4, 16
    cos, sin = D.rope_tables(cfg, S + 2, "cpu")
    tok = torch.randint(0, cfg.vocab, (B,), generator=torch.Generator().manual_seed(1))
    pos = torch.tensor([S])
    caches = [D.new_cache(cfg, B, S + 2, "cpu") for _ in range(2)]
    for li in range(cfg.n_layers):
        for j in range(2):
            x = _t(*caches[0][li][j].shape, seed=10 + 2 * li + j)
            caches[0][li][j].copy_(x)
            caches[1][li][j].copy_(x)
    got, n = _run(D.decode_step_static, tok, pos, params, cos, sin, caches[0], cfg,
                  passes=(fuse_swiglu, fuse_decode_norm, fuse_residual))
    # per layer: the attention norm into the QKV projection, the MLP norm
    # into the SwiGLU projection, two residual adds; the final norm into
    # the LM head
    assert n == {"fuse_swiglu": 2, "fuse_decode_norm": 2 * 2 + 1, "fuse_residual": 2 * 2}
    want = D.decode_step_static(tok, pos, params, cos, sin, caches[1], cfg)
    torch.testing.assert_close(got.float(), want.float(), rtol=1e-2, atol=1e-2)


def test_spyre_wrapper_calls_folded_ops(fake_device):
    code = _compile(lambda h, nw, w: _norm_proj(h, nw, w),
                    [((4, 512), torch.float16), ((512,), torch.float16),
                     ((1024, 512), torch.float16)])
    assert "torch.ops.spyre.rms_norm_mm.default(" in code
    assert "extern_kernels.mm(" not in code
    code = _compile(lambda h, a, w: h + F.linear(a, w),
                    [((4, 1, 256), torch.float16), ((4, 1, 512), torch.float16),
                     ((256, 512), torch.float16)])
    assert "extern_kernels.addmm(" in code
