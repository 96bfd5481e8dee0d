"""The `torch.ops.spyre.*` custom operators (reference
torch_spyre/_inductor/customops.py:22-154, decompositions.py:21-58).

CPU: the op bodies (`*_impl`, the same code the spyre registrations run)
are pinned against numpy float64 statistics and the oracle's LayerNorm /
RMSNorm; the stick layout of their results against the descriptor rules;
the compiled forms against Inductor's output on fake spyre tensors (compact
fuses to one copy kernel, spyre::layer_norm to one Welford row kernel, the
statistics ops stay extern calls).  GPU: the registered ops on spyre
tensors, eager and compiled, against the same references.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import torch_spyre  # noqa: F401
from torch_spyre._inductor import Unsupported
from torch_spyre._inductor import customops as C
from torch_spyre._inductor import decompositions as D
from torch_spyre._inductor.stickify import StickFormat, elems_per_stick

from oracle import ops as O

from helpers import assert_close_fp, randn
from test_compile_codegen import _compile, _kernels, fake_device  # noqa: F401

DEV = "spyre"


def _stats_np(x: np.ndarray):
    x = x.astype(np.float64)
    return x.mean(-1), (x * x).mean(-1), x.var(-1)


# ---------------------------------------------------------------------------
# CPU: op algebra and layouts
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(6, 256), (3, 5, 130), (64,)])
def test_exx2_sticks_hold_both_moments(shape):
    x = randn(shape, k=0, scale=2.0, mean=0.5)
    n = shape[-1]
    s = C.exx2_impl(x, 1.0 / n, False)
    eps = elems_per_stick(x.dtype)
    assert list(s.shape) == list(shape[:-1]) and s.dtype == x.dtype
    if s.dim():
        assert s.stride(-1) == eps
    m1, m2, _ = _stats_np(x.float().numpy())
    np.testing.assert_allclose(s.float().numpy(), m1, rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(C._slot(s, 1).float().numpy(), m2, rtol=2e-3, atol=2e-3)
    z = C.exx2_impl(x, 1.0 / n, True)
    assert z.float().abs().max() == 0
    np.testing.assert_allclose(C._slot(z, 1).float().numpy(), m2, rtol=2e-3, atol=2e-3)


def test_layernormscale_and_norm_compose_to_layer_norm_and_rms_norm():
    R, N = 16, 512
    x = randn((R, N), k=1)
    w = randn((N,), k=2, scale=0.1, mean=1.0)
    b = randn((N,), k=3, scale=0.1)
    s = C.exx2_impl(x, 1.0 / N, False)
    r = C.layernormscale_impl(s, 1e-5)
    assert r.stride(-1) == elems_per_stick(x.dtype)
    _, _, var = _stats_np(x.float().numpy())
    np.testing.assert_allclose(r.float().numpy(), 1 / np.sqrt(var + 1e-5), rtol=5e-3)
    y = C.layernormnorm_impl(x, s, r, w, b)
    assert_close_fp(y, O.layernorm(x.numpy(), w.numpy(), b.numpy(), 1e-5)[0], what="LN chain")
    # zero-mean statistics turn the same chain into RMSNorm
    z = C.exx2_impl(x, 1.0 / N, True)
    y2 = C.layernormnorm_impl(x, z, C.layernormscale_impl(z, 1e-5), w, None)
    assert_close_fp(y2, O.rmsnorm(x.numpy(), w.numpy(), 1e-5)[0], what="RMS chain")


def test_layernormscale_rejects_dense_statistics():
    with pytest.raises(Unsupported):
        C.layernormscale_impl(torch.ones(4, 3, dtype=torch.float16), 1e-5)


def test_swap_slice_compact_on_cpu():
    x = torch.arange(100, dtype=torch.float16)
    s = C.swap_impl(x)
    assert s.stride() == (64,) and torch.equal(s, x)
    assert s.untyped_storage().nbytes() >= 100 * 128
    assert torch.equal(torch.ops.spyre.compact(x), x)
    for bad in (torch.ops.spyre.compact, C.swap_impl):
        with pytest.raises(Unsupported):
            bad(torch.ones(2, 2))


def test_layer_norm_op_and_hook_on_cpu():
    x = randn((8, 64), k=4, dtype=torch.float32)
    torch.testing.assert_close(torch.ops.spyre.layer_norm(x, [64], None, None, 1e-5),
                               F.layer_norm(x, [64]))
    with pytest.raises(Unsupported):
        torch.ops.spyre.layer_norm(x, [8, 64], None, None, 1e-5)
    # the F.layer_norm replacement passes non-spyre tensors through
    assert F.layer_norm is D.spyre_layer_norm
    torch.testing.assert_close(F.layer_norm(x, [8, 64]), D._orig_layer_norm(x, [8, 64]))


def test_ops_are_spyre_only_where_the_reference_says():
    for name in ("swap", "slice", "exx2", "layernormscale", "layernormnorm"):
        assert hasattr(torch.ops.spyre, name)
    with pytest.raises(NotImplementedError):
        torch.ops.spyre.swap(torch.arange(3.0))


# ---------------------------------------------------------------------------
# CPU: what Inductor generates for them on fake spyre tensors
# ---------------------------------------------------------------------------
def test_compact_compiles_to_one_copy_kernel(fake_device):  # noqa: F811
    code = _compile(lambda x: torch.ops.spyre.compact(x), [((1000,), torch.float16)])
    assert len(_kernels(code)) == 1


def test_spyre_layer_norm_compiles_to_one_fused_kernel(fake_device):  # noqa: F811
    code = _compile(lambda x, r, w, b: torch.ops.spyre.layer_norm(x + r, [4096], w, b, 1e-5),
                    [((64, 4096), torch.float16), ((64, 4096), torch.float16),
                     ((4096,), torch.float16), ((4096,), torch.float16)])
    assert len(_kernels(code)) == 1 and "block_welford" in code


def test_statistics_ops_are_extern_calls(fake_device):  # noqa: F811
    def chain(x):
        s = torch.ops.spyre.exx2(x, 1.0 / 256, False)
        return torch.ops.spyre.layernormnorm(x, s, torch.ops.spyre.layernormscale(s, 1e-5),
                                             None, None)

    code = _compile(chain, [((32, 256), torch.float16)])
    for op in ("exx2", "layernormscale", "layernormnorm"):
        assert f"torch.ops.spyre.{op}.default" in code


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
@pytest.mark.gpu
def test_custom_ops_eager_on_spyre():
    print("[case] spyre custom ops eager", flush=True)
    R, N = 64, 4096
    x = randn((R, N), k=5)
    w = randn((N,), k=6, scale=0.02, mean=1.0)
    b = randn((N,), k=7, scale=0.02)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    s = torch.ops.spyre.exx2(xd, 1.0 / N, False)
    assert s.device.type == DEV and s.stride() == (64,)
    m1, m2, var = _stats_np(x.float().numpy())
    np.testing.assert_allclose(s.cpu().float().numpy(), m1, rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(C._slot(s, 1).cpu().float().numpy(), m2, rtol=2e-3, atol=2e-3)
    r = torch.ops.spyre.layernormscale(s, 1e-5)
    np.testing.assert_allclose(r.cpu().float().numpy(), 1 / np.sqrt(var + 1e-5), rtol=5e-3)
    y = torch.ops.spyre.layernormnorm(xd, s, r, wd, bd)
    want = O.layernorm(x.numpy(), w.numpy(), b.numpy(), 1e-5)[0]
    assert_close_fp(y, want, what="spyre LN chain")
    assert_close_fp(torch.ops.spyre.layer_norm(xd, [N], wd, bd, 1e-5), want, what="spyre.layer_norm")
    assert_close_fp(F.layer_norm(xd, [N], wd, bd, 1e-5), want, what="F.layer_norm hook")
    v = torch.arange(300, dtype=torch.float16)
    sw = torch.ops.spyre.swap(v.to(DEV))
    assert sw.stride() == (64,) and torch.equal(sw.cpu(), v)
    assert torch.equal(torch.ops.spyre.slice(sw).cpu(), v)
    assert torch.equal(torch.ops.spyre.compact(v.to(DEV)).cpu(), v)


@pytest.mark.gpu
def test_custom_ops_compiled_on_spyre():
    print("[case] spyre custom ops compiled", flush=True)
    torch._dynamo.reset()
    R, N = 512, 4096
    x, r = randn((R, N), k=8), randn((R, N), k=9)
    w = randn((N,), k=10, scale=0.02, mean=1.0)
    b = randn((N,), k=11, scale=0.02)
    xd, rd, wd, bd = (t.to(DEV) for t in (x, r, w, b))
    y = torch.compile(lambda a, c, g, e: torch.ops.spyre.layer_norm(a + c, [N], g, e, 1e-5))(
        xd, rd, wd, bd)
    want = O.layernorm(x.numpy(), w.numpy(), b.numpy(), 1e-5, residual=r.numpy())[0]
    assert_close_fp(y, want, what="compiled spyre.layer_norm")
    ln = torch.nn.LayerNorm(N, eps=1e-5).half().to(DEV)
    with torch.no_grad():
        y2 = torch.compile(ln)(xd)
    assert_close_fp(y2, O.layernorm(x.numpy(), np.ones(N, np.float32), np.zeros(N, np.float32),
                                    1e-5)[0], what="compiled nn.LayerNorm")
    v = torch.arange(1000, dtype=torch.float16)
    assert torch.equal(torch.compile(lambda t: torch.ops.spyre.compact(t))(v.to(DEV)).cpu(), v)

    def chain(t):
        s = torch.ops.spyre.exx2(t, 1.0 / N, True)
        return torch.ops.spyre.layernormnorm(t, s, torch.ops.spyre.layernormscale(s, 1e-5), None,
                                             None)

    assert_close_fp(torch.compile(chain)(xd), O.rmsnorm(x.numpy(), np.ones(N, np.float32),
                                                         1e-5)[0], what="compiled RMS chain")
