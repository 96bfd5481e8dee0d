"""torch.compile on "spyre" tensors (MI355X): the generated, hiprtc-compiled
HIP kernels and the extern MFMA GEMM calls, checked against the numpy oracle
and torch's CPU ops at rtol = atol = 1e-2 (fp16 outputs).

The reference's compiled-path tests (tests/_inductor/test_building_blocks.py
:33-89, test_inductor_ops.py) compare torch.compile on its device with the
CPU; the cases here are the BASELINE configs' compiled flows: c1 softmax,
c2 matmul / bmm, c3 norms and the GELU chain with a row-sum, plus the
reference's building blocks (softplus, single-head attention).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import torch_spyre  # noqa: F401

from oracle import ops as O

from helpers import assert_close_fp, randn, uniform

pytestmark = pytest.mark.gpu

DEV = "spyre"
TOL = dict(rtol=1e-2, atol=1e-2)


def _log(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(autouse=True)
def _fresh_dynamo():
    torch._dynamo.reset()
    yield


def test_c1_softmax_compiled_vs_oracle():
    _log("compiled softmax [512,4096]")
    x = randn((512, 4096), k=0, scale=4.0)
    f = torch.compile(lambda a: torch.softmax(a, dim=-1))
    y = f(x.to(DEV))
    assert_close_fp(y, O.softmax(x.numpy()), what="compiled softmax")
    # same result as the eager spyre kernel, and repeatable
    torch.testing.assert_close(f(x.to(DEV)).cpu(), y.cpu(), rtol=0, atol=0)


@pytest.mark.parametrize("dim", [0, 1, -1])
def test_building_block_softmax_dims(dim):
    # reference tests/_inductor/test_building_blocks.py:33-36
    _log(f"compiled softmax [512,1024] dim={dim}")
    x = randn((512, 1024), k=1)
    y = torch.compile(lambda a: torch.softmax(a, dim=dim))(x.to(DEV))
    torch.testing.assert_close(y.cpu(), torch.softmax(x.float(), dim=dim).half(), **TOL)


@pytest.mark.parametrize("R", [512, 8192])
def test_c3_norms_and_gelu_chain_compiled_vs_oracle(R):
    """The compiled c3 programs the benchmark times, at [512, 4096] and at
    the config's [8192, 4096]."""
    _log(f"compiled c3 at [{R},4096]")
    C = 4096
    x, r = randn((R, C), k=0), randn((R, C), k=1)
    w = randn((C,), k=2, scale=0.02, mean=1.0)
    b = randn((C,), k=3, scale=0.02)
    xd, rd, wd, bd = (t.to(DEV) for t in (x, r, w, b))

    h, y = torch.compile(lambda a, c, g: (lambda s: (s, torch.rms_norm(s, [C], g, 1e-5)))(a + c))(
        xd, rd, wd)
    ey, eh = O.rmsnorm(x.numpy(), w.numpy(), 1e-5, residual=r.numpy())[:2]
    assert_close_fp(h, eh, what="compiled residual add")
    assert_close_fp(y, ey, what="compiled add+rmsnorm")

    h2, y2 = torch.compile(
        lambda a, c, g, e: (lambda s: (s, F.layer_norm(s, [C], g, e, 1e-5)))(a + c))(xd, rd, wd, bd)
    ly, lh = O.layernorm(x.numpy(), w.numpy(), b.numpy(), 1e-5, residual=r.numpy())[:2]
    assert_close_fp(h2, lh, what="compiled residual add (LN)")
    assert_close_fp(y2, ly, what="compiled add+layernorm")

    g, rs = torch.compile(lambda a, s, c: (lambda t: (t, t.sum(-1)))(F.gelu(a * s + c)))(xd, wd, bd)
    eg, ers = O.gelu_affine_rowsum(x.numpy(), w.numpy(), b.numpy())
    assert_close_fp(g, eg, what="compiled gelu chain")
    # a row-sum of 4096 fp16 values: fp16 output rounding is ~0.1 at |sum|~300
    np.testing.assert_allclose(rs.cpu().float().numpy(), ers, rtol=2e-2, atol=0.5)


def test_compiled_variance_and_gelu_edges():
    # LayerNorm's per-thread variance is summed around a data point, so a
    # large mean with a small spread keeps its precision (fp32 in and out,
    # against float64 on the CPU); the looped form (rows longer than the
    # register-held ones) goes the same way
    for cols in (4096, 40960):
        _log(f"compiled layer_norm fp32, mean 100, std 0.1, [32,{cols}]")
        g = torch.Generator().manual_seed(11)
        x = 100 + 0.1 * torch.randn(32, cols, generator=g)
        y = torch.compile(lambda a: F.layer_norm(a, [cols], eps=1e-5), dynamic=False)(x.to(DEV))
        ref = F.layer_norm(x.double(), [cols], eps=1e-5).float()
        torch.testing.assert_close(y.cpu(), ref, rtol=0, atol=2e-4)
    # the erf form of GELU (one call in the generated code) over its
    # breakpoints and special values, against torch's CPU gelu (fp32)
    _log("compiled gelu special values")
    v = [-float("inf"), -30.0, -5.6, -5.5, -5.4, -3.0, -0.5, -1e-3, 0.0, 1e-3, 0.5, 3.0, 5.4,
         5.5, 5.6, 30.0, float("nan"), float("inf")]
    x = torch.tensor(v + torch.linspace(-8, 8, 4096 - len(v)).tolist()).reshape(2, 2048)
    y = torch.compile(lambda a: F.gelu(a), dynamic=False)(x.to(DEV)).cpu()
    torch.testing.assert_close(y, F.gelu(x), rtol=0, atol=1e-6, equal_nan=True)


def test_c2_matmul_and_bmm_compiled():
    _log("compiled mm / bmm")
    A, B = uniform((1024, 2048), k=0), uniform((2048, 512), k=1)
    C = torch.compile(lambda a, b: a @ b)(A.to(DEV), B.to(DEV))
    assert_close_fp(C, O.gemm(A.numpy(), B.numpy()), what="compiled mm")
    Q, K = uniform((8, 256, 128), k=2), uniform((8, 128, 256), k=3)
    S = torch.compile(lambda q, k: torch.softmax(torch.bmm(q, k) * 0.088, dim=-1))(
        Q.to(DEV), K.to(DEV))
    ref = torch.softmax(torch.bmm(Q.float(), K.float()).half().float() * 0.088, -1).half()
    torch.testing.assert_close(S.cpu(), ref, **TOL)


def test_c2_compiled_mm_4096_vs_oracle_sample():
    """The compiled c2 product the benchmark reports, M = N = K = 4096, a
    sample of rows against the oracle."""
    _log("compiled mm 4096^3 (row sample vs oracle)")
    A, B = uniform((4096, 4096), k=0), uniform((4096, 4096), k=1)
    C = torch.compile(lambda a, b: a @ b)(A.to(DEV), B.to(DEV))
    rows = torch.arange(0, 4096, 257)
    assert_close_fp(C.index_select(0, rows.to(DEV)), O.gemm(A[rows].numpy(), B.numpy()),
                    what="compiled c2 mm sampled rows")


def test_building_block_softplus_and_attention():
    # reference tests/_inductor/test_building_blocks.py:38-89
    _log("compiled softplus / single-head attention")
    x = randn((512, 1024), k=4)
    sp = torch.compile(lambda a: F.softplus(a))(x.to(DEV))
    torch.testing.assert_close(sp.cpu(), F.softplus(x.float()).half(), **TOL)
    q, k, v = randn((256, 128), k=5), randn((256, 128), k=6), randn((256, 128), k=7)

    def attn(q, k, v):
        s = q @ k.transpose(-2, -1) * (1.0 / 128 ** 0.5)
        return torch.softmax(s, dim=-1) @ v

    o = torch.compile(attn)(q.to(DEV), k.to(DEV), v.to(DEV))
    ref = attn(q.float(), k.float(), v.float()).half()
    torch.testing.assert_close(o.cpu(), ref, rtol=2e-2, atol=2e-2)


def test_pointwise_chain_and_broadcast_compiled():
    _log("compiled pointwise chain")
    x = randn((333, 77), k=8, dtype=torch.float32)
    y = randn((77,), k=9, dtype=torch.float32)
    f = torch.compile(lambda a, b: (torch.sigmoid(a * 2 + b).relu() - 1) * torch.tanh(a))
    torch.testing.assert_close(f(x.to(DEV), y.to(DEV)).cpu(),
                               (torch.sigmoid(x * 2 + y).relu() - 1) * torch.tanh(x),
                               rtol=1e-5, atol=1e-5)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_pointwise_group_form_compiled(dtype):
    # 8 consecutive elements per thread with 16-byte accesses: rotate-half
    # (masked loads whose shifted index leaves the buffer at its first and
    # last rows), a permuted store, row broadcasts; results bit-exact
    # against torch on the CPU (pure data movement, negation and one
    # rounding per output)
    _log(f"compiled group-form pointwise {dtype}")
    x = randn((3, 16, 4, 64), k=30, dtype=dtype)
    c = randn((16, 64), k=31, dtype=dtype)
    f = torch.compile(lambda a, cs: (a * cs[:, None, :] + _rotate_half(a) * cs[:, None, :]).transpose(1, 2)
                      .contiguous())
    got = f(x.to(DEV), c.to(DEV)).cpu()
    ref = ((x.float() * c.float()[:, None, :] + _rotate_half(x.float()) * c.float()[:, None, :])
           .to(dtype).transpose(1, 2).contiguous())
    # each output is one fp32 multiply-add of the same two products, rounded once
    torch.testing.assert_close(got.float(), ref.float(), rtol=1e-2, atol=1e-2)
    g = torch.compile(lambda a: _rotate_half(a))
    torch.testing.assert_close(g(x.to(DEV)).cpu(), _rotate_half(x), rtol=0, atol=0)
    # a buffer whose last group ends exactly at the end of the allocation,
    # and a row of 40 elements (groups never straddle rows: 40 % 8 == 0)
    y = randn((5, 40), k=32, dtype=dtype)
    h = torch.compile(lambda a: torch.cat([a[:, 20:] * 2, -a[:, :20]], dim=-1))
    torch.testing.assert_close(h(y.to(DEV)).cpu(), torch.cat([y[:, 20:] * 2, -y[:, :20]], dim=-1),
                               rtol=0, atol=0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_pointwise_group_form_gathered_rows(dtype):
    # rows gathered by an index tensor (negative indices wrap, as in torch)
    # read as whole 8-element groups; bit-exact against torch on the CPU
    _log(f"compiled group-form gathered rows {dtype}")
    t = randn((50, 40), k=34, dtype=dtype)
    r = randn((7, 40), k=35, dtype=dtype)
    i = torch.tensor([0, 49, -1, -50, 17, 3, 3])
    f = torch.compile(lambda tt, ii, rr: tt[ii] + rr)
    torch.testing.assert_close(f(t.to(DEV), i.to(DEV), r.to(DEV)).cpu(), t[i] + r, rtol=0, atol=0)


def test_pointwise_group_form_unaligned_views():
    # buffers that are not 16-byte aligned (views at an odd element offset)
    # take the element path of the group form
    _log("compiled group-form pointwise, unaligned views")
    base = randn((1, 8 * 64 + 3), k=33, dtype=torch.float16)
    dev = base.to(DEV)
    f = torch.compile(lambda a, b: a * 2 + b)
    a, b = dev[0, 1:1 + 8 * 64], dev[0, 3:3 + 8 * 64]
    torch.testing.assert_close(f(a, b).cpu(), base[0, 1:1 + 512] * 2 + base[0, 3:3 + 512],
                               rtol=0, atol=0)


@pytest.mark.parametrize("sk", [77, 130])
def test_fused_masked_attention_any_key_count(sk):
    # a mask whose rows are not a multiple of 8 keys long goes through the
    # fused kernel (the op pads its rows) and matches the oracle
    _log(f"compiled fused masked attention sk={sk}")
    from torch_spyre._inductor import customops  # noqa: F401  (torch.ops.spyre.attention)

    b, mq = 2, 256
    q, k, v = randn((b, mq, 128), k=70), randn((b, sk, 128), k=71), randn((b, sk, 128), k=72)
    mask = torch.full((mq, sk), float("-inf")).triu(1 + sk - mq if sk > mq else 1)
    mask[:, 0] = 0.0  # every row keeps a key
    mask = mask.half()
    scale = 1.0 / 128 ** 0.5

    def fn(q, k, v, m):
        s = torch.bmm(q, k.transpose(1, 2)) * scale + m
        return torch.bmm(torch.softmax(s, dim=-1), v)

    out = torch.compile(fn)(q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV))
    want = O.attention(q.numpy(), k.numpy(), v.numpy(), scale, mask.numpy())
    assert_close_fp(out, want, what=f"fused masked attention sk={sk}")
    # and the op itself, called directly with the unpadded mask
    direct = torch.ops.spyre.attention(q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV), scale)
    assert_close_fp(direct, want, what=f"spyre.attention sk={sk}")
