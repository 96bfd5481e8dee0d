"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each oracle function is checked against (a) the known answers the reference's
own tests hold, (b) PyTorch's CPU kernels -- the comparator the reference uses
(tests/_inductor/utils_inductor.py:186-198) -- and (c) closed forms /
invariants / brute force, chosen so a dropped term, a wrong index or a
transposed operand fails.  CPU only.
"""

import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import layout as L
from oracle import ops as O

from helpers import golden, randn, uniform

# --------------------------------------------------------------------------
# SpyreTensorLayout golden vectors: tests/tensor/test_tensor_layout.py:28-94
# --------------------------------------------------------------------------
GOLDEN_STL = [(c["host_size"], c["dim_order"], c["device_size"], c["device_strides"], c["dim_map"])
              for c in golden("spyre_tensor_layout")["cases"]]


@pytest.mark.parametrize("host,order,dsize,dstrides,dmap", GOLDEN_STL)
def test_stl_golden(host, order, dsize, dstrides, dmap):
    ds, dst, dm = L.stl_init(host, 2, order)
    assert ds == dsize
    assert dst == dstrides
    assert dm == dmap


def test_stl_str_golden():
    g = golden("spyre_tensor_layout")["str"]
    ds, dst, dm = L.stl_init(g["host_size"], 2)
    assert L.stl_to_string(ds, dst, dm) == g["text"]


@pytest.mark.parametrize("eb", [1, 2, 4, 8])
def test_stl_closed_form(eb):
    rng = np.random.default_rng(1)
    for _ in range(50):
        n = int(rng.integers(1, 5))
        host = [int(x) for x in rng.integers(1, 200, size=n)]
        order = [int(x) for x in rng.permutation(n)]
        ds, dst, dm = L.stl_init(host, eb, order)
        e = 128 // eb
        assert ds[0] == math.ceil(host[order[-1]] / e) and ds[-1] == e
        assert ds[1:-1] == [host[d] for d in order[:-1]]
        assert dm == [order[-1]] + order[:-1] + [order[-1]]
        assert dst[-1] == 1 and all(dst[i] == dst[i + 1] * ds[i + 1] for i in range(n))


# --------------------------------------------------------------------------
# Allocation sizing: tests/test_spyre.py:171-176 (128 B for a 2-element fp16)
# --------------------------------------------------------------------------
def test_alloc_golden():
    for c in golden("allocation")["cases"]:
        assert L.alloc_nbytes(c["host_size"], c["elem_bytes"]) == c["nbytes"]
    assert L.alloc_nbytes([], 2) == 128
    assert L.alloc_nbytes([512, 4096], 2) == 512 * 4096 * 2
    assert L.alloc_nbytes([8192, 4096], 2) == 64 * 2**20


def test_alloc_closed_form_and_reference_deviation():
    rng = np.random.default_rng(2)
    for _ in range(200):
        n = int(rng.integers(1, 4))
        host = [int(x) for x in rng.integers(1, 300, size=n)]
        eb = int(rng.choice([1, 2, 4]))
        e = 128 // eb
        want = 128 * math.ceil(host[-1] / e) * int(np.prod(host[:-1]))
        assert L.alloc_nbytes(host, eb) == want
        # Never smaller than the dense bytes, and equal for multiples of a stick.
        assert L.alloc_nbytes(host, eb) >= int(np.prod(host)) * eb
    # The reference rule gives one stick to any ragged stick dim, which is
    # smaller than the data for lengths > one stick (spyre_mem.cpp:109-118).
    assert L.alloc_nbytes_reference([100], 2) == 128
    assert L.alloc_nbytes([100], 2) == 256
    assert L.alloc_nbytes_reference([2], 2) == L.alloc_nbytes([2], 2) == 128


# --------------------------------------------------------------------------
# Stick permutation: C restatement vs a brute-force walk over host elements
# --------------------------------------------------------------------------
def _brute_pack(host: np.ndarray, order):
    """Walks host elements, places each at its device offset computed from
    the SpyreTensorLayout strides (dim_map), zero padding elsewhere."""
    eb = host.dtype.itemsize
    ds, dst, dm = L.stl_init(list(host.shape), eb, order)
    e = ds[-1]
    out = np.zeros(int(np.prod(ds)), dtype=host.dtype)
    sd = order[-1]
    for idx in itertools.product(*[range(s) for s in host.shape]):
        off = (idx[sd] // e) * dst[0] + (idx[sd] % e) * dst[-1]
        for j in range(1, len(ds) - 1):
            off += idx[dm[j]] * dst[j]
        out[off] = host[idx]
    return out.view(np.uint8)


@pytest.mark.parametrize("dtype", [np.uint8, np.float16, np.float32, np.int64])
def test_stick_pack_brute_force(dtype):
    rng = np.random.default_rng(3)
    for _ in range(12):
        n = int(rng.integers(1, 4))
        shape = [int(x) for x in rng.integers(1, 9, size=n)]
        shape[-1] = int(rng.integers(1, 150))
        order = [int(x) for x in rng.permutation(n)]
        host = (rng.standard_normal(shape) * 100).astype(dtype)
        packed = L.stick_pack(host, order)
        np.testing.assert_array_equal(packed, _brute_pack(host, order))
        back = L.stick_unpack(packed, shape, dtype, order)
        np.testing.assert_array_equal(back.view(np.uint8), host.view(np.uint8))


def test_stick_pack_strided_source_and_kpanel():
    a = np.arange(7 * 200, dtype=np.float16).reshape(7, 200)
    # Transposed view as the source: strides are honoured.
    t = a.T  # [200, 7]
    np.testing.assert_array_equal(L.stick_pack(t, [0, 1]), _brute_pack(np.ascontiguousarray(t), [0, 1]))
    # dim_order [0, 1] on [M, K] = K panels of 64: device[p, m, e] = A[m, 64p + e].
    dev = L.stick_pack(a, [0, 1]).view(np.float16).reshape(4, 7, 64)
    for p in range(4):
        for m in range(7):
            for e in range(64):
                k = 64 * p + e
                assert dev[p, m, e] == (a[m, k] if k < 200 else 0)


# --------------------------------------------------------------------------
# Softmax
# --------------------------------------------------------------------------
def test_softmax_reference_kat():
    # tests/test_ops.py:430-436: rows of arange(64), softmax over dim 1.
    x = np.tile(np.arange(64, dtype=np.float16), (3, 1))
    got = O.softmax(x, axis=1)
    i = np.arange(64, dtype=np.float64)
    want = np.exp(i - 63) / np.exp(i - 63).sum()
    np.testing.assert_allclose(got, np.tile(want, (3, 1)), rtol=1e-6, atol=1e-9)


def test_softmax_vs_torch_and_invariants():
    x = randn((64, 333), k=1, scale=4.0)
    got = O.softmax(x.numpy(), axis=-1)
    ref = F.softmax(x.float(), dim=-1).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(got.sum(-1), 1.0, rtol=1e-5)
    shifted = O.softmax(x.numpy().astype(np.float32) + 7.0, axis=-1)
    np.testing.assert_allclose(shifted, got, rtol=1e-4, atol=1e-7)
    # dim 0 as well (test_building_blocks.py:33-36 uses dims 0/1/-1)
    np.testing.assert_allclose(O.softmax(x.numpy(), axis=0), F.softmax(x.float(), 0).numpy(),
                               rtol=1e-5, atol=1e-7)
    lg = O.softmax(x.numpy(), axis=-1, log=True)
    np.testing.assert_allclose(lg, F.log_softmax(x.float(), -1).numpy(), rtol=1e-5, atol=1e-5)


def test_softmax_masked_one_hot_and_causal():
    x = np.full((2, 8), -np.inf, dtype=np.float32)
    x[0, 3] = 5.0
    x[1, 0] = -2.0
    np.testing.assert_array_equal(O.softmax(x), np.eye(8, dtype=np.float32)[[3, 0]])
    s = randn((3 * 5, 9), k=2).numpy()  # 3 heads, q_len 5, k_len 9 -> offset 4
    got = O.softmax(s, scale=0.5, causal_q_len=5, causal_offset=4)
    t = torch.from_numpy(s).float().view(3, 5, 9) * 0.5
    mask = torch.ones(5, 9, dtype=torch.bool).tril(diagonal=4)
    ref = F.softmax(t.masked_fill(~mask, float("-inf")), -1).reshape(15, 9).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-7)


# --------------------------------------------------------------------------
# Norms
# --------------------------------------------------------------------------
def test_rmsnorm_vs_torch_and_invariant():
    x, r = randn((16, 200), k=1), randn((16, 200), k=2)
    w = randn((200,), k=3, scale=0.02, mean=1.0)
    y, h = O.rmsnorm(x.numpy(), w.numpy(), 1e-5, residual=r.numpy())
    h_ref = (x + r)  # fp16 add rounds like the kernel's h
    np.testing.assert_array_equal(h, h_ref.float().numpy())
    ref = F.rms_norm(h_ref.float(), (200,), w.float(), 1e-5).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)
    y1, _ = O.rmsnorm(x.numpy(), None, 0.0)
    np.testing.assert_allclose(np.sqrt((y1.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-5)


def test_rmsnorm_linear_vs_torch_composite():
    # the folded norm: unrounded, it is torch's rms_norm then linear; with
    # fp16 staging it moves only the rounding of x * w; swiglu splits the
    # stacked product; eps matters for rows of tiny values
    x = randn((5, 256), k=21)
    x[3] *= 1e-3
    nw = randn((256,), k=22, scale=0.1, mean=1.0)
    w = randn((96, 256), k=23, scale=0.05)
    ref = F.linear(F.rms_norm(x.float(), (256,), nw.float(), 1e-5), w.float()).numpy()
    got = O.rmsnorm_linear(x.numpy(), nw.numpy(), w.numpy(), 1e-5, act_dtype=None)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    wrong_eps = O.rmsnorm_linear(x.numpy(), nw.numpy(), w.numpy(), 1e-6, act_dtype=None)
    assert np.abs(wrong_eps[3] - ref[3]).max() > 1e-2
    half = O.rmsnorm_linear(x.numpy(), nw.numpy(), w.numpy(), 1e-5)
    np.testing.assert_allclose(half, ref, rtol=1e-2, atol=1e-2)
    assert np.abs(half - ref).max() > 0
    sw = O.rmsnorm_linear(x.numpy(), nw.numpy(), w.numpy(), 1e-5, act_dtype=None, swiglu=True)
    np.testing.assert_allclose(sw, F.silu(torch.from_numpy(ref[:, :48])).numpy() * ref[:, 48:],
                               rtol=1e-5, atol=1e-6)


def test_layernorm_vs_torch_and_invariants():
    x, r = randn((16, 300), k=4), randn((16, 300), k=5)
    w = randn((300,), k=6, scale=0.02, mean=1.0)
    b = randn((300,), k=7, scale=0.02)
    y, h, mean, rstd = O.layernorm(x.numpy(), w.numpy(), b.numpy(), 1e-5, residual=r.numpy())
    hr = (x + r).float()
    ref = F.layer_norm(hr, (300,), w.float(), b.float(), 1e-5).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)
    _, m_ref, rs_ref = torch.native_layer_norm(hr, (300,), None, None, 1e-5)
    np.testing.assert_allclose(mean, m_ref.squeeze(-1).numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rstd, rs_ref.squeeze(-1).numpy(), rtol=1e-5)
    y0, *_ = O.layernorm(x.numpy(), None, None, 0.0)
    np.testing.assert_allclose(y0.mean(-1), 0.0, atol=1e-5)
    np.testing.assert_allclose(y0.var(-1), 1.0, rtol=1e-4)


def test_planted_mistakes_fail():
    """Mutations of the oracle formulas (made here, not in oracle/) must be
    caught by the torch comparison: unbiased variance, missing residual
    rounding... each shifts the result beyond tolerance."""
    x = randn((8, 64), k=8)
    hr = x.float()
    ref = F.layer_norm(hr, (64,), None, None, 1e-5).numpy()
    h = x.numpy().astype(np.float64)
    unbiased = (h - h.mean(-1, keepdims=True)) / np.sqrt(h.var(-1, ddof=1, keepdims=True) + 1e-5)
    assert not np.allclose(unbiased, ref, rtol=1e-5, atol=1e-5)
    sm = F.softmax(hr, -1).numpy()
    no_norm = np.exp(h - h.max(-1, keepdims=True))
    assert not np.allclose(no_norm, sm, rtol=1e-2, atol=1e-2)


# --------------------------------------------------------------------------
# GELU chain
# --------------------------------------------------------------------------
def test_gelu_known_values_and_torch():
    v = O.gelu(np.array([0.0, 1.0, -1.0, 3.0], dtype=np.float32))
    np.testing.assert_allclose(v, [0.0, 0.8413447460685429, -0.15865525393145707,
                                   2.9959502751228433], rtol=1e-6, atol=1e-7)
    x = randn((32, 257), k=9)
    s = randn((257,), k=10, scale=0.02, mean=1.0)
    b = randn((257,), k=11, scale=0.02)
    y, r = O.gelu_affine_rowsum(x.numpy(), s.numpy(), b.numpy())
    ref = F.gelu(x.float() * s.float() + b.float())
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(r, ref.sum(-1).numpy(), rtol=1e-5, atol=1e-4)


# --------------------------------------------------------------------------
# GEMM
# --------------------------------------------------------------------------
def test_mm_reference_kat_exact():
    # tests/test_ops.py:265-275: arange(15).view(3,5) @ arange(35).view(5,7).
    a = np.arange(15, dtype=np.float16).reshape(3, 5)
    b = np.arange(35, dtype=np.float16).reshape(5, 7)
    want = np.array([[sum((5 * i + k) * (7 * k + j) for k in range(5)) for j in range(7)]
                     for i in range(3)], dtype=np.float64)
    np.testing.assert_array_equal(O.gemm(a, b), want.astype(np.float32))


def test_gemm_vs_torch_and_brute_force():
    a, b = uniform((9, 13), k=1), uniform((13, 6), k=2)
    c = uniform((6,), k=3)
    got = O.gemm(a.numpy(), b.numpy(), alpha=0.5, beta=2.0, c=c.numpy())
    ref = torch.addmm(c.float(), a.float(), b.float(), beta=2.0, alpha=0.5).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    brute = np.array([[0.5 * sum(float(a[i, k]) * float(b[k, j]) for k in range(13)) +
                       2.0 * float(c[j]) for j in range(6)] for i in range(9)])
    np.testing.assert_allclose(got, brute, rtol=1e-5, atol=1e-5)
    # A transposed operand gives a different answer (catches swapped operands).
    sq_a, sq_b = uniform((8, 8), k=4), uniform((8, 8), k=5)
    assert not np.allclose(O.gemm(sq_a.numpy(), sq_b.numpy()), O.gemm(sq_a.numpy().T, sq_b.numpy()))
    assert np.allclose(O.gemm(sq_a.numpy(), sq_b.numpy(), epilogue="relu"),
                       np.maximum(torch.mm(sq_a.float(), sq_b.float()).numpy(), 0), atol=1e-6)


def test_bmm_vs_torch():
    a, b = uniform((3, 5, 17), k=6), uniform((3, 17, 4), k=7)
    np.testing.assert_allclose(O.gemm(a.numpy(), b.numpy()), torch.bmm(a.float(), b.float()).numpy(),
                               rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------
# RoPE
# --------------------------------------------------------------------------
def test_rope_vs_torch_and_norm_preserved():
    x = randn((6, 2, 16), k=12)
    pos = np.arange(3, 9)
    got = O.rope(x.numpy(), pos, 1e4)
    inv = 1.0 / (1e4 ** (torch.arange(0, 16, 2).float() / 16))
    ang = torch.from_numpy(pos).float()[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[:, None, :]
    xf = x.float()
    rot = torch.cat([-xf[..., 8:], xf[..., :8]], -1)
    ref = (xf * cos + rot * sin).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    pair = lambda z: z[..., :8] ** 2 + z[..., 8:] ** 2  # noqa: E731
    np.testing.assert_allclose(pair(got), pair(xf.numpy()), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(O.rope(x.numpy(), np.zeros(6), 1e4), xf.numpy(), atol=0)


def test_attention_vs_torch_sdpa():
    # oracle.attention against torch's own fused attention routine on the CPU
    # (fp32): causal with stacked query heads, an additive mask, and a
    # transposed-operand mistake that must fail
    g = torch.Generator().manual_seed(7)
    q = torch.randn(3, 4 * 16, 32, generator=g)
    k = torch.randn(3, 16, 32, generator=g)
    v = torch.randn(3, 16, 32, generator=g)
    scale = 1 / math.sqrt(32)
    got = O.attention(q.numpy(), k.numpy(), v.numpy(), scale, causal_q_len=16)
    # stacked heads: row r is query r % 16 of head r // 16
    qh = q.view(3, 4, 16, 32)
    want = F.scaled_dot_product_attention(qh, k[:, None], v[:, None], is_causal=True)
    np.testing.assert_allclose(got, want.reshape(3, 64, 32).numpy(), rtol=1e-5, atol=1e-5)
    mask = torch.randn(64, 16, generator=g)
    mask[mask < -1] = float("-inf")
    mask[:, 0] = 0.0  # every row keeps a key
    got = O.attention(q.numpy(), k.numpy(), v.numpy(), scale, mask=mask.numpy())
    want = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-5, atol=1e-5)
    bad = O.attention(q.numpy(), v.numpy(), k.numpy(), scale, mask=mask.numpy())
    assert not np.allclose(bad, want.numpy(), rtol=1e-3, atol=1e-3)


def test_round_to_bfloat16_matches_torch():
    x = np.concatenate([randn((4096,), k=31, scale=50.0).float().numpy(),
                        np.array([0.0, -0.0, 1.0, 3.0039062, -3.0039062, 65504.0, 1e-40,
                                  np.inf, -np.inf], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O._round_to(x, "bfloat16"), want)
