"""Parity of every HIP kernel with the CPU oracle, called through the C-ABI
(include/spyre_hip.h) on device buffers.  Device memory comes from torch
(plumbing only); the computation is the library's.

Bars: bit-exact for layout / copy / gather / integer work; rtol = atol = 1e-2
against the oracle's fp32 result rounded to the output dtype for fp16 / bf16
floating point (fp32 outputs: 1e-4)."""

import ctypes
import math

import numpy as np
import pytest
import torch

from torch_spyre import _capi

from oracle import layout as L
from oracle import ops as O

from helpers import assert_close_fp, np32, randn, uniform

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _p(t):
    return t.data_ptr() if t is not None else None


def _sync():
    torch.cuda.synchronize()


def _log(msg):
    print(f"[case] {msg}", flush=True)


DT = {torch.float16: _capi.F16, torch.bfloat16: _capi.BF16, torch.float32: _capi.F32}


# ---------------------------------------------------------------------------
# softmax
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols", [(512, 4096), (3, 64), (5, 1), (7, 1000), (33, 7),
                                       (4, 2048), (2, 8192), (2, 12000), (2, 32768), (3, 40000),
                                       (2, 70000)])
def test_softmax_shapes(rows, cols):
    _log(f"softmax {rows}x{cols}")
    x = randn((rows, cols), k=0, scale=4.0)
    xd = x.to(DEV)
    yd = torch.empty_like(xd)
    _capi.call("sph_softmax_rows_f16", _p(xd), _p(yd), rows, cols, _stream())
    _sync()
    assert_close_fp(yd, O.softmax(x.numpy()), what="softmax")
    np.testing.assert_allclose(np32(yd).sum(-1), 1.0, rtol=2e-2)


def test_softmax_reference_kat():
    _log("softmax arange KAT")
    x = torch.arange(0, 64, dtype=torch.float16).unsqueeze(0).repeat(3, 1)
    xd = x.to(DEV)
    yd = torch.empty_like(xd)
    _capi.call("sph_softmax_rows_f16", _p(xd), _p(yd), 3, 64, _stream())
    _sync()
    torch.testing.assert_close(yd.cpu(), torch.softmax(x.float(), 1).half(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("in_dt,out_dt", [(torch.bfloat16, torch.bfloat16),
                                          (torch.float32, torch.float32),
                                          (torch.float16, torch.float32)])
def test_softmax_dtypes_log_scale_strided(in_dt, out_dt):
    _log(f"softmax dtypes {in_dt}->{out_dt}")
    rows, cols, ld = 37, 300, 320
    big = randn((rows, ld), k=1, scale=3.0, dtype=in_dt)
    xd = big.to(DEV)
    yd = torch.zeros(rows, ld + 8, dtype=out_dt, device=DEV)
    for flags in (0, _capi.SOFTMAX_LOG):
        _capi.call("sph_softmax_rows", DT[in_dt], DT[out_dt], _p(xd), ld, _p(yd), ld + 8,
                   rows, cols, 0.5, flags, 0, 0, _stream())
        _sync()
        want = O.softmax(big[:, :cols].float().numpy(), scale=0.5, log=bool(flags))
        tol = 1e-4 if out_dt == torch.float32 and in_dt == torch.float32 else 1e-2
        assert_close_fp(yd[:, :cols], want, out_dtype=out_dt, rtol=tol, atol=tol,
                        what=f"softmax flags={flags}")
        assert torch.all(yd[:, cols:].cpu() == 0)  # nothing written past cols


@pytest.mark.parametrize("in_dt,out_dt", [(torch.float16, torch.float16),
                                          (torch.bfloat16, torch.bfloat16),
                                          (torch.float32, torch.float32),
                                          (torch.float16, torch.float32)])
@pytest.mark.parametrize("cols", [512, 2048, 4096])
def test_softmax_whole_rows(in_dt, out_dt, cols):
    # rows of exactly one register configuration's width take the path
    # without per-chunk bounds tests: strided rows, a partial last group of
    # rows (several rows per workgroup at 512 / 2048 columns), log, scale and
    # the causal mask
    rows, ld = 9, cols + 64
    _log(f"softmax whole rows {in_dt}->{out_dt} cols={cols}")
    big = randn((rows, ld), k=4, scale=3.0, dtype=in_dt)
    xd = big.to(DEV)
    for flags, q_len in ((0, 0), (_capi.SOFTMAX_LOG, 0), (_capi.SOFTMAX_CAUSAL, 3)):
        yd = torch.zeros(rows, ld, dtype=out_dt, device=DEV)
        off = cols - 3 - 100 if q_len else 0
        _capi.call("sph_softmax_rows", DT[in_dt], DT[out_dt], _p(xd), ld, _p(yd), ld,
                   rows, cols, 0.5, flags, q_len, off, _stream())
        _sync()
        want = O.softmax(big[:, :cols].float().numpy(), scale=0.5, log=flags == _capi.SOFTMAX_LOG,
                         causal_q_len=q_len, causal_offset=off)
        tol = 1e-4 if out_dt == torch.float32 and in_dt == torch.float32 else 1e-2
        assert_close_fp(yd[:, :cols], want, out_dtype=out_dt, rtol=tol, atol=tol,
                        what=f"softmax whole rows flags={flags}")
        assert torch.all(yd[:, cols:].cpu() == 0)


@pytest.mark.parametrize("q_len,k_len", [(5, 9), (2048, 2048), (1, 1152), (7, 64)])
def test_softmax_causal(q_len, k_len):
    _log(f"softmax causal {q_len}x{k_len}")
    heads = 4 if q_len < 2048 else 2
    x = randn((heads * q_len, k_len), k=2)
    xd = x.to(DEV)
    yd = torch.empty_like(xd)
    off = k_len - q_len
    _capi.call("sph_softmax_rows", _capi.F16, _capi.F16, _p(xd), k_len, _p(yd), k_len,
               heads * q_len, k_len, 0.125, _capi.SOFTMAX_CAUSAL, q_len, off, _stream())
    _sync()
    want = O.softmax(x.numpy(), scale=0.125, causal_q_len=q_len, causal_offset=off)
    assert_close_fp(yd, want, what="causal softmax")


# ---------------------------------------------------------------------------
# norms
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols", [(8192, 4096), (3, 64), (17, 100), (4, 4097),
                                       (2, 20000), (2, 40000), (2, 70000), (64, 1)])
@pytest.mark.parametrize("residual", [False, True])
def test_rmsnorm(rows, cols, residual):
    _log(f"rmsnorm {rows}x{cols} residual={residual}")
    x = randn((rows, cols), k=0)
    r = randn((rows, cols), k=1) if residual else None
    w = randn((cols,), k=2, scale=0.02, mean=1.0)
    xd, wd = x.to(DEV), w.to(DEV)
    rd = r.to(DEV) if residual else None
    yd = torch.empty_like(xd)
    hd = torch.empty_like(xd) if residual else None
    rstd = torch.empty(rows, dtype=torch.float32, device=DEV)
    _capi.call("sph_rmsnorm", _capi.F16, _capi.F16, _p(xd), _p(rd), _p(wd), _p(yd), _p(hd),
               _p(rstd), rows, cols, 1e-5, _stream())
    _sync()
    y, h = O.rmsnorm(x.numpy(), w.numpy(), 1e-5, residual=r.numpy() if residual else None)
    assert_close_fp(yd, y, what="rmsnorm y")
    if residual:
        # h is a plain fp16 add: bit-exact
        assert torch.equal(hd.cpu(), (x + r))


@pytest.mark.parametrize("rows,cols", [(8192, 4096), (5, 300), (3, 8), (2, 20000), (2, 70000)])
@pytest.mark.parametrize("residual", [False, True])
def test_layernorm(rows, cols, residual):
    _log(f"layernorm {rows}x{cols} residual={residual}")
    x = randn((rows, cols), k=3)
    r = randn((rows, cols), k=4) if residual else None
    w = randn((cols,), k=5, scale=0.02, mean=1.0)
    b = randn((cols,), k=6, scale=0.02)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    rd = r.to(DEV) if residual else None
    yd = torch.empty_like(xd)
    hd = torch.empty_like(xd) if residual else None
    mean = torch.empty(rows, dtype=torch.float32, device=DEV)
    rstd = torch.empty(rows, dtype=torch.float32, device=DEV)
    _capi.call("sph_layernorm", _capi.F16, _capi.F16, _p(xd), _p(rd), _p(wd), _p(bd), _p(yd),
               _p(hd), _p(mean), _p(rstd), rows, cols, 1e-5, _stream())
    _sync()
    y, h, m, rs = O.layernorm(x.numpy(), w.numpy(), b.numpy(), 1e-5,
                              residual=r.numpy() if residual else None)
    assert_close_fp(yd, y, what="layernorm y")
    np.testing.assert_allclose(mean.cpu().numpy(), m, rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(rstd.cpu().numpy(), rs, rtol=1e-3, atol=1e-3)
    if residual:
        assert torch.equal(hd.cpu(), (x + r))


def test_norm_fp32_weight_and_bf16():
    _log("norm fp32 weight / bf16")
    x = randn((9, 256), k=7)
    w = randn((256,), k=8, scale=0.02, mean=1.0, dtype=torch.float32)
    xd, wd = x.to(DEV), w.to(DEV)
    yd = torch.empty_like(xd)
    _capi.call("sph_rmsnorm", _capi.F16, _capi.F32, _p(xd), None, _p(wd), _p(yd), None, None,
               9, 256, 1e-6, _stream())
    _sync()
    assert_close_fp(yd, O.rmsnorm(x.numpy(), w.numpy(), 1e-6)[0])
    xb = randn((9, 256), k=9, dtype=torch.bfloat16)
    xbd = xb.to(DEV)
    ybd = torch.empty_like(xbd)
    _capi.call("sph_layernorm", _capi.BF16, _capi.F32, _p(xbd), None, _p(wd), None, _p(ybd),
               None, None, None, 9, 256, 1e-5, _stream())
    _sync()
    assert_close_fp(ybd, O.layernorm(xb.float().numpy(), w.numpy(), None, 1e-5)[0],
                    out_dtype=torch.bfloat16, rtol=2e-2, atol=2e-2)


# ---------------------------------------------------------------------------
# GELU chain
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols", [(8192, 4096), (3, 100), (2, 70000), (7, 2048), (5, 8192),
                                       (2, 16384), (2, 50000)])
def test_gelu_affine_rowsum(rows, cols):
    _log(f"gelu_rowsum {rows}x{cols}")
    x = randn((rows, cols), k=0)
    s = randn((cols,), k=1, scale=0.02, mean=1.0)
    b = randn((cols,), k=2, scale=0.02)
    xd, sd, bd = x.to(DEV), s.to(DEV), b.to(DEV)
    yd = torch.empty_like(xd)
    rd = torch.empty(rows, dtype=torch.float16, device=DEV)
    _capi.call("sph_gelu_affine_rowsum_f16", _p(xd), _p(sd), _p(bd), _p(yd), _p(rd), rows, cols,
               _stream())
    _sync()
    y, r = O.gelu_affine_rowsum(x.numpy(), s.numpy(), b.numpy())
    assert_close_fp(yd, y, what="gelu y")
    assert_close_fp(rd, r, what="gelu rowsum")


def test_gelu_whole_row_bf16_and_tails():
    # whole-row path (cols = 2048 * k) in bf16, and the GELU tails: x over
    # [-12, 12] against the oracle's erf form (the device evaluates erfc by
    # Abramowitz & Stegun 7.1.26, absolute error below 5e-7)
    _log("gelu whole-row bf16 / tails")
    rows, cols = 6, 4096
    x = (torch.linspace(-12, 12, rows * cols).view(rows, cols)).to(torch.bfloat16)
    s = torch.ones(cols, dtype=torch.bfloat16)
    b = torch.zeros(cols, dtype=torch.bfloat16)
    xd, sd, bd = x.to(DEV), s.to(DEV), b.to(DEV)
    yd = torch.empty_like(xd)
    rd = torch.empty(rows, dtype=torch.bfloat16, device=DEV)
    _capi.call("sph_gelu_affine_rowsum", _capi.BF16, _p(xd), _p(sd), _p(bd), 1.0, 0.0, _p(yd),
               _p(rd), rows, cols, _stream())
    _sync()
    y, r = O.gelu_affine_rowsum(x.float().numpy(), s.float().numpy(), b.float().numpy())
    assert_close_fp(yd, y, out_dtype=torch.bfloat16, rtol=2e-2, atol=2e-2, what="gelu bf16 y")
    assert_close_fp(rd, r, out_dtype=torch.bfloat16, rtol=2e-2, atol=2e-2, what="gelu bf16 rowsum")
    xf = torch.linspace(-12, 12, 4 * 2048).view(4, 2048).half()
    xd = xf.to(DEV)
    yd = torch.empty_like(xd)
    _capi.call("sph_gelu_affine_rowsum", _capi.F16, _p(xd), None, None, 1.0, 0.0, _p(yd), None,
               4, 2048, _stream())
    _sync()
    y, _ = O.gelu_affine_rowsum(xf.float().numpy(), np.float32(1.0), np.float32(0.0))
    assert_close_fp(yd, y, rtol=1e-3, atol=1e-3, what="gelu tails")


def test_gelu_scalar_affine():
    _log("gelu scalar s,b")
    x = randn((4, 512), k=3)
    xd = x.to(DEV)
    yd = torch.empty_like(xd)
    rd = torch.empty(4, dtype=torch.float16, device=DEV)
    _capi.call("sph_gelu_affine_rowsum", _capi.F16, _p(xd), None, None, 1.5, -0.25, _p(yd),
               _p(rd), 4, 512, _stream())
    _sync()
    y, r = O.gelu_affine_rowsum(x.numpy(), np.float32(1.5), np.float32(-0.25))
    assert_close_fp(yd, y)
    assert_close_fp(rd, r)


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
def _gemm(a, b, trans_a=False, trans_b=False, alpha=1.0, beta=0.0, c=None, crow=0, ccol=0,
          epi=0, dtype=torch.float16):
    """a/b are device tensors holding op(A)/op(B) in their storage layout."""
    m = a.shape[1] if trans_a else a.shape[0]
    k = a.shape[0] if trans_a else a.shape[1]
    n = b.shape[0] if trans_b else b.shape[1]
    d = torch.empty(m, n, dtype=dtype, device=DEV)
    _capi.call("sph_gemm", DT[dtype], int(trans_a), int(trans_b), m, n, k, alpha, _p(a),
               a.stride(0), _p(b), b.stride(0), beta, _p(c), crow, ccol, _p(d), n, epi, _stream())
    _sync()
    return d


def test_gemm_reference_kat_exact():
    _log("gemm arange KAT")
    x = torch.arange(15, dtype=torch.float16).view(3, 5)
    y = torch.arange(35, dtype=torch.float16).view(5, 7)
    d = _gemm(x.to(DEV), y.to(DEV))
    want = O.gemm(x.numpy(), y.numpy())
    assert torch.equal(d.cpu().float(), torch.from_numpy(want))  # exact in fp32 accumulate


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 4096), (256, 256, 64), (300, 200, 70),
                                   (1, 1, 1), (5, 7, 3), (129, 65, 257), (2048, 1024, 128),
                                   (64, 49155, 64)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_shapes_transposes(m, n, k, ta, tb):
    _log(f"gemm {m}x{n}x{k} ta={ta} tb={tb}")
    A = uniform((m, k), k=1)
    B = uniform((k, n), k=2)
    a_store = A.t().contiguous() if ta else A
    b_store = B.t().contiguous() if tb else B
    d = _gemm(a_store.to(DEV), b_store.to(DEV), ta, tb)
    assert_close_fp(d, O.gemm(A.numpy(), B.numpy()), what=f"gemm ta={ta} tb={tb}")


@pytest.mark.parametrize("epi,name", [(0, "none"), (1, "relu"), (2, "gelu"), (3, "silu")])
def test_gemm_bias_alpha_beta_epilogue(epi, name):
    _log(f"gemm epilogue {name}")
    m, n, k = 96, 80, 136
    A, B = uniform((m, k), k=3), uniform((k, n), k=4)
    bias = uniform((n,), k=5)
    d = _gemm(A.to(DEV), B.to(DEV), alpha=0.5, beta=1.5, c=bias.to(DEV), crow=0, ccol=1, epi=epi)
    want = O.gemm(A.numpy(), B.numpy(), alpha=0.5, beta=1.5, c=bias.numpy()[None, :], epilogue=name)
    assert_close_fp(d, want, what=f"epilogue {name}")
    C = uniform((m, n), k=6)
    d2 = _gemm(A.to(DEV), B.to(DEV), beta=-1.0, c=C.to(DEV), crow=n, ccol=1)
    assert_close_fp(d2, O.gemm(A.numpy(), B.numpy(), beta=-1.0, c=C.numpy()))


@pytest.mark.parametrize("m,n,k,tb,pad", [(256, 512, 192, False, 0), (512, 256, 320, True, 0),
                                          (256, 256, 64, True, 8), (512, 768, 128, False, 64),
                                          (2048, 4096, 12800, True, 0), (768, 1024, 4096, False, 0),
                                          (512, 384, 192, False, 0), (256, 128, 64, True, 8),
                                          (2048, 4096, 512, False, 0), (1024, 640, 256, True, 0),
                                          (2048, 8192, 1216, False, 8), (4096, 4096, 64, True, 0),
                                          (4096, 4096, 4096, False, 0)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_whole_tile_direct_load(m, n, k, tb, pad, dtype):
    # whole 256-row tiles with K-contiguous A run the direct-to-LDS kernel,
    # 256 or 128 columns wide (n = 384, 128, 640 only fit 128; 2048 x 4096
    # picks 128 for a full round of tiles): odd and even K-tile counts (k/64 =
    # 1, 2, 3, 5, 8, 19, 64, 200), row-major and K-contiguous B, leading
    # dimensions wider than the matrix (pad); c2's 4096^3 through the C-ABI
    _log(f"gemm direct-load {m}x{n}x{k} tb={tb} pad={pad} {dtype}")
    A = uniform((m, k), k=21, dtype=dtype)
    B = uniform((k, n), k=22, dtype=dtype)
    if k > 2048:
        B = (B.float() * 0.05).to(dtype)
    bst = B.t().contiguous() if tb else B
    a_buf = torch.zeros(m, k + pad, dtype=dtype)
    a_buf[:, :k] = A
    b_buf = torch.zeros(bst.shape[0], bst.shape[1] + pad, dtype=dtype)
    b_buf[:, :bst.shape[1]] = bst
    ad, bd = a_buf.to(DEV), b_buf.to(DEV)
    d = torch.empty(m, n, dtype=dtype, device=DEV)
    _capi.call("sph_gemm", DT[dtype], 0, int(tb), m, n, k, 1.0, _p(ad), k + pad, _p(bd),
               bst.shape[1] + pad, 0.0, None, 0, 0, _p(d), n, 0, _stream())
    _sync()
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(d, O.gemm(A.float().numpy(), B.float().numpy()), out_dtype=dtype,
                    what="direct-load gemm", **tol)


@pytest.mark.parametrize("batch,m,n,k,tb,pad", [(1, 128, 128, 64, False, 0), (2, 256, 384, 64, True, 8),
                                                (3, 384, 128, 128, False, 64), (4, 128, 256, 128, True, 0),
                                                (32, 2048, 2048, 128, True, 0),
                                                (9, 768, 1280, 128, False, 64),
                                                (40, 1664, 256, 64, True, 8),
                                                (24, 512, 768, 64, True, 8),
                                                (12, 1024, 2048, 64, False, 0)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_short_k(batch, m, n, k, tb, pad, dtype):
    # K = 64 / 128 on whole 128x128 tiles: the short-K kernel (attention
    # scores), batched, both B layouts, padded leading dimensions.  From 512
    # tiles up the persistent ring kernel runs: runs of 2-6 tiles that start
    # and end inside tile rows (540 / 576 / 1536 tiles), 2-tile rows that
    # switch A panels every other tile (1040 tiles).
    _log(f"gemm short-K b={batch} {m}x{n}x{k} tb={tb} pad={pad} {dtype}")
    A = uniform((batch, m, k), k=31, dtype=dtype)
    B = uniform((batch, k, n), k=32, dtype=dtype)
    bst = B.transpose(1, 2).contiguous() if tb else B
    a_buf = torch.zeros(batch, m, k + pad, dtype=dtype)
    a_buf[:, :, :k] = A
    b_buf = torch.zeros(batch, bst.shape[1], bst.shape[2] + pad, dtype=dtype)
    b_buf[:, :, :bst.shape[2]] = bst
    ad, bd = a_buf.to(DEV), b_buf.to(DEV)
    out = torch.empty(batch, m, n, dtype=dtype, device=DEV)
    lda, ldb = k + pad, bst.shape[2] + pad
    _capi.call("sph_gemm_strided_batched", DT[dtype], 0, int(tb), batch, m, n, k, 1.0, _p(ad), lda,
               a_buf[0].numel(), _p(bd), ldb, b_buf[0].numel(), 0.0, None, 0, 0, 0, _p(out), n,
               m * n, 0, _stream())
    _sync()
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(out, O.gemm(A.float().numpy(), B.float().numpy()), out_dtype=dtype,
                    what="short-K gemm", **tol)


@pytest.mark.parametrize("tb", [False, True])
def test_gemm_whole_tile_epilogue_and_batch(tb):
    # direct-load kernel with alpha / beta / per-column C / SiLU, and batched
    _log(f"gemm direct-load epilogue/batch tb={tb}")
    m, n, k = 512, 256, 256
    A, B = uniform((m, k), k=23), uniform((k, n), k=24)
    bias = uniform((n,), k=25)
    bst = B.t().contiguous() if tb else B
    d = _gemm(A.to(DEV), bst.to(DEV), trans_b=tb, alpha=0.5, beta=1.5, c=bias.to(DEV), crow=0,
              ccol=1, epi=3)
    want = O.gemm(A.numpy(), B.numpy(), alpha=0.5, beta=1.5, c=bias.numpy()[None, :],
                  epilogue="silu")
    assert_close_fp(d, want, what="direct-load silu epilogue")
    batch = 3
    Ab, Bb = uniform((batch, m, k), k=26), uniform((batch, k, n), k=27)
    ad = Ab.to(DEV)
    bd = (Bb.transpose(1, 2).contiguous() if tb else Bb).to(DEV)
    out = torch.empty(batch, m, n, dtype=torch.float16, device=DEV)
    _capi.call("sph_gemm_strided_batched", _capi.F16, 0, int(tb), batch, m, n, k, 1.0, _p(ad), k,
               m * k, _p(bd), k if tb else n, k * n, 0.0, None, 0, 0, 0, _p(out), n, m * n, 0,
               _stream())
    _sync()
    assert_close_fp(out, O.gemm(Ab.numpy(), Bb.numpy()), what="direct-load batched")


@pytest.mark.parametrize("batch,m,n,k,pad,epi,dtype", [
    (1, 2048, 6144, 4096, 0, 0, torch.float16),     # c4 QKV: 256 tiles of 256 x 192
    (1, 4096, 6144, 512, 8, 2, torch.float16),      # 512 tiles, padded rows, GELU
    (1, 2048, 6144, 1216, 0, 3, torch.bfloat16),    # bf16, SiLU, 19 K tiles
    (2, 1024, 6144, 256, 0, 0, torch.float16)])     # batched: 2 x 128 tiles
def test_gemm_192_wide_tiles(batch, m, n, k, pad, epi, dtype):
    # K-contiguous B whose 256-wide tiles leave a partial round and whose
    # 192-wide ones fill whole rounds runs 256 x 192 tiles (8 waves of 128 x
    # 48): alpha, beta * C (a bias row), activation; with and without a
    # workspace (the 192-wide tiles take precedence over a split-K tail)
    _log(f"gemm 192-wide {batch}x{m}x{n}x{k} pad={pad} epi={epi} {dtype}")
    A = uniform((batch, m, k), k=31, dtype=dtype)
    W = (uniform((batch, n, k), k=32, dtype=dtype).float() * 0.05).to(dtype)
    bias = uniform((n,), k=33, dtype=dtype)
    a_buf = torch.zeros(batch, m, k + pad, dtype=dtype)
    a_buf[:, :, :k] = A
    w_buf = torch.zeros(batch, n, k + pad, dtype=dtype)
    w_buf[:, :, :k] = W
    ad, wd, bd = a_buf.to(DEV), w_buf.to(DEV), bias.to(DEV)
    want = O.gemm(A.float().numpy(), np.swapaxes(W.float().numpy(), 1, 2), alpha=0.75, beta=0.5,
                  c=bias.float().numpy()[None, None, :],
                  epilogue={0: "none", 2: "gelu", 3: "silu"}[epi])
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    lib = _capi.lib()
    nws = lib.sph_gemm_workspace_bytes(1, m, n, k) if batch == 1 else 0
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=DEV)
    outs = []
    for w_ptr, w_n in ((None, 0), (_p(ws), nws)):
        d = torch.empty(batch, m, n, dtype=dtype, device=DEV)
        _capi.call("sph_gemm_ex", DT[dtype], 0, 1, batch, m, n, k, 0.75, _p(ad), k + pad,
                   a_buf[0].numel(), _p(wd), k + pad, w_buf[0].numel(), 0.5, _p(bd), 0, 1, 0,
                   _p(d), n, m * n, epi, w_ptr if w_n else None, w_n, _stream())
        _sync()
        assert_close_fp(d, want, out_dtype=dtype, what="192-wide gemm", **tol)
        outs.append(d)
    assert torch.equal(outs[0], outs[1]), "the workspace changed the 192-wide result"


@pytest.mark.parametrize("batch,m,n,k,tb,pad,epi,dtype", [
    (1, 2048, 4096, 4096, 1, 0, 0, torch.float16),   # c4 O (no workspace): 256 tiles of 256 x 128
    (1, 2048, 4096, 4096, 0, 0, 3, torch.bfloat16),  # row-major B, bf16, SiLU
    (2, 1024, 2048, 1024, 1, 8, 2, torch.float16),   # batched, padded rows, GELU
    (3, 512, 1024, 512, 0, 8, 3, torch.bfloat16),    # batched row-major B, bf16
    (1, 512, 384, 192, 0, 0, 0, torch.float16)])     # N % 256 != 0: 6 tiles, 3 K tiles
def test_gemm_128_wide_tiles(batch, m, n, k, tb, pad, epi, dtype):
    # shapes whose 256-wide tiles leave most CUs idle and that have no
    # split-K workspace run 256 x 128 tiles (8 waves of 128 x 32): alpha,
    # beta * C (a bias row), activation
    _log(f"gemm 128-wide {batch}x{m}x{n}x{k} tb={tb} pad={pad} epi={epi} {dtype}")
    A = uniform((batch, m, k), k=34, dtype=dtype)
    ld_b = (k if tb else n) + pad
    W = (uniform((batch, n, k) if tb else (batch, k, n), k=35, dtype=dtype).float() * 0.05).to(dtype)
    bias = uniform((n,), k=36, dtype=dtype)
    a_buf = torch.zeros(batch, m, k + pad, dtype=dtype)
    a_buf[:, :, :k] = A
    w_buf = torch.zeros(*W.shape[:2], ld_b, dtype=dtype)
    w_buf[:, :, :W.shape[2]] = W
    ad, wd, bd = a_buf.to(DEV), w_buf.to(DEV), bias.to(DEV)
    wf = W.float().numpy()
    want = O.gemm(A.float().numpy(), np.swapaxes(wf, 1, 2) if tb else wf, alpha=0.75, beta=0.5,
                  c=bias.float().numpy()[None, None, :],
                  epilogue={0: "none", 2: "gelu", 3: "silu"}[epi])
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    d = torch.empty(batch, m, n, dtype=dtype, device=DEV)
    _capi.call("sph_gemm_ex", DT[dtype], 0, tb, batch, m, n, k, 0.75, _p(ad), k + pad,
               a_buf[0].numel(), _p(wd), ld_b, w_buf[0].numel(), 0.5, _p(bd), 0, 1, 0,
               _p(d), n, m * n, epi, None, 0, _stream())
    _sync()
    assert_close_fp(d, want, out_dtype=dtype, what="128-wide gemm", **tol)


@pytest.mark.parametrize("m,n,k,c_lay,epi,dtype,split", [
    (4096, 4096, 1024, "row", 0, torch.float16, False),      # 256-wide tiles: 16-byte C reads
    (1024, 2048, 1024, "row", 3, torch.bfloat16, False),     # 128-wide tiles, bf16
    (2048, 6144, 512, "row", 2, torch.float16, False),       # 192-wide tiles
    (4096, 4096, 1024, "row_off", 0, torch.float16, False),  # C rows not 16-byte aligned
    (512, 2048, 1024, "col", 3, torch.float16, False),       # column-major C: per element
    (200, 328, 96, "row", 2, torch.bfloat16, False),         # register-staged kernel, ragged
    (768, 512, 2048, "row", 3, torch.float16, True),         # split-K tail: C in the reduce
    (768, 512, 2048, "col", 2, torch.bfloat16, True)])
def test_gemm_full_c_epilogue(m, n, k, c_lay, epi, dtype, split):
    # D = epi(alpha A B^T + beta C) with a whole matrix C (a residual): the
    # epilogue reads row-major, 16-byte aligned C rows 16 bytes a lane ahead
    # of the stores, other layouts element by element; with a workspace the
    # split-K reduce applies the same epilogue
    _log(f"gemm full C {m}x{n}x{k} {c_lay} epi={epi} {dtype} split={split}")
    A = uniform((m, k), k=37, dtype=dtype)
    W = (uniform((n, k), k=38, dtype=dtype).float() * 0.05).to(dtype)
    Cm = uniform((m, n), k=39, dtype=dtype)
    ad, wd = A.to(DEV), W.to(DEV)
    if c_lay == "col":
        cbuf = Cm.t().contiguous().to(DEV)           # C[i, j] at j * m + i
        c_ptr, ldc_r, ldc_c = _p(cbuf), 1, m
    else:
        off = 1 if c_lay == "row_off" else 0
        cbuf = torch.zeros(m * n + off, dtype=dtype)
        cbuf[off:] = Cm.reshape(-1)
        cbuf = cbuf.to(DEV)
        c_ptr, ldc_r, ldc_c = _p(cbuf) + off * cbuf.element_size(), n, 1
    want = O.gemm(A.float().numpy(), W.float().numpy().T, alpha=0.75, beta=0.5,
                  c=Cm.float().numpy(), epilogue={0: "none", 2: "gelu", 3: "silu"}[epi])
    nws = _capi.lib().sph_gemm_workspace_bytes(1, m, n, k) if split else 0
    assert (nws > 0) == split
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=DEV)
    d = torch.empty(m, n, dtype=dtype, device=DEV)
    _capi.call("sph_gemm_ex", DT[dtype], 0, 1, 1, m, n, k, 0.75, _p(ad), k, 0, _p(wd), k, 0,
               0.5, c_ptr, ldc_r, ldc_c, 0, _p(d), n, 0, epi, _p(ws) if nws else None, nws,
               _stream())
    _sync()
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(d, want, out_dtype=dtype, what=f"gemm full C ({c_lay})", **tol)


def test_gemm_bf16_and_unaligned_ld():
    _log("gemm bf16 / unaligned")
    A, B = uniform((70, 45), k=7, dtype=torch.bfloat16), uniform((45, 33), k=8, dtype=torch.bfloat16)
    d = _gemm(A.to(DEV), B.to(DEV), dtype=torch.bfloat16)
    assert_close_fp(d, O.gemm(A.float().numpy(), B.float().numpy()), out_dtype=torch.bfloat16,
                    rtol=2e-2, atol=2e-2)
    # row-major views with odd leading dims (no 16-byte vector path)
    big = uniform((70, 51), k=9)
    Av = big.to(DEV)[:, 3:48]
    Bd = uniform((45, 33), k=10).to(DEV)
    m, k, n = 70, 45, 33
    dd = torch.empty(m, n, dtype=torch.float16, device=DEV)
    _capi.call("sph_gemm", _capi.F16, 0, 0, m, n, k, 1.0, Av.data_ptr(), 51, _p(Bd), 33, 0.0, None,
               0, 0, _p(dd), n, 0, _stream())
    _sync()
    assert_close_fp(dd, O.gemm(big[:, 3:48].numpy(), Bd.cpu().numpy()))


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (4, 1024, 4096), (4, 12800, 4096),
                                   (4, 4096, 12800), (3, 49155, 64), (8, 777, 2056),
                                   (13, 33, 8), (16, 520, 136)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_small_m_weight_layout(m, n, k, dtype):
    # decode-step shapes: x[M,K] @ W[N,K]^T, both K-contiguous (streaming
    # small-M kernel), including K tails (k % 2048 != 0) and odd N
    _log(f"gemm small-M {m}x{n}x{k} {dtype}")
    X = uniform((m, k), k=11, dtype=dtype)
    W = (uniform((n, k), k=12) * 0.05).to(dtype)
    d = _gemm(X.to(DEV), W.to(DEV), trans_b=True, dtype=dtype)
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(d, O.gemm(X.float().numpy(), W.float().numpy().T), out_dtype=dtype,
                    what=f"small-M {dtype}", **tol)


@pytest.mark.parametrize("m,n,k", [(4, 25600, 4096), (4, 49155, 4096), (5, 16400, 2056),
                                   (8, 4100, 8192), (2, 32770, 1024), (3, 4097, 8192),
                                   (1, 4100, 8200), (4, 6144, 4096), (4, 4096, 4096),
                                   (4, 4096, 12800), (4, 2100, 4096), (2, 1030, 16384),
                                   (8, 2050, 8200)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_stream_decode_shapes(m, n, k, dtype):
    # the persistent weight-stream kernel (batch 1, M <= 8, K >= 1024):
    # K not a multiple of the 512-element lane sweep, N off the 16 waves of
    # a workgroup, several rows per wave; leftover rows split along K over
    # 2 to 16 waves (N % 4096 of 1024, 16, 3, 2 rows), every row split
    # (N below one round), no leftover (N = 4096), whole rounds of 12 or 10
    # waves per workgroup (N = 6144, 25600); K at the LDS staging
    # limits (16384 for M <= 4, 8192 for M <= 8) and past them (M = 8,
    # K = 8200: the small-M kernel)
    _log(f"gemm stream {m}x{n}x{k} {dtype}")
    X = uniform((m, k), k=21, dtype=dtype)
    W = (uniform((n, k), k=22) * 0.05).to(dtype)
    d = _gemm(X.to(DEV), W.to(DEV), trans_b=True, dtype=dtype)
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(d, O.gemm(X.float().numpy(), W.float().numpy().T), out_dtype=dtype,
                    what=f"stream {dtype}", **tol)


@pytest.mark.parametrize("n,k", [(8192, 4096), (6144, 4096), (4096, 12800)])
def test_gemm_stream_epilogue(n, k):
    _log(f"gemm stream epilogue n={n} k={k}")
    m = 4
    X, W = uniform((m, k), k=23), uniform((n, k), k=24) * 0.02
    bias = uniform((n,), k=25)
    d = _gemm(X.to(DEV), W.to(DEV), trans_b=True, alpha=0.5, beta=1.5, c=bias.to(DEV), crow=0,
              ccol=1, epi=3)
    want = O.gemm(X.numpy(), W.numpy().T, alpha=0.5, beta=1.5, c=bias.numpy()[None, :],
                  epilogue="silu")
    assert_close_fp(d, want, what="stream silu epilogue")
    # the decode residual: D = x W^T + H with a full [m, n] H
    H = uniform((m, n), k=26)
    d2 = _gemm(X.to(DEV), W.to(DEV), trans_b=True, beta=1.0, c=H.to(DEV), crow=n, ccol=1)
    assert_close_fp(d2, O.gemm(X.numpy(), W.numpy().T, beta=1.0, c=H.numpy()),
                    what="stream residual epilogue")


@pytest.mark.parametrize("m,n,k,pad", [(256, 128, 64, 0), (512, 384, 256, 8), (1024, 1280, 4096, 0),
                                       (768, 256, 1024, 16), (256, 1280, 2048, 8),
                                       (4, 12800, 4096, 0), (1, 300, 64, 8),
                                       (8, 1000, 2056, 0), (5, 4100, 8192, 16)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_swiglu(m, n, k, pad, dtype):
    # silu(x Wg^T) * (x Wu^T) from one [2n, k] weight (gate rows first),
    # padded leading dims on every operand; whole 256-row tiles (direct-load
    # GEMM) and decode rows (m <= 8, weight-stream kernel)
    _log(f"gemm swiglu {m}x{n}x{k} pad={pad} {dtype}")
    X = uniform((m, k), k=31, dtype=dtype)
    W = (uniform((2 * n, k), k=32) * 0.05).to(dtype)
    xd = torch.zeros(m, k + pad, dtype=dtype, device=DEV)
    xd[:, :k] = X.to(DEV)
    wd = torch.zeros(2 * n, k + pad, dtype=dtype, device=DEV)
    wd[:, :k] = W.to(DEV)
    d = torch.full((m, n + pad), 7.0, dtype=dtype, device=DEV)
    nws = _capi.lib().sph_gemm_swiglu_workspace_bytes(m, n, k)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=DEV)
    _capi.call("sph_gemm_swiglu", DT[dtype], m, n, k, _p(xd), k + pad, _p(wd), k + pad, _p(d),
               n + pad, _p(ws), nws, _stream())
    _sync()
    xf, wf = X.float().numpy(), W.float().numpy()
    want = O.silu(O.gemm(xf, wf[:n].T)) * O.gemm(xf, wf[n:].T)
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(d[:, :n], want, out_dtype=dtype, what=f"swiglu {dtype}", **tol)
    if pad:
        assert bool((d[:, n:] == 7.0).all()), "padding columns written"


@pytest.mark.parametrize("m,n,k,tb,epi,dtype", [
    (2048, 4096, 12800, True, 0, torch.float16),   # 128 tiles, 2 K slices (c4 down shape)
    (1024, 4096, 8192, False, 3, torch.bfloat16),  # row-major B, bf16: 64 tiles, 4 slices
    (768, 512, 2048, False, 2, torch.float16),     # 6 tiles, 8 K slices
    (512, 1024, 12800, True, 0, torch.float16),    # 8 tiles, 200 K tiles in 8 slices
    (256, 256, 2048, True, 3, torch.float16),      # one tile
    (2048, 10240, 2048, True, 0, torch.float16),   # 320 tiles: a full round, then 64 in 4 slices
    (2048, 10240, 2048, False, 2, torch.bfloat16)])
def test_gemm_splitk_tail(m, n, k, tb, epi, dtype):
    # sph_gemm_ex with a workspace: the partial last round of 256 x 256
    # tiles runs as K slices plus a reduce (alpha, beta*C with a bias row,
    # activation applied there); against the oracle and the call without a
    # workspace
    _log(f"gemm split-K tail {m}x{n}x{k} tb={tb} epi={epi} {dtype}")
    lib = _capi.lib()
    nws = lib.sph_gemm_workspace_bytes(1, m, n, k)
    assert nws > 0, "shape should take a split"
    X = uniform((m, k), k=61).to(dtype)
    W = (uniform((n, k) if tb else (k, n), k=62) * 0.05).to(dtype)
    bias = uniform((n,), k=63).to(dtype)
    xd, wd, bd = X.to(DEV), W.to(DEV), bias.to(DEV)
    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    outs = []
    for rep, (w_ptr, w_n) in enumerate(((_p(ws), nws), (None, 0), (_p(ws), nws))):
        d = torch.empty(m, n, dtype=dtype, device=DEV)
        _capi.call("sph_gemm_ex", DT[dtype], 0, int(tb), 1, m, n, k, 0.75, _p(xd), k, 0, _p(wd),
                   k if tb else n, 0, 0.5, _p(bd), 0, 1, 0, _p(d), n, 0, epi, w_ptr, w_n, _stream())
        _sync()
        outs.append(d)
    b_ = W.float().numpy().T if tb else W.float().numpy()
    want = O.gemm(X.float().numpy(), b_, alpha=0.75, beta=0.5, c=bias.float().numpy()[None, :],
                  epilogue={0: "none", 2: "gelu", 3: "silu"}[epi])
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(outs[0], want, out_dtype=dtype, what="split-K tail", **tol)
    close = dict(rtol=2e-3, atol=2e-3) if dtype == torch.float16 else dict(rtol=1.6e-2, atol=1e-2)
    torch.testing.assert_close(outs[0].float(), outs[1].float(), **close)
    # the same call again: the reduce sums the slices in a fixed order
    assert torch.equal(outs[0], outs[2]), "second call with the workspace differs"


@pytest.mark.parametrize("m,n,k,swiglu,pad,dtype", [
    (4, 6144, 4096, 0, 0, torch.float16),      # QKV shape: small-M kernel
    (4, 12800, 4096, 1, 0, torch.float16),     # gate / up: weight stream, SwiGLU
    (4, 49155, 4096, 0, 8, torch.float16),     # LM head: weight stream
    (1, 200, 264, 0, 8, torch.bfloat16),       # narrow, ragged, one row
    (8, 1000, 8192, 1, 0, torch.bfloat16),     # longest rows, eight rows
    (3, 25600, 1024, 0, 0, torch.float16)])
def test_gemm_rmsnorm(m, n, k, swiglu, pad, dtype):
    # rms_norm(x) W^T with the norm as the prologue of the decode GEMM:
    # against the oracle's fold (x * w staged in the activation type, sums
    # scaled by 1 / rms) at fp16's output rounding, and the exact composite
    # at the north star's 1e-2; row 1 is tiny so eps carries weight
    _log(f"gemm rmsnorm {m}x{n}x{k} swiglu={swiglu} pad={pad} {dtype}")
    X = uniform((m, k), k=71) * 3
    if m > 1:
        X[1] *= 1e-3
    X = X.to(dtype)
    nw = (1 + 0.1 * uniform((k,), k=72)).to(dtype)
    N = 2 * n if swiglu else n
    W = (uniform((N, k), k=73) * 0.05).to(dtype)
    xd = torch.zeros(m, k + pad, dtype=dtype, device=DEV)
    xd[:, :k] = X.to(DEV)
    wd = torch.zeros(N, k + pad, dtype=dtype, device=DEV)
    wd[:, :k] = W.to(DEV)
    nwd = nw.to(DEV)
    d = torch.full((m, n + pad), 7.0, dtype=dtype, device=DEV)
    _capi.call("sph_gemm_rmsnorm", DT[dtype], m, n, k, _p(xd), k + pad, _p(nwd), 1e-5, _p(wd),
               k + pad, _p(d), n + pad, swiglu, _stream())
    _sync()
    xf, nf, wf = X.float().numpy(), nw.float().numpy(), W.float().numpy()
    act = np.float16 if dtype == torch.float16 else "bfloat16"
    fold = O.rmsnorm_linear(xf, nf, wf, 1e-5, act_dtype=act, swiglu=bool(swiglu))
    tight = dict(rtol=4e-3, atol=1e-3) if dtype == torch.float16 else dict(rtol=1.6e-2, atol=4e-3)
    assert_close_fp(d[:, :n], fold, out_dtype=dtype, what="rmsnorm fold", **tight)
    exact = O.rmsnorm_linear(xf, nf, wf, 1e-5, act_dtype=None, swiglu=bool(swiglu))
    if dtype == torch.float16:
        assert_close_fp(d[:, :n], exact, out_dtype=dtype, what="rmsnorm composite")
    else:
        # bf16 staging carries 2^-9 per term, as the eager path's rounded
        # normalized activations do: relative L2 against the exact result
        got = d[:, :n].float().cpu().numpy()
        rel = np.linalg.norm(got - exact) / np.linalg.norm(exact)
        assert rel <= 1e-2, f"rmsnorm composite (bf16): relative L2 {rel:.2e}"
    if pad:
        assert bool((d[:, n:] == 7.0).all()), "padding columns written"


def test_gemm_rmsnorm_op_and_rejects():
    # the ATen op on spyre tensors (decode rows: one kernel; more rows: the
    # norm and the product as separate ops) against the CPU composite
    _log("spyre rms_norm_mm op")
    for m in (4, 12):
        x = (uniform((m, 512), k=81) * 2).half()
        nw = (1 + 0.1 * uniform((512,), k=82)).half()
        w = (uniform((384, 512), k=83) * 0.05).half()
        for sw in (False, True):
            got = torch.ops.spyre.rms_norm_mm(x.to("spyre"), nw.to("spyre"), 1e-5,
                                              w.to("spyre"), sw).cpu()
            want = torch.ops.spyre.rms_norm_mm(x.float(), nw.float(), 1e-5, w.float(), sw)
            torch.testing.assert_close(got.float(), want, rtol=1e-2, atol=1e-2)
    x = torch.zeros(9, 64, dtype=torch.float16, device=DEV)
    w = torch.zeros(64, 64, dtype=torch.float16, device=DEV)
    nw = torch.zeros(64, dtype=torch.float16, device=DEV)
    d = torch.zeros(9, 64, dtype=torch.float16, device=DEV)
    rc = _capi.lib().sph_gemm_rmsnorm(_capi.F16, 9, 64, 64, _p(x), 64, _p(nw),
                                      ctypes.c_float(1e-5), _p(w), 64, _p(d), 64, 0, _stream())
    assert rc == 1002  # SPH_ERR_UNSUPPORTED: more than 8 rows


def test_gemm_swiglu_rejects_unfit_shapes():
    x = torch.zeros(200, 64, dtype=torch.float16, device=DEV)
    w = torch.zeros(256, 64, dtype=torch.float16, device=DEV)
    d = torch.zeros(200, 128, dtype=torch.float16, device=DEV)
    rc = _capi.lib().sph_gemm_swiglu(_capi.F16, 200, 128, 64, _p(x), 64, _p(w), 64, _p(d), 128,
                                     None, 0, _stream())
    assert rc == 1002  # SPH_ERR_UNSUPPORTED: m % 256 != 0


def test_gemm_small_m_epilogue_and_batch():
    _log("gemm small-M epilogue / batched")
    m, n, k = 4, 200, 264
    X, W = uniform((m, k), k=13), uniform((n, k), k=14) * 0.1
    bias = uniform((n,), k=15)
    d = _gemm(X.to(DEV), W.to(DEV), trans_b=True, alpha=0.5, beta=1.5, c=bias.to(DEV), crow=0,
              ccol=1, epi=3)
    want = O.gemm(X.numpy(), W.numpy().T, alpha=0.5, beta=1.5, c=bias.numpy()[None, :],
                  epilogue="silu")
    assert_close_fp(d, want, what="small-M silu epilogue")
    # batched decode attention scores: q [b, 4, 128] x K[b, L, 128]^T
    b, L = 32, 1030
    Q, K = uniform((b, 4, 128), k=16), uniform((b, L, 128), k=17)
    qd, kd = Q.to(DEV), K.to(DEV)
    out = torch.empty(b, 4, L, dtype=torch.float16, device=DEV)
    _capi.call("sph_gemm_strided_batched", _capi.F16, 0, 1, b, 4, L, 128, 1.0, _p(qd), 128,
               4 * 128, _p(kd), 128, L * 128, 0.0, None, 0, 0, 0, _p(out), L, 4 * L, 0, _stream())
    _sync()
    assert_close_fp(out, O.gemm(Q.numpy(), K.numpy().transpose(0, 2, 1)), what="small-M batched")


@pytest.mark.parametrize("batch,m,n,k,tb", [(32, 2048, 2048, 128, False), (32, 2048, 128, 2048, False),
                                            (4, 100, 36, 72, True), (3, 5, 7, 9, False)])
def test_bmm(batch, m, n, k, tb):
    _log(f"bmm {batch}x{m}x{n}x{k} tb={tb}")
    A = uniform((batch, m, k), k=1)
    B = uniform((batch, k, n), k=2)
    ad = A.to(DEV)
    bd = (B.transpose(1, 2).contiguous() if tb else B).to(DEV)
    d = torch.empty(batch, m, n, dtype=torch.float16, device=DEV)
    ldb = k if tb else n
    _capi.call("sph_gemm_strided_batched", _capi.F16, 0, int(tb), batch, m, n, k, 1.0, _p(ad), k,
               m * k, _p(bd), ldb, k * n, 0.0, None, 0, 0, 0, _p(d), n, m * n, 0, _stream())
    _sync()
    assert_close_fp(d, O.gemm(A.numpy(), B.numpy()), what="bmm")


# ---------------------------------------------------------------------------
# fused attention
# ---------------------------------------------------------------------------
def _attention(q, k, v, scale, mask=None, causal_q=0, causal_off=0, dtype=torch.float16,
               ld_pad=0, workspace=True):
    """q [b, mq, 128], k / v [b, sk, 128] (device, contiguous); mask [mq, sk]
    or [b, mq, sk] on the device, or None.  Rows of q/k/v/o get ld_pad extra
    elements when set; `workspace` passes room for the mask-block pre-pass."""
    b, mq, d = q.shape
    sk = k.shape[1]

    def padded(t):
        if not ld_pad:
            return t, t.shape[-1]
        buf = torch.zeros(t.shape[0], t.shape[1], d + ld_pad, dtype=t.dtype, device=t.device)
        buf[..., :d] = t
        return buf, d + ld_pad

    (qp, ldq), (kp, ldk), (vp_, ldv) = padded(q), padded(k), padded(v)
    o = torch.empty(b, mq, d + ld_pad, dtype=dtype, device=DEV)
    ldm = mask.stride(-2) if mask is not None else 0
    sm = mask.stride(0) if mask is not None and mask.dim() == 3 else 0
    ws, nws = None, 0
    if workspace and mask is not None:
        nws = _capi.lib().sph_attention_workspace_bytes(b, mq, sk, sm)
        ws = torch.full((nws,), 0xAB, dtype=torch.uint8, device=DEV)  # stale contents
    _capi.call("sph_attention_fwd", DT[dtype], b, mq, sk, d, _p(qp), ldq, qp[0].numel(), _p(kp),
               ldk, kp[0].numel(), _p(vp_), ldv, vp_[0].numel(), _p(mask), ldm, sm, causal_q,
               causal_off, scale, _p(o), d + ld_pad, o[0].numel(), _p(ws), nws, _stream())
    _sync()
    return o[..., :d]


@pytest.mark.parametrize("b,mq,sk,causal_q,masked,pad", [(2, 256, 256, 256, False, 0),
                                                        (3, 512, 128, 128, False, 8),
                                                        (2, 128, 200, 0, True, 0),
                                                        (1, 384, 320, 96, True, 16),
                                                        (2, 256, 64, 0, False, 0)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_attention_fused(b, mq, sk, causal_q, masked, pad, dtype):
    # causal with stacked query heads (mq = heads * causal_q), additive masks
    # with -inf entries and key counts off the 64-key block, padded rows
    _log(f"attention b={b} mq={mq} sk={sk} causal_q={causal_q} mask={masked} pad={pad} {dtype}")
    q = randn((b, mq, 128), k=41, dtype=dtype)
    k = randn((b, sk, 128), k=42, dtype=dtype)
    v = randn((b, sk, 128), k=43, dtype=dtype)
    scale = 1 / math.sqrt(128)
    mask = None
    if masked:
        m = randn((mq, sk), k=44)
        m[m < -1.2] = float("-inf")
        m[:, 0] = 0.0
        mask = m.to(dtype)
    off = sk - causal_q if causal_q else 0
    got = _attention(q.to(DEV), k.to(DEV), v.to(DEV), scale,
                     mask.to(DEV) if mask is not None else None, causal_q, off, dtype, pad)
    want = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), scale,
                       mask=None if mask is None else mask.float().numpy(),
                       causal_q_len=causal_q, causal_offset=off)
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(got, want, out_dtype=dtype, what="fused attention", **tol)


def _block_mask(kind, b, mq, sk, causal_q=0):
    """Additive masks whose 128 x 64 blocks cover every class the pre-pass
    tells apart (all zero, mixed, all -inf), as [mq, sk] or [b, mq, sk]."""
    if kind == "causal":       # stacked heads, each a causal run of causal_q rows
        r = torch.arange(mq)[:, None] % causal_q + (sk - causal_q)
        return torch.where(torch.arange(sk)[None, :] <= r, 0.0, float("-inf"))
    if kind == "window":       # keys (pos - 100, pos]: all -inf blocks at the front
        pos = torch.arange(mq)[:, None] % sk
        c = torch.arange(sk)[None, :]
        return torch.where((c <= pos) & (c > pos - 100), 0.0, float("-inf"))
    if kind == "holes":        # zero mask with all -inf key blocks in the middle, per batch
        m = torch.zeros(b, mq, sk)
        for i in range(b):
            m[i, :, 64 * (i + 1):64 * (i + 2)] = float("-inf")
        m[:, 5, 3] = -0.75     # one mixed block
        return m
    if kind == "zero":
        return torch.zeros(mq, sk)
    raise ValueError(kind)


@pytest.mark.parametrize("kind,b,mq,sk,causal_q", [("causal", 2, 512, 256, 128),
                                                    ("causal", 1, 256, 200, 200),
                                                    ("window", 2, 384, 384, 0),
                                                    ("holes", 3, 256, 320, 0),
                                                    ("zero", 2, 128, 136, 0)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_attention_mask_blocks(kind, b, mq, sk, causal_q, dtype):
    # the mask-block pre-pass: same result as without it (bit-exact: skipped
    # blocks are all -inf, unloaded ones all zero) and as the oracle
    _log(f"attention mask blocks {kind} b={b} mq={mq} sk={sk} {dtype}")
    q = randn((b, mq, 128), k=51, dtype=dtype)
    k = randn((b, sk, 128), k=52, dtype=dtype)
    v = randn((b, sk, 128), k=53, dtype=dtype)
    m = _block_mask(kind, b, mq, sk, causal_q).to(dtype)
    args = (q.to(DEV), k.to(DEV), v.to(DEV), 1 / math.sqrt(128), m.to(DEV), 0, 0, dtype)
    got = _attention(*args)
    plain = _attention(*args, workspace=False)
    assert torch.equal(got, plain), "mask-block pre-pass changed the result"
    want = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 1 / math.sqrt(128),
                       mask=m.float().numpy())
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    assert_close_fp(got, want, out_dtype=dtype, what=f"attention {kind} mask", **tol)


def test_attention_causal_mask_matches_causal_positions():
    # c4's attention with its additive causal mask (stacked heads) takes
    # the same blocks, in the same order, as the causal-position mode
    _log("attention c4 causal mask vs positions")
    q = randn((8, 8192, 128), k=55).to(DEV)
    k = randn((8, 2048, 128), k=56).to(DEV)
    v = randn((8, 2048, 128), k=57).to(DEV)
    m = _block_mask("causal", 8, 8192, 2048, 2048).half().to(DEV)
    by_mask = _attention(q, k, v, 1 / math.sqrt(128), m, 0, 0)
    by_pos = _attention(q, k, v, 1 / math.sqrt(128), None, 2048, 0)
    assert torch.equal(by_mask, by_pos)


def test_attention_fused_c4_shape():
    # the c4 layer's attention: 8 KV heads, 4 query heads stacked per KV
    # head (mq = 4 * 2048), causal over 2048 keys; one batch element
    # checked against the oracle, all 8 run
    _log("attention c4 shape")
    q = randn((8, 8192, 128), k=45)
    k = randn((8, 2048, 128), k=46)
    v = randn((8, 2048, 128), k=47)
    got = _attention(q.to(DEV), k.to(DEV), v.to(DEV), 1 / math.sqrt(128), None, 2048, 0)
    want = O.attention(q[:1].numpy(), k[:1].numpy(), v[:1].numpy(), 1 / math.sqrt(128),
                       causal_q_len=2048)
    assert_close_fp(got[:1], want, what="c4 attention")
    assert torch.isfinite(got.float()).all()


# ---------------------------------------------------------------------------
# pointwise engine
# ---------------------------------------------------------------------------
def _pw(op, out, ins, alpha=0.0, beta=0.0):
    shape = list(out.shape)
    ops = [_capi.operand(out.data_ptr(), _capi.torch_dtype_code(out.dtype), out.stride())]
    for t in ins:
        t = t.expand(shape) if t.dim() <= len(shape) else t
        ops.append(_capi.operand(t.data_ptr(), _capi.torch_dtype_code(t.dtype), t.stride()))
    arr = (_capi.Operand * len(ops))(*ops)
    _capi.call("sph_pointwise", op, len(ins), arr, len(shape), _capi.i64_array(shape), alpha, beta,
               _stream())
    _sync()


UNARY = [(20, torch.neg), (21, torch.abs), (22, torch.exp), (24, lambda t: torch.sqrt(t.abs())),
         (26, torch.reciprocal), (27, torch.sigmoid), (28, torch.tanh), (29, torch.relu),
         (30, torch.nn.functional.gelu), (32, torch.nn.functional.silu), (33, torch.sin),
         (34, torch.cos), (35, torch.erf), (48, torch.square)]


@pytest.mark.parametrize("op,fn", UNARY)
def test_pointwise_unary(op, fn):
    _log(f"pointwise unary {op}")
    x = randn((67, 256), k=1)
    if op == 24:
        x = x.abs()
    xd = x.to(DEV)
    out = torch.empty_like(xd)
    _pw(op, out, [xd])
    want = fn(x.float()).numpy()
    assert_close_fp(out, want, what=f"unary {op}")


BINARY = [(2, lambda a, b: a + 2 * b, 2.0), (3, lambda a, b: a - b, 1.0), (4, torch.mul, 0.0),
          (5, torch.div, 0.0), (13, torch.maximum, 0.0), (14, torch.minimum, 0.0),
          (81, lambda a, b: torch.nn.functional.silu(a) * b, 0.0)]


@pytest.mark.parametrize("op,fn,alpha", BINARY)
def test_pointwise_binary_broadcast_strided(op, fn, alpha):
    _log(f"pointwise binary {op}")
    a = randn((67, 256), k=2)
    b = randn((256,), k=3)
    if op == 5:
        b = torch.where(b.abs() < 0.1, torch.full_like(b, 0.5), b)
    ad, bd = a.to(DEV), b.to(DEV)
    out = torch.empty_like(ad)
    _pw(op, out, [ad, bd.unsqueeze(0)], alpha)
    assert_close_fp(out, fn(a.float(), b.float()).numpy(), what=f"binary {op}")
    # transposed (non-contiguous) input and output
    a2 = randn((256, 67), k=9)
    if op == 5:
        a2 = torch.where(a2.abs() < 0.1, torch.full_like(a2, 0.5), a2)
    a2t = a2.to(DEV).t()
    out_t = torch.empty(256, 67, dtype=torch.float16, device=DEV).t()
    _pw(op, out_t, [ad, a2t], alpha)
    assert_close_fp(out_t, fn(a.float(), a2.t().float()).numpy(), what=f"binary {op} strided")


def test_pointwise_compare_where_cast_fill():
    _log("pointwise compare/where/cast/fill")
    x, y = randn((256,), k=4), randn((256,), k=5)
    xd, yd = x.to(DEV), y.to(DEV)
    eq = torch.empty(256, dtype=torch.bool, device=DEV)
    for op, fn in [(60, torch.eq), (65, torch.ge), (62, torch.lt)]:
        _pw(op, eq, [xd, yd])
        assert torch.equal(eq.cpu(), fn(x, y))
    ge = torch.empty(256, dtype=torch.bool, device=DEV)
    _pw(65, ge, [xd, yd])
    w = torch.empty_like(xd)
    _pw(80, w, [ge, xd, yd])
    assert torch.equal(w.cpu(), torch.where(x >= y, x, y))
    # casts are bit-exact with torch's
    f32 = torch.empty(256, dtype=torch.float32, device=DEV)
    _pw(0, f32, [xd])
    assert torch.equal(f32.cpu(), x.float())
    big = (randn((256,), k=6, dtype=torch.float32) * 1000)
    bd = big.to(DEV)
    for dt in (torch.float16, torch.bfloat16, torch.int32, torch.int8, torch.int64):
        o = torch.empty(256, dtype=dt, device=DEV)
        _pw(0, o, [bd])
        if dt == torch.int8:
            continue  # out-of-range float -> int8 is undefined behaviour in C and torch
        assert torch.equal(o.cpu(), big.to(dt)), dt
    fill = torch.empty(3, 5, dtype=torch.float16, device=DEV)
    _pw(1, fill, [], alpha=3.5)
    assert torch.equal(fill.cpu(), torch.full((3, 5), 3.5, dtype=torch.float16))
    ints = torch.arange(-5, 5, dtype=torch.int64)
    io = torch.empty(10, dtype=torch.int64, device=DEV)
    _pw(2, io, [ints.to(DEV), ints.to(DEV)], alpha=3.0)
    assert torch.equal(io.cpu(), ints + 3 * ints)


# ---------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------
def _reduce(op, x, dims, out_dtype=None, keep_out=False):
    shape = list(x.shape)
    out_shape = [1 if i in dims else s for i, s in enumerate(shape)]
    out = torch.empty(out_shape, dtype=out_dtype or x.dtype, device=DEV)
    ost = [0 if i in dims else s for i, s in enumerate(out.stride())]
    i_op = _capi.operand(x.data_ptr(), _capi.torch_dtype_code(x.dtype), x.stride())
    o_op = _capi.operand(out.data_ptr(), _capi.torch_dtype_code(out.dtype), ost)
    mask = sum(1 << d for d in dims)
    _capi.call("sph_reduce", op, i_op, o_op, len(shape), _capi.i64_array(shape), mask, _stream())
    _sync()
    return out


@pytest.mark.parametrize("dims", [[0], [1], [0, 1], [2], [0, 2]])
def test_reduce_sum_mean_max(dims):
    _log(f"reduce dims={dims}")
    x = randn((6, 67, 40), k=7)
    xd = x.to(DEV)
    for op, fn in [(0, lambda t: t.sum(dims, keepdim=True)), (1, lambda t: t.mean(dims, keepdim=True)),
                   (2, lambda t: t.amax(dims, keepdim=True)), (3, lambda t: t.amin(dims, keepdim=True))]:
        out = _reduce(op, xd, dims)
        assert_close_fp(out, fn(x.float()).numpy(), what=f"reduce op={op}")


def test_reduce_argmax_ties_nan_and_ints():
    _log("reduce argmax / ints")
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [float("nan"), 5.0, float("nan"), 1.0],
                      [-1.0, -1.0, -2.0, -3.0]], dtype=torch.float16)
    xd = x.to(DEV)
    am = _reduce(4, xd, [1], out_dtype=torch.int64)
    assert torch.equal(am.cpu().view(-1), torch.argmax(x.float(), 1))
    an = _reduce(5, xd, [1], out_dtype=torch.int64)
    assert torch.equal(an.cpu().view(-1), torch.argmin(x.float(), 1))
    logits = randn((4, 49155), k=8)
    ld = logits.to(DEV)
    am2 = _reduce(4, ld, [1], out_dtype=torch.int64)
    assert torch.equal(am2.cpu().view(-1), torch.argmax(logits.float(), 1))
    ints = torch.arange(64, dtype=torch.int32).view(8, 8)
    s = _reduce(0, ints.to(DEV), [0], out_dtype=torch.int64)
    assert torch.equal(s.cpu(), ints.long().sum(0, keepdim=True))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("start", [0, 1, 3, 7])
def test_reduce_long_rows_vector_path(dtype, start):
    """Rows of >= 8192 contiguous elements (the LM-head argmax shape) take
    the vectorised one-workgroup-per-row path: rows that start off a
    16-byte boundary, ties placed in the unaligned head, the body and the
    tail, NaNs, and every op of that path against torch on the CPU."""
    _log(f"reduce long rows dtype={dtype} start={start}")
    n = 49155
    base = randn((5, n + 8), k=11).to(dtype)
    top = torch.tensor(9.0, dtype=dtype)
    base[0, start + 1] = top            # tie between the head ...
    base[0, start + 30000] = top        # ... and the body
    base[1, start + n - 1] = top        # maximum in the tail
    base[1, start + 40] = top           # ... tied with an earlier body element
    base[2, start + 5000] = float("nan")
    base[2, start + 7000] = float("nan")
    base[3, start + 2] = -top           # minimum in the head
    x = base[:, start:start + n]        # rows start `start` elements in
    xd = base.to(DEV)[:, start:start + n]
    xf = x.float()
    for op, fn in [(4, lambda t: torch.argmax(t, 1, keepdim=True)),
                   (5, lambda t: torch.argmin(t, 1, keepdim=True))]:
        got = _reduce(op, xd, [1], out_dtype=torch.int64)
        assert torch.equal(got.cpu(), fn(xf)), f"op {op}"
    for op, fn in [(2, lambda t: t.amax(1, keepdim=True)), (3, lambda t: t.amin(1, keepdim=True))]:
        got = _reduce(op, xd, [1])
        torch.testing.assert_close(got.cpu().float(), fn(xf).to(dtype).float(), rtol=0, atol=0,
                                   equal_nan=True, msg=f"op {op}")
    fin = base[[0, 1, 3, 4], start:start + n].contiguous().to(DEV)   # rows without NaN
    ff = base[[0, 1, 3, 4], start:start + n].float()
    for op, fn in [(0, lambda t: t.sum(1, keepdim=True)), (1, lambda t: t.mean(1, keepdim=True))]:
        got = _reduce(op, fin, [1], out_dtype=torch.float32)
        torch.testing.assert_close(got.cpu(), fn(ff.double()).float(), rtol=1e-4, atol=1e-3)


# ---------------------------------------------------------------------------
# data movement
# ---------------------------------------------------------------------------
def test_gather_rows_embedding():
    _log("gather rows")
    table = randn((49155, 4096), k=1)
    idx = torch.randint(0, 49155, (2048,), generator=torch.Generator().manual_seed(5))
    td, idd = table.to(DEV), idx.to(DEV)
    out = torch.empty(2048, 4096, dtype=torch.float16, device=DEV)
    _capi.call("sph_gather_rows", _p(td), 49155, 4096, 2, _p(idd), 1, 2048, _p(out), None,
               _stream())
    _sync()
    assert torch.equal(out.cpu(), table[idx])
    # ragged rows, int32 indices, out-of-range: a zero row and the report
    # word set (a device-accessible int32 the caller clears and reads)
    t2 = randn((10, 3), k=2)
    i2 = torch.tensor([9, 0, 10, -1, 4], dtype=torch.int32)
    o2 = torch.empty(5, 3, dtype=torch.float16, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    # keep the device copies referenced until the kernel has run: a dropped
    # temporary's block is reused by the next allocation
    t2d, i2d = t2.to(DEV), i2.to(DEV)
    _capi.call("sph_gather_rows", _p(t2d), 10, 3, 2, _p(i2d), 0, 5, _p(o2), _p(flag), _stream())
    _sync()
    want = torch.stack([t2[9], t2[0], torch.zeros(3, dtype=torch.float16),
                        torch.zeros(3, dtype=torch.float16), t2[4]])
    assert torch.equal(o2.cpu(), want)
    assert int(flag.cpu()[0]) == 1
    # in-range indices leave the word alone
    flag.zero_()
    _capi.call("sph_gather_rows", _p(t2d), 10, 3, 2, _p(i2d), 0, 2, _p(o2), _p(flag), _stream())
    _sync()
    assert int(flag.cpu()[0]) == 0


@pytest.mark.parametrize("upper,diag", [(0, 0), (1, 0), (0, -2), (1, 3)])
def test_tri(upper, diag):
    _log(f"tri upper={upper} diag={diag}")
    x = randn((3, 9, 13), k=3)
    xd = x.to(DEV)
    y = torch.empty_like(xd)
    _capi.call("sph_tri", upper, diag, 2, _p(xd), _p(y), 3, 9, 13, _stream())
    _sync()
    want = torch.triu(x, diag) if upper else torch.tril(x, diag)
    assert torch.equal(y.cpu(), want)


def test_rope():
    _log("rope")
    x = randn((2048, 32, 128), k=4)
    pos = torch.arange(2048, dtype=torch.int64)
    xd, pd = x.to(DEV), pos.to(DEV)
    y = torch.empty_like(xd)
    _capi.call("sph_rope", _capi.F16, _p(xd), _p(y), _p(pd), 2048, 32, 128, 1e4, _stream())
    _sync()
    assert_close_fp(y, O.rope(x.numpy(), pos.numpy(), 1e4), what="rope")


@pytest.mark.parametrize("shape,order,dtype", [([512, 256], [0, 1], torch.float16),
                                               ([512, 256], [1, 0], torch.float16),
                                               ([512, 8, 256], [2, 1, 0], torch.float16),
                                               ([3, 100], [0, 1], torch.float32),
                                               ([2, 3, 5, 70], [1, 3, 0, 2], torch.int8),
                                               ([4096, 4096], [1, 0], torch.float16)])
def test_stick_pack_unpack_bit_exact(shape, order, dtype):
    _log(f"stick {shape} {order} {dtype}")
    if dtype.is_floating_point:
        x = randn(shape, k=5, dtype=dtype)
    else:
        x = torch.randint(-100, 100, shape, generator=torch.Generator().manual_seed(7)).to(dtype)
    eb = x.element_size()
    nbytes = L.stick_nbytes(shape, eb, order)
    xd = x.to(DEV)
    dev = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=DEV)
    _capi.call("sph_stick_pack", _p(xd), _p(dev), len(shape), _capi.i64_array(shape),
               _capi.i64_array(list(xd.stride())), _capi.i32_array(order), eb, _stream())
    _sync()
    np.testing.assert_array_equal(dev.cpu().numpy(), L.stick_pack(x.numpy(), order))
    back = torch.zeros_like(xd)
    _capi.call("sph_stick_unpack", _p(dev), _p(back), len(shape), _capi.i64_array(shape),
               _capi.i64_array(list(back.stride())), _capi.i32_array(order), eb, _stream())
    _sync()
    assert torch.equal(back.cpu().view(torch.uint8) if dtype != torch.int8 else back.cpu(),
                       x.view(torch.uint8) if dtype != torch.int8 else x)


# ---------------------------------------------------------------------------
# decode-step attention (sph_attention_decode; sph_attention_fwd routes
# mq <= 16 there)
# ---------------------------------------------------------------------------
def _decode(q, k, v, scale, mask=None, ldm=None, v_dim_major=False, causal_q=0, causal_off=0,
            workspace=True, dtype=torch.float16, via_fwd=False):
    """q [b, mq, 128], k [b, sk, 128], v [b, sk, 128] (values; stored
    dim-major [b, 128, sk] when v_dim_major) on the device."""
    b, mq, d = q.shape
    sk = k.shape[1]
    o = torch.empty(b, mq, d, dtype=dtype, device=DEV)
    if v_dim_major:
        skp = (sk + 7) // 8 * 8  # dim-major rows padded to 16 bytes
        vt = torch.zeros(b, d, skp, dtype=dtype, device=DEV)
        vt[..., :sk] = v.transpose(1, 2)
        vks, vds, sv = 1, skp, vt[0].numel()
        vbuf = vt
    else:
        vks, vds, sv, vbuf = d, 1, v[0].numel(), v
    if ldm is None:
        ldm = mask.stride(-2) if mask is not None else 0
    sm = mask.stride(0) if mask is not None and mask.dim() == 3 else 0
    nws = _capi.lib().sph_attention_decode_workspace_bytes(b, mq, sk)
    ws = torch.full((max(nws, 1),), 0xAB, dtype=torch.uint8, device=DEV) if workspace else None
    if via_fwd:
        assert not v_dim_major
        _capi.call("sph_attention_fwd", DT[dtype], b, mq, sk, d, _p(q), d, q[0].numel(), _p(k), d,
                   k[0].numel(), _p(vbuf), d, sv, _p(mask), ldm, sm, causal_q, causal_off, scale,
                   _p(o), d, o[0].numel(), _p(ws), nws if workspace else 0, _stream())
    else:
        _capi.call("sph_attention_decode", DT[dtype], b, mq, sk, d, _p(q), d, q[0].numel(), _p(k),
                   d, k[0].numel(), _p(vbuf), vks, vds, sv, _p(mask), ldm, sm, causal_q,
                   causal_off, scale, _p(o), d, o[0].numel(), _p(ws), nws if workspace else 0,
                   _stream())
    _sync()
    return o


@pytest.mark.parametrize("b,mq,sk", [(32, 4, 1152), (1, 1, 1), (3, 16, 63), (2, 7, 130),
                                     (4, 4, 64), (64, 8, 2000)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_attention_decode_vs_oracle(b, mq, sk, dtype):
    _log(f"decode attention b={b} mq={mq} sk={sk} {dtype}")
    q = randn((b, mq, 128), k=61, dtype=dtype)
    k = randn((b, sk, 128), k=62, dtype=dtype)
    v = randn((b, sk, 128), k=63, dtype=dtype)
    # one mask row for every query row (a decode step's key positions):
    # the last 5 keys dropped (all keys when sk <= 5 would drop every key)
    row = torch.zeros(sk, dtype=dtype)
    if sk > 5:
        row[sk - 5:] = float("-inf")
    scale = 1 / math.sqrt(128)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    want = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), scale,
                       mask=row.float().numpy())
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    outs = []
    for vdm in (False, True):
        for ws in (True, False):
            got = _decode(qd, kd, vd, scale, mask=row.to(DEV), ldm=0, v_dim_major=vdm,
                          workspace=ws, dtype=dtype)
            assert_close_fp(got, want, out_dtype=dtype, what=f"decode vdm={vdm} ws={ws}", **tol)
            outs.append(got)
    # a full [mq, sk] mask, and the prefill entry routing to the same path
    full = row.expand(mq, sk).contiguous().to(DEV)
    got = _decode(qd, kd, vd, scale, mask=full, dtype=dtype, via_fwd=True)
    torch.testing.assert_close(got, outs[0], rtol=0, atol=0)
    # no mask
    got = _decode(qd, kd, vd, scale, dtype=dtype)
    want = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), scale)
    assert_close_fp(got, want, out_dtype=dtype, what="decode no mask", **tol)


def _step_call(qkv, cs, sn, pos_d, err, kc, vc, H, Hkv, L, scale, v_dim_major, out, ws):
    dt = DT[qkv.dtype]
    if v_dim_major:  # vc [B, Hkv, 128, L]
        vks, vds = 1, vc.stride(2)
    else:            # vc [B, Hkv, L, 128]
        vks, vds = vc.stride(2), 1
    _capi.call("sph_decode_attention_step", dt, qkv.shape[0], H, Hkv, 128, _p(qkv),
               qkv.stride(0), _p(cs), _p(sn), cs.stride(0), _p(pos_d), _p(err), _p(kc),
               kc.stride(0), kc.stride(1), kc.stride(2), _p(vc), vc.stride(0), vc.stride(1),
               vks, vds, L, scale, _p(out), out.stride(0), _p(ws), ws.numel(), _stream())
    _sync()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,H,Hkv,L,v_dim_major", [(4, 32, 8, 1152, True), (4, 32, 8, 1152, False),
                                                   (2, 8, 8, 200, True), (1, 16, 2, 65, False),
                                                   (3, 24, 3, 130, False), (3, 24, 3, 136, True),
                                                   (2, 16, 4, 70, True)])
def test_decode_attention_step_vs_oracle(dtype, B, H, Hkv, L, v_dim_major):
    """The fused decode step (RoPE of q / k at pos, cache append, attention
    over keys 0..pos) against the oracle's restatement, for a sequence of
    positions on the same caches (first key, chunk edges, the last slot):
    out at 1e-2, the appended value bit-exact, the appended key within one
    element-type step of the oracle's rounding, every other cache entry
    unchanged; a position past the cache sets the error word and writes
    nothing."""
    from oracle import decoder as OD

    _log(f"decode step B={B} H={H} Hkv={Hkv} L={L} vdm={v_dim_major} {dtype}")
    D = 128
    kc = randn((B, Hkv, L, D), k=81).to(dtype)     # earlier steps' contents
    vc = randn((B, Hkv, L, D), k=82).to(dtype)
    ang = torch.arange(L, dtype=torch.float32)[:, None] * \
        (1e4 ** (-torch.arange(0, D, 2, dtype=torch.float32) / D))[None, :]
    ang = torch.cat([ang, ang], -1)
    cs, sn = ang.cos().to(dtype), ang.sin().to(dtype)
    kcd = kc.to(DEV)
    vcd = (vc.transpose(2, 3).contiguous() if v_dim_major else vc).to(DEV)
    csd, snd = cs.to(DEV), sn.to(DEV)
    scale = 1.0 / math.sqrt(D)
    nws = _capi.lib().sph_decode_attention_step_workspace_bytes(B, H, Hkv, L)
    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.empty(B, H * D, dtype=dtype, device=DEV)
    want_k, want_v = kc.float().numpy(), vc.float().numpy()
    act = np.float16 if dtype == torch.float16 else "bfloat16"
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.float16 else dict(rtol=2e-2, atol=2e-2)
    positions = sorted({0, 63, 64, min(1000, L - 2), L - 1})
    for n, pos in enumerate(positions):
        qkv = randn((B, (H + 2 * Hkv) * D), k=90 + n).to(dtype)
        pos_d = torch.tensor([pos], dtype=torch.int64, device=DEV)
        _step_call(qkv.to(DEV), csd, snd, pos_d, err, kcd, vcd, H, Hkv, L, scale, v_dim_major,
                   out, ws)
        o_want, want_k2, want_v2 = OD.decode_step_attention(
            qkv.float().numpy(), cs.float().numpy(), sn.float().numpy(), pos, want_k, want_v,
            H, Hkv, scale, act=act)
        assert_close_fp(out, o_want, out_dtype=dtype, what=f"decode step out pos={pos}", **tol)
        got_k = kcd.cpu().float().numpy()
        got_v = vcd.cpu().float()
        got_v = (got_v.transpose(2, 3) if v_dim_major else got_v).numpy()
        # the appended value is a copy; the appended key is RoPE in fp32
        # rounded once (one step of the element type apart at most)
        assert np.array_equal(got_v[:, :, pos], want_v2[:, :, pos])
        step = np.abs(want_k2[:, :, pos]) * (2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7)
        assert np.all(np.abs(got_k[:, :, pos] - want_k2[:, :, pos]) <= step + 1e-6)
        others = np.ones(L, bool)
        others[pos] = False
        assert np.array_equal(got_k[:, :, others], want_k2[:, :, others])
        assert np.array_equal(got_v[:, :, others], want_v2[:, :, others])
        # later positions read what this call stored
        want_k, want_v = got_k, got_v
        assert int(err.cpu()[0]) == 0
    # a position outside the cache: error word 2, caches untouched
    before_k, before_v = kcd.clone(), vcd.clone()
    for bad in (L, -1):
        pos_d = torch.tensor([bad], dtype=torch.int64, device=DEV)
        _step_call(qkv.to(DEV), csd, snd, pos_d, err, kcd, vcd, H, Hkv, L, scale, v_dim_major,
                   out, ws)
        assert int(err.cpu()[0]) == 2
        err.zero_()
        assert torch.equal(kcd, before_k) and torch.equal(vcd, before_v)
    # and the next valid call still merges correctly (arrival counts intact)
    pos = positions[-2]
    qkv = randn((B, (H + 2 * Hkv) * D), k=99).to(dtype)
    pos_d = torch.tensor([pos], dtype=torch.int64, device=DEV)
    _step_call(qkv.to(DEV), csd, snd, pos_d, err, kcd, vcd, H, Hkv, L, scale, v_dim_major, out,
               ws)
    o_want, _, _ = OD.decode_step_attention(qkv.float().numpy(), cs.float().numpy(),
                                            sn.float().numpy(), pos, want_k, want_v, H, Hkv,
                                            scale, act=act)
    assert_close_fp(out, o_want, out_dtype=dtype, what="decode step after errors", **tol)


@pytest.mark.parametrize("v_dim_major", [True, False])
def test_decode_attention_step_ignores_slots_past_pos(v_dim_major):
    """Cache slots after the step's position may hold anything (an
    uninitialised or recycled cache): NaN, +Inf and -Inf there leave the
    output equal to the oracle's over keys 0..pos, and finite."""
    from oracle import decoder as OD

    _log(f"decode step with NaN / Inf past pos, vdm={v_dim_major}")
    B, H, Hkv, L, D = 2, 16, 4, 136, 128
    dtype = torch.float16
    ang = torch.arange(L, dtype=torch.float32)[:, None] * \
        (1e4 ** (-torch.arange(0, D, 2, dtype=torch.float32) / D))[None, :]
    ang = torch.cat([ang, ang], -1)
    cs, sn = ang.cos().to(dtype), ang.sin().to(dtype)
    csd, snd = cs.to(DEV), sn.to(DEV)
    scale = 1.0 / math.sqrt(D)
    nws = _capi.lib().sph_decode_attention_step_workspace_bytes(B, H, Hkv, L)
    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.empty(B, H * D, dtype=dtype, device=DEV)
    junk = torch.tensor([float("nan"), float("inf"), float("-inf")], dtype=dtype)
    for n, pos in enumerate((0, 10, 63, 64, 100, L - 2)):
        kc = randn((B, Hkv, L, D), k=120 + n).to(dtype)
        vc = randn((B, Hkv, L, D), k=130 + n).to(dtype)
        idx = torch.arange(B * Hkv * (L - pos - 1) * D) % 3
        kc[:, :, pos + 1:] = junk[idx].view(B, Hkv, L - pos - 1, D)
        vc[:, :, pos + 1:] = junk[(idx + 1) % 3].view(B, Hkv, L - pos - 1, D)
        kcd = kc.to(DEV)
        vcd = (vc.transpose(2, 3).contiguous() if v_dim_major else vc).to(DEV)
        qkv = randn((B, (H + 2 * Hkv) * D), k=140 + n).to(dtype)
        pos_d = torch.tensor([pos], dtype=torch.int64, device=DEV)
        _step_call(qkv.to(DEV), csd, snd, pos_d, err, kcd, vcd, H, Hkv, L, scale, v_dim_major,
                   out, ws)
        o_want, _, _ = OD.decode_step_attention(
            qkv.float().numpy(), cs.float().numpy(), sn.float().numpy(), pos,
            kc.float().numpy(), vc.float().numpy(), H, Hkv, scale, act=np.float16)
        assert bool(torch.isfinite(out).all()), f"pos={pos}"
        assert_close_fp(out, o_want, out_dtype=dtype, what=f"junk past pos={pos}",
                        rtol=1e-2, atol=1e-2)
        assert int(err.cpu()[0]) == 0


def test_attention_decode_causal_and_empty_rows():
    _log("decode attention causal / all-masked rows")
    b, mq, sk = 3, 6, 300
    q = randn((b, mq, 128), k=64)
    k = randn((b, sk, 128), k=65)
    v = randn((b, sk, 128), k=66)
    scale = 0.1
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    # causal positions: row r sees keys <= r % 3 + 200
    got = _decode(qd, kd, vd, scale, causal_q=3, causal_off=200)
    want = O.attention(q.numpy(), k.numpy(), v.numpy(), scale, causal_q_len=3, causal_offset=200)
    assert_close_fp(got, want, what="decode causal")
    # per-row masks with one row masked everywhere: that row is NaN, the
    # others are unaffected
    m = torch.zeros(b, mq, sk, dtype=torch.float16)
    m[:, 2, :] = float("-inf")
    m[:, 4, 100:] = float("-inf")
    got = _decode(qd, kd, vd, scale, mask=m.to(DEV))
    want = O.attention(q.numpy(), k.numpy(), v.numpy(), scale, mask=m.float().numpy())
    assert torch.isnan(got[:, 2].cpu().float()).all()
    keep = [0, 1, 3, 4, 5]
    assert_close_fp(got[:, keep], want[:, keep], what="decode masked rows")
