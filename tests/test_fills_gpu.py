"""Device fills against their oracle (oracle/philox.py) and torch's CPU ops:
the Philox random fills (uniform_, normal_, random_) and dropout, arange and
cumsum, through the C-ABI and as torch ops on spyre tensors.

The reference runs all of these on the CPU (cumsum:
codegen/inputs/spyre_torch_ops.cpp:502-505; native_dropout an identity stub,
:180-186).  Bars: integer draws, uniforms, masks, arange of integers and
integer-valued floats, and cumsum along columns are bit-exact; normals are
within float32 transcendental error; cumsum of long last-dim rows (a
workgroup scan) is exact for integers and within rounding for floats.
"""

import numpy as np
import pytest
import torch

import torch_spyre  # noqa: F401
from torch_spyre import _capi

from oracle import philox as P

from helpers import randn

pytestmark = pytest.mark.gpu

DEV = "spyre"
NP = {torch.float16: np.float16, torch.bfloat16: "bfloat16", torch.float32: np.float32,
      torch.float64: np.float64, torch.int32: np.int32, torch.int64: np.int64,
      torch.uint8: np.uint8, torch.int8: np.int8}


def _log(msg):
    print(f"[case] {msg}", flush=True)


def _np(t):
    t = t.cpu()
    return t.float().numpy() if t.dtype == torch.bfloat16 else t.numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("kind", ["uniform", "normal"])
def test_random_fill_capi_vs_oracle(kind, dtype):
    n, seed, off = 10007, 0x1234_5678_9ABC_DEF0, 12345
    _log(f"sph_random_fill {kind} {dtype} n={n}")
    out = torch.empty(n, dtype=dtype, device="cuda")
    code = _capi.torch_dtype_code(dtype)
    k = P.UNIFORM if kind == "uniform" else P.NORMAL
    a, b = (-1.5, 2.5) if kind == "uniform" else (0.5, 2.0)
    _capi.call("sph_random_fill", k, code, out.data_ptr(), n, seed, off, a, b, 0, 0,
               torch.cuda.current_stream().cuda_stream)
    got = _np(out)
    want = (P.uniform if kind == "uniform" else P.normal)(n, NP[dtype], seed, off, a, b)
    want = np.asarray(want, np.float64)
    if kind == "uniform":
        np.testing.assert_array_equal(got.astype(np.float64), want)
    else:
        # float32 log / sincos on the device against float64 here, then the
        # output rounding: one unit in the last place of the output type
        eps = {torch.float32: 2e-6, torch.float16: 2 ** -10, torch.bfloat16: 2 ** -7,
               torch.float64: 1e-12}[dtype]
        np.testing.assert_allclose(got.astype(np.float64), want, rtol=eps, atol=eps * 4)
    assert lib_blocks(k, code, n) == P.n_blocks(k, NP[dtype] if dtype != torch.bfloat16
                                                 else np.float32, n)


def lib_blocks(kind, code, n, irange=0):
    return _capi.lib().sph_random_blocks(kind, code, n, irange)


@pytest.mark.parametrize("dtype,ifrom,irange", [(torch.int64, -5, 11), (torch.int32, 0, 1 << 31),
                                                (torch.uint8, 0, 256), (torch.int64, 7, 1 << 40),
                                                (torch.float16, 0, 2049)])
def test_random_integers_capi_vs_oracle(dtype, ifrom, irange):
    n, seed, off = 4099, 99, 3
    _log(f"sph_random_fill int {dtype} [{ifrom}, +{irange})")
    out = torch.empty(n, dtype=dtype, device="cuda")
    code = _capi.torch_dtype_code(dtype)
    _capi.call("sph_random_fill", P.INT, code, out.data_ptr(), n, seed, off, 0.0, 0.0, ifrom,
               irange, torch.cuda.current_stream().cuda_stream)
    want = P.integers(n, NP[dtype], seed, off, ifrom, irange)
    np.testing.assert_array_equal(_np(out), np.asarray(want))


def test_generator_state_seed_and_offsets():
    _log("spyre generator: manual_seed, consecutive fills, reseed")
    torch.spyre.manual_seed(123)
    a = torch.empty(1000, device=DEV).uniform_()
    b = torch.empty(998, device=DEV).uniform_()
    c = torch.empty(3, 5, device=DEV, dtype=torch.float64).normal_(1.0, 3.0)
    np.testing.assert_array_equal(_np(a), P.uniform(1000, np.float32, 123, 0, 0.0, 1.0))
    np.testing.assert_array_equal(_np(b), P.uniform(998, np.float32, 123, 250, 0.0, 1.0))
    np.testing.assert_allclose(_np(c).reshape(-1), P.normal(15, np.float64, 123, 250 + 250, 1.0,
                                                             3.0), rtol=1e-12, atol=1e-12)
    torch.spyre.manual_seed(123)
    again = torch.empty(1000, device=DEV).uniform_()
    assert torch.equal(again.cpu(), a.cpu())
    # torch.rand / randn on the device draw from the same generator
    torch.spyre.manual_seed(7)
    r = torch.randn(64, 33, device=DEV)
    np.testing.assert_allclose(_np(r).reshape(-1), P.normal(64 * 33, np.float32, 7, 0, 0.0, 1.0),
                               rtol=2e-6, atol=8e-6)


def test_fills_of_views_and_explicit_generators():
    _log("fills of non-contiguous views; CPU generators")
    torch.spyre.manual_seed(5)
    base = torch.zeros(40, 60, device=DEV)
    view = base[:, ::3]  # [40, 20], not contiguous
    view.uniform_(2.0, 3.0)
    got = base.cpu()
    want = P.uniform(800, np.float32, 5, 0, 2.0, 3.0).reshape(40, 20)
    np.testing.assert_array_equal(got[:, ::3].numpy(), want)
    assert not got[:, 1::3].any() and not got[:, 2::3].any()
    g1, g2 = torch.Generator().manual_seed(9), torch.Generator().manual_seed(9)
    x = torch.empty(500, device=DEV).normal_(generator=g1)
    y = torch.empty(500, device=DEV).normal_(generator=g2)
    assert torch.equal(x.cpu(), y.cpu())
    v = torch.empty(10000, dtype=torch.int64, device=DEV).random_(3, 17)
    vc = v.cpu()
    assert int(vc.min()) == 3 and int(vc.max()) == 16
    h = torch.empty(10000, dtype=torch.float16, device=DEV).random_()
    hc = h.cpu().float()
    assert float(hc.min()) >= 0 and float(hc.max()) <= 2048 and torch.equal(hc, hc.round())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_dropout_vs_oracle(dtype):
    _log(f"native_dropout {dtype}")
    x = randn((37, 129), k=12, dtype=dtype)
    torch.spyre.manual_seed(31)
    p = 0.3
    y, m = torch.native_dropout(x.to(DEV), p, True)
    want_y, want_m = P.dropout(x.float().numpy(), p, np.float32(1 / (1 - p)), 31, 0)
    np.testing.assert_array_equal(m.cpu().numpy(), want_m)
    wy = torch.from_numpy(want_y).to(dtype)
    assert torch.equal(y.cpu(), wy)
    assert 0.65 < m.cpu().float().mean().item() < 0.75


@pytest.mark.parametrize("start,end,step,dtype", [
    (0, 1152, 1, torch.int64), (-7, 100, 3, torch.int32), (5, -20, -4, torch.int64),
    (0, 2048, 1, torch.float16), (0.0, 100.0, 0.5, torch.float32), (-3.0, 3.0, 0.25, torch.float64),
    (0, 300, 1, torch.bfloat16), (1.0, 2.0, 0.1, torch.float32), (3, 3, 1, torch.int64),
    (0, 100, 7, torch.uint8)])
def test_arange_vs_torch_cpu(start, end, step, dtype):
    _log(f"arange({start}, {end}, {step}) {dtype}")
    got = torch.arange(start, end, step, dtype=dtype, device=DEV).cpu()
    want = torch.arange(start, end, step, dtype=dtype)
    assert got.shape == want.shape
    od = NP[dtype]
    np.testing.assert_array_equal(_np(got), np.asarray(P.arange(start, step, want.numel(), od),
                                                       dtype=_np(got).dtype))
    if step == 0.1:
        torch.testing.assert_close(got, want, rtol=2 ** -23, atol=0)
    else:
        assert torch.equal(got, want)


def test_arange_errors():
    with pytest.raises(RuntimeError):
        torch.arange(0, 10, 0, device=DEV)
    with pytest.raises(RuntimeError):
        torch.arange(10, 0, 1, device=DEV)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64,
                                   torch.int32, torch.int64, torch.uint8, torch.bool])
@pytest.mark.parametrize("shape,dim", [((7, 300), 1), ((300, 5), 0), ((4, 6, 50), 1),
                                       ((4096, 33), -1), ((2, 3, 1000), 0)])
def test_cumsum_columns_bit_exact(dtype, shape, dim):
    # walked sequentially per column: the CPU kernel's order, so bit-exact
    _log(f"cumsum {shape} dim={dim} {dtype}")
    g = torch.Generator().manual_seed(0xAFFE)
    if dtype.is_floating_point:
        x = (torch.randn(*shape, generator=g) * 3).to(dtype)
    elif dtype == torch.bool:
        x = torch.randint(0, 2, shape, generator=g).bool()
    else:
        x = torch.randint(0, 100, shape, generator=g).to(dtype)
    got = torch.cumsum(x.to(DEV), dim).cpu()
    want = torch.cumsum(x, dim)
    assert got.dtype == want.dtype
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32, torch.float32, torch.float16])
def test_cumsum_long_rows(dtype):
    # few long last-dim rows: one workgroup scan per row
    _log(f"cumsum long rows {dtype}")
    g = torch.Generator().manual_seed(3)
    if dtype.is_floating_point:
        x = torch.rand(3, 100_003, generator=g).to(dtype)
    else:
        x = torch.randint(-50, 50, (3, 100_003), generator=g).to(dtype)
    got = torch.cumsum(x.to(DEV), -1).cpu()
    want = torch.cumsum(x, -1)
    if dtype.is_floating_point:
        ref = torch.cumsum(x.double(), -1)
        # sums of up to 1e5 positive terms: the CPU's sequential order and a
        # tree order each carry about sqrt(n) ulps of the running sum
        scale = ref.abs().max().item()
        tol = (1e-3 if dtype == torch.float16 else 1e-5) * scale
        assert (got.double() - ref).abs().max().item() <= tol
        assert (want.double() - ref).abs().max().item() <= tol
    else:
        assert torch.equal(got, want)


def test_cumsum_dtypes_inplace_views_and_edges():
    _log("cumsum dtype promotion, in place, views, 0-d, empty")
    x = torch.arange(12, dtype=torch.int32).reshape(3, 4)
    got = torch.cumsum(x.to(DEV), 1)
    assert got.dtype == torch.int64 and torch.equal(got.cpu(), torch.cumsum(x, 1))
    f = torch.cumsum(x.to(DEV), 0, dtype=torch.float32)
    assert torch.equal(f.cpu(), torch.cumsum(x, 0, dtype=torch.float32))
    y = torch.randn(5, 8).to(DEV)
    yt = y.t()  # non-contiguous input
    assert torch.equal(torch.cumsum(yt, 1).cpu(), torch.cumsum(y.cpu().t(), 1))
    z = y.clone()
    z.cumsum_(1)
    assert torch.equal(z.cpu(), torch.cumsum(y.cpu(), 1))
    s = torch.tensor(2.5).to(DEV)
    assert torch.equal(torch.cumsum(s, 0).cpu(), torch.cumsum(torch.tensor(2.5), 0))
    e = torch.empty(0, 4).to(DEV)
    assert torch.cumsum(e, 1).shape == (0, 4)
