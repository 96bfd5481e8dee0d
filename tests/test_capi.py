"""C-ABI library: loads, exports every declared entry point, validates
arguments on the host.  CPU only: nothing here launches a kernel (every call
below fails argument validation before any HIP call)."""

import ctypes

import pytest

from torch_spyre import _capi

from oracle import layout as L


def test_library_exports_every_declared_function():
    lib = _capi.lib()
    declared = _capi.header_functions()
    assert len(declared) >= 20
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, f"declared in include/spyre_hip.h but not exported: {missing}"
    # every declared function has a ctypes signature in the binding
    assert set(declared) <= set(_capi._SIGS), set(declared) - set(_capi._SIGS)


def test_abi_version():
    assert _capi.lib().sph_abi_version() == 1


@pytest.mark.parametrize("shape,order,eb", [([128], [0], 2), ([512, 256], [0, 1], 2),
                                            ([512, 256], [1, 0], 2), ([3, 5, 100], [2, 0, 1], 4),
                                            ([7], [0], 1)])
def test_stick_nbytes_matches_oracle(shape, order, eb):
    got = _capi.lib().sph_stick_nbytes(len(shape), _capi.i64_array(shape),
                                       _capi.i32_array(order), eb)
    assert got == L.stick_nbytes(shape, eb, order)


def test_host_side_argument_errors():
    lib = _capi.lib()
    rc = lib.sph_gemm(_capi.F16, 0, 0, -1, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 0, 0,
                      None, 4, 0, None)
    assert rc == 1001
    assert b"negative" in lib.sph_last_error()
    rc = lib.sph_gemm(_capi.F32, 0, 0, 4, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 0, 0,
                      None, 4, 0, None)
    assert rc == 1002
    rc = lib.sph_softmax_rows(_capi.F16, _capi.F16, None, 2, None, 2, 4, 8, 1.0, 0, 0, 0, None)
    assert rc == 1001  # ld < cols
    with pytest.raises(_capi.SpyreKernelError, match="dim_order"):
        _capi.call("sph_stick_pack", None, None, 2, _capi.i64_array([2, 2]),
                   _capi.i64_array([2, 1]), _capi.i32_array([0, 0]), 2, None)
    rc = lib.sph_pointwise(999, 1, None, 1, None, 0.0, 0.0, None)
    assert rc == 1001
    # zero-size work is a no-op that succeeds without touching the device
    assert lib.sph_gemm_f16(0, 4, 4, None, None, None, None) == 0
    assert lib.sph_softmax_rows_f16(None, None, 0, 8, None) == 0
    assert ctypes.c_int(lib.sph_tri(0, 0, 2, None, None, 0, 4, 4, None)).value == 0


@pytest.mark.parametrize("batch,m,n,k,split", [
    (1, 4096, 4096, 4096, False),    # 256 tiles: one whole round
    (1, 2048, 4096, 4096, True),     # c4 O: a 2-way split beats 128-wide tiles on cold weights
    (1, 2048, 4096, 2048, False),    # K = 2048: a round of 128-wide tiles beats the split
    (1, 2048, 4096, 12800, True),    # c4 down: the split tail beats 128-wide tiles
    (1, 2048, 25600, 4096, True),    # c4 gate/up: 800 tiles, a 32-tile tail in 8 slices
    (1, 256, 256, 2048, True),       # one tile in 8 slices
    (2, 2048, 4096, 12800, False),   # batched: never split
    (1, 2048, 4096, 1024, False)])   # K < 2048: slices too short
def test_gemm_workspace_bytes(batch, m, n, k, split):
    # host-side sizing of the split-K workspace (no device call): nonzero
    # exactly where the GEMM would split its last round along K
    got = _capi.lib().sph_gemm_workspace_bytes(batch, m, n, k)
    assert (got > 0) == split, got
    if split:
        assert got % (256 * 256 * 4) == 0 and got <= 256 * 256 * 256 * 4
