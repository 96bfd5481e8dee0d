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
