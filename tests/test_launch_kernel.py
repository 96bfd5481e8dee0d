"""torch_spyre._C.launch_kernel, the compiled path's launcher.

The reference binds launch_kernel(g2_path, args) with the output as the
last argument (torch_spyre/csrc/module.cpp:63,176) and its runner calls it
as launch_kernel(g2, actuals) (torch_spyre/_inductor/runtime/
kernel_runner.py:36-40).  Here the same two-argument call takes a kernel
handle (launch shape stored at load) or the path of a gfx950 code object
whose launch description sits beside it (`path`.launch); the explicit
five-argument form remains.  Argument errors are raised on the host before
any HIP call, so they are CPU tests; the launches themselves are GPU tests.
"""

import os

import pytest
import torch

import torch_spyre  # noqa: F401
from torch_spyre import _C
from torch_spyre._inductor.runtime.hiprtc import compile_source, write_launchable
from torch_spyre._inductor.runtime.kernel_runner import launch_description
from torch_spyre._inductor.runtime import KernelSpec, TensorArg

# out[i] = 2 a[i] + 1 for i < 1000 (the output is the last parameter)
SRC = r"""
extern "C" __global__ void spyre_kernel(const float* __restrict__ a, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 1000) out[i] = a[i] * 2.0f + 1.0f;
}
"""


def test_unknown_handle_and_missing_files(tmp_path):
    with pytest.raises(RuntimeError, match="unknown kernel handle"):
        _C.launch_kernel(10 ** 9, [torch.zeros(1)])
    with pytest.raises(RuntimeError, match="cannot read code object"):
        _C.launch_kernel(str(tmp_path / "missing.co"), [torch.zeros(1)])
    co = tmp_path / "k.co"
    co.write_bytes(b"\x7fELF-not-loaded-before-the-checks")
    with pytest.raises(RuntimeError, match="cannot read launch description"):
        _C.launch_kernel(str(co), [torch.zeros(1)])


@pytest.mark.parametrize("line,msg", [("spyre_kernel 4 256", "malformed"),
                                      ("spyre_kernel 4 256 3 10 10", "fewer than 3"),
                                      ("spyre_kernel 0 256 1 10", "no launch shape"),
                                      ("spyre_kernel 4 2048 1 10", "bad launch shape")])
def test_malformed_launch_descriptions(tmp_path, line, msg):
    co = tmp_path / "k.co"
    co.write_bytes(b"\x7fELF")
    (tmp_path / "k.co.launch").write_text(line + "\n")
    with pytest.raises(RuntimeError, match=msg):
        _C.launch_kernel(str(co), [torch.zeros(1)])


def test_handle_argument_checks():
    h = _C.load_kernel(b"\x7fELF", "spyre_kernel")  # no launch shape stored
    with pytest.raises(RuntimeError, match="without a launch shape"):
        _C.launch_kernel(h, [torch.zeros(1)])
    h = _C.load_kernel(b"\x7fELF", "spyre_kernel", 4, 256, [1000, 1000])
    with pytest.raises(RuntimeError, match="needs tensor arguments"):
        _C.launch_kernel(h, [])
    with pytest.raises(RuntimeError, match="one extent per argument"):
        _C.launch_kernel(h, [torch.zeros(1)])
    with pytest.raises(RuntimeError, match="is not on spyre"):
        _C.launch_kernel(h, [torch.zeros(1000), torch.zeros(1000)])
    with pytest.raises(RuntimeError, match="bad launch shape"):
        _C.launch_kernel(h, [torch.zeros(1)], 0, 256, [-1])
    with pytest.raises(RuntimeError, match="bad launch shape"):
        _C.load_kernel(b"\x7fELF", "spyre_kernel", 1, 4096, [])
    with pytest.raises(RuntimeError, match="empty code object"):
        _C.load_kernel(b"", "spyre_kernel")


def test_launch_description_format():
    spec = KernelSpec(op="pointwise", is_reduction=False, dimensions=[1000],
                      args=[TensorArg(True, 0, torch.float32, 1000),
                            TensorArg(False, 1, torch.float32, None)],
                      grid=4, block=256, source=SRC)
    assert launch_description(spec) == "spyre_kernel 4 256 2 1000 -1 0\n"


@pytest.mark.gpu
def test_two_argument_forms_launch_a_compiled_kernel():
    code = compile_source(SRC, "launch_test.hip")
    path = write_launchable(code, "spyre_kernel 4 256 2 1000 1000\n")
    assert os.path.exists(path) and os.path.exists(path + ".launch")
    a = torch.randn(1000, generator=torch.Generator().manual_seed(0xAFFE))
    want = a * 2 + 1  # exact in fp32 (one rounding of 2a + 1, as on the device)
    ad = a.to("spyre")
    out = torch.empty(1000, device="spyre")
    _C.launch_kernel(path, [ad, out])  # the reference's form, output last
    assert torch.equal(out.cpu(), want)
    h = _C.load_kernel(code, "spyre_kernel", 4, 256, [1000, 1000])
    out2 = torch.zeros(1000, device="spyre")
    _C.launch_kernel(h, [ad, out2])
    assert torch.equal(out2.cpu(), want)
    out3 = torch.zeros(1000, device="spyre")
    _C.launch_kernel(h, [ad, out3], 4, 256, [1000, 1000])
    assert torch.equal(out3.cpu(), want)
    # the stored extents bound every argument: a short output is refused
    # before the launch
    with pytest.raises(RuntimeError):
        _C.launch_kernel(path, [ad, torch.empty(500, device="spyre")])
