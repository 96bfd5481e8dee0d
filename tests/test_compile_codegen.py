"""The spyre torch.compile backend on the CPU host: Inductor lowers graphs
over fake spyre tensors, SpyreKernel generates HIP for the fused groups,
hiprtc compiles them for gfx950 and the code objects are registered with
torch_spyre._C.  Nothing is launched (no GPU here); the GPU parity of the
same kernels is in test_compile_gpu.py.

Checks the structure the backend promises: one kernel per fused row
reduction (softmax = max, sum and normalise phases in one kernel; LayerNorm
= Welford + normalise; GELU chain + row-sum), matrix products as extern
calls to the MFMA GEMM, per-argument extents for the launch-time bounds
check, and the fusions the reference forbids (choices.py:58-83).
"""

import os
import re

import pytest
import torch
import torch.nn.functional as F

import torch_spyre  # noqa: F401
from torch_spyre.utils import device_interface as di


@pytest.fixture
def fake_device(monkeypatch):
    # No GPU on this host: fake tensors need a device index and Inductor's
    # heuristics need the device's properties (MI355X values).
    monkeypatch.setattr(torch.spyre, "current_device", lambda: 0)
    monkeypatch.setattr(di.SpyreInterface.Worker, "get_device_properties", staticmethod(
        lambda device=None: di.SpyreDeviceProperties("spyre", 0, "AMD Instinct MI355X",
                                                     "gfx950", 256, 288 << 30, 64)))
    yield


def _compile(fn, specs):
    from torch._inductor import config
    from torch._inductor.compile_fx import compile_fx
    from torch._subclasses.fake_tensor import FakeTensorMode

    n = len(specs)
    names = ", ".join(f"a{i}" for i in range(n))
    ns = {}
    exec(f"def forward(self, {names}):\n    return self.fn({names})\n", ns)
    mod = type("M", (torch.nn.Module,), {"forward": ns["forward"]})()
    mod.fn = fn
    gm = torch.fx.symbolic_trace(mod)
    with FakeTensorMode():
        args = [torch.empty(s, dtype=d, device="spyre") for s, d in specs]
    codes = []
    from torch._inductor.graph import GraphLowering

    orig = GraphLowering.compile_to_module

    def capture(self):
        mod = orig(self)
        with open(mod.__file__) as f:
            codes.append(f.read())
        return mod

    GraphLowering.compile_to_module = capture
    try:
        with config.patch({"fx_graph_cache": False}):
            compile_fx(gm, args)
    finally:
        GraphLowering.compile_to_module = orig
    return "\n".join(codes)


def _kernels(code):
    return re.findall(r"async_compile\.hip\('([^']+)'", code)


def test_softmax_is_one_three_phase_kernel(fake_device):
    code = _compile(lambda x: torch.softmax(x, -1), [((512, 4096), torch.float16)])
    ks = _kernels(code)
    assert len(ks) == 1, ks
    assert code.count("block_reduce<spy::MaxF") == 1 and code.count("block_reduce<spy::SumF") == 1
    assert code.count("for (int64_t r0_cnt") == 3
    assert "extent=2097152" in code  # 512*4096 elements bound both arguments
    # each generated kernel carries a name of its own (kind + source hash)
    sym = re.search(r"symbol='(spyre_red_[0-9a-f]{10})'", code).group(1)
    assert f") {sym}(" in code


def test_layernorm_gelu_rmsnorm_fuse(fake_device):
    code = _compile(lambda x, w, b: F.layer_norm(x, [4096], w, b, 1e-5),
                    [((64, 4096), torch.float16), ((4096,), torch.float16), ((4096,), torch.float16)])
    assert len(_kernels(code)) == 1 and "block_welford" in code
    code = _compile(lambda x, s, b: (lambda y: (y, y.sum(-1)))(F.gelu(x * s + b)),
                    [((64, 4096), torch.float16), ((4096,), torch.float16), ((4096,), torch.float16)])
    assert len(_kernels(code)) == 1 and "spy::gelu_erf(" in code
    code = _compile(lambda x, r, w: (lambda h: (h, torch.rms_norm(h, [4096], w, 1e-5)))(x + r),
                    [((64, 4096), torch.float16), ((64, 4096), torch.float16), ((4096,), torch.float16)])
    assert len(_kernels(code)) == 1


def _source(code):
    src = re.search(r"source='(.*?)',\n", code, re.S).group(1)
    return src.encode().decode("unicode_escape")


def test_row_phases_reuse_stored_values(fake_device):
    # add + LayerNorm: the residual sum is stored once and the normalise
    # phase takes it from registers, not by reading the output back
    code = _compile(lambda x, r, w, b: (lambda h: (h, F.layer_norm(h, [4096], w, b, 1e-5)))(x + r),
                    [((64, 4096), torch.float16)] * 2 + [((4096,), torch.float16)] * 2)
    src = _source(code)
    out = re.search(r"(out_ptr\d+)\[r0_1 \+ 4096LL\*x0\] = ", src).group(1)
    assert src.count(f"{out}[") == 1, src  # the store only
    assert "welford_acc_add" in src and "welford_finish" in src and "welford_add(" not in src


def test_gelu_peephole_only_on_the_erf_form(fake_device):
    specs = [((64, 4096), torch.float16)]
    # the tanh form and a near miss (a different scale inside erf) keep the generic code
    for fn in (lambda x: F.gelu(x, approximate="tanh"),
               lambda x: x * 0.5 * (1 + torch.erf(x * 0.7))):
        assert "gelu_erf" not in _compile(fn, specs)
    assert "spy::gelu_erf(" in _compile(lambda x: x * 0.5 * (1 + torch.erf(x * 0.7071067811865476)), specs)


def test_matmul_is_extern_mfma_call(fake_device):
    code = _compile(lambda a, b: a @ b, [((256, 512), torch.float16), ((512, 384), torch.float16)])
    assert "extern_kernels.mm(" in code and not _kernels(code)
    code = _compile(lambda a, b: torch.softmax(torch.bmm(a, b), -1),
                    [((4, 64, 32), torch.float16), ((4, 32, 64), torch.float16)])
    assert "extern_kernels.bmm(" in code and len(_kernels(code)) == 1


def test_pointwise_chain_fuses_into_one_kernel(fake_device):
    code = _compile(lambda x, y: torch.sigmoid(x * 2 + y).relu() - 1,
                    [((1000, 3), torch.float32), ((1000, 3), torch.float32)])
    assert len(_kernels(code)) == 1
    # 3000 elements: whole groups of 8 consecutive elements per thread
    assert "if (spy_xb >= 3000LL) return;" in code


def test_pointwise_group_form(fake_device):
    # contiguous loads and stores of 8 consecutive elements become one wide
    # access each (runtime alignment test, element fallback)
    code = _compile(lambda x, y: torch.sigmoid(x * 2 + y), [((64, 256), torch.float16)] * 2)
    assert "spy::load8f(in_ptr0" in code and "spy::load8f(in_ptr1" in code
    assert "spy::store8v<_Float16, false>(out_ptr0" in code and "spy_al" in code
    # a permute that keeps the innermost dimension: the permuted store is
    # contiguous too
    code = _compile(lambda x: x.permute(1, 0, 2).contiguous() + 1, [((16, 32, 128), torch.float16)])
    assert "spy::load8f(" in code and "spy::store8v<" in code
    # a row broadcast ([N] over [M, N]) is contiguous along the row
    code = _compile(lambda x, b: x * b, [((64, 256), torch.float16), ((256,), torch.float16)])
    assert code.count("spy::load8f(") == 2
    # a column broadcast ([M, 1]) is the same value for the whole group: one
    # element load, no wide one
    code = _compile(lambda x, b: x * b, [((64, 256), torch.float16), ((64, 1), torch.float16)])
    assert code.count("spy::load8f(") == 1 and "spy::store8v<" in code


def test_pointwise_group_form_not_used(fake_device):
    # element count not a multiple of 8
    code = _compile(lambda x: x * 2 + 1, [((7, 5), torch.float16)])
    assert "spy::load8f" not in code and "spy_xb" not in code
    # a row broadcast over an innermost dimension of 6: a group of 8 would
    # wrap the row
    code = _compile(lambda x, b: x * b, [((8, 6), torch.float16), ((6,), torch.float16)])
    assert "spy::load8f" not in code and "spy_xb" not in code
    # a gather whose index changes along the innermost dimension (columns
    # picked by an index tensor) keeps the element form, and so the whole
    # kernel keeps the block-strided layout
    code = _compile(lambda x, i: x[:, i] * 2,
                    [((16, 64), torch.float16), ((64,), torch.int64)])
    assert "spy::load8f" not in code and "spy_xb" not in code


def test_pointwise_group_form_gathered_rows(fake_device):
    # an embedding row: the token index is the same for the 8 elements of a
    # group (its load is indexed by the row only), so the gathered row is
    # read as whole groups, by the group's first element, after the index
    # (and its bounds check) is computed
    code = _compile(lambda t, e, r: F.embedding(t, e) + r,
                    [((4, 16), torch.int64), ((100, 64), torch.float16),
                     ((4, 16, 64), torch.float16)])
    assert "#define SPY_GLD0 if (spy_v == 0) spy::load8f(in_ptr1" in code
    assert "spy_bad |=" in code and "spy::store8v<" in code


def test_scatter_keeps_element_stores(fake_device):
    # a scatter's index is computed in the element loop: the store stays an
    # element store inside that loop (a grouped store after the loop would
    # name a variable out of scope, and hiprtc rejects the kernel)
    cases = [
        (lambda c, p, k: c.index_copy(1, p, k),
         [((8, 64, 128), torch.float16), ((1,), torch.int64), ((8, 1, 128), torch.float16)]),
        (lambda c, p, k: c.index_put((p,), k),
         [((64, 128), torch.float16), ((4,), torch.int64), ((4, 128), torch.float16)]),
    ]
    for fn, specs in cases:
        code = _compile(fn, specs)
        assert _kernels(code)
        assert not re.search(r"store8v<[^>]*>\(out_ptr\d+ \+ \([^)]*tmp\d+", code)
        assert re.search(r"out_ptr\d+\[[^\]]*tmp\d+[^\]]*\] = spy::cvt", code)


def test_pointwise_group_form_in_place(fake_device):
    # an in-place update reads and writes the same buffer as whole groups
    def fn(x, y):
        x.mul_(2).add_(y)
        return x
    code = _compile(fn, [((32, 64), torch.float16), ((32, 64), torch.float16)])
    assert "spy::store8v<" in code


def test_transposing_copy_uses_flat_index(fake_device):
    code = _compile(lambda x: x.transpose(1, 2).contiguous() * 2,
                    [((4, 96, 64), torch.float16)])
    assert len(_kernels(code)) == 1 and "yindex" not in code


def test_unsupported_dynamic_shapes_raise(fake_device):
    from torch_spyre._inductor import Unsupported

    assert issubclass(Unsupported, RuntimeError)


def test_compiled_graph_cache_key_covers_the_backend_sources(monkeypatch):
    # Inductor reuses a cached compiled graph while the custom pass's uuid is
    # unchanged: the uuid must hash every source of the backend, so changed
    # kernel generation, scheduling or device runtime code is never served
    # from a stale cache
    from torch_spyre._inductor import passes

    seen = {}

    def fake_hash(files):
        seen["files"] = [os.path.basename(f) for f in files]
        return b"h"

    monkeypatch.setattr(passes, "get_hash_for_files", fake_hash)
    passes.CustomPostPasses().uuid()
    for name in ("spyre_kernel.py", "spyre_inductor_rt.h", "scheduling.py", "lowering.py",
                 "fuse_attention.py", "fuse_transpose.py", "__init__.py"):
        assert name in seen["files"], name
