"""The stick-layout descriptor algebra (torch_spyre._inductor.stickify) on
the CPU.

Reference: torch_spyre/_inductor/stickify.py:30-245.  The rules are pinned
independently of their formulas:
  * spyre_strides against a brute-force placement that walks the elements
    in dim_order-major order and gives each stick (or, for sparse formats,
    each element) the next free 128-byte slot;
  * reduction result sizes against torch's CPU reduction, and dim orders
    against the strides left after indexing the reduced dims away from a
    tensor laid out in that dim order;
  * pointwise result sizes against torch.broadcast_shapes, and the format
    rule on every DENSE/SPARSE pairing of tiny shapes.
"""

import itertools

import pytest
import torch

import torch_spyre  # noqa: F401
from torch_spyre._inductor import Unsupported
from torch_spyre._inductor.stickify import (BYTES_IN_STICK, SpyreDCI, SpyreFixedLayout,
                                            StickFormat, elems_per_stick,
                                            spyre_matmul_result_shape,
                                            spyre_pointwise_result_shape,
                                            spyre_reduction_result_shape, tensor_get_dci)


def _laid_out(size, order, dtype=torch.float32):
    """A CPU tensor of `size` whose memory order is `order` (outermost
    first), built by permuting a contiguous tensor."""
    phys = torch.empty([size[d] for d in order], dtype=dtype)
    inv = [order.index(d) for d in range(len(size))]
    return phys.permute(inv)


def _brute_offsets(size, order, dtype, fmt):
    """Element offsets by placement: walk elements with dim_order[-1]
    fastest; a DENSE layout packs them, a sparse one gives each element the
    start of its own stick."""
    eps = elems_per_stick(dtype)
    offs = {}
    pos = 0
    for idx in itertools.product(*[range(size[d]) for d in order]):
        full = [0] * len(size)
        for d, i in zip(order, idx):
            full[d] = i
        offs[tuple(full)] = pos
        pos += 1 if fmt == StickFormat.DENSE else eps
    return offs


@pytest.mark.parametrize("fmt", [StickFormat.DENSE, StickFormat.SPARSE, StickFormat.SPARSE_MULTI])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.int8])
def test_spyre_strides_brute_force(fmt, dtype):
    for size in ([5], [3, 4], [2, 3, 5], [2, 1, 3, 2]):
        for order in itertools.permutations(range(len(size))):
            st = SpyreDCI(list(order), format=fmt).spyre_strides(size, dtype)
            for idx, off in _brute_offsets(size, list(order), dtype, fmt).items():
                assert sum(i * s for i, s in zip(idx, st)) == off, (size, order, fmt)


def test_elems_per_stick_and_generic_dci():
    assert BYTES_IN_STICK == 128
    assert [elems_per_stick(d) for d in (torch.float16, torch.bfloat16, torch.float32, torch.int8)] \
        == [64, 64, 32, 128]
    t = torch.empty(512, 4096, dtype=torch.float16)
    d = SpyreDCI.generic_stick_dci(t)
    assert d.dim_order == [0, 1] and d.get_stick_dims() == [1] and d.format == StickFormat.DENSE
    assert d.is_stick_dim(1) and not d.is_stick_dim(0) and d.is_stick_dim([0, 1])
    assert d.spyre_strides([512, 4096], torch.float16) == list(t.stride())
    with pytest.raises(Unsupported):
        SpyreDCI([0, 1], num_stick_dims=2)


def test_dci_from_strides():
    assert tensor_get_dci(torch.empty(4, 6)).dim_order == [0, 1]
    assert tensor_get_dci(torch.empty(4, 6).t()).dim_order == [1, 0]
    col = torch.empty(10, 64, dtype=torch.float16)[:, 0]  # one element per stick
    assert tensor_get_dci(col).format == StickFormat.SPARSE
    t = torch.empty(3)
    t.spyre_dci = SpyreDCI([0], format=StickFormat.SPARSE_MULTI)
    assert tensor_get_dci(t).format == StickFormat.SPARSE_MULTI
    torch_spyre._inductor.stickify.install_spyre_tensors()
    assert torch.empty(2, 3).get_dci().dim_order == [0, 1]


def test_reduction_result_vs_torch():
    for size in ([2, 3], [2, 3, 4], [2, 3, 4, 5]):
        n = len(size)
        for order in itertools.permutations(range(n)):
            x = _laid_out(size, list(order))
            assert tensor_get_dci(x).dim_order == list(order)
            for k in range(1, n):
                for axes in itertools.combinations(range(n), k):
                    stick = order[-1] in axes
                    if stick and len(axes) > 1:
                        with pytest.raises(Unsupported):
                            spyre_reduction_result_shape(x, list(axes))
                        continue
                    for keep in (False, True):
                        rs, rd = spyre_reduction_result_shape(x, list(axes), keep)
                        y = x.sum(dim=axes, keepdim=keep)
                        assert rs == list(y.shape)
                        assert rd.format == (StickFormat.SPARSE if stick else StickFormat.DENSE)
                        if not keep:
                            kept = x[tuple(0 if d in axes else slice(None) for d in range(n))]
                            assert rd.dim_order == SpyreDCI.from_tensor(kept).dim_order, \
                                (size, order, axes)
                        else:
                            assert rd.dim_order == list(order)


def test_reduction_negative_axis_and_config_shape():
    x = torch.empty(512, 4096, dtype=torch.float16)
    rs, rd = spyre_reduction_result_shape(x, -1)
    assert rs == [512] and rd.dim_order == [0] and rd.format == StickFormat.SPARSE
    rs, rd = spyre_reduction_result_shape(x, 0)
    assert rs == [4096] and rd.format == StickFormat.DENSE
    # a SPARSE input reduced over a non-stick dim keeps its format
    s = torch.empty(6, 4)
    s.spyre_dci = SpyreDCI([0, 1], format=StickFormat.SPARSE)
    assert spyre_reduction_result_shape(s, 0)[1].format == StickFormat.SPARSE


def test_pointwise_result_shapes_and_formats():
    shapes = [[], [1], [3], [4, 3], [4, 1], [1, 3], [2, 4, 3], [2, 1, 1]]
    for a, b in itertools.product(shapes, repeat=2):
        x, y = torch.empty(a), torch.empty(b)
        try:
            want = list(torch.broadcast_shapes(tuple(a), tuple(b)))
        except RuntimeError:
            with pytest.raises(RuntimeError):
                spyre_pointwise_result_shape(x, y)
            continue
        rs, rd = spyre_pointwise_result_shape(x, y)
        assert rs == want and rd.dim_order == list(range(len(want)))
        assert rd.format == StickFormat.DENSE
    # DENSE [4,3] with a SPARSE operand broadcast along the stick dim: DENSE
    x = torch.empty(4, 3)
    s = torch.empty(4, 1)
    s.spyre_dci = SpyreDCI([0, 1], format=StickFormat.SPARSE)
    assert spyre_pointwise_result_shape(x, s)[1].format == StickFormat.DENSE
    assert spyre_pointwise_result_shape(s, x)[1].format == StickFormat.DENSE
    # ranks differ: the sparse [4,1] against DENSE [2,4,3] aligns from the right
    assert spyre_pointwise_result_shape(torch.empty(2, 4, 3), s)[1].format == StickFormat.DENSE
    # sparse operand NOT broadcast along the stick dim: unsupported
    s2 = torch.empty(4, 3)
    s2.spyre_dci = SpyreDCI([0, 1], format=StickFormat.SPARSE)
    with pytest.raises(Unsupported):
        spyre_pointwise_result_shape(x, s2)
    # both sparse: passes through
    assert spyre_pointwise_result_shape(s2, s)[1].format == StickFormat.SPARSE


def test_matmul_result_shape():
    a, b = torch.empty(6, 4), torch.empty(4, 5)
    rs, rd = spyre_matmul_result_shape(a, b)
    assert rs == [6, 5] and rd.dim_order == [0, 1] and rd.format == StickFormat.DENSE
    with pytest.raises(Unsupported):
        spyre_matmul_result_shape(a, torch.empty(5, 4).t())
    s = torch.empty(4, 5)
    s.spyre_dci = SpyreDCI([0, 1], format=StickFormat.SPARSE)
    with pytest.raises(Unsupported):
        spyre_matmul_result_shape(a, s)


def test_fixed_layout_carries_dci():
    d = SpyreDCI([1, 0])
    lay = d.spyre_layout(torch.device("spyre", 0), [8, 64], torch.float16)
    assert isinstance(lay, SpyreFixedLayout)
    assert list(lay.stride) == [1, 8] and lay.dci is d
    assert "dci=SpyreDCI(dim_order=[1, 0]" in str(lay)
