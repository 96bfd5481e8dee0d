"""The reference's compiled-op test matrix on spyre tensors
(tests/_inductor/test_inductor_ops.py:58-232), shapes and ops as there.

The reference compares torch.compile on its device with its eager device
result (exactly) and with the CPU at rtol = atol = 0.1 (compare /
compare_with_cpu, tests/_inductor/utils_inductor.py:186-231).  Here every
case is compared with torch's CPU result in fp32 cast to the output dtype at
the north star's rtol = atol = 1e-2, and with the eager spyre result at the
same tolerance; data movement (transposes) and selections (where, max) must
match the CPU bit for bit.  Inputs are fp16 as the reference's
cached_randn, from seeded generators.
"""

import pytest
import torch

import torch_spyre  # noqa: F401

from helpers import randn

pytestmark = pytest.mark.gpu

DEV = "spyre"
FP16_EPS = torch.finfo(torch.float16).eps
TOL = dict(rtol=1e-2, atol=1e-2, equal_nan=True)

UNARY = {"abs": torch.abs, "exp": torch.exp, "reciprocal": torch.reciprocal, "relu": torch.relu,
         "tanh": torch.tanh}
BINARY = {"add": torch.add, "mul": torch.mul, "sub": torch.sub, "div": torch.div}
ALIAS = {"double": lambda x: x + x, "square": lambda x: x * x, "cube": lambda x: x * x * x,
         "triple": lambda x: x + x + x}


def _log(msg):
    print(f"[case] {msg}", flush=True)


def _compare(fn, *args, exact=False):
    torch._dynamo.reset()
    dev = [a.to(DEV) for a in args]
    got = torch.compile(fn)(*dev).cpu()
    want = fn(*[a.float() if a.is_floating_point() else a for a in args])
    want = want.to(got.dtype)
    if exact:
        assert torch.equal(got, fn(*args)), "compiled result differs from the CPU's"
    else:
        torch.testing.assert_close(got.float(), want.float(), **TOL)
    eager = fn(*dev).cpu()
    torch.testing.assert_close(got.float(), eager.float(), **TOL)


def _abs(shape, k):
    return randn(shape, k=k).abs()


@pytest.mark.parametrize("shape", [(64,), (67, 256)])
@pytest.mark.parametrize("name", ["sqrt", "rsqrt", "log"])
def test_unary_domain_ops(name, shape):
    # sqrt on |x|; rsqrt and log on |x| + eps (reference :60-95)
    _log(f"compiled {name} {shape}")
    x = _abs(shape, 1) + (0 if name == "sqrt" else FP16_EPS)
    _compare(getattr(torch, name), x.half())


@pytest.mark.parametrize("shape", [(256,), (67, 256)])
@pytest.mark.parametrize("name", list(UNARY))
def test_pointwise_unary(name, shape):
    _log(f"compiled {name} {shape}")
    x = randn(shape, k=2)
    if name == "reciprocal":
        x[x == 0] = FP16_EPS  # the reference's division-by-zero sidestep
    _compare(UNARY[name], x)


@pytest.mark.parametrize("shape", [(256,), (67, 256)])
@pytest.mark.parametrize("name", list(BINARY))
def test_pointwise_binary(name, shape):
    _log(f"compiled {name} {shape}")
    a, b = randn(shape, k=3), randn(shape, k=4)
    if name == "div":
        b[b == 0] = FP16_EPS
    _compare(BINARY[name], a, b)


def test_add_broadcast():
    _log("compiled add broadcast (256,) + (67, 256)")
    _compare(lambda x, y: torch.add(x[None, :], y), randn((256,), k=5), randn((67, 256), k=6))


@pytest.mark.parametrize("name", ["mm", "matmul"])
def test_mm(name):
    _log(f"compiled {name} 67x256 . 256x128")
    _compare(getattr(torch, name), randn((67, 256), k=7), randn((256, 128), k=8))


@pytest.mark.parametrize("dim", [0, 1])
@pytest.mark.parametrize("name", ["sum", "max"])
def test_reduce_2d(name, dim):
    # the reference runs dim 0 only (its eager dim-1 result is not readable)
    _log(f"compiled {name} over dim {dim} of 67x256")
    x = randn((67, 256), k=9)
    if name == "max":
        _compare(lambda x: torch.max(x, dim=dim)[0], x, exact=True)
    else:
        _compare(lambda x: torch.sum(x, dim=dim), x)


@pytest.mark.parametrize("dim", [0, 1])
def test_max_sub_broadcast(dim):
    _log(f"compiled x - max(x, {dim}) on 128x256")

    def fn(x):
        return x - torch.unsqueeze(torch.max(x, dim=dim)[0], dim=dim)

    _compare(fn, randn((128, 256), k=10))


@pytest.mark.parametrize("shape", [(256,), (67, 256)])
@pytest.mark.parametrize("name", list(ALIAS))
def test_alias_operands(name, shape):
    _log(f"compiled alias {name} {shape}")
    _compare(ALIAS[name], randn(shape, k=11))


def test_transpose_2d():
    _log("compiled x.t().contiguous() 1088x320")
    _compare(lambda x: x.t().contiguous(), randn((1088, 320), k=12), exact=True)


@pytest.mark.parametrize("d0,d1", [(0, 2), (1, 2)])
def test_transpose_3d(d0, d1):
    _log(f"compiled transpose({d0}, {d1}).contiguous() 512x256x128")
    _compare(lambda x: torch.transpose(x, d0, d1).contiguous(), _abs((512, 256, 128), 13),
             exact=True)


@pytest.mark.parametrize("cond", ["eq", "ge"])
def test_where(cond):
    _log(f"compiled where({cond})")
    x, y = randn((256,), k=14), randn((256,), k=15)
    y[::7] = x[::7]  # some equal pairs, so eq selects both ways
    op = (lambda a, b: a == b) if cond == "eq" else (lambda a, b: a >= b)
    _compare(lambda a, b: torch.where(op(a, b), a, b), x, y, exact=True)


@pytest.mark.parametrize("shape,dims", [((1088, 320), (1, 0)), ((512, 256, 128), (2, 1, 0)),
                                        ((512, 256, 128), (0, 2, 1)),
                                        ((8, 2048, 32, 128), (0, 2, 1, 3)),
                                        ((7, 100, 33), (0, 2, 1))])
def test_eager_transposing_copies_bit_exact(shape, dims):
    # eager .contiguous() of a permuted view: the tiled transpose when the
    # innermost dimension moves, the elementwise copy otherwise
    _log(f"eager permute{dims}.contiguous() {shape}")
    x = randn(shape, k=16)
    got = x.to(DEV).permute(*dims).contiguous()
    assert got.is_contiguous()
    assert torch.equal(got.cpu(), x.permute(*dims).contiguous())
