"""The oracle of the device fills (oracle/philox.py) on the CPU.

Philox4x32-10 is pinned by its published known-answer vectors (Random123's
kat_vectors for philox4x32_10) and by torch's own Philox engine
(ATen/core/PhiloxRNGEngine.h, compiled here with g++) over a sweep of seeds
and counter offsets; the distributions by their moments and
Kolmogorov-Smirnov tests; arange and cumsum by torch's CPU kernels, which
are what the reference runs for them (its cumsum is a CPU fallback,
codegen/inputs/spyre_torch_ops.cpp:502-505).
"""

import os
import shutil
import subprocess

import numpy as np
import pytest
import scipy.stats
import torch

from oracle import philox as P

# (counter, key, output) from Random123's kat_vectors, philox4x32 10 rounds
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = P.philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
    assert [int(v) for v in got] == list(want)


def test_philox_matches_torch_engine(tmp_path):
    gxx = shutil.which("g++")
    inc = os.path.join(os.path.dirname(torch.__file__), "include")
    hdr = os.path.join(inc, "ATen", "core", "PhiloxRNGEngine.h")
    if gxx is None or not os.path.exists(hdr):
        pytest.skip("g++ or torch's PhiloxRNGEngine.h not available")
    src = tmp_path / "t.cpp"
    src.write_text(r"""
#include <ATen/core/PhiloxRNGEngine.h>
#include <cstdio>
#include <cstdlib>
int main(int argc, char** argv) {
  for (int a = 1; a + 1 < argc; a += 2) {
    unsigned long long seed = strtoull(argv[a], 0, 0), off = strtoull(argv[a + 1], 0, 0);
    at::Philox4_32 e(seed, 0, off);  // counter (lo off, hi off, 0, 0), key (lo seed, hi seed)
    unsigned w0 = e(), w1 = e(), w2 = e(), w3 = e();
    printf("%u %u %u %u\n", w0, w1, w2, w3);
  }
}
""")
    exe = tmp_path / "t"
    subprocess.run([gxx, "-std=c++17", "-O1", f"-I{inc}", str(src), "-o", str(exe)], check=True)
    cases = [(0, 0), (1, 0), (0xAFFE, 7), (0x123456789ABCDEF0, (1 << 32) + 5),
             ((1 << 64) - 1, (1 << 64) - 2), (42, 123456789)]
    out = subprocess.run([str(exe)] + [str(v) for c in cases for v in c], check=True,
                         capture_output=True, text=True).stdout.split("\n")
    for (seed, off), line in zip(cases, out):
        want = [int(v) for v in line.split()]
        got = [int(v) for v in P.blocks(seed, off, 1)[0]]
        assert got == want, (seed, off)


def test_planted_wrong_constant_fails_the_known_answer():
    # a dropped key increment (one plausible slip) changes the first vector
    orig = P.W1
    try:
        P.W1 = 0
        got = P.philox4x32_10(np.array([KAT[0][0]], dtype=np.uint32), KAT[0][1])[0]
        assert [int(v) for v in got] != list(KAT[0][2])
    finally:
        P.W1 = orig


def test_block_layout_and_offsets():
    # a fill at offset o continues a fill at offset 0 exactly where it ends
    a = P.uniform(64, np.float32, 5, 0, 0.0, 1.0)
    b = P.uniform(32, np.float32, 5, 8, 0.0, 1.0)
    np.testing.assert_array_equal(a[32:], b)
    assert P.n_blocks(P.UNIFORM, np.float32, 10) == 3
    assert P.n_blocks(P.UNIFORM, np.float64, 10) == 5
    assert P.n_blocks(P.INT, np.int64, 10, irange=1 << 40) == 5


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16, "bfloat16"])
def test_uniform_distribution(dtype):
    u = np.asarray(P.uniform(200_000, dtype, 0xAFFE, 3, -2.0, 3.0), np.float64)
    assert u.min() >= -2.0 and u.max() < 3.0
    assert abs(u.mean() - 0.5) < 0.02 and abs(u.var() - 25 / 12) < 0.03
    if dtype in (np.float32, np.float64):
        assert scipy.stats.kstest((u + 2) / 5, "uniform").pvalue > 1e-3


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_normal_distribution(dtype):
    z = np.asarray(P.normal(200_001, dtype, 0xAFFE, 0, 1.5, 2.0), np.float64)
    assert abs(z.mean() - 1.5) < 0.02 and abs(z.std() - 2.0) < 0.02
    assert scipy.stats.kstest((z - 1.5) / 2.0, "norm").pvalue > 1e-3


def test_integer_ranges():
    v = P.integers(100_000, np.int64, 9, 0, -5, 11)
    assert v.min() == -5 and v.max() == 5
    counts = np.bincount(v + 5)
    assert scipy.stats.chisquare(counts).pvalue > 1e-3
    w = P.integers(1000, np.int64, 9, 0, 0, 1 << 40)  # 64-bit draws
    assert w.min() >= 0 and w.max() < (1 << 40) and w.max() > (1 << 39)


@pytest.mark.parametrize("start,end,step,dtype", [
    (0, 10, 1, torch.int64), (-7, 100, 3, torch.int32), (5, -20, -4, torch.int64),
    (0, 2048, 1, torch.float16), (0.0, 100.0, 0.5, torch.float32), (-3.0, 3.0, 0.25, torch.float64),
    (0, 300, 1, torch.bfloat16), (1.0, 2.0, 0.1, torch.float32)])
def test_arange_oracle_vs_torch(start, end, step, dtype):
    want = torch.arange(start, end, step, dtype=dtype)
    nd = "bfloat16" if dtype == torch.bfloat16 else torch.empty(0, dtype=dtype).numpy().dtype
    got = P.arange(start, step, want.numel(), nd)
    w = want.float().numpy() if dtype == torch.bfloat16 else want.numpy()
    if step == 0.1:  # a step that is not a binary fraction: one ulp apart at most
        np.testing.assert_allclose(np.asarray(got, np.float64), w, rtol=2 ** -23, atol=0)
    else:
        np.testing.assert_array_equal(np.asarray(got), w)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64,
                                   torch.int32, torch.int64, torch.uint8])
@pytest.mark.parametrize("shape,dim", [((7, 300), 1), ((300, 5), 0), ((4, 6, 50), 1)])
def test_cumsum_oracle_vs_torch(dtype, shape, dim):
    g = torch.Generator().manual_seed(0xAFFE)
    if dtype.is_floating_point:
        x = (torch.randn(*shape, generator=g) * 3).to(dtype)
    else:
        x = torch.randint(0, 100, shape, generator=g).to(dtype)
    want = torch.cumsum(x, dim)
    od = {torch.float16: np.float16, torch.bfloat16: "bfloat16", torch.float32: np.float32,
          torch.float64: np.float64}.get(want.dtype, np.int64)
    xn = x.float().numpy() if dtype == torch.bfloat16 else x.numpy()
    got = P.cumsum(xn, dim, od)
    wn = want.float().numpy() if want.dtype == torch.bfloat16 else want.numpy()
    np.testing.assert_array_equal(np.asarray(got, dtype=wn.dtype), wn)
