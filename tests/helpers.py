"""Seeded inputs and comparison helpers shared by the tests and the bench.

Inputs follow the reference's seeding convention (seed 0xAFFE,
tests/_inductor/test_inductor_ops.py:50, examples/softmax.py:18): the k-th
tensor of a case is drawn on the CPU in fp32 from
torch.Generator().manual_seed(0xAFFE + k), then cast.
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

SEED = 0xAFFE
GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name: str):
    """A section of tests/golden/reference_vectors.json (the reference
    tests' known answers)."""
    with open(os.path.join(GOLDEN_DIR, "reference_vectors.json")) as f:
        return json.load(f)[name]


def gen(k: int) -> torch.Generator:
    return torch.Generator().manual_seed(SEED + k)


def randn(shape, k=0, scale=1.0, mean=0.0, dtype=torch.float16):
    return (torch.randn(*shape, generator=gen(k), dtype=torch.float32) * scale + mean).to(dtype)


def uniform(shape, k=0, lo=-1.0, hi=1.0, dtype=torch.float16):
    return (torch.rand(*shape, generator=gen(k), dtype=torch.float32) * (hi - lo) + lo).to(dtype)


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu").float().numpy()


def assert_close_fp(actual: torch.Tensor, expected_f32: np.ndarray, out_dtype=torch.float16,
                    rtol=1e-2, atol=1e-2, what=""):
    """Device result vs the oracle's fp32 result rounded to the output dtype,
    at the tolerance the north-star sets for fp16 (rtol = atol = 1e-2)."""
    exp = torch.from_numpy(np.ascontiguousarray(expected_f32)).to(out_dtype)
    act = actual.detach().to("cpu")
    torch.testing.assert_close(act.float(), exp.float(), rtol=rtol, atol=atol, equal_nan=True,
                               msg=lambda m: f"{what}: {m}")
