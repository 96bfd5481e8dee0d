"""numpy restatement of the device fills: the Philox4x32-10 random fills and
dropout, arange and cumsum.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference has no device implementation of these: it runs cumsum on the
CPU (codegen/inputs/spyre_torch_ops.cpp:502-505), arange and the random
fills through the CPU path, and native_dropout is an identity stub
(:180-186).  So arange and cumsum follow torch's CPU semantics (the
reference's CPU fallback is at::cumsum itself), and the random fills follow
the generator the device uses:

Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as
easy as 1, 2, 3", SC'11): ten rounds on a 4 x 32-bit counter under a 2 x
32-bit key; a round takes the products M0 c0 and M1 c2 (M0 = 0xD2511F53,
M1 = 0xCD9E8D57) to the new counter (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2),
hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)), and the key advances by (0x9E3779B9,
0xBB67AE85) between rounds.  Block j of a fill is the output for counter
(lo(offset + j), hi(offset + j), 0, 0) and key (lo(seed), hi(seed));
element i of a fill of 32-bit draws takes word i % 4 of block i // 4, a
fill of 64-bit draws the word pair 2(i % 2), 2(i % 2) + 1 of block i // 2
(first word high).

Pinned by tests/test_philox_oracle.py: the published known-answer vectors of
Philox4x32-10 (Random123's kat_vectors), torch's own Philox engine
(ATen/core/PhiloxRNGEngine.h, compiled on the host) on a sweep of seeds and
offsets, torch's CPU arange / cumsum, and the distributions' moments.
"""

from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = np.uint64(0xFFFFFFFF)

UNIFORM, NORMAL, INT = 0, 1, 2


def philox4x32_10(ctr, key):
    """ctr: uint32 [..., 4]; key: (k0, k1) -> uint32 [..., 4]."""
    c = [np.asarray(ctr, dtype=np.uint64)[..., i] for i in range(4)]
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for _ in range(10):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        c = [((p1 >> np.uint64(32)) ^ c[1] ^ np.uint64(k0)) & MASK32, p1 & MASK32,
             ((p0 >> np.uint64(32)) ^ c[3] ^ np.uint64(k1)) & MASK32, p0 & MASK32]
        k0 = (k0 + W0) & 0xFFFFFFFF
        k1 = (k1 + W1) & 0xFFFFFFFF
    return np.stack(c, axis=-1).astype(np.uint32)


def blocks(seed: int, offset: int, count: int) -> np.ndarray:
    """The fill's blocks 0..count-1: uint32 [count, 4]."""
    j = np.arange(count, dtype=np.uint64) + np.uint64(offset)
    ctr = np.stack([j & MASK32, j >> np.uint64(32), np.zeros_like(j), np.zeros_like(j)], axis=-1)
    return philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))


def n_blocks(kind: int, dtype, n: int, irange: int = 0) -> int:
    wide = irange > 0xFFFFFFFF if kind == INT else np.dtype(dtype) == np.float64
    return (n + 1) // 2 if wide else (n + 3) // 4


def _words32(seed, offset, n):
    return blocks(seed, offset, (n + 3) // 4).reshape(-1)[:n]


def _words64(seed, offset, n):
    b = blocks(seed, offset, (n + 1) // 2).astype(np.uint64)
    pairs = np.stack([(b[:, 0] << np.uint64(32)) | b[:, 1], (b[:, 2] << np.uint64(32)) | b[:, 3]],
                     axis=-1)
    return pairs.reshape(-1)[:n]


def _cast(x, dtype):
    if dtype == "bfloat16":
        import torch

        return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).float().numpy()
    return np.asarray(x).astype(dtype)


def uniform(n, dtype, seed, offset, a, b):
    """a + u (b - a), u in [0, 1): top 24 bits of each word (float32
    arithmetic, each step rounded), or top 53 bits of each 64-bit draw for
    float64; a value that rounds to b in the output type becomes a."""
    if dtype != "bfloat16" and np.dtype(dtype) == np.float64:
        u = (_words64(seed, offset, n) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        x = u * (np.float64(b) - np.float64(a)) + np.float64(a)
        return np.where(x >= b, np.float64(a), x)
    u = (_words32(seed, offset, n) >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)
    fa, fb = np.float32(a), np.float32(b)
    x = (u * (fb - fa)).astype(np.float32) + fa
    back = _cast(x, dtype).astype(np.float32)
    return _cast(np.where(back >= fb, fa, x), dtype)


def normal(n, dtype, seed, offset, mean, std):
    """mean + std * z, z from Box-Muller on word pairs: u1 in (0, 1] from
    the first word, u2 in [0, 1) from the second, z = sqrt(-2 ln u1) times
    cos(2 pi u2), then sin(2 pi u2).  Computed in float64 here (the device
    uses float32 transcendentals for 2- and 4-byte outputs)."""
    if dtype != "bfloat16" and np.dtype(dtype) == np.float64:
        d = _words64(seed, offset, 2 * ((n + 1) // 2)).reshape(-1, 2)
        u1 = ((d[:, 0] >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
        u2 = (d[:, 1] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    else:
        w = _words32(seed, offset, 4 * ((n + 3) // 4)).reshape(-1, 2).astype(np.uint64)
        u1 = ((w[:, 0] >> np.uint64(8)) + np.uint64(1)).astype(np.float64) * 2.0 ** -24
        u2 = (w[:, 1] >> np.uint64(8)).astype(np.float64) * 2.0 ** -24
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    z = np.stack([r * np.cos(t), r * np.sin(t)], axis=-1).reshape(-1)[:n]
    return _cast(mean + std * z, dtype)


def integers(n, dtype, seed, offset, ifrom, irange):
    """ifrom + draw % irange, 32-bit draws for ranges up to 2^32, 64-bit
    draws above."""
    if irange > 0xFFFFFFFF:
        d = _words64(seed, offset, n)
    else:
        d = _words32(seed, offset, n).astype(np.uint64)
    v = (np.uint64(ifrom & 0xFFFFFFFFFFFFFFFF) + d % np.uint64(irange)).astype(np.int64)
    return _cast(v.astype(np.float64), dtype) if (dtype == "bfloat16" or
                                                   np.dtype(dtype).kind == "f") else v.astype(dtype)


def dropout(x, p, scale, seed, offset):
    """(y, mask): element i kept when its uniform (word i % 4 of block
    offset + i // 4, top 24 bits) is >= p; y = x * scale where kept."""
    x = np.asarray(x)
    n = x.size
    u = (_words32(seed, offset, n) >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)
    keep = (u >= np.float32(p)).reshape(x.shape)
    y = np.where(keep, x.astype(np.float32) * np.float32(scale), np.float32(0))
    return y, keep


def arange(start, step, n, dtype):
    """start + step * i as torch's CPU arange accumulates: int64 for integer
    outputs, float32 for float16 / bfloat16, float64 for float32 / float64."""
    i = np.arange(n)
    if dtype != "bfloat16" and np.dtype(dtype).kind in "iu":
        return (np.int64(start) + np.int64(step) * i.astype(np.int64)).astype(dtype)
    if dtype == "bfloat16" or np.dtype(dtype) == np.float16:
        v = np.float32(start) + (np.float32(step) * i.astype(np.float32)).astype(np.float32)
        return _cast(v, dtype)
    return (np.float64(start) + np.float64(step) * i.astype(np.float64)).astype(dtype)


def cumsum(x, axis, out_dtype):
    """Sequential inclusive prefix sum along `axis` in torch's CPU
    accumulation type (float32 for float16 / bfloat16, float64 for float32 /
    float64, int64 for integers), each partial sum rounded to out_dtype."""
    x = np.asarray(x)
    if out_dtype == "bfloat16" or np.dtype(out_dtype) == np.float16:
        return _cast(np.cumsum(x.astype(np.float32), axis=axis, dtype=np.float32), out_dtype)
    if np.dtype(out_dtype).kind == "f":
        return np.cumsum(x.astype(np.float64), axis=axis, dtype=np.float64).astype(out_dtype)
    return np.cumsum(x.astype(np.int64), axis=axis, dtype=np.int64).astype(out_dtype)
