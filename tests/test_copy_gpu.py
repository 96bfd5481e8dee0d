"""Host<->device copies of the spyre device on MI355X (the copy engine of
csrc/aten/spyre_copy.cpp), called as user code calls them: Tensor.to,
copy_ with and without non_blocking.

Reference: the reference's copies (torch_spyre/csrc/spyre_mem.cpp:661-703)
ignore non_blocking and round trips hold to rtol 2e-3 (test_spyre.py:
138-152).  Here every copy is bit-exact.  The engine's edges are covered:
sizes around the 16 MiB staging chunk and its 4-buffer ring, the source
changing right after a staged host-to-device copy, pinned host memory with
non_blocking in both directions (torch's pinned memory and views into it at
an offset), and copies that convert dtype or layout on the way.
"""

import pytest
import torch

import torch_spyre  # noqa: F401  (registers the backend)

pytestmark = pytest.mark.gpu

DEV = "spyre"
CHUNK = 16 << 20  # staging chunk bytes


def _log(msg):
    print(f"[case] {msg}", flush=True)


def _bytes(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, (n,), dtype=torch.uint8, generator=g)


@pytest.mark.parametrize("nbytes", [1, 4095, CHUNK - 2, CHUNK, CHUNK + 2, 3 * CHUNK + 1234,
                                    5 * CHUNK - 6])
def test_pageable_round_trip_across_chunks(nbytes):
    _log(f"pageable round trip {nbytes} B")
    x = _bytes(nbytes, 1)
    d = x.to(DEV)
    assert torch.equal(d.cpu(), x)
    if nbytes % 2 == 0:  # fp16 view of the same bytes, converted on the way back
        h = x.view(torch.float16)
        assert torch.equal(h.to(DEV).cpu().view(torch.uint8), x)


def test_staging_ring_reuse_and_source_reuse():
    # more chunks than staging buffers in flight, interleaved with reads;
    # each source is overwritten right after its copy returns
    _log("staging ring reuse")
    n = 2 * CHUNK + 999
    srcs, devs = [], []
    for i in range(6):
        x = _bytes(n, 10 + i)
        srcs.append(x.clone())
        devs.append(x.to(DEV))
        x.fill_(0)  # a staged copy no longer reads the source
        if i % 2:
            assert torch.equal(devs[i - 1].cpu(), srcs[i - 1])
    for d, s in zip(devs, srcs):
        assert torch.equal(d.cpu(), s)


def test_pinned_non_blocking_both_ways():
    _log("pinned non_blocking")
    n = 3 * CHUNK + 77
    x = _bytes(n, 20)
    xp = x.pin_memory()
    d = torch.empty(n, dtype=torch.uint8, device=DEV)
    d.copy_(xp, non_blocking=True)
    torch.spyre.synchronize()
    xp.fill_(0)  # after the synchronise the device copy is complete
    back = torch.empty(n, dtype=torch.uint8).pin_memory()
    back.copy_(d, non_blocking=True)
    torch.spyre.synchronize()
    assert torch.equal(back, x)
    # pageable destination with non_blocking: complete on return
    back2 = torch.empty(n, dtype=torch.uint8)
    back2.copy_(d, non_blocking=True)
    assert torch.equal(back2, x)


def test_pinned_views_at_offsets():
    _log("pinned views")
    base = _bytes(CHUNK + 4096, 30).pin_memory()
    view = base[1000:1000 + CHUNK]
    d = torch.empty(CHUNK, dtype=torch.uint8, device=DEV)
    d.copy_(view, non_blocking=True)
    torch.spyre.synchronize()
    assert torch.equal(d.cpu(), view)
    out = torch.zeros(CHUNK + 4096, dtype=torch.uint8).pin_memory()
    out[17:17 + CHUNK].copy_(d, non_blocking=True)
    torch.spyre.synchronize()
    assert torch.equal(out[17:17 + CHUNK], view)
    assert int(out[:17].sum()) == 0 and int(out[17 + CHUNK:].sum()) == 0


def test_pinned_source_dropped_while_in_flight():
    # the engine keeps the pinned storage alive until its copy completes
    _log("pinned keep-alive")
    n = 4 * CHUNK
    x = _bytes(n, 40)
    d = torch.empty(n, dtype=torch.uint8, device=DEV)
    xp = x.pin_memory()
    d.copy_(xp, non_blocking=True)
    del xp
    torch.spyre.synchronize()
    assert torch.equal(d.cpu(), x)


def test_converting_and_strided_copies():
    _log("converting / strided copies")
    g = torch.Generator().manual_seed(50)
    x = torch.randn(1024, 3000, generator=g)
    d = torch.empty(1024, 3000, dtype=torch.float16, device=DEV)
    d.copy_(x)  # fp32 host -> fp16 device (converted on the host)
    assert torch.equal(d.cpu(), x.half())
    t = x.t()  # strided host source
    dt = t.to(DEV)
    assert torch.equal(dt.cpu(), t)
    dv = torch.zeros(3000, 2048, dtype=torch.float32, device=DEV)
    dv[:, ::2].copy_(t)  # strided device destination
    assert torch.equal(dv[:, ::2].cpu(), t)
    assert int(dv[:, 1::2].cpu().abs().sum()) == 0
    h = torch.empty(1024, 3000, dtype=torch.float64)
    h.copy_(d)  # device fp16 -> host fp64 (converted on the host)
    assert torch.equal(h, x.half().double())
