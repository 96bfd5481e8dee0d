"""sph_attention_fwd_noalloc, the entry point that allocates nothing, against
sph_attention_fwd with a caller-allocated workspace, through the C-ABI.

Bit for bit on two calls in a row, the second smaller, for a masked prefill
call (its mask-block classes and job order live in the static scratch) and
a decode call (its key-split partials do); an unmasked prefill call (no
workspace at all); and a shape whose workspace exceeds the scratch is
refused before any launch with SPH_ERR_TOO_LARGE.
"""

import math

import pytest
import torch

from torch_spyre import _capi

from helpers import randn

pytestmark = pytest.mark.gpu

D = 128
SCALE = 1 / math.sqrt(D)


def _log(msg):
    print(f"[case] {msg}", flush=True)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _operands(b, mq, sk, seed, masked, ldm=None):
    q = randn((b, mq, D), k=seed).cuda()
    k = randn((b, sk, D), k=seed + 1).cuda()
    v = randn((b, sk, D), k=seed + 2).cuda()
    mask = None
    if masked:
        ldm = ldm or sk
        m = torch.zeros(mq, ldm)
        m[:, :sk] = torch.full((mq, sk), float("-inf")).triu(1 + max(sk - mq, 0))
        m[:, 0] = 0.0  # every row keeps a key
        mask = m.half().cuda()
    return q, k, v, mask, (ldm or sk)


def _call(name, q, k, v, mask, ldm, ws=None):
    b, mq, _ = q.shape
    sk = k.shape[1]
    o = torch.full_like(q, float("nan"))
    args = [_capi.F16, b, mq, sk, D, q.data_ptr(), D, mq * D, k.data_ptr(), D, sk * D,
            v.data_ptr(), D, sk * D, mask.data_ptr() if mask is not None else None,
            ldm if mask is not None else 0, 0, 0, 0, SCALE, o.data_ptr(), D, mq * D]
    if name == "sph_attention_fwd":
        args += [ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0]
    _capi.call(name, *args, _stream())
    torch.cuda.synchronize()
    return o


def _with_workspace(q, k, v, mask, ldm):
    lib = _capi.lib()
    b, mq, _ = q.shape
    n = lib.sph_attention_workspace_bytes(b, mq, k.shape[1], 0)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
    return _call("sph_attention_fwd", q, k, v, mask, ldm, ws)


@pytest.mark.parametrize("kind", ["prefill_masked", "decode", "prefill_unmasked"])
def test_noalloc_matches_workspace_entry_twice(kind):
    shapes = {"prefill_masked": [(2, 512, 640, None), (1, 256, 300, 304)],
              "decode": [(32, 4, 1152, None), (8, 4, 200, None)],
              "prefill_unmasked": [(2, 512, 640, None), (1, 256, 300, None)]}[kind]
    for i, (b, mq, sk, ldm) in enumerate(shapes):
        _log(f"no-alloc attention {kind} call {i + 1}: b={b} mq={mq} sk={sk}")
        q, k, v, mask, ld = _operands(b, mq, sk, 80 + 10 * i, kind == "prefill_masked", ldm)
        want = _with_workspace(q, k, v, mask, ld)
        got = _call("sph_attention_fwd_noalloc", q, k, v, mask, ld)
        assert not torch.isnan(want).any()
        assert torch.equal(got, want), f"{kind} call {i + 1}"


def test_noalloc_refuses_shapes_beyond_the_scratch():
    lib = _capi.lib()
    cap = lib.sph_attention_fwd_noalloc_max_bytes()
    assert cap == 4 << 20
    b, mq, sk = 64, 16, 2048  # decode: 64 x 32 splits x 16 rows of fp32 partials
    need = lib.sph_attention_workspace_bytes(b, mq, sk, 0)
    assert need > cap
    _log(f"no-alloc attention refuses b={b} mq={mq} sk={sk} ({need} bytes)")
    q, k, v, _, _ = _operands(b, mq, sk, 99, False)
    o = torch.zeros_like(q)
    rc = lib.sph_attention_fwd_noalloc(_capi.F16, b, mq, sk, D, q.data_ptr(), D, mq * D,
                                       k.data_ptr(), D, sk * D, v.data_ptr(), D, sk * D, None,
                                       0, 0, 0, 0, SCALE, o.data_ptr(), D, mq * D, _stream())
    assert rc == 1003  # SPH_ERR_TOO_LARGE
    assert b"static scratch" in lib.sph_last_error()
    torch.cuda.synchronize()
    assert not o.any()  # nothing was launched
