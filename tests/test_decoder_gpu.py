"""The decoder workload (configs c4 / c5) on the spyre device, eager and
under torch.compile, against the numpy oracle (oracle/decoder.py) at the
device's fp16 rounding points (eager: every op output; compiled: every
fused kernel's output), rtol = atol = 1e-2.

c4 runs at its full shape (hidden 4096, 32/8 heads, SwiGLU 12800, seq
2048).  The c5 flow (prefill into the contiguous KV cache, then greedy
decode) runs on a 2-layer model of the same layer shape with a short
prompt; its logits are compared teacher-forced (the CPU's tokens are fed
to both), and the greedy tokens must agree with the oracle's argmax
wherever the oracle's top-2 logits are separated by more than the
tolerance.
"""

import dataclasses

import numpy as np
import pytest
import torch

import torch_spyre  # noqa: F401

from oracle import decoder as OD
from torch_spyre.examples import decoder as D

pytestmark = pytest.mark.gpu

DEV = "spyre"
SMALL = D.DecoderConfig(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, intermediate=1280,
                        vocab=1000, n_layers=2)


def _log(msg):
    print(f"[case] {msg}", flush=True)


def _np(params):
    return {"embed": params["embed"].float().numpy(),
            "layers": [{k: v.float().numpy() for k, v in w.items()} for w in params["layers"]],
            "final_norm": params["final_norm"].float().numpy(),
            "lm_head": params["lm_head"].float().numpy()}


def _to(params, dev):
    return {"embed": params["embed"].to(dev),
            "layers": [{k: v.to(dev) for k, v in w.items()} for w in params["layers"]],
            "final_norm": params["final_norm"].to(dev), "lm_head": params["lm_head"].to(dev)}


def _tokens(B, S, vocab, seed=0):
    return torch.randint(0, vocab, (B, S), generator=torch.Generator().manual_seed(0xAFFE + seed))


def _block(cfg, S, compiled):
    params = D.init_params(cfg, "cpu", seed=0xAFFE)
    tok = _tokens(1, S, cfg.vocab)
    dp = _to(params, DEV)
    cos, sin = D.rope_tables(cfg, S, DEV)
    mask = D.causal_mask(cfg, S, DEV)
    fn = D.block_forward
    if compiled:
        torch._dynamo.reset()
        fn = torch.compile(D.block_forward)
    h = fn(tok.to(DEV), dp, cos, sin, mask, cfg).cpu().float().numpy()
    want = OD.block(tok.numpy(), _np(params), cfg, act=np.float16, fused=compiled)
    return h, want


@pytest.mark.parametrize("compiled", [False, True])
def test_small_block_vs_oracle(compiled):
    _log(f"decoder block small compiled={compiled}")
    h, want = _block(dataclasses.replace(SMALL, n_layers=1), 256, compiled)
    np.testing.assert_allclose(h, want, rtol=1e-2, atol=1e-2)


def _violations(a, b, tol=1e-2):
    d = np.abs(a - b)
    return float(np.mean(d > tol + tol * np.abs(b))), float(d.max())


def test_c4_block_compiled_vs_oracle():
    """At the full c4 shape two correct fp16 programs differ beyond 1e-2 at
    a few elements per million: an fp16 score of |s| ~ 60 carries an error
    of 0.03 before the 1/sqrt(128) scale, and a one-ulp difference in q, k
    or a SwiGLU product moves the K = 12800 down projection by ~0.005.  The
    gate is therefore calibrated on the oracle itself: the device may not
    differ from the compiled-program oracle by more than the oracle's
    eager-rounding variant differs from it (fraction beyond rtol = atol =
    1e-2, and the largest deviation), with rtol = atol = 1e-2 holding for
    all but 1e-4 of the elements."""
    _log("c4 decoder layer compiled, seq 2048")
    params = D.init_params(D.C4, "cpu", seed=0xAFFE)
    tok = _tokens(1, 2048, D.C4.vocab)
    h, want = _block(D.C4, 2048, True)
    eager = OD.block(tok.numpy(), _np(params), D.C4, act=np.float16, fused=False)
    frac_dev, max_dev = _violations(h, want)
    frac_floor, max_floor = _violations(eager, want)
    print(f"device vs oracle: {frac_dev:.2e} beyond 1e-2, max {max_dev:.4f}; "
          f"oracle eager vs fused: {frac_floor:.2e}, max {max_floor:.4f}", flush=True)
    assert frac_dev <= 1e-4
    assert frac_dev <= max(frac_floor, 1e-6) and max_dev <= max(max_floor, 1e-2)


@pytest.mark.parametrize("compiled", [False, True])
def test_c5_flow_teacher_forced_vs_oracle(compiled):
    """compiled = prefill layers and the static decode step under
    torch.compile (the decode step's fused kernels round like the eager
    ops except RoPE and SiLU*up, which the fused oracle models)."""
    _log(f"c5 flow (2 layers of the c4 shape) compiled={compiled}")
    cfg = dataclasses.replace(D.C5, n_layers=2)
    params = D.init_params(cfg, "cpu", seed=0xAFFE + 1)
    prompt = _tokens(4, 64, cfg.vocab, seed=1)
    teacher = _tokens(4, 6, cfg.vocab, seed=2)
    layer_fn = decode_fn = None
    if compiled:
        torch._dynamo.reset()
        layer_fn = torch.compile(D.layer_forward)
        decode_fn = torch.compile(D.decode_step_static)
    toks, logits = D.generate(prompt.to(DEV), _to(params, DEV), cfg, 6, DEV, layer_fn=layer_fn,
                              teacher=teacher.to(DEV), decode_fn=decode_fn)
    want = OD.generate_teacher_forced(prompt.numpy(), teacher.numpy(), _np(params), cfg,
                                      fused=compiled)
    got = logits.cpu().float().numpy()
    if not compiled:
        np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)
    else:
        # the noise-floor gate of the c4 test (two fp16 rounding regimes of
        # the oracle bound the device's deviation)
        eager = OD.generate_teacher_forced(prompt.numpy(), teacher.numpy(), _np(params), cfg,
                                           fused=False)
        frac_dev, max_dev = _violations(got, want)
        frac_floor, max_floor = _violations(eager, want)
        print(f"device vs oracle: {frac_dev:.2e}, max {max_dev:.4f}; "
              f"floor: {frac_floor:.2e}, max {max_floor:.4f}", flush=True)
        assert frac_dev <= 1e-4
        assert frac_dev <= max(frac_floor, 1e-5) and max_dev <= max(max_floor, 1e-2) * 1.5
    # greedy tokens: equal to the oracle's argmax wherever that argmax is
    # decided by more than the tolerance
    top2 = np.sort(want, axis=-1)[..., -2:]
    decided = (top2[..., 1] - top2[..., 0]) > 2e-2
    oracle_tok = want.argmax(-1)[:-1].T
    dev_tok = toks.cpu().numpy()
    sel = decided[:-1].T
    assert sel.sum() > 0
    assert np.array_equal(dev_tok[sel], oracle_tok[sel])
