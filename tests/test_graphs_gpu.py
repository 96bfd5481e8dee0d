"""HIP graphs of the spyre stream (torch.spyre.SpyreGraph / torch.spyre.graph).

Every replay is checked against the same work done eagerly, with eager work
and host synchronisations between replays, and the private pool's buffers
are checked not to be reused by allocations outside the graph.  The decode
loop of the c5 flow (torch.compile'd static decode step + argmax + position
update in one graph) must produce exactly the tokens and logits of the
same loop without the graph.
"""

import dataclasses

import pytest
import torch

import torch_spyre  # noqa: F401
from torch_spyre.examples import decoder as D

from helpers import randn

pytestmark = pytest.mark.gpu

DEV = "spyre"


def _log(msg):
    print(f"[case] {msg}", flush=True)


def test_graph_replays_eager_ops():
    _log("graph of eager ops")
    a = randn((64, 300), k=0).to(DEV)
    w = randn((300, 200), k=1).to(DEV)

    def fn():
        return torch.softmax(torch.mm(a, w) * 0.5 + 1.0, dim=-1)

    fn()  # load kernels
    torch.spyre.synchronize()
    g = torch.spyre.SpyreGraph()
    with torch.spyre.graph(g):
        out = fn()
    for i in range(4):
        a.copy_(randn((64, 300), k=10 + i).to(DEV))
        g.replay()
        torch.spyre.synchronize()
        # eager work between replays must not touch the graph's buffers
        junk = [torch.full((64, 200), 7.0, device=DEV, dtype=torch.float16) for _ in range(3)]
        want = fn()
        assert torch.equal(out.cpu(), want.cpu()), f"replay {i}"
        del junk
    g.reset()


def test_graph_of_compiled_function():
    _log("graph of a compiled function")
    torch._dynamo.reset()
    x = randn((512, 1024), k=2).to(DEV)
    r = randn((512, 1024), k=3).to(DEV)
    wt = randn((1024,), k=4, mean=1.0, scale=0.02).to(DEV)
    f = torch.compile(lambda a, b, c: torch.rms_norm(a + b, [1024], c, 1e-5) * 2)
    f(x, r, wt)
    torch.spyre.synchronize()
    g = torch.spyre.SpyreGraph()
    with torch.spyre.graph(g):
        y = f(x, r, wt)
    for i in range(3):
        x.copy_(randn((512, 1024), k=20 + i).to(DEV))
        g.replay()
        assert torch.equal(y.cpu(), f(x, r, wt).cpu()), f"replay {i}"
    g.reset()


def test_graph_decode_loop_matches_ungraphed():
    _log("graph decode loop (2 layers of the c5 shape)")
    torch._dynamo.reset()
    cfg = dataclasses.replace(D.C5, n_layers=2)
    params = D.init_params(cfg, DEV, seed=0xAFFE + 3)
    prompt = torch.randint(0, cfg.vocab, (4, 64),
                           generator=torch.Generator().manual_seed(5)).to(DEV)
    dec = torch.compile(D.decode_step_static)
    t1, l1 = D.generate(prompt, params, cfg, 6, DEV, decode_fn=dec)
    t2, l2 = D.generate(prompt, params, cfg, 6, DEV, decode_fn=dec, use_graph=True)
    assert torch.equal(t1.cpu(), t2.cpu())
    assert torch.equal(l1.cpu(), l2.cpu())
