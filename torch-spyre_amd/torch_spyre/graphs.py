"""HIP graphs of the spyre stream (the launch-bound decode loop's path).

The counterpart of torch.cuda.CUDAGraph / torch.cuda.graph for the spyre
device: everything the captured code launches on the device's spyre stream
(eager spyre ops, kernels of torch.compile'd spyre graphs, copies between
spyre tensors) is recorded once and replayed with one hipGraphLaunch.
Tensors allocated during the capture come from a private pool that stays
reserved for the graph, so each replay reads the same inputs and writes the
same outputs: update inputs in place between replays and read outputs
before the next replay.  Code that synchronises with the host (`.item()`,
`.cpu()`, copies from host memory) cannot be captured.  Kernels launched for
the first time load their code objects, so run the captured code once
before capturing it.
"""

from __future__ import annotations

import contextlib

import torch


class SpyreGraph:
    def __init__(self):
        from torch_spyre import _C

        self._g = _C.Graph()

    def capture_begin(self):
        self._g.capture_begin()

    def capture_end(self):
        self._g.capture_end()

    def replay(self):
        self._g.replay()

    def reset(self):
        self._g.reset()

    def pool(self) -> int:
        return self._g.pool()


@contextlib.contextmanager
def graph(g: SpyreGraph):
    """`with torch.spyre.graph(g): ...` captures the body into `g`."""
    g.capture_begin()
    try:
        yield g
    except BaseException:
        g.reset()
        raise
    g.capture_end()
