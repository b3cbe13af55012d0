"""Graph replay wrapper for the per-slice transform (hipGraph on ROCm).

Graphed(fn, *example) runs fn three times on a side stream (so lazy
allocations and library handles are created outside the graph), then
records one call on private copies of the example inputs. Each call copies
the new inputs in, replays the graph and returns clones of the recorded
outputs. Inference only: capture does not record autograd.
Reference surface: graphed.py:35-57.
"""
import torch


def _leaves(t):
    if torch.is_tensor(t):
        yield t
    elif isinstance(t, (list, tuple)):
        for u in t:
            yield from _leaves(u)


def _map(t, fn):
    if torch.is_tensor(t):
        return fn(t)
    if isinstance(t, tuple):
        return tuple(_map(u, fn) for u in t)
    if isinstance(t, list):
        return [_map(u, fn) for u in t]
    return t


class Graphed:
    def __init__(self, fn, *example):
        if not torch.cuda.is_available():
            raise RuntimeError("graph replay needs a GPU")
        self._fn = fn
        self._in = _map(example, lambda t: t.clone())
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(3):
                fn(*self._in)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self._out = fn(*self._in)

    @torch.no_grad()
    def replay(self):
        """Replay on the recorded inputs, return the recorded output buffers."""
        self.graph.replay()
        return self._out

    @torch.no_grad()
    def __call__(self, *args):
        for dst, src in zip(_leaves(self._in), _leaves(args)):
            dst.copy_(src)
        self.graph.replay()
        return _map(self._out, lambda t: t.clone())
