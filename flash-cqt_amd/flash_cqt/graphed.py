"""Graph replay wrapper for the per-slice transform (hipGraph on ROCm).

Graphed(fn, *example) records fn once on private copies of the example
inputs and then serves each call by copying the new inputs into those
copies, replaying the graph and returning clones of the recorded outputs.
Inference only: capture does not record autograd.

Before recording, fn runs a few times on a side stream (PyTorch's capture
recipe), so that lazily created workspaces, tables and library handles exist
outside the graph. A call must pass inputs of the recorded shapes (dtype and
device are converted by the copy); a shape mismatch raises instead of being
broadcast into the recorded buffers.
Reference surface: graphed.py:35-57.
"""
import torch


def _leaves(t):
    """Tensors of a nested list / tuple, in order."""
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


def _check_inputs(recorded, given):
    """Raise unless `given` holds as many tensors as `recorded`, each of the
    recorded shape."""
    if len(given) != len(recorded):
        raise ValueError(f"graph recorded {len(recorded)} input tensors, got {len(given)}")
    for i, (r, g) in enumerate(zip(recorded, given)):
        if tuple(g.shape) != tuple(r.shape):
            raise ValueError(f"input {i}: shape {tuple(g.shape)}, graph recorded {tuple(r.shape)}")


class Graphed:
    def __init__(self, fn, *example, warmup=3):
        if not torch.cuda.is_available():
            raise RuntimeError("graph replay needs a GPU")
        self._fn = fn
        self._in = _map(example, lambda t: t.clone())
        self._slots = list(_leaves(self._in))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(max(1, warmup)):
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
        given = list(_leaves(args))
        _check_inputs(self._slots, given)
        for dst, src in zip(self._slots, given):
            dst.copy_(src)
        self.graph.replay()
        return _map(self._out, lambda t: t.clone())
