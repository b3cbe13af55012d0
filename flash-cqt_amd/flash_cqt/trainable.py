"""TrainableCQT: OctCQT-shaped fwd/bwd on the fused HIP engine, with autograd.

Same surface as the reference (trainable.py:28-191):
    t = TrainableCQT(cqt)         # cqt: OctCQT at audio_len 65536
    blocks, side = t.fwd(x)       # x [..., 65536], leading dims preserved
    y = t.bwd(blocks, side)       # gradients flow both ways
The transform is linear, so each backward is the transpose run on the same
engines with other tables: the analysis transpose is the scatter engine with
the analysis-adjoint gains plus the packed inverse tail; the synthesis
transpose is the packed FFT plus the route engine with the dual-window
record (flash_cqt/tables.py). Nothing is saved for backward.

Coefficients live in one interleaved complex64 buffer [B, ncoef]; the
returned blocks are views into it (no per-group copies), and bwd reads that
buffer in place when it is handed the same views back (the reference
concatenates the blocks, trainable.py:161-164).
"""
import torch

from . import _native
from .fused import FusedOctCQT, N


class TrainableCQT:
    """Differentiable octave CQT on the fused engine."""

    def __init__(self, cqt, device="cuda"):
        self.f = FusedOctCQT(cqt, device)
        self.cqt = cqt
        self.dev = self.f.dev
        self.gspec = self.f.gspec
        self.ncoef = self.f.ncoef
        self.ngroups = len(cqt.groups)

    # ------------------------------------------------ engine directions
    # The inputs reaching these are [B, N] float32 or [B, ncoef] complex64,
    # contiguous and on the engine's device (fwd/bwd and the autograd
    # Functions make them so); outputs are fresh buffers of the right size.
    # So the launches go straight to the C ABI with the engine's cached
    # workspace and table pointers.

    def _launch_analysis(self, x, table):
        B = x.shape[0]
        f = self.f
        f._workspace(B)
        p = f._wp[B]
        kc = torch.empty(B, self.ncoef, dtype=torch.complex64, device=self.dev)
        _native.check(f.lib.fcqt_analysis(f._ct, f._tp[table], x.data_ptr(), kc.data_ptr(), None,
                                          _native.INTERLEAVED, p["X"], p["W"], B,
                                          _native.stream_handle(self.dev.index)), "analysis")
        return kc

    def _launch_synthesis(self, kc, table, fbuf):
        B = kc.shape[0]
        f = self.f
        f._fbuf(table, B)                  # the table's scatter buffer (FA on first adjoint use)
        p = f._wp[B]
        y = torch.empty(B, N, dtype=torch.float32, device=self.dev)
        _native.check(f.lib.fcqt_synthesis(f._ct, f._tp[table], f._tp["ovf_" + table], kc.data_ptr(), None,
                                           _native.INTERLEAVED, p[fbuf], p["W"], y.data_ptr(), B,
                                           _native.stream_handle(self.dev.index)), "synthesis")
        return y

    def _analysis(self, x):
        return self._launch_analysis(x, "route")

    def _synthesis(self, kc):
        return self._launch_synthesis(kc, "scat", "F")

    def _adj_analysis(self, gk):
        return self._launch_synthesis(gk, "scat_a", "FA")

    def _adj_synthesis(self, gy):
        return self._launch_analysis(gy, "route_b")

    # ---------------------------------------------------- public surface

    def fwd(self, x):
        """x [..., N] real -> (blocks, side) complex views, gradients flow."""
        lead = x.shape[:-1]
        xf = x.reshape(-1, N)
        if xf.dtype != torch.float32:
            xf = xf.float()
        if xf.device != self.dev:
            raise ValueError(f"x is on {xf.device}, engine on {self.dev}")
        if xf.shape[0] < 1:
            raise ValueError("x needs at least one slice")
        kc = _Analysis.apply(xf.contiguous(), self)
        # one narrow per group (not a multi-output split): the blocks stay
        # single views, which autograd lets a caller modify in place
        views = [kc.narrow(1, off, b * M).view(*lead, b, M) for b, M, off in self.gspec]
        return views[:self.ngroups], views[self.ngroups:]

    def _base_of(self, parts, B):
        """The [B, ncoef] complex64 buffer whose consecutive group views the
        parts are (as fwd returns them), else None."""
        base = parts[0]._base
        if base is None or base.device != self.dev or base.dtype != torch.complex64 \
                or base.shape != (B, self.ncoef) or not base.is_contiguous():
            return None
        ptr = base.data_ptr()
        for c, (b, M, off) in zip(parts, self.gspec):
            if c._base is not base or c.data_ptr() != ptr + 8 * off or c.stride()[-2:] != (M, 1) \
                    or c.shape[-2:] != (b, M):
                return None
        return base

    def bwd(self, blocks, side=None):
        """Inverse of fwd; side=None treats the DC and Nyquist bands as zero."""
        lead = blocks[0].shape[:-2]
        B = 1
        for d in lead:
            B *= d
        if side is not None and B >= 1:
            flat = self._base_of(list(blocks) + list(side), B)
            if flat is not None:
                return _Synthesis.apply(flat, self).reshape(*lead, N)
        parts = [c.reshape(B, -1) for c in list(blocks)]
        if side is not None:
            parts += [c.reshape(B, -1) for c in list(side)]
        else:
            nside = sum(b * M for b, M, _ in self.gspec[self.ngroups:])
            parts.append(torch.zeros(B, nside, dtype=torch.complex64, device=self.dev))
        flat = torch.cat([p.to(torch.complex64) for p in parts], dim=-1)
        if flat.shape[-1] != self.ncoef:
            raise ValueError(f"blocks carry {flat.shape[-1]} coefficients, expected {self.ncoef}")
        if flat.device != self.dev:
            raise ValueError(f"blocks are on {flat.device}, engine on {self.dev}")
        return _Synthesis.apply(flat.contiguous(), self).reshape(*lead, N)


class _Analysis(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, eng):
        ctx.eng = eng
        return eng._analysis(x)

    @staticmethod
    def backward(ctx, gk):
        return ctx.eng._adj_analysis(gk.to(torch.complex64).contiguous()), None


class _Synthesis(torch.autograd.Function):
    @staticmethod
    def forward(ctx, kc, eng):
        ctx.eng = eng
        return eng._synthesis(kc)

    @staticmethod
    def backward(ctx, gy):
        return ctx.eng._adj_synthesis(gy.float().contiguous()), None
