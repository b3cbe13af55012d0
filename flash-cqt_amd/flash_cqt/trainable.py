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
returned blocks are views into it (no per-group copies).
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

    def _analysis(self, x):
        kc = torch.empty(x.shape[0], self.ncoef, dtype=torch.complex64, device=self.dev)
        self.f.analysis(x, kc, None, _native.INTERLEAVED, table="route")
        return kc

    def _synthesis(self, kc):
        y = torch.empty(kc.shape[0], N, dtype=torch.float32, device=self.dev)
        self.f.synthesis(kc, None, _native.INTERLEAVED, y, table="scat")
        return y

    def _adj_analysis(self, gk):
        gx = torch.empty(gk.shape[0], N, dtype=torch.float32, device=self.dev)
        self.f.synthesis(gk, None, _native.INTERLEAVED, gx, table="scat_a")
        return gx

    def _adj_synthesis(self, gy):
        gk = torch.empty(gy.shape[0], self.ncoef, dtype=torch.complex64, device=self.dev)
        self.f.analysis(gy, gk, None, _native.INTERLEAVED, table="route_b")
        return gk

    # ---------------------------------------------------- public surface

    def fwd(self, x):
        """x [..., N] real -> (blocks, side) complex views, gradients flow."""
        lead = x.shape[:-1]
        xf = x.reshape(-1, N)
        if xf.dtype != torch.float32:
            xf = xf.float()
        kc = _Analysis.apply(xf.contiguous(), self)
        views = [kc[:, off:off + b * M].view(*lead, b, M) for b, M, off in self.gspec]
        return views[:self.ngroups], views[self.ngroups:]

    def bwd(self, blocks, side=None):
        """Inverse of fwd; side=None treats the DC and Nyquist bands as zero."""
        lead = blocks[0].shape[:-2]
        B = 1
        for d in lead:
            B *= d
        parts = [c.reshape(B, -1) for c in list(blocks)]
        if side is not None:
            parts += [c.reshape(B, -1) for c in list(side)]
        else:
            nside = sum(b * M for b, M, _ in self.gspec[self.ngroups:])
            parts.append(torch.zeros(B, nside, dtype=torch.complex64, device=self.dev))
        flat = torch.cat([p.to(torch.complex64) for p in parts], dim=-1)
        if flat.shape[-1] != self.ncoef:
            raise ValueError(f"blocks carry {flat.shape[-1]} coefficients, expected {self.ncoef}")
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
