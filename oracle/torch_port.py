"""Pure-torch float32 port of the reference transform for the host CPU.

TEST INFRASTRUCTURE: used by tests/ as an autograd reference and by
bench.py's cpu_baseline leg as the timed host-core baseline (the reference's
own OctCQT algorithm on the box's cores, torch.fft = pocketfft on CPU).
Tables come from cqt_oracle (bit-identical to the reference's); the ops
follow oct_cqt.py:84-117: rfft -> gather x window -> ifft per group;
fft x dual window -> one index_add on the real/imag planes -> irfft.
"""
import torch

from .cqt_oracle import OctCQT as _OracleTables


class TorchPortOctCQT:
    def __init__(self, num_octs=(3, 4, 2), bins_per_oct=(8, 16, 32), fs=44100, audio_len=65536):
        tab = _OracleTables(list(num_octs), list(bins_per_oct), fs, audio_len)
        self.nn = tab.nn
        self.Ls = tab.Ls
        conv = lambda g: (torch.from_numpy(g[0]), torch.from_numpy(g[1]), torch.from_numpy(g[2]),
                          torch.from_numpy(g[3]), torch.from_numpy(g[4]))
        self.groups = [conv(g) for g in tab.groups]
        self.side_groups = [conv(g) for g in tab.side_groups]
        self.pos_flat = torch.from_numpy(tab.pos_flat)

    def fwd(self, x):
        ft = torch.fft.rfft(x)
        blocks = [torch.fft.ifft(ft[..., idx] * gv) for idx, gv, _, _, _ in self.groups]
        side = []
        for idx, gv, _, _, conj in self.side_groups:
            a = ft[..., idx]
            side.append(torch.fft.ifft(torch.where(conj, a.conj(), a) * gv))
        return blocks, side

    def bwd(self, blocks, side):
        lead = blocks[0].shape[:-2]
        n = 1
        for s in lead:
            n *= s
        srcs = [(torch.fft.fft(c) * gdv).reshape(*lead, -1)
                for c, (_, _, _, gdv, _) in zip(list(blocks) + list(side), self.groups + self.side_groups)]
        src = torch.cat(srcs, dim=-1).reshape(n, -1)
        fr = torch.zeros(n, self.nn // 2 + 1, dtype=src.dtype)
        torch.view_as_real(fr).index_add_(1, self.pos_flat, torch.view_as_real(src))
        return torch.fft.irfft(fr, n=self.nn).reshape(*lead, self.nn)
