"""Invertible octave-mode CQT over one buffer, pure torch.

This is the transform definition the engine accelerates (reference
oct_cqt.py:18-117), kept as the reference's public `OctCQT` API. It runs on
any torch device: on a GPU its torch.fft calls dispatch to hipFFT/rocFFT,
which makes it the "library call" baseline the fused engine is measured
against. The fused HIP path (FusedOctCQT, TrainableCQT) never calls it.

Forward: one rfft, then per octave group a gather of the spectrum at the
window's bins times the analysis window and an inverse FFT of the group's
block length. The DC and Nyquist side bands wrap around bins 0 and nn/2, so
taps past nn/2 read the conjugate of the mirrored bin.
Inverse: FFT of each block times the dual window (times the block length),
one scatter-add into the half spectrum (bins past nn/2 are implied by
Hermitian symmetry and skipped), one irfft.
"""
import numpy as np
import torch

from .filterbank import FlexOctBank


def _group_tables(bank, band_ids, Lo, nn):
    """Gather index, window, scatter position, dual window and conj mask of a
    group of bands sharing block length Lo (numpy; values in the bank's
    dtype, float32 or float64, as the reference's enc_dec_group builds them
    in self.dtype, oct_cqt.py:36-67).

    A window of length Lg centred on bin c is laid out in fft order inside
    the block: taps 0..r-1 hold bins c..c+r-1, taps Lo-l..Lo-1 hold bins
    c-l..c-1 (r = ceil(Lg/2), l = floor(Lg/2)); the rest stay zero.
    """
    nb = len(band_ids)
    vt = bank.np_dtype
    idx = np.zeros((nb, Lo), dtype=np.int64)
    gv = np.zeros((nb, Lo), dtype=vt)
    gdv = np.zeros((nb, Lo), dtype=vt)
    for k, bi in enumerate(band_ids):
        rng = bank.np_wins[bi]
        Lg = rng.shape[0]
        r, l = (Lg + 1) // 2, Lg // 2
        centred = np.fft.fftshift(bank.np_g[bi])
        idx[k, :r], idx[k, Lo - l:] = rng[l:], rng[:l]
        gv[k, :r], gv[k, Lo - l:] = centred[l:], centred[:l]
        dual = bank.np_gd[bi] * vt(Lo)
        gdv[k, :r], gdv[k, Lo - l:] = dual[:r], dual[r:]
    half = nn // 2
    pos = idx.copy()
    conj = idx > half
    idx = np.where(conj, nn - idx, idx)
    live = pos <= half
    gdv = (gdv * live).astype(vt)
    pos = np.where(live, pos, 0)
    return idx, gv, pos, gdv, conj


class OctCQT:
    """Octave-mode CQT with exact DC / Nyquist side bands (reference API).

    groups / side_groups hold (idx, gv, pos, gdv, conj) torch tensors on
    `device`; np_groups / np_side_groups the same as numpy arrays.
    """

    def __init__(self, num_octs, bins_per_oct, fs=44100, audio_len=44100,
                 device="cpu", dtype=torch.float32):
        self.bank = FlexOctBank(num_octs, bins_per_oct, fs, audio_len,
                                device=device, dtype=dtype)
        bank = self.bank
        self.Ls = audio_len
        self.nn = bank.nn
        self.device = torch.device(device)
        self.dtype = dtype
        self.numocts = len(bank.oct_bins)
        self.oct_bins = bank.oct_bins
        self.size_per_oct = bank.size_per_oct
        self.frqs_hz = bank.frqs_hz

        self.np_groups = []
        first = 1
        for b, Lo in zip(self.oct_bins, self.size_per_oct):
            grp = _group_tables(bank, range(first, first + b), Lo, self.nn)
            assert not grp[4].any(), "octave windows never wrap"
            self.np_groups.append(grp)
            first += b
        self.np_side_groups = [_group_tables(bank, [0], bank.M0, self.nn),
                               _group_tables(bank, [bank.fbins + 1], bank.Mnyq, self.nn)]

        def to_dev(grp):
            idx, gv, pos, gdv, conj = grp
            d = self.device
            return (torch.as_tensor(idx, device=d), torch.as_tensor(gv, device=d).to(dtype),
                    torch.as_tensor(pos, device=d), torch.as_tensor(gdv, device=d).to(dtype),
                    torch.as_tensor(conj, device=d))

        self.groups = [to_dev(g) for g in self.np_groups]
        self.side_groups = [to_dev(g) for g in self.np_side_groups]
        self.pos_flat = torch.cat([g[2].reshape(-1) for g in self.groups + self.side_groups])

    def fwd(self, x):
        """x [..., Ls] real -> (blocks, side)
        blocks[i] is [..., oct_bins[i], size_per_oct[i]] complex,
        side is (dc, nyq), each [..., 1, M] complex."""
        assert x.shape[-1] == self.Ls
        spec = torch.fft.rfft(x)
        blocks = [torch.fft.ifft(spec[..., idx] * gv) for idx, gv, _, _, _ in self.groups]
        side = []
        for idx, gv, _, _, conj in self.side_groups:
            taps = spec[..., idx]
            side.append(torch.fft.ifft(torch.where(conj, taps.conj(), taps) * gv))
        return blocks, side

    def bwd(self, blocks, side=None):
        """Inverse of fwd; side=None drops the DC and Nyquist bands."""
        lead = blocks[0].shape[:-2]
        rows = 1
        for s in lead:
            rows *= s
        parts = [(torch.fft.fft(c) * gdv).reshape(*lead, -1)
                 for c, (_, _, _, gdv, _) in zip(blocks, self.groups)]
        if side is not None:
            parts += [(torch.fft.fft(c) * gdv).reshape(*lead, -1)
                      for c, (_, _, _, gdv, _) in zip(side, self.side_groups)]
            pos = self.pos_flat
        else:
            pos = self.pos_flat[:sum(p.shape[-1] for p in parts)]
        src = torch.cat(parts, dim=-1).reshape(rows, -1)
        half = torch.zeros(rows, self.nn // 2 + 1, dtype=src.dtype, device=src.device)
        # real and imaginary planes scattered separately (no complex index_add needed)
        torch.view_as_real(half).index_add_(1, pos, torch.view_as_real(src))
        sig = torch.fft.irfft(half, n=self.nn)
        return sig.reshape(*lead, self.nn)[..., :self.Ls]
