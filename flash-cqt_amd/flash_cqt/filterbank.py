"""Flexible octave filterbank of the octave-mode CQT: centre frequencies,
window lengths, per-octave block lengths, analysis and dual windows.

Follows FlexOctBank, filterbank.py:26-122 of the reference, so that every
table is bit-identical (pinned by tests against golden vectors recorded from
the reference). Two details of that recipe are reproduced on purpose:
  * the per-octave power-of-two block length is also written into the
    mirrored half of the length vector one position too low
    (filterbank.py:110), so the Nyquist side band gets the top octave's
    block length (2048 for [3,4,2]/[8,16,32], read at filterbank.py:122) and
    the frame diagonal is weighted with that shifted vector;
  * windows are built from the un-rounded lengths, only the block lengths
    are rounded to powers of two (roundings at filterbank.py:74-76, 85-94).
The windows and the frame diagonal are built in the bank's dtype, as the
reference's hannwin(...).to(dtype) and nsdual(dtype=...) do
(filterbank.py:114-117): float32 by default, float64 for a float64 bank.
"""
import math

import numpy as np
import torch

from .ref_util import hann_fft_order, window_ranges, painless_dual


def next_power_of_2(x):
    return 1 if x == 0 else 2 ** math.ceil(math.log2(x))


def _group_bins(n_oct, bins, fmax, nyq, scale):
    """Kept centre bins and window lengths of one octave group.

    Groups below Nyquist are laid out over one extra octave that is then
    dropped (the consumer rule of the multi-resolution CQT); the first kept
    bin's length is fmin/q, every other bin spans its two neighbours.
    """
    eps = 1e-6
    if fmax < nyq:
        top, n_lay = 2.0 * fmax - eps, n_oct + 1
    else:
        top, n_lay = fmax - eps, n_oct
    bottom = top / 2.0 ** n_lay
    n_all = n_lay * bins
    step = 2.0 ** ((math.log2(top) - math.log2(bottom)) / (n_all - 1))
    q = math.sqrt(step) / (step - 1.0) / 2.0
    f = bottom * step ** np.arange(n_all + 1)
    f[-1] = min(f[-1], nyq)
    f *= scale
    keep = n_oct * bins
    lens = np.zeros(keep)
    lens[0] = np.round(f[0] / q)
    for k in range(1, keep):
        lens[k] = np.round(f[k + 1] - f[k - 1])
    return f[:keep], lens


class FlexOctBank:
    """Analysis windows, dual windows and octave layout for one audio_len.

    Attributes mirror the reference bank: num_octs, bins_per_oct, fs, Ls,
    oct_bins, size_per_oct, M (int64 block lengths, torch), g / gd (window
    and dual lists, torch on `device`), wins (index ranges, torch), nn,
    fbins, frqs_hz, M0, Mnyq. Host numpy copies are kept in np_g, np_gd,
    np_wins, np_M for the table builder.
    """

    def __init__(self, num_octs, bins_per_oct, fs, audio_len, min_win=4,
                 device="cpu", dtype=torch.float32):
        num_octs = [num_octs] if isinstance(num_octs, int) else list(num_octs)
        bins_per_oct = [bins_per_oct] if isinstance(bins_per_oct, int) else list(bins_per_oct)
        assert len(num_octs) == len(bins_per_oct)
        self.num_octs, self.bins_per_oct = num_octs, bins_per_oct
        self.fs, self.Ls = fs, audio_len
        self.device, self.dtype = torch.device(device), dtype

        nyq = fs / 2.0
        scale = float(audio_len) / fs
        K = len(num_octs)
        centres, lens = [], []
        for j in range(K):
            fmax = fs * 2.0 ** (-1 - sum(num_octs[j + 1:]))
            c, m = _group_bins(num_octs[j], bins_per_oct[j], fmax, nyq, scale)
            centres.append(c)
            lens.append(m)
        frq = np.concatenate(centres)
        Ms = np.concatenate(lens)
        lbas = len(frq)

        # dc and nyquist side windows
        M0 = np.round(2.0 * frq[0])
        Mnyq = np.round(nyq * scale - frq[-2])

        # centre positions over the full spectrum; the last kept bin is moved
        # halfway to nyquist (and mirrored) before rounding
        half = np.concatenate(((0.0,), frq, (nyq * scale,)))
        pos = np.concatenate((half, audio_len - half[-2:0:-1]))
        pos[lbas] = (pos[lbas - 1] + pos[lbas + 1]) / 2.0
        pos[lbas + 2] = audio_len - pos[lbas]
        rpos = np.round(pos).astype(int)

        M_raw = np.concatenate(((M0,), Ms, (Mnyq,), Ms[::-1]))
        np.clip(M_raw, min_win, None, out=M_raw)

        self.oct_bins = [b for n, b in zip(num_octs, bins_per_oct) for _ in range(n)]
        self.size_per_oct = []
        M = M_raw.copy()
        start = 1
        for b in self.oct_bins:
            p2 = next_power_of_2(M_raw[start:start + b].max())
            self.size_per_oct.append(int(p2))
            M[start:start + b] = p2
            M[len(M) - start - b:len(M) - start] = p2   # mirrored write, one slot low
            start += b

        self.np_M = M.astype(np.int64)
        self.np_M_raw = M_raw
        # window values in the bank's dtype: float64 stays as built, every
        # other dtype is built from float32 windows (the reference's
        # .to(dtype) of the float64 window), then cast on the device
        self.np_dtype = np.float64 if dtype == torch.float64 else np.float32
        self.np_g = [hann_fft_order(int(m)).astype(self.np_dtype) for m in M_raw]
        self.np_wins, self.nn = window_ranges([len(g) for g in self.np_g], rpos, audio_len)
        assert self.nn == audio_len
        self.np_gd, self.np_diag = painless_dual(self.np_g, self.np_wins, self.nn, self.np_M,
                                                 dtype=self.np_dtype)

        dev = self.device
        self.M = torch.as_tensor(self.np_M, dtype=torch.int64, device=dev)
        self.g = [torch.as_tensor(g, device=dev).to(dtype) for g in self.np_g]
        self.gd = [torch.as_tensor(g, device=dev).to(dtype) for g in self.np_gd]
        self.wins = [torch.as_tensor(w, device=dev) for w in self.np_wins]
        self.fbins = lbas
        self.frqs_hz = frq / scale
        self.M0 = int(M[0])
        self.Mnyq = int(M[lbas + 1])
