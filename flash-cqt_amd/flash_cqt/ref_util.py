"""Window helpers of the nonstationary Gabor bank: Hann window, window index
ranges and the painless dual frame.

The numbers must be bit-identical to the reference bank (ref_util.py:16-52),
because the windows are the transform's definition: same float64 Hann
recipe (scale, cos, +1, *0.5, ref_util.py:16-22), same frame diagonal
accumulated band by band in band order, in the bank's dtype (float32 for a
float32 bank, float64 for a float64 one, ref_util.py:43-52). Everything is
computed with numpy on the host and returned as numpy arrays; callers move
the results to their device.
"""
import numpy as np


def hann_fft_order(length):
    """float64 Hann window of `length` with its peak at index 0 (fft order)."""
    r = np.arange(length, dtype=np.float64)
    r *= np.pi * 2. / length
    r = np.cos(r)
    r += 1.
    r *= 0.5
    return r


def window_ranges(lengths, centre_bins, total):
    """Absolute bin indices (mod nn) covered by each window, and nn.

    Window i of length Lg is centred on its centre position and covers
    [centre - Lg//2, centre + Lg - Lg//2). The centre positions are the
    cumulative sum of the rounded centre-frequency increments, started at
    the wrap-around increment of the last centre (ref_util.py:25-40).
    """
    inc = np.concatenate(((np.mod(-centre_bins[-1], total),), np.diff(centre_bins)))
    centres = np.cumsum(inc)
    nn = int(centres[-1])
    centres = centres - inc[0]
    out = []
    for Lg, c in zip(lengths, centres):
        lo = c - Lg // 2
        out.append(np.mod(np.arange(lo, lo + Lg, dtype=np.int64), nn))
    return out, nn


def painless_dual(windows, ranges, nn, block_lengths, dtype=np.float32):
    """Canonical dual windows of a painless frame, computed in `dtype`
    (the bank's dtype: float32 by default, float64 for a float64 bank).

    The frame operator is diagonal: d[k] = sum_i M_i |g_i(k)|^2 over the
    windows covering bin k (g in natural order), and the dual of window i is
    g_i / d over its own support, back in fft order (ref_util.py:43-52).
    Returns (duals, diagonal).
    """
    d = np.zeros(nn, dtype=dtype)
    for g, m, rng in zip(windows, block_lengths, ranges):
        d[rng] = d[rng] + np.square(np.fft.fftshift(g)) * dtype(m)
    duals = [g / np.fft.ifftshift(d[rng]) for g, rng in zip(windows, ranges)]
    return duals, d


# names the reference exports
def hannwin(l, device="cpu"):
    """Reference-compatible alias: float64 torch Hann window (ref_util.py:16-22)."""
    import torch
    return torch.as_tensor(hann_fft_order(l), device=torch.device(device))


def calcwinrange(g, rfbas, Ls, device="cpu"):
    """Reference-compatible: (index ranges as int64 tensors, nn) of windows g
    centred at the bins rfbas (ref_util.py:25-40); window_ranges does the work."""
    import torch
    ranges, nn = window_ranges([len(gi) for gi in g], np.asarray(rfbas), Ls)
    return [torch.as_tensor(r, device=torch.device(device)) for r in ranges], nn


def nsdual(g, wins, nn, M=None, dtype=None, device="cpu"):
    """Reference-compatible: dual windows (torch tensors) of windows g over
    ranges wins with block lengths M (ref_util.py:43-52); the frame diagonal
    accumulates in `dtype` (float32 by default, as the reference's)."""
    import torch
    if M is None:
        raise ValueError("nsdual needs the block lengths M")
    dt = {torch.float64: np.float64, torch.float32: np.float32, None: np.float32}[dtype]
    gn = [gi.detach().cpu().numpy() if torch.is_tensor(gi) else np.asarray(gi) for gi in g]
    wn = [w.detach().cpu().numpy() if torch.is_tensor(w) else np.asarray(w) for w in wins]
    mn = [int(m) for m in (M.tolist() if torch.is_tensor(M) else M)]
    duals, _ = painless_dual(gn, wn, int(nn), mn, dtype=dt)
    return [torch.as_tensor(d, device=torch.device(device)) for d in duals]
