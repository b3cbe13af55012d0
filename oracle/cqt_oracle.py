"""numpy restatement of the reference CQT transform (test oracle, CPU only).

TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may use this module, and only as the checker.

Tables (windows, dual windows, gather/scatter indices) are built in float32
with the same operation order as the reference, so they are bit-identical to
the reference's tables (pinned by tests/golden fixtures); a float64 bank
(dtype=np.float64, the reference's OctCQT(dtype=torch.float64)) is built the
same way in float64 and pinned by the painless-frame identity and the
round trip it then reconstructs to near machine precision. The transforms
themselves are evaluated in float64 (numpy pocketfft), which makes this
oracle more accurate than the reference's own float32 torch path: any
implementation of the same algorithm in fp32 lands ~130-145 dB from it.
"""
import math

import numpy as np


# ---------------------------------------------------------------- helpers

def snr_db(ref, test):
    """10 log10(|ref|^2 / |ref - test|^2) over all elements, complex aware."""
    ref = np.asarray(ref)
    test = np.asarray(test)
    e = np.sum(np.abs(ref.astype(np.complex128)) ** 2)
    d = np.sum(np.abs(ref.astype(np.complex128) - test.astype(np.complex128)) ** 2)
    return float("inf") if d == 0 else float(10.0 * np.log10(e / d))


# ----------------------------------------------- ref_util.py restatement

def hannwin(l):
    """Hann window with its peak at index 0, float64.

    Follows hannwin, ref_util.py:16-22 (same operation order: scale, cos,
    +1, *0.5).
    """
    r = np.arange(l, dtype=np.float64)
    r *= np.pi * 2. / l
    r = np.cos(r)
    r += 1.
    r *= 0.5
    return r


def calcwinrange(lengths, rfbas, Ls):
    """Window index ranges (mod nn) and the total length nn.

    Follows calcwinrange, ref_util.py:25-40.
    """
    shift = np.concatenate(((np.mod(-rfbas[-1], Ls),), rfbas[1:] - rfbas[:-1]))
    timepos = np.cumsum(shift)
    nn = timepos[-1]
    timepos = timepos - shift[0]
    wins = []
    for Lg, tp in zip(lengths, timepos):
        wr = np.arange(-(Lg // 2) + tp, Lg - (Lg // 2) + tp, dtype=np.int64)
        wins.append(np.mod(wr, nn))
    return wins, int(nn)


def nsdual(g, wins, nn, M, dtype=np.float32):
    """Painless dual windows in `dtype`, frame operator diagonal weighted by M.

    Follows nsdual, ref_util.py:43-52: the diagonal is accumulated band by
    band in `dtype` (float32 for the default bank, float64 for a float64
    one) in band order, then each window is divided by the ifftshifted
    diagonal over its own support.
    """
    x = np.zeros(nn, dtype=dtype)
    for gi, mii, sl in zip(g, M, wins):
        xa = np.square(np.fft.fftshift(gi))
        xa = xa * dtype(mii)
        x[sl] = x[sl] + xa
    gd = [gi / np.fft.ifftshift(x[wi]) for gi, wi in zip(g, wins)]
    return gd, x


def next_power_of_2(x):
    return 1 if x == 0 else 2 ** math.ceil(math.log2(x))


# -------------------------------------------- filterbank.py restatement

class FlexOctBank:
    """Analysis windows, dual windows and octave layout for one audio_len.

    Follows FlexOctBank, filterbank.py:26-122, including the mirrored
    block-size write one position too low (filterbank.py:110), which makes
    Mnyq (filterbank.py:122) the top octave's block length (2048 for the
    [3,4,2]/[8,16,32] layout) and weights the frame-operator diagonal with
    the shifted M vector. Windows and the diagonal are built in `dtype`
    (filterbank.py:114-117: hannwin(...).to(dtype), nsdual(dtype=...)):
    float32 by default, float64 for a float64 bank.
    """

    def __init__(self, num_octs, bins_per_oct, fs, audio_len, min_win=4, dtype=np.float32):
        if isinstance(num_octs, int):
            num_octs = [num_octs]
        if isinstance(bins_per_oct, int):
            bins_per_oct = [bins_per_oct]
        assert len(num_octs) == len(bins_per_oct)
        self.num_octs = list(num_octs)
        self.bins_per_oct = list(bins_per_oct)
        self.fs = fs
        self.Ls = audio_len

        nf = fs / 2.0
        eps = 1e-6
        scale = float(audio_len) / fs
        K = len(num_octs)
        fmaxs = [fs * 2.0 ** (-1 - sum(num_octs[j + 1:])) for j in range(K)]

        frq, Ms = [], []
        for j in range(K):
            n, b = num_octs[j], bins_per_oct[j]
            if fmaxs[j] < nf:
                fmax_g = 2.0 * fmaxs[j] - eps
                n_g = n + 1
            else:
                fmax_g = fmaxs[j] - eps
                n_g = n
            fmin_g = fmax_g / 2.0 ** n_g
            nb_g = n_g * b
            odiv = (math.log2(fmax_g) - math.log2(fmin_g)) / (nb_g - 1)
            p = 2.0 ** odiv
            q = math.sqrt(p) / (p - 1.0) / 2.0
            f_all = fmin_g * p ** np.arange(nb_g + 1)
            f_all[-1] = min(f_all[-1], nf)
            f_all *= scale
            keep = n * b
            M_g = np.zeros(keep)
            M_g[0] = np.round(f_all[0] / q)
            for k in range(1, keep):
                M_g[k] = np.round(f_all[k + 1] - f_all[k - 1])
            frq.extend(f_all[:keep])
            Ms.extend(M_g)

        lbas = len(frq)
        frq = np.array(frq)
        Ms = np.array(Ms)
        M0 = np.round(2.0 * frq[0])
        Mnyq = np.round(nf * scale - frq[-2])

        fbas = np.concatenate(((0.0,), frq, (nf * scale,)))
        fbas = np.concatenate((fbas, audio_len - fbas[-2:0:-1]))
        fbas[lbas] = (fbas[lbas - 1] + fbas[lbas + 1]) / 2.0
        fbas[lbas + 2] = audio_len - fbas[lbas]
        rfbas = np.round(fbas).astype(int)

        M_raw = np.concatenate(((M0,), Ms, (Mnyq,), Ms[::-1]))
        np.clip(M_raw, min_win, None, out=M_raw)

        self.oct_bins = [b for n, b in zip(num_octs, bins_per_oct) for _ in range(n)]
        self.size_per_oct = []
        M = M_raw.copy()
        idx = 1
        for b in self.oct_bins:
            value = next_power_of_2(M_raw[idx:idx + b].max())
            self.size_per_oct.append(int(value))
            M[idx:idx + b] = value
            M[len(M) - idx - b:len(M) - idx] = value
            idx += b

        self.M_raw = M_raw
        self.M = M.astype(np.int64)
        self.rfbas = rfbas
        self.dtype = dtype
        self.g = [hannwin(int(m)).astype(dtype) for m in M_raw]
        self.wins, self.nn = calcwinrange([len(gi) for gi in self.g], rfbas, audio_len)
        assert self.nn == audio_len
        self.gd, self.diag = nsdual(self.g, self.wins, self.nn, self.M, dtype=dtype)
        self.fbins = lbas
        self.frqs_hz = frq / scale
        self.M0 = int(M[0])
        self.Mnyq = int(M[lbas + 1])


# ---------------------------------------------- oct_cqt.py restatement

class OctCQT:
    """Invertible octave-mode CQT over one buffer (oracle).

    Tables follow oct_cqt.py:36-82 (in the bank's dtype: float32 by default,
    bit-identical to the reference, or float64);
    fwd follows oct_cqt.py:84-96 and bwd oct_cqt.py:98-117, both evaluated in
    float64. Adjoints are derived from the real inner product (see the
    function docstrings); they are the gradients torch autograd produces
    through the reference transform.
    """

    def __init__(self, num_octs, bins_per_oct, fs=44100, audio_len=44100, dtype=np.float32):
        self.bank = FlexOctBank(num_octs, bins_per_oct, fs, audio_len, dtype=dtype)
        bank = self.bank
        self.Ls = audio_len
        self.nn = bank.nn
        self.oct_bins = bank.oct_bins
        self.size_per_oct = bank.size_per_oct
        self.frqs_hz = bank.frqs_hz
        nn = self.nn
        half = nn // 2

        def enc_dec_group(band_idx, Lo):
            nb = len(band_idx)
            idx = np.zeros((nb, Lo), dtype=np.int64)
            gv = np.zeros((nb, Lo), dtype=dtype)
            pos = np.zeros((nb, Lo), dtype=np.int64)
            gdv = np.zeros((nb, Lo), dtype=dtype)
            for k, bi in enumerate(band_idx):
                wr = bank.wins[bi]
                Lg = wr.shape[0]
                r, l = (Lg + 1) // 2, Lg // 2
                gs = np.fft.fftshift(bank.g[bi])
                idx[k, :r] = wr[l:]
                idx[k, Lo - l:] = wr[:l]
                gv[k, :r] = gs[l:]
                gv[k, Lo - l:] = gs[:l]
                gd = bank.gd[bi] * dtype(Lo)
                gdv[k, :r] = gd[:r]
                gdv[k, Lo - l:] = gd[r:]
                pos[k, :r] = wr[l:]
                pos[k, Lo - l:] = wr[:l]
            conj = idx > half
            idx = np.where(conj, nn - idx, idx)
            valid = pos <= half
            gdv = (gdv * valid).astype(dtype)
            pos = np.where(valid, pos, 0)
            return idx, gv, pos, gdv, conj

        self.groups = []
        start = 1
        for i, b in enumerate(self.oct_bins):
            grp = enc_dec_group(range(start, start + b), self.size_per_oct[i])
            assert not grp[4].any()
            self.groups.append(grp)
            start += b
        self.side_groups = [enc_dec_group([0], bank.M0),
                            enc_dec_group([bank.fbins + 1], bank.Mnyq)]
        self.pos_flat = np.concatenate([g[2].reshape(-1) for g in self.groups]
                                       + [g[2].reshape(-1) for g in self.side_groups])

    @property
    def all_groups(self):
        return list(self.groups) + list(self.side_groups)

    @property
    def gspec(self):
        """(bins, M, coefficient offset) per group in flat buffer order."""
        out, off = [], 0
        for idx, *_ in self.all_groups:
            b, M = idx.shape
            out.append((b, M, off))
            off += b * M
        return out

    @property
    def ncoef(self):
        return sum(g[0].size for g in self.all_groups)

    # forward / inverse -------------------------------------------------

    def fwd(self, x):
        """x [..., Ls] real -> (blocks, side), complex128 (oct_cqt.py:84-96)."""
        x = np.asarray(x, dtype=np.float64)
        assert x.shape[-1] == self.Ls
        ft = np.fft.rfft(x, axis=-1)
        blocks = [np.fft.ifft(ft[..., idx] * gv.astype(np.float64), axis=-1)
                  for idx, gv, _, _, _ in self.groups]
        side = []
        for idx, gv, _, _, conj in self.side_groups:
            a = ft[..., idx]
            a = np.where(conj, np.conj(a), a) * gv.astype(np.float64)
            side.append(np.fft.ifft(a, axis=-1))
        return blocks, side

    def bwd(self, blocks, side=None):
        """Inverse of fwd (oct_cqt.py:98-117); side None drops the side bands."""
        lead = blocks[0].shape[:-2]
        n = int(np.prod(lead)) if lead else 1
        srcs = [(np.fft.fft(np.asarray(c, dtype=np.complex128), axis=-1)
                 * gdv.astype(np.float64)).reshape(*lead, -1)
                for c, (_, _, _, gdv, _) in zip(blocks, self.groups)]
        if side is not None:
            srcs += [(np.fft.fft(np.asarray(c, dtype=np.complex128), axis=-1)
                      * gdv.astype(np.float64)).reshape(*lead, -1)
                     for c, (_, _, _, gdv, _) in zip(side, self.side_groups)]
            pos = self.pos_flat
        else:
            pos = self.pos_flat[:sum(s.shape[-1] for s in srcs)]
        src = np.concatenate(srcs, axis=-1).reshape(n, -1)
        fr = np.zeros((n, self.nn // 2 + 1), dtype=np.complex128)
        for i in range(n):
            fr[i] = (np.bincount(pos, weights=src[i].real, minlength=self.nn // 2 + 1)
                     + 1j * np.bincount(pos, weights=src[i].imag, minlength=self.nn // 2 + 1))
        sig = np.fft.irfft(fr, n=self.nn, axis=-1)
        return sig.reshape(*lead, self.nn)[..., :self.Ls]

    # flat coefficient buffers -------------------------------------------

    def flatten(self, blocks, side):
        """blocks + side -> one [..., ncoef] complex buffer in gspec order."""
        allb = list(blocks) + list(side)
        lead = allb[0].shape[:-2]
        return np.concatenate([c.reshape(*lead, -1) for c in allb], axis=-1)

    def unflatten(self, flat):
        """[..., ncoef] complex -> (blocks, side) views in gspec order."""
        lead = flat.shape[:-1]
        vs = [flat[..., off:off + b * M].reshape(*lead, b, M) for b, M, off in self.gspec]
        ng = len(self.groups)
        return vs[:ng], vs[ng:]

    # adjoints (gradients) -------------------------------------------------

    def fwd_adjoint(self, gblocks, gside):
        """Transpose of fwd under the real inner product.

        For a real loss with coefficient cotangents G (torch's complex
        gradient convention, G = dL/dRe C + i dL/dIm C) this returns dL/dx.
        Derivation: C = ifft_M(a) has transpose fft_M(G)/M; a tap
        a = g X[k] scatters g*abar into Xbar[k] (conj taps scatter g*conj);
        X = rfft(x) has transpose xbar[n] = Re sum_{k=0..L} Xbar[k]
        e^{+2 pi i k n / N} = (N/2) irfft(Xbar with bins 0 and L doubled).
        """
        L = self.nn // 2
        lead = gblocks[0].shape[:-2]
        Y = np.zeros(lead + (L + 1,), dtype=np.complex128)
        Yf = Y.reshape(-1, L + 1)
        for G, (idx, gv, _, _, conj) in zip(list(gblocks) + list(gside), self.all_groups):
            M = idx.shape[1]
            abar = np.fft.fft(np.asarray(G, dtype=np.complex128), axis=-1) / M
            abar = np.where(conj, np.conj(abar), abar) * gv.astype(np.float64)
            ab = abar.reshape(-1, idx.size)
            fl = idx.reshape(-1)
            for i in range(Yf.shape[0]):
                Yf[i] += (np.bincount(fl, weights=ab[i].real, minlength=L + 1)
                          + 1j * np.bincount(fl, weights=ab[i].imag, minlength=L + 1))
        Y[..., 0] *= 2.0
        Y[..., L] *= 2.0
        return (self.nn / 2.0) * np.fft.irfft(Y, n=self.nn, axis=-1)

    def bwd_adjoint(self, u):
        """Transpose of bwd (with side bands) under the real inner product.

        u [..., N] real cotangent of the output -> coefficient gradients
        (blocks, side). Derivation: irfft has transpose (2/N) rfft with bins
        0 and L halved; the scatter F[pos] += gdv D has transpose
        Dbar = gdv Fbar[pos]; D = fft_M(C) has transpose M ifft_M(Dbar).
        """
        L = self.nn // 2
        U = np.fft.rfft(np.asarray(u, dtype=np.float64), axis=-1) * (2.0 / self.nn)
        U[..., 0] *= 0.5
        U[..., L] *= 0.5
        outs = []
        for idx, gv, pos, gdv, conj in self.all_groups:
            M = idx.shape[1]
            Db = U[..., pos] * gdv.astype(np.float64)
            outs.append(M * np.fft.ifft(Db, axis=-1))
        ng = len(self.groups)
        return outs[:ng], outs[ng:]


# ------------------------------------------ packed real FFT identities

def packed_spectrum(x):
    """Z = FFT_L(x[0::2] + i x[1::2]) in natural order (bench/packedfft.py:73-85)."""
    x = np.asarray(x, dtype=np.float64)
    z = x[..., 0::2] + 1j * x[..., 1::2]
    return np.fft.fft(z, axis=-1)


def untangle(Z, k):
    """X[k] = cA(k) Z[k mod L] + cB(k) conj Z[(L-k) mod L], the rfft of x.

    cA = (1 - i W_N^k)/2, cB = (1 + i W_N^k)/2 with N = 2L (derived from
    Z = E + iO, conj Z[-k] = E - iO, X = E + W_N^k O).
    """
    L = Z.shape[-1]
    N = 2 * L
    k = np.asarray(k)
    W = np.exp(-2j * np.pi * k / N)
    cA = 0.5 * (1.0 - 1j * W)
    cB = 0.5 * (1.0 + 1j * W)
    return cA * Z[..., k % L] + cB * np.conj(Z[..., (L - k) % L])


# ----------------------------------------------- sliced.py restatement

def makewnd(sl_len, tr_area):
    """Tukey slice window, float32 (sliced.py:26-38)."""
    hhop = sl_len // 4
    htr = tr_area // 2
    w = hannwin(2 * tr_area).astype(np.float32)
    tw = np.empty(sl_len, dtype=np.float32)
    tw[:hhop - htr] = 0
    tw[hhop - htr:hhop + htr] = w[tr_area:]
    tw[hhop + htr:3 * hhop - htr] = 1
    tw[3 * hhop - htr:3 * hhop + htr] = w[:tr_area]
    tw[3 * hhop + htr:] = 0
    return tw


class SlicedCQT:
    """50%-overlap Tukey-sliced OctCQT (oracle), follows sliced.py:41-209."""

    def __init__(self, num_octs=(3, 4, 2), bins_per_oct=(8, 16, 32), fs=44100,
                 sl_len=65536, tr_area=None):
        assert sl_len % 4 == 0
        if tr_area is None:
            tr_area = sl_len // 4
        assert tr_area % 2 == 0 and 0 < tr_area * 2 <= sl_len
        self.fs = fs
        self.sl_len = sl_len
        self.tr_area = tr_area
        self.H = sl_len // 4
        self.hop = sl_len // 2
        self.cqt = OctCQT(list(num_octs), list(bins_per_oct), fs=fs, audio_len=sl_len)
        self.oct_bins = self.cqt.oct_bins
        self.size_per_oct = self.cqt.size_per_oct
        self.tw = makewnd(sl_len, tr_area).astype(np.float64)
        self._roll = [m // 4 for m in self.size_per_oct]

    def num_slices(self, L):
        nb = -(-L // self.H)
        return (nb + 1) // 2 + 1

    def slice(self, x):
        """[B, C, L] -> windowed, rolled slices [B, C, S, sl_len] (sliced.py:106-117)."""
        x = np.asarray(x, dtype=np.float64)
        B, C, L = x.shape
        H = self.H
        S = self.num_slices(L)
        nb = -(-L // H)
        xp = np.concatenate([np.zeros((B, C, 2 * H)), x,
                             np.zeros((B, C, nb * H - L + 3 * H))], axis=-1)
        sl = np.stack([xp[..., 2 * H * s:2 * H * s + 4 * H] for s in range(S)], axis=2) * self.tw
        out = np.empty_like(sl)
        out[:, :, 0::2] = np.roll(sl[:, :, 0::2], -H, axis=-1)
        out[:, :, 1::2] = np.roll(sl[:, :, 1::2], +H, axis=-1)
        return out

    def arrange(self, blocks, fwd):
        """Quarter roll of each octave block's time axis (sliced.py:119-130)."""
        out = []
        s = 1 if fwd else -1
        for c, r in zip(blocks, self._roll):
            o = np.empty_like(c)
            o[:, :, 0::2] = np.roll(c[:, :, 0::2], s * r, axis=-1)
            o[:, :, 1::2] = np.roll(c[:, :, 1::2], -s * r, axis=-1)
            out.append(o)
        return out

    def fwd(self, x):
        """x [B, C, L] -> (blocks [B,C,b,S*M], side [B,C,S,1,M]) (sliced.py:134-146)."""
        B, C, _ = np.shape(x)
        sl = self.slice(x)
        S = sl.shape[2]
        blocks, side = self.cqt.fwd(sl)
        blocks = self.arrange(blocks, fwd=True)
        blocks = [c.transpose(0, 1, 3, 2, 4).reshape(B, C, b, S * m)
                  for c, b, m in zip(blocks, self.oct_bins, self.size_per_oct)]
        return blocks, side

    def bwd(self, blocks, side=None, length=None):
        """Inverse of fwd with overlap-add (sliced.py:148-167)."""
        B, C = blocks[0].shape[:2]
        m0 = self.size_per_oct[0]
        S = blocks[0].shape[-1] // m0
        blocks = [c.reshape(B, C, b, S, m).transpose(0, 1, 3, 2, 4)
                  for c, b, m in zip(blocks, self.oct_bins, self.size_per_oct)]
        blocks = self.arrange(blocks, fwd=False)
        y = self.cqt.bwd(blocks, side)
        H = self.H
        yr = np.empty_like(y)
        yr[:, :, 0::2] = np.roll(y[:, :, 0::2], +H, axis=-1)
        yr[:, :, 1::2] = np.roll(y[:, :, 1::2], -H, axis=-1)
        out = np.zeros((B, C, (S + 1) * 2 * H))
        out[..., :S * 2 * H] += yr[..., :2 * H].reshape(B, C, -1)
        out[..., 2 * H:] += yr[..., 2 * H:].reshape(B, C, -1)
        out = out[..., 2 * H:]
        if length is not None:
            out = out[..., :length]
        return out
