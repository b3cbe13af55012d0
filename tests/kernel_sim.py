"""numpy simulator of the HIP kernels' schedules (test infrastructure).

Replays, thread by thread (vectorised over threads), the exact index
arithmetic of flash-cqt_amd/csrc: the Stockham stages of fcqt_fft.hpp with
the padded LDS layout, the column / row passes of packed_fft.hip and the
band prologue / epilogue of bands.hip, using the product's own tables
(flash_cqt/tables.py). Butterfly codelets are exact DFTs here; every LDS and
global index is asserted in bounds. This is the CPU gate that runs before
any GPU time, like the reference's schedule reference
(bench/radix_reference.py) and table gates (bench/radix_gpu.py:51-120).
"""
import numpy as np

from flash_cqt import tables as T

L = T.L
N = T.N


def pad16(i):
    return i + (i >> 4)


class Plan:
    def __init__(self, M):
        self.M = M
        self.T = M // 16
        self.R2 = 16 if M >= 256 else M // 16
        self.R3 = M // 256 if M > 256 else 1
        self.RL = self.R3 if M > 256 else self.R2
        self.QL = 16 // self.RL
        self.OS = M // self.RL
        self.US = M + M // 16 + 1


def _dft(a, R, sign):
    """DFT of length R over the last axis; sign -1 forward, +1 unscaled inverse."""
    return np.fft.fft(a, axis=-1) if sign < 0 else np.fft.ifft(a, axis=-1) * R


_TWS = None


def tws():
    global _TWS
    if _TWS is None:
        t = T.stage_twiddles()
        _TWS = t[:, 0].astype(np.complex128) + 1j * t[:, 1].astype(np.complex128)
    return _TWS


def tw_off(ns, r):
    off = 0
    for a, b in T.STAGE_ORDER:
        if (a, b) == (ns, r):
            return off
        off += a * b
    raise KeyError((ns, r))


def stage_write(v, s, t, M, R, NS, base):
    """v [U, T, 16] -> LDS s (flat) at base[u] + pad16(pos)."""
    P = Plan(M)
    Q = 16 // R
    for q in range(Q):
        j = t + P.T * q
        b = (j // NS) * NS * R + (j & (NS - 1))
        for r in range(R):
            idx = pad16(b + r * NS)
            assert idx.max() < P.US - 1 + 1 and idx.min() >= 0
            s[base[:, None] + idx[None, :]] = v[:, :, q * R + r]


def stage_read(s, t, M, R, NS, sign, base):
    P = Plan(M)
    Q = 16 // R
    stride = M // R
    out = np.empty((base.size, P.T, 16), dtype=np.complex128)
    for q in range(Q):
        j = t + P.T * q
        a = np.empty((base.size, P.T, R), dtype=np.complex128)
        for r in range(R):
            idx = pad16(j + r * stride)
            assert idx.max() < P.US and idx.min() >= 0
            a[:, :, r] = s[base[:, None] + idx[None, :]]
        if NS > 1:
            k = j & (NS - 1)
            off = tw_off(NS, R)
            rows = off + np.arange(R)[None, :] * NS + k[:, None]
            assert rows.max() < T.TW_STAGE_LEN
            w = tws()[rows]
            if sign > 0:
                w = np.conj(w)
            a = a * w[None, :, :]
        out[:, :, q * R:(q + 1) * R] = _dft(a, R, sign)
    return out


def fft_unit(v, M, sign):
    """v [U, T, 16] with v[u, t, r] = x_u[t + T r] -> v[u, t, q RL + r] = X_u[t + T q + r OS]."""
    P = Plan(M)
    U = v.shape[0]
    t = np.arange(P.T)
    s = np.full(U * P.US, np.nan + 0j)
    base = np.arange(U) * P.US
    v = _dft(v, 16, sign)
    stage_write(v, s, t, M, 16, 1, base)
    v = stage_read(s, t, M, P.R2, 16, sign, base)
    if P.R3 > 1:
        stage_write(v, s, t, M, 16, 16, base)
        v = stage_read(s, t, M, P.R3, 256, sign, base)
    return v


def unit_output_index(M):
    """[T, 16] natural output index held by (thread, register slot)."""
    P = Plan(M)
    t = np.arange(P.T)[:, None]
    out = np.empty((P.T, 16), dtype=np.int64)
    for q in range(P.QL):
        for r in range(P.RL):
            out[:, q * P.RL + r] = t[:, 0] + P.T * q + r * P.OS
    return out


# ------------------------------------------------------------ packed FFT

def _c(t):
    return t[:, 0].astype(np.complex128) + 1j * t[:, 1].astype(np.complex128)


# Tile shapes of the pass kernels (packed_fft.hip): wide (the default) and
# the narrow shapes that batches up to NARROW_MAX_BATCH run.
WIDE = dict(cols=16, rows=16, inv_cols=32)
NARROW = dict(cols=8, rows=8, inv_cols=16)
NARROW_MAX_BATCH = 16
FOLD_LISTS = 256 // WIDE["inv_cols"]


def col_fwd(x, cpw=16):
    """k_col_fwd with CPW columns per workgroup: x [B, N] real -> Y [B, L]
    (rows k1, columns n2); every element of Y written exactly once."""
    x = np.asarray(x, dtype=np.float64)
    B = x.shape[0]
    z = x[:, 0::2] + 1j * x[:, 1::2]
    twp = _c(T.pass_twiddles())
    Y = np.empty((B, L), dtype=np.complex128)
    hits = np.zeros(L, dtype=np.int64)
    tid = np.arange(8 * cpw)
    c_of, t_of = tid & (cpw - 1), tid // cpw
    assert t_of.max() < 8
    c = np.arange(cpw)
    tt = np.arange(8)
    for b in range(B):
        for cg in range(256 // cpw):
            n2 = cg * cpw + c
            assert np.array_equal(np.sort(cg * cpw + c_of), np.repeat(n2, 8))
            v = np.empty((cpw, 8, 16), dtype=np.complex128)    # [unit=c, t, r]
            for r in range(16):
                idx = 256 * (tt[None, :] + 8 * r) + n2[:, None]
                assert idx.max() < L
                v[:, :, r] = z[b][idx]
            v = fft_unit(v, 128, -1)
            for q in range(2):
                for r in range(8):
                    k1 = tt + 8 * q + 16 * r
                    o = k1[None, :] * 256 + n2[:, None]
                    assert o.max() < L
                    Y[b][o] = v[:, :, q * 8 + r] * twp[o]
                    if b == 0:
                        np.add.at(hits, o.ravel(), 1)
    assert np.all(hits == 1)
    return Y


def fwd_row(w, rho, rpw=16):
    hp = rpw // 2
    p = hp * w + (rho & (hp - 1))
    return p if rho < hp else (64 if p == 0 else 128 - p)


def row_fwd(Y, rpw=16):
    """k_row_fwd with RPW rows per workgroup: paired row FFTs + untangle ->
    X [B, L+1] (rfft); each bin written exactly once, by the lane mapping
    of the kernel's store loop."""
    B = Y.shape[0]
    twn = _c(T.half_twiddles())
    X = np.full((B, L + 1), np.nan + 0j)
    hits = np.zeros(L + 1, dtype=np.int64)
    t = np.arange(16)
    tid = np.arange(16 * rpw)
    rho2_of, kg_of = tid & (rpw - 1), tid // rpw
    assert kg_of.max() < 16
    for b in range(B):
        for w in range(128 // rpw):
            rows = np.array([fwd_row(w, rho, rpw) for rho in range(rpw)])
            v = np.empty((rpw, 16, 16), dtype=np.complex128)
            for r in range(16):
                v[:, :, r] = Y[b][rows[:, None] * 256 + (t[None, :] + 16 * r)]
            v = fft_unit(v, 256, -1)
            Zr = np.empty((rpw, 256), dtype=np.complex128)       # LDS: row rho, column k2
            for r in range(16):
                Zr[:, t + 16 * r] = v[:, :, r]
            for rho2, kg in zip(rho2_of, kg_of):
                k1 = rows[rho2]
                k2 = kg + 16 * np.arange(16)
                k = k1 + 128 * k2
                z = Zr[rho2, k2]
                if k1 == 0:
                    zm = Zr[rho2, (256 - k2) & 255]
                elif k1 == 64:
                    zm = Zr[rho2, 255 - k2]
                else:
                    assert rows[rho2 ^ (rpw // 2)] == 128 - k1
                    zm = Zr[rho2 ^ (rpw // 2), 255 - k2]
                wn = twn[k]
                ca = 0.5 * (1 + wn.imag) - 0.5j * wn.real
                cb = 0.5 * (1 - wn.imag) + 0.5j * wn.real
                X[b][k] = ca * z + cb * np.conj(zm)
                if b == 0:
                    np.add.at(hits, k, 1)
            if w == 0:
                assert rows[0] == 0
                z0 = Zr[0, 0]
                X[b][L] = z0.real - z0.imag
                if b == 0:
                    hits[L] += 1
    assert np.all(hits == 1)
    assert not np.isnan(X).any()
    return X


def packed_fft_fwd(x, shape=WIDE):
    """Forward passes of packed_fft.hip: x [B, N] -> X = rfft(x) [B, L+1]."""
    return row_fwd(col_fwd(x, shape["cols"]), shape["rows"])


def _row_pass(Y, inverse, rpw=16):
    """k_row_inv with RPW rows per workgroup: row FFTs, stored through the
    kernel's lane mapping at k1 + 128 k2 (each element exactly once)."""
    B = Y.shape[0]
    out = np.empty((B, L), dtype=np.complex128)
    hits = np.zeros(L, dtype=np.int64)
    t = np.arange(16)
    tid = np.arange(16 * rpw)
    rho2_of, kg_of = tid & (rpw - 1), tid // rpw
    for b in range(B):
        for rg in range(128 // rpw):
            k1 = rg * rpw + np.arange(rpw)
            v = np.empty((rpw, 16, 16), dtype=np.complex128)
            for r in range(16):
                v[:, :, r] = Y[b][(k1[:, None] * 256) + (t[None, :] + 16 * r)]
            v = fft_unit(v, 256, -1)
            Zr = np.empty((rpw, 256), dtype=np.complex128)
            for r in range(16):
                Zr[:, t + 16 * r] = v[:, :, r]
            for u in range(16):
                k2 = kg_of + 16 * u
                o = rg * rpw + rho2_of + 128 * k2
                assert o.max() < L
                out[b][o] = Zr[rho2_of, k2]
                if b == 0:
                    np.add.at(hits, o, 1)
    assert np.all(hits == 1)
    if inverse:
        return out / L
    return out


def staged_bins(Fs, fold):
    """Bin values [L+1] as k_col_inv stages them: dense slots bin and
    FSTRIDE + bin, plus the two overflow slots of every bin on a workgroup's
    fold list (each listed bin once, owned by the workgroup of its column)."""
    dense = Fs[0:L + 1] + Fs[T.FSTRIDE:T.FSTRIDE + L + 1]
    out = dense.copy()
    seen = set()
    for w in range(T.INV_WGS):
        for ent in fold[w * T.FOLD_PER_WG:(w + 1) * T.FOLD_PER_WG].tolist():
            if ent < 0:
                continue
            b, k = ent & 0xFFFF, min(ent >> 16, T.OVF_CAP - 1)
            assert b not in seen
            seen.add(b)
            assert b == L or T.inverse_column_wg(b & 255) == w
            o = 2 * T.FSTRIDE + 2 * k
            out[b] += Fs[o] + Fs[o + 1]
    return out


def inv_col(w, c, cpw=32):
    h = cpw // 2
    p = h * w + (c & (h - 1))
    return p if c < h else (128 if p == 0 else 256 - p)


US128 = Plan(128).US


def col_inv_stage(Fs, fold, w, cpw=32):
    """LDS of inverse column workgroup w (CPW columns) after its staging
    phase, by the kernel's own arithmetic: slot c holds column
    inv_col(w, c) at [c US + n1] (plane sum), bin L at [128] of slot 0 in
    workgroup 0, and each fold-list entry of the containing wide list is
    added at the position the kernel computes, if this workgroup owns it.
    Returns (lds, entries used)."""
    h = cpw // 2
    nthreads = 8 * cpw
    share = (256 // cpw) // FOLD_LISTS
    nent = T.FOLD_PER_WG // nthreads
    assert share * FOLD_LISTS == 256 // cpw and nent * nthreads == T.FOLD_PER_WG
    lds = np.full(cpw * US128, np.nan + 0j)
    n1 = np.arange(128)
    for c in range(cpw):
        col = inv_col(w, c, cpw)
        lds[c * US128 + n1] = Fs[256 * n1 + col] + Fs[T.FSTRIDE + 256 * n1 + col]
        if col == 0:
            assert c == 0 and w == 0
            lds[128] = Fs[L] + Fs[T.FSTRIDE + L]
    used = []
    lst = fold[(w // share) * T.FOLD_PER_WG:(w // share + 1) * T.FOLD_PER_WG]
    for tid in range(nthreads):
        for e in range(nent):
            ent = int(lst[tid + e * nthreads])
            if ent < 0:
                continue
            b = ent & 0xFFFF
            pos = -1
            if b >= L:
                if w == 0:
                    pos = 128
            else:
                cl, r1 = b & 255, b >> 8
                pp = (0 if cl == 128 else cl) if cl <= 128 else 256 - cl
                if pp // h == w:
                    pos = ((0 if cl < 128 else h) + (pp & (h - 1))) * US128 + r1
                    assert inv_col(w, pos // US128, cpw) == cl and pos % US128 == r1
            if pos >= 0:
                assert 0 <= pos < cpw * US128
                k = min(ent >> 16, T.OVF_CAP - 1)
                o = 2 * T.FSTRIDE + 2 * k
                lds[pos] += Fs[o] + Fs[o + 1]
                used.append(ent)
    return lds, used


def packed_fft_inv(F, ovf=None, shape=WIDE):
    """k_col_inv (paired columns, retangle from staged bins) + k_row_inv.
    F is a plain half spectrum [B, L+1] or, with the fold lists, the slot
    buffer [B, FROW] (then staged through col_inv_stage, and every fold
    entry must be consumed exactly once)."""
    cpw, rpw = shape["inv_cols"], shape["rows"]
    h = cpw // 2
    F = np.asarray(F, dtype=np.complex128)
    B = F.shape[0]
    twn = _c(T.half_twiddles())
    twp = _c(T.pass_twiddles())
    Y = np.empty((B, L), dtype=np.complex128)
    hits = np.zeros(L, dtype=np.int64)
    tt = np.arange(8)
    n1s = np.arange(128)
    for b in range(B):
        used = []
        if ovf is None:
            plain = np.zeros(T.FROW, dtype=np.complex128)
            plain[:L + 1] = F[b]
        for w in range(256 // cpw):
            cols = np.array([inv_col(w, c, cpw) for c in range(cpw)])
            if ovf is None:
                lds, _ = col_inv_stage(plain, np.full(T.INV_WGS * T.FOLD_PER_WG, -1), w, cpw)
            else:
                lds, u = col_inv_stage(F[b], ovf, w, cpw)
                used += u
            raw = lds.reshape(cpw, US128)
            if w == 0:
                raw[0, 0] = raw[0, 0].real      # bins 0 and L are real for irfft
                raw[0, 128] = raw[0, 128].real
            v = np.empty((cpw, 8, 16), dtype=np.complex128)
            for r in range(16):
                n1 = tt + 8 * r
                for c in range(cpw):
                    col = cols[c]
                    i = 256 * n1 + col
                    f0 = raw[c, n1].copy()
                    if col == 0:
                        f1 = raw[c, 128 - n1]
                    elif col == 128:
                        f1 = raw[c, 127 - n1]
                    else:
                        assert cols[c ^ h] == 256 - col
                        f1 = raw[c ^ h, 127 - n1]
                    e = 0.5 * (f0 + np.conj(f1))
                    d = 0.5 * (f0 - np.conj(f1))
                    o = d * np.conj(twn[i])
                    v[c, :, r] = np.conj(e + 1j * o)
            assert not np.isnan(v).any()
            v = fft_unit(v, 128, -1)
            for q in range(2):
                for r in range(8):
                    k1 = tt + 8 * q + 16 * r
                    o = k1[None, :] * 256 + cols[:, None]
                    Y[b][o] = v[:, :, q * 8 + r] * twp[o]
                    if b == 0:
                        np.add.at(hits, o.ravel(), 1)
        if ovf is not None:
            listed = [e for e in np.asarray(ovf).tolist() if e >= 0]
            assert sorted(used) == sorted(listed)
    assert np.all(hits == 1)
    zp = _row_pass(Y, inverse=True, rpw=rpw)
    y = np.empty((B, N))
    y[:, 0::2] = zp.real
    y[:, 1::2] = -zp.imag
    return y


# ----------------------------------------------------------- band engines

def _decode(rec):
    """8-byte scatter record -> (slot, gr, gi)."""
    slot = (rec[:, 0].view(np.uint32) & 0x3FFFFFFF).astype(np.int64)
    mode = rec[:, 0].view(np.uint32) >> 30
    gr = rec[:, 1].view(np.float32).astype(np.float64)
    gi = np.where(mode == 0, gr, np.where(mode == 1, -gr, 0.0))
    return slot, gr, gi


def route_bands(X, weights, bands, tasks, ncoef):
    """bands.hip route_band on X [B, L+1] -> coefficients [B, ncoef]."""
    B = X.shape[0]
    out = np.full((B, ncoef), np.nan + 0j)
    wt = weights.astype(np.float64)
    for M, first, nb, band0 in tasks.tolist():
        P = Plan(M)
        U = T.POINTS_PER_TASK // M
        assert nb <= U and band0 + nb <= bands.shape[0]
        t = np.arange(P.T)
        for b in range(B):
            v = np.zeros((U, P.T, 16), dtype=np.complex128)
            for u in range(nb):
                cb = first + u * M
                c, r_, l_, _ = bands[band0 + u].tolist()
                k, cj = T.tap_bins(c, r_, l_, M)
                assert k.max() <= L
                for r in range(16):
                    j = t + P.T * r
                    live = k[j] >= 0
                    xv = X[b][np.clip(k[j], 0, L)]
                    xv = np.where(cj[j], np.conj(xv), xv)
                    v[u, :, r] = np.where(live, wt[cb + j] * xv, 0)
            v = fft_unit(v, M, +1)
            oi = unit_output_index(M)
            for u in range(nb):
                cb = first + u * M
                assert cb + oi.max() < ncoef
                out[b][cb + oi] = v[u]
    return out


def scatter_bands(C, scat, tasks, ncoef):
    """bands.hip scatter_band: C [B, ncoef] -> slot buffer [B, FROW]; asserts
    that no slot is written twice."""
    B = C.shape[0]
    F = np.zeros((B, T.FROW), dtype=np.complex128)
    target, gr, gi = _decode(scat)
    for M, first, nb, _ in tasks.tolist():
        P = Plan(M)
        U = T.POINTS_PER_TASK // M
        t = np.arange(P.T)
        oi = unit_output_index(M)
        for b in range(B):
            v = np.zeros((U, P.T, 16), dtype=np.complex128)
            for u in range(nb):
                cb = first + u * M
                for r in range(16):
                    v[u, :, r] = C[b][cb + t + P.T * r]
            v = fft_unit(v, M, -1)
            for u in range(nb):
                cb = first + u * M
                j = (cb + oi).reshape(-1)
                d = v[u].reshape(-1)
                live = gr[j] != 0
                slot = np.minimum(target[j], T.FROW - 1)[live]
                F[b][slot] = gr[j][live] * d[live].real + 1j * gi[j][live] * d[live].imag
    tl = target[gr != 0]
    assert np.unique(tl).size == tl.size, "two taps share a slot"
    return F


# ---------------------------------------------------------------- sliced framing

def sliced_frames(sig, win, S, first=0, origin=0, pairs=False):
    """The sliced column pass's read, index for index (sliced_pair and, with
    pairs=True, sliced_pair_vec in fcqt_passes.hpp): slice g = first + s of
    each signal row, sample j = x[2H (g - 1) + jj] win[jj], jj = (j + H) mod N
    for even g and (j - H) mod N for odd g, x[i] = sig[i - origin] inside the
    row and 0 outside. The pair form reads samples (i, i + 1), i even, with
    one load at i clamped to [0, len - 2]; it needs an even length and origin.
    Returns [nsig * S, N] float32 and asserts every clamped read in range."""
    H = N // 4
    nsig, length = sig.shape
    out = np.zeros((nsig * S, N), dtype=np.float32)
    j = np.arange(N)
    if pairs:
        assert length >= 2 and length % 2 == 0 and origin % 2 == 0
    for row in range(nsig):
        for s in range(S):
            g = first + s
            s0 = 2 * H * (g - 1) - origin
            sh = N - H if g & 1 else H
            jj = (j + sh) & (N - 1)
            i = s0 + jj
            if pairs:
                ie, je = i[0::2], jj[0::2]                 # pair starts: jj even
                assert (ie % 2 == 0).all() and (je % 2 == 0).all() and (jj[1::2] == je + 1).all()
                ic = np.clip(ie, 0, length - 2)
                assert ic.min() >= 0 and ic.max() + 1 < length
                inside = (ie >= 0) & (ie <= length - 2)
                assert ((ie + 1 < length) == inside)[ie >= 0].all()   # pairs never straddle the end
                a = np.where(inside, sig[row, ic], 0.0).astype(np.float32)
                c = np.where(inside, sig[row, ic + 1], 0.0).astype(np.float32)
                o = np.empty(N, np.float32)
                o[0::2] = win[je] * a
                o[1::2] = win[je + 1] * c
                out[row * S + s] = o
                continue
            ic = np.clip(i, 0, length - 1)
            assert ic.min() >= 0 and ic.max() < length
            a = sig[row, ic] * ((i >= 0) & (i < length)).astype(np.float32)
            out[row * S + s] = win[jj] * a
    return out


def stream_frames(prev, nxt, win, first, pairs=True):
    """fcqt_stream_analysis's framing read: slice `first` of each row from
    two buffers, samples [0, hop) of the slice in prev and [hop, N) in nxt
    (SliceRow.at), s0 = 0 (origin = hop (first - 1)), with the pair loads of
    sliced_pair_vec or the scalar reads of sliced_pair. Asserts that every
    read stays inside its own buffer's row. Returns [nsig, N] float32."""
    H = N // 4
    hop = 2 * H
    nsig = prev.shape[0]
    assert prev.shape == nxt.shape == (nsig, hop)
    j = np.arange(N)
    sh = N - H if first & 1 else H
    jj = (j + sh) & (N - 1)
    out = np.zeros((nsig, N), np.float32)

    def at(row, i):
        i = np.asarray(i)
        a = i < hop
        assert (i[a] >= 0).all() and (i[a] < hop).all() and (i[~a] - hop >= 0).all() and (i[~a] - hop < hop).all()
        return np.where(a, prev[row, np.clip(i, 0, hop - 1)], nxt[row, np.clip(i - hop, 0, hop - 1)])
    for row in range(nsig):
        i = jj                                   # s0 = 0: the slice is exactly [prev, nxt]
        if pairs:
            ie = i[0::2]
            assert ((ie < hop) == (ie + 1 < hop)).all()        # a pair never straddles the split
            ic = np.clip(ie, 0, N - 2)
            o = np.empty(N, np.float32)
            o[0::2] = win[jj[0::2]] * at(row, ic)
            o[1::2] = win[jj[1::2]] * at(row, ic + 1)
            out[row] = o
        else:
            out[row] = win[jj] * at(row, i)
    return out


def overlap_add(y, nsig, S, length, vec4=False):
    """k_overlap_add (one sample per thread) or k_overlap_add4 (four per
    thread, length % 4 == 0): out[sig][p] = sum of the two slices covering
    p + 2H, each read at its un-rolled index; asserts the four-sample reads
    stay inside one slice row."""
    H = N // 4
    out = np.zeros((nsig, length), np.float32)
    if vec4:
        assert length % 4 == 0
    for sig in range(nsig):
        p = np.arange(0, length, 4) if vec4 else np.arange(length)
        q = p + 2 * H
        sh = q // (2 * H)
        for k in range(2):
            s = sh - 1 + k
            ok = (s >= 0) & (s < S)
            jv = q - 2 * H * s
            jj = (jv + np.where(s & 1, H, N - H)) & (N - 1)
            if vec4:
                assert (jj % 4 == 0).all() and (jj[ok] + 3 < N).all()
                for e in range(4):
                    rows = (sig * S + s[ok]) * N + jj[ok] + e
                    out[sig, p[ok] + e] += y.reshape(-1)[rows]
            else:
                out[sig, p[ok]] += y.reshape(-1)[(sig * S + s[ok]) * N + jj[ok]]
    return out


def row_inv_ola(y, nsig, S, length):
    """The inverse row pass with the overlap-add fused into its store
    (k_row_inv_ola): a launch over the even slices, then one over the odd
    slices. Slice s's sample jj goes to p = 2H (s - 1) + j, j = (jj + H) mod N
    (even s) or (jj - H) mod N (odd s), if 0 <= p < length. Even slices store
    0 + v; odd slices add to what the even launch stored, except in their
    second half when no slice s + 1 exists, where they store 0 + v. Asserts
    every output sample is stored exactly once before it is added to, and at
    most once added to, in launch order."""
    H = N // 4
    hop = 2 * H
    out = np.full((nsig, length), np.nan, np.float32)
    stored = np.zeros((nsig, length), np.int64)
    added = np.zeros((nsig, length), np.int64)
    jj = np.arange(N)
    for odd in (0, 1):
        for sig in range(nsig):
            for s in range(odd, S, 2):
                j = (jj + (N - H if odd else H)) & (N - 1)
                p = hop * (s - 1) + j
                ok = (p >= 0) & (p < length)
                v = y[sig * S + s][ok].astype(np.float32)
                pp = p[ok]
                if odd:
                    add = (j[ok] < hop) | (s + 1 < S)
                    assert (stored[sig, pp[add]] == 1).all() and (added[sig, pp[add]] == 0).all()
                    out[sig, pp[add]] = out[sig, pp[add]] + v[add]
                    added[sig, pp[add]] += 1
                    st = ~add
                    assert (stored[sig, pp[st]] == 0).all()
                    out[sig, pp[st]] = np.float32(0) + v[st]
                    stored[sig, pp[st]] += 1
                else:
                    assert (stored[sig, pp] == 0).all()
                    out[sig, pp] = np.float32(0) + v
                    stored[sig, pp] += 1
    assert (stored == 1).all()
    return out


def stream_overlap(y, tail, k):
    """k_stream_overlap: y [nsig, N] one inverse slice k per signal; returns
    (out or None, new tail)."""
    H = N // 4
    p = np.arange(2 * H)
    sh = H if k & 1 else N - H
    a = y[:, (p + sh) & (N - 1)]
    b = y[:, (p + 2 * H + sh) & (N - 1)]
    return (tail + a if k > 0 else None), b


# ------------------------------------------------------------ XCD mapping

def xcd_remap(lin, G):
    """fcqt_fft.hpp xcd_remap: dispatch id -> logical id, each of the 8 XCDs
    (ids lin & 7) receiving one contiguous range."""
    q, rem = G >> 3, G & 7
    x, i = lin & 7, lin >> 3
    return x * (q + 1) + i if x < rem else rem * (q + 1) + (x - rem) * q + i


def xcd_remap_reverse(lin, G):
    """fcqt_fft.hpp xcd_remap_reverse: the same ranges, walked from the end."""
    q, rem = G >> 3, G & 7
    x, i = lin & 7, lin >> 3
    n = q + 1 if x < rem else q
    start = x * (q + 1) if x < rem else rem * (q + 1) + (x - rem) * q
    return start + (n - 1 - i)


def band_place(lg, ntasks, batch, slice_major):
    """fcqt_fft.hpp band_place: logical band workgroup -> (task, slice),
    task-major (lg = task * batch + b) or slice-major (lg = b * ntasks + task)."""
    if slice_major:
        return lg % ntasks, lg // ntasks
    return lg // batch, lg % batch
