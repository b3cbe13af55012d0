"""Host-side builder of the factored engine's tables (float64 -> fp32).

Everything the kernels need that does not depend on the batch:
  route    analysis route records in the band kernels' order
           [task][slot][thread] (kernel_taps): {bin, signed weight bits},
           the tap's gather bin and fp32 weight window / M (route_taps: the
           weights in natural tap order), negated for the taps that read
           the conjugate (the weights are >= 0, so the sign bit carries the
           conjugation: the kernel takes |w| Re X and w Im X). The kernel gathers
           the real FFT X (computed by the forward passes, untangle included)
           at the tap's bin, conjugated for taps past nn/2 (DC/Nyquist bands),
           multiplies by the weight and runs the band's unscaled inverse DFT.
           The band's 1/M is folded in (exact: M is a power of two).
  route_b  synthesis-adjoint route records (route_b_taps: the weights): dual
           window times
           (2/N)(1 - [k in {0, L}]/2) (the transpose of irfft is (2/N) rfft
           with bins 0 and L halved; the band's transpose of the forward DFT
           is the unscaled inverse DFT).
  bands    per band {centre bin c, r, l, side}: tap j < r reads bin c + j,
           tap j >= M - l reads bin c + j - M (mod N; bins past N/2 fold to
           N - k with conjugation), the taps between lie outside the window.
           side = 1 marks the bands whose taps reach bin 0 or N/2 or beyond
           (DC, Nyquist); the others take the kernel's no-wrap path.
  scat     synthesis record per tap, 2 x int32 {slot | mode << 30, gain},
           in the band kernels' output order (scat_taps: natural tap order):
           the half spectrum is F[pos] = sum over taps of gdv DFT(C).
  scat_a   analysis-adjoint record {slot of idx | mode << 30, gr} with
           gr = g (N/2)/M (1 + edge), gi = -+gr (1 - edge): the transpose of
           rfft is (N/2) irfft with bins 0 and L doubled, of a conj tap the
           conjugate, of the band's 1/M inverse DFT the forward DFT / M.
           Scatter without atomics: the live taps of one bin (at most 4) are
           ranked; ranks 0 and 1 own the bin's slot in dense plane 0 or 1
           (F[r FSTRIDE + bin]: the taps of one band and rank are contiguous,
           so a band writes whole cache lines), ranks 2-3 own two slots of a
           compact overflow area indexed by the bin's position among the bins
           of degree > 2. Every slot has one writer, the set of written slots
           is fixed by the table, and slots never written stay zero, so F
           needs zeroing only once.
  ovf_*    per scatter table, int32 [8][512] fold lists for the inverse
           column pass: workgroup w (columns 16w..16w+15 and their mirrors)
           adds the overflow slots of the bins of degree > 2 in its columns;
           entry = bin | overflow index << 16, -1 = none.
  tasks    band tasks {M, first coefficient, band count, first band}:
           consecutive bands of one group, at most POINTS / M per task.
  slice_groups  per task {off_g, bins_g, roll, 0} of its group, for the
           SlicedCQT block layout (see fcqt_route_bands_sliced).
  tw_pass  W_L^(k1 n2) at k1*256 + n2 (column pass of the packed FFT).
  tw_half  W_N^i, i < L (retangle of the inverse).
  tw_stage Stockham stage twiddles W_{NS R}^(r k) in [r][k] rows for
           (NS, R) = (16,2) (16,4) (16,8) (16,16) (256,2) (256,4) (256,8):
           the lanes of one load share r and take consecutive k, so a load
           touches one 128-byte line per 16 lanes.
Semantics follow fused.py:303-476 (records, adjoint constants); the layout
(natural order, folded scales, 64-lane-friendly rows) is this engine's own.
Every angle is taken from an exact integer residue in float64 and rounded
once to fp32.
"""
import numpy as np

N = 65536
L = N // 2
FSTRIDE = L + 64            # complex elements per half-spectrum plane (>= L + 1)
OVF_CAP = 4096              # bins with more than two contributing taps, per table
FROW = 2 * FSTRIDE + 2 * OVF_CAP   # complex elements per batch row of F
INV_COLS_PER_WG = 32        # inverse column pass: 16 columns + their 16 mirrors per workgroup
INV_WGS = 256 // INV_COLS_PER_WG    # 8 inverse column workgroups per slice
FOLD_PER_WG = 512           # fold-list entries per inverse column workgroup
XSTRIDE = L + 64            # complex elements per row of the real-FFT spectrum X
POINTS_PER_TASK = 2048      # 128 threads x 16 values per band workgroup
STAGE_ORDER = ((16, 2), (16, 4), (16, 8), (16, 16), (256, 2), (256, 4), (256, 8))
TW_STAGE_LEN = sum(ns * r for ns, r in STAGE_ORDER)
BAND_LENGTHS = (32, 64, 128, 256, 512, 1024, 2048)


def _unit_roots(e, n):
    """W_n^e = exp(-2 pi i e / n) for integer residues e, complex128."""
    ang = -2.0 * np.pi * (np.asarray(e, dtype=np.int64) % n).astype(np.float64) / n
    return np.cos(ang) + 1j * np.sin(ang)


def _as_pairs(c):
    """complex -> float32 [..., 2] (re, im)."""
    c = np.asarray(c)
    return np.stack([c.real, c.imag], axis=-1).astype(np.float32)


def _bits(f):
    return np.asarray(f, dtype=np.float32).view(np.int32)


def stage_twiddles():
    rows = []
    for ns, r in STAGE_ORDER:
        rr = np.arange(r)[:, None]
        k = np.arange(ns)[None, :]
        rows.append(_unit_roots(rr * k, ns * r).reshape(-1))
    out = np.concatenate(rows)
    assert out.size == TW_STAGE_LEN
    return _as_pairs(out)


def pass_twiddles():
    k1 = np.arange(128)[:, None]
    n2 = np.arange(256)[None, :]
    return _as_pairs(_unit_roots(k1 * n2, L).reshape(-1))


def half_twiddles():
    return _as_pairs(_unit_roots(np.arange(L), N))


def band_tasks(gspec, points=POINTS_PER_TASK):
    tasks = []
    band0 = 0
    for b, M, off in gspec:
        assert M in BAND_LENGTHS, f"band length {M} not supported by the engine"
        per = max(1, points // M)
        for first in range(0, b, per):
            tasks.append([M, off + first * M, min(per, b - first), band0 + first])
        band0 += b
    return np.asarray(tasks, dtype=np.int32)


def kernel_taps(tasks, out=False):
    """Natural tap index of every (task, slot, thread) of the band kernels,
    [ntasks, 16, 128] int64, -1 = padding (units past the task's bands).
    Thread tid = u T + t (T = M / 16) works on unit (band) u. Inputs
    (out=False): slot r holds tap t + T r. Outputs (out=True): slot q RL + r
    holds output t + T q + r OS of the transform (the layout fft_unit leaves)."""
    tasks = np.asarray(tasks)
    res = np.full((tasks.shape[0], 16, 128), -1, dtype=np.int64)
    slots = np.arange(16)
    for ti, (M, off, nb, _) in enumerate(tasks.tolist()):
        T = M // 16
        tid = np.arange(128)
        u, t = tid // T, tid % T
        if not out:
            j = t[None, :] + T * slots[:, None]
        else:
            R2 = 16 if M >= 256 else M // 16
            RL = M // 256 if M > 256 else R2
            j = t[None, :] + T * (slots // RL)[:, None] + (slots % RL)[:, None] * (M // RL)
        res[ti] = np.where(u[None, :] < nb, off + u[None, :] * M + j, -1)
    return res


def _kernel_order(rec_taps, taps):
    """[ncoef, 2] int32 per-tap records -> [ntasks * 16 * 128, 2] in kernel
    order; padding slots get (0, 0) (weight or gain 0: no effect)."""
    out = np.zeros(taps.shape + (2,), dtype=np.int32)
    live = taps >= 0
    out[live] = rec_taps[taps[live]]
    return out.reshape(-1, 2)


def band_descriptors(groups, nn=N):
    """{c, r, l, 0} per band, recovered from the group gather tables: the
    live taps j < r hold bins c..c+r-1 (c = the window centre) and the live
    taps j >= M - l hold bins c-l..c-1 (mod nn)."""
    rows = []
    for idx, gv, pos, gdv, conj in groups:
        b, M = idx.shape
        unwrapped = np.where(conj, nn - idx, idx)     # bins before the conj fold
        for i in range(b):
            live = gv[i] != 0
            j = np.flatnonzero(live)
            lo = j[j < M // 2]
            hi = j[j >= M // 2]
            r = int(lo.max()) + 1 if lo.size else 0
            l = int(M - hi.min()) if hi.size else 0
            c = int(unwrapped[i, 0])
            # side flag: taps may wrap mod nn or fold past nn/2 (DC, Nyquist)
            k = c + np.concatenate([np.arange(r), np.arange(M - l, M) - M])
            side = int(bool(np.any(k <= 0) or np.any(k >= nn // 2)))
            rows.append([c, r, l, side])
    return np.asarray(rows, dtype=np.int32)


def slice_groups(tasks, gspec, noct):
    """Per task {off_g, bins_g, roll, 0} of the task's group (first
    coefficient, band count, 1 for the noct octave groups whose SlicedCQT
    blocks are quarter-rolled, 0 for the side groups)."""
    out = []
    for M, first, _, _ in np.asarray(tasks).tolist():
        for gi, (b, Mg, off) in enumerate(gspec):
            if off <= first < off + b * Mg:
                assert Mg == M and (first - off) % M == 0
                out.append([off, b, 1 if gi < noct else 0, 0])
                break
        else:
            raise AssertionError("task outside every group")
    return np.asarray(out, dtype=np.int32)


def build(groups, nn=N, noct=None):
    """Tables for the fused engine from OctCQT group tables.

    groups: list of numpy (idx, gv, pos, gdv, conj) in coefficient order
    (octave groups, then DC, then Nyquist), as OctCQT.np_groups +
    np_side_groups; noct: number of octave groups (default: all but the two
    side groups). Returns a dict of numpy arrays.
    """
    assert nn == N, "the fused engine is built for 65536-sample slices"
    gspec, off = [], 0
    for idx, *_ in groups:
        b, M = idx.shape
        gspec.append((b, M, off))
        off += b * M
    ncoef = off

    k = np.concatenate([g[0].reshape(-1) for g in groups]).astype(np.int64)
    g = np.concatenate([g[1].reshape(-1) for g in groups]).astype(np.float64)
    pos = np.concatenate([g[2].reshape(-1) for g in groups]).astype(np.int64)
    gd = np.concatenate([g[3].reshape(-1) for g in groups]).astype(np.float64)
    cf = np.concatenate([g[4].reshape(-1) for g in groups]).astype(bool)
    Mt = np.concatenate([np.full(i.size, i.shape[1], dtype=np.float64) for i, *_ in groups])
    assert k.min() >= 0 and k.max() <= L and pos.min() >= 0 and pos.max() <= L

    edge = (k == 0) | (k == L)
    g32 = g.astype(np.float32).astype(np.float64)
    gd32 = gd.astype(np.float32).astype(np.float64)
    # exact power-of-two scales of the fp32 window values
    route = (g32 / Mt).astype(np.float32)
    route_b = (gd32 * (2.0 / N) * (1.0 - 0.5 * edge)).astype(np.float32)

    scat, ovf = scatter_table(pos, gd32, gd32)

    gr = g32 * (N / 2.0) / Mt * (1.0 + edge)
    gi = gr * np.where(cf, -1.0, 1.0) * (1.0 - edge)
    scat_a, ovf_a = scatter_table(k, gr, gi)

    tasks = band_tasks(gspec)
    bands = band_descriptors(groups)
    check_tasks(tasks, ncoef, bands)
    check_band_taps(bands, groups)
    tin, tout = kernel_taps(tasks), kernel_taps(tasks, out=True)
    assert not np.any(np.signbit(route)) and not np.any(np.signbit(route_b)), "route weights must be >= 0"
    kbin = k.astype(np.int32)
    route_rec = lambda w: _kernel_order(np.stack([kbin, _bits(np.where(cf, -w, w))], axis=1), tin)
    return dict(route=route_rec(route), route_b=route_rec(route_b), route_taps=route, route_b_taps=route_b,
                scat=_kernel_order(scat, tout), scat_a=_kernel_order(scat_a, tout),
                scat_taps=scat, scat_a_taps=scat_a, tasks=tasks, bands=bands,
                slice_groups=slice_groups(tasks, gspec, len(groups) - 2 if noct is None else noct),
                ovf_scat=ovf, ovf_scat_a=ovf_a,
                tw_pass=pass_twiddles(), tw_half=half_twiddles(), tw_stage=stage_twiddles(),
                gspec=gspec, ncoef=ncoef, coef_span=coef_span(tasks))


def coef_span(tasks):
    """One past the last coefficient any task touches (the C descriptor's
    coef_span: launches are refused unless it is at most ncoef)."""
    return int(max(int(t[1]) + int(t[2]) * int(t[0]) for t in np.asarray(tasks)))


def scatter_table(bins, gr, gi):
    """Slot-assigned scatter records {target | mode << 30, gr} and the fold
    lists (mode 0: gi = gr, 1: gi = -gr, 2: gi = 0; gr = 0 marks a tap
    without slot).

    Live taps (gr or gi nonzero) are ranked per bin in coefficient order;
    target = rank FSTRIDE + bin for ranks 0-1 (dense planes), and
    2 FSTRIDE + 2 * overflow_index(bin) + rank - 2 for ranks 2-3."""
    bins = np.asarray(bins, dtype=np.int64)
    n = bins.size
    live = (np.asarray(gr) != 0) | (np.asarray(gi) != 0)
    order = np.lexsort((np.arange(n), bins))          # by bin, then tap index
    order = order[live[order]]
    sb = bins[order]
    first = np.ones(sb.size, dtype=bool)
    first[1:] = sb[1:] != sb[:-1]
    start = np.flatnonzero(first)
    run = np.cumsum(first) - 1
    rank = np.arange(sb.size) - start[run]
    deg = np.bincount(bins[live], minlength=L + 1)
    assert rank.max() <= 3, "more than four taps on one bin"
    obins = np.flatnonzero(deg > 2)
    assert obins.size <= OVF_CAP, "overflow area too small"
    oidx = np.full(L + 1, -1, dtype=np.int64)
    oidx[obins] = np.arange(obins.size)
    target = np.zeros(n, dtype=np.int64)
    tl = np.where(rank < 2, rank * FSTRIDE + sb, 2 * FSTRIDE + 2 * oidx[sb] + (rank - 2))
    target[order] = tl
    assert target.max() < FROW
    gr = np.where(live, gr, 0.0)
    gi = np.where(live, gi, 0.0)
    mode = np.where(gi == gr, 0, np.where(gi == -gr, 1, 2))
    assert np.all((mode != 2) | (gi == 0)), "gi must be gr, -gr or 0"
    assert np.all(~live | (gr != 0)), "a live tap needs a nonzero gr"
    rec = np.zeros((n, 2), dtype=np.int32)
    rec[:, 0] = target | (mode << 30)
    rec[:, 1] = _bits(gr)
    ovf = fold_lists(obins)
    return rec, ovf


def inverse_column_wg(col):
    """Workgroup of the inverse column pass that owns column col (0..255):
    workgroup w holds columns 16w..16w+15 and their mirrors 256 - p; pair 0
    is {0, 128}."""
    p = col if col < 128 else (0 if col == 128 else 256 - col)
    return p // 16


def fold_lists(obins):
    """Per inverse-column workgroup list of (bin | overflow index << 16)."""
    lists = [[] for _ in range(INV_WGS)]
    for k, b in enumerate(np.asarray(obins).tolist()):
        w = 0 if b == L else inverse_column_wg(b & 255)
        lists[w].append(b | (k << 16))
    out = np.full((INV_WGS, FOLD_PER_WG), -1, dtype=np.int64)
    for w, lst in enumerate(lists):
        assert len(lst) <= FOLD_PER_WG, "fold list overflow"
        out[w, :len(lst)] = lst
    return out.astype(np.int32).reshape(-1)


def check_tasks(tasks, ncoef, bands, points=POINTS_PER_TASK):
    """Reject a task table the kernels could not execute in bounds."""
    assert tasks.ndim == 2 and tasks.shape[1] == 4 and tasks.shape[0] >= 1
    for M, first, nb, band0 in tasks.tolist():
        assert M in BAND_LENGTHS
        assert 1 <= nb <= max(1, points // M)
        assert 0 <= first and first + nb * M <= ncoef
        assert 0 <= band0 and band0 + nb <= bands.shape[0]


def tap_bins(c, r, l, M, nn=N):
    """Bin and conj flag of every tap j of a band (-1 outside the window),
    exactly as the band kernel derives them."""
    j = np.arange(M)
    live = (j < r) | (j >= M - l)
    k = c + np.where(j < r, j, j - M)
    k = np.where(k < 0, k + nn, k)
    cj = k > nn // 2
    k = np.where(cj, nn - k, k)
    return np.where(live, k, -1), cj & live


def check_band_taps(bands, groups, nn=N):
    """The descriptor rule must reproduce the gather table on every live tap,
    and both weight rows (window and dual window) must be exactly zero on
    the dead taps r <= j < M - l: the band kernels gather a clamped bin there
    and rely on the zero weight instead of a select."""
    bi = 0
    for idx, gv, pos, gdv, conj in groups:
        b, M = idx.shape
        for i in range(b):
            c, r, l, _ = bands[bi].tolist()
            k, cj = tap_bins(c, r, l, M, nn)
            dead = np.zeros(M, dtype=bool)
            dead[r:M - l] = True
            assert not np.any(gv[i][dead]) and not np.any(gdv[i][dead]), "nonzero weight on a dead tap"
            live = gv[i] != 0
            assert np.array_equal(k[live], idx[i][live]), "band descriptor disagrees with the gather table"
            assert np.array_equal(cj[live], conj[i][live])
            assert not np.any((k < 0) & live)
            bi += 1


# ------------------------------------------------------------ table image
# A flat, versioned image of every batch-invariant table, for callers of the
# C ABI that do not run Python at load time: write it once here
# (image_bytes / save_image), then fcqt_image_check validates it on the host
# and fcqt_tables_upload copies it into caller-allocated device memory and
# fills the descriptors (include/flashcqt.h). Layout, little endian:
#   header   "FCQT", u32 format version, u32 section count, u32 0
#   sections u32 id, u32 element bytes, u64 element count, u64 byte offset
#   data     each section at a 256-byte aligned offset from the image start
# The device copy keeps the same offsets, so a table's device address is
# the device base plus its offset.

IMAGE_MAGIC = b"FCQT"
IMAGE_VERSION = 1
IMAGE_ALIGN = 256
# section id -> (name in build(), element type)
IMAGE_SECTIONS = {
    1: ("tw_pass", np.float32), 2: ("tw_half", np.float32), 3: ("tw_stage", np.float32),
    4: ("tasks", np.int32), 5: ("route", np.int32), 6: ("route_b", np.int32),
    7: ("scat", np.int32), 8: ("scat_a", np.int32), 9: ("ovf_scat", np.int32),
    10: ("ovf_scat_a", np.int32), 11: ("slice_groups", np.int32), 12: ("ncoef", np.int64),
}


def image_bytes(built):
    """The table image of build()'s output, as bytes."""
    import struct
    arrays = []
    for sid, (name, dt) in IMAGE_SECTIONS.items():
        v = built[name]
        a = np.asarray([v] if np.ndim(v) == 0 else v, dtype=dt).reshape(-1)
        arrays.append((sid, np.ascontiguousarray(a)))
    head = 16 + 24 * len(arrays)
    off = -(-head // IMAGE_ALIGN) * IMAGE_ALIGN
    secs, blobs = [], []
    for sid, a in arrays:
        secs.append(struct.pack("<IIQQ", sid, a.itemsize, a.size, off))
        blobs.append((off, a.tobytes()))
        off += -(-a.nbytes // IMAGE_ALIGN) * IMAGE_ALIGN
    out = bytearray(off)
    out[:16] = IMAGE_MAGIC + struct.pack("<III", IMAGE_VERSION, len(arrays), 0)
    out[16:head] = b"".join(secs)
    for o, b in blobs:
        out[o:o + len(b)] = b
    return bytes(out)


def save_image(built, path):
    """Write build()'s tables as a table image file."""
    with open(path, "wb") as f:
        f.write(image_bytes(built))
