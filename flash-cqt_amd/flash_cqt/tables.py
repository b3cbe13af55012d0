"""Host-side builder of the factored engine's tables (float64 -> fp32).

Everything the kernels need that does not depend on the batch:
  route    analysis record per tap, 4 x int32:
             {p1 | p2 << 16, Re A / M, Im A / M, g / M}
           the kernel computes v = A Z[p1] + (g - A) conj Z[p2] on the packed
           spectrum Z = FFT_L(x[0::2] + i x[1::2]) (natural order) and then
           the unscaled inverse DFT of the band. A = g cA(k) with
           cA = (1 - i W_N^k)/2; conj taps (DC/Nyquist bands past nn/2) use
           A = g conj cB(k), cB = 1 - cA, and swap p1/p2. The band's 1/M is
           folded in (exact: M is a power of two).
  route_b  synthesis-adjoint record, same form with the dual window times
           (2/N)(1 - [k in {0, L}]/2) (the transpose of irfft is (2/N) rfft
           with bins 0 and L halved; the band's transpose of the forward DFT
           is the unscaled inverse DFT).
  scat     synthesis record per tap {pos, gdv, gdv, 0}: F[pos] += gdv DFT(C).
  scat_a   analysis-adjoint record {idx, gr, gi, 0} with
           gr = g (N/2)/M (1 + edge), gi = -+gr (1 - edge): the transpose of
           rfft is (N/2) irfft with bins 0 and L doubled, of a conj tap the
           conjugate, of the band's 1/M inverse DFT the forward DFT / M.
  tasks    band tasks {M, first coefficient, band count, 0}: consecutive
           bands of one group, at most POINTS / M per task.
  tw_pass  W_L^(k1 n2) at k1*256 + n2 (column pass of the packed FFT).
  tw_half  W_N^i, i < L (retangle of the inverse).
  tw_stage Stockham stage twiddles W_{NS R}^(r k) in [k][r] rows for
           (NS, R) = (16,2) (16,4) (16,8) (16,16) (256,2) (256,4) (256,8).
Semantics follow fused.py:303-476 (records, adjoint constants); the layout
(natural order, folded scales, 64-lane-friendly rows) is this engine's own.
Every angle is taken from an exact integer residue in float64 and rounded
once to fp32.
"""
import numpy as np

N = 65536
L = N // 2
FSTRIDE = L + 64            # complex elements per row of the half-spectrum buffer
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
        k = np.arange(ns)[:, None]
        rr = np.arange(r)[None, :]
        rows.append(_unit_roots(k * rr, ns * r).reshape(-1))
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
    for b, M, off in gspec:
        assert M in BAND_LENGTHS, f"band length {M} not supported by the engine"
        per = max(1, points // M)
        for first in range(0, b, per):
            tasks.append([M, off + first * M, min(per, b - first), 0])
    return np.asarray(tasks, dtype=np.int32)


def build(groups, nn=N):
    """Tables for the fused engine from OctCQT group tables.

    groups: list of numpy (idx, gv, pos, gdv, conj) in coefficient order
    (octave groups, then DC, then Nyquist), as OctCQT.np_groups +
    np_side_groups. Returns a dict of numpy arrays.
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

    W = _unit_roots(k, N)
    cA = 0.5 * (1.0 - 1j * W)
    cB = 0.5 * (1.0 + 1j * W)
    q1 = k % L
    q2 = (L - k) % L
    p1 = np.where(cf, q2, q1)
    p2 = np.where(cf, q1, q2)
    pp = (p1 | (p2 << 16)).astype(np.int64)
    pp = np.where(pp >= 2 ** 31, pp - 2 ** 32, pp).astype(np.int32)
    edge = (k == 0) | (k == L)

    def record(a, w):
        # fp32 rounding of A and the window first, then exact power-of-two scales
        rec = np.empty((ncoef, 4), dtype=np.int32)
        rec[:, 0] = pp
        rec[:, 1] = _bits(a.real)
        rec[:, 2] = _bits(a.imag)
        rec[:, 3] = _bits(w)
        return rec

    A = np.where(cf, g * np.conj(cB), g * cA)
    A32 = A.astype(np.complex64).astype(np.complex128)
    g32 = g.astype(np.float32).astype(np.float64)
    route = record(A32 / Mt, g32 / Mt)

    Ad = np.where(cf, gd * np.conj(cB), gd * cA)
    Ad32 = Ad.astype(np.complex64).astype(np.complex128)
    gd32 = gd.astype(np.float32).astype(np.float64)
    cb = (2.0 / N) * (1.0 - 0.5 * edge)
    route_b = record(Ad32 * cb, gd32 * cb)

    scat = np.zeros((ncoef, 4), dtype=np.int32)
    scat[:, 0] = pos
    scat[:, 1] = _bits(gd32)
    scat[:, 2] = _bits(gd32)

    gr = g32 * (N / 2.0) / Mt * (1.0 + edge)
    gi = gr * np.where(cf, -1.0, 1.0) * (1.0 - edge)
    scat_a = np.zeros((ncoef, 4), dtype=np.int32)
    scat_a[:, 0] = k
    scat_a[:, 1] = _bits(gr)
    scat_a[:, 2] = _bits(gi)

    tasks = band_tasks(gspec)
    check_tasks(tasks, ncoef)
    return dict(route=route, route_b=route_b, scat=scat, scat_a=scat_a, tasks=tasks,
                tw_pass=pass_twiddles(), tw_half=half_twiddles(), tw_stage=stage_twiddles(),
                gspec=gspec, ncoef=ncoef)


def check_tasks(tasks, ncoef, points=POINTS_PER_TASK):
    """Reject a task table the kernels could not execute in bounds."""
    assert tasks.ndim == 2 and tasks.shape[1] == 4 and tasks.shape[0] >= 1
    for M, first, nb, _ in tasks.tolist():
        assert M in BAND_LENGTHS
        assert 1 <= nb <= max(1, points // M)
        assert 0 <= first and first + nb * M <= ncoef
