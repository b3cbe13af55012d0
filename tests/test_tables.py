"""CPU gates of the product's transform definition and factored tables.

The package's OctCQT tables must equal the reference tables bit for bit
(golden hashes); its pure-torch fwd/bwd must agree with the oracle; and the
factored tables, replayed through the kernels' exact schedule
(tests/kernel_sim.py), must reproduce the oracle's analysis, synthesis and
both adjoints (the analogue of the reference's CPU table gates,
bench/radix_gpu.py:51-120 and bench/autograd_check.py)."""
import pathlib

import numpy as np
import pytest
import torch

import kernel_sim as ks
from golden.golden_inputs import inputs
from oracle.cqt_oracle import snr_db
from test_oracle import group_hashes

N = 65536
ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_package_tables_bit_exact(pkg_cqt_cpu, golden):
    c = pkg_cqt_cpu
    assert group_hashes(c.np_groups + c.np_side_groups) == golden["group_table_sha256"].tolist()
    assert np.array_equal(c.bank.M.numpy(), golden["bank_M"])
    torch_groups = [tuple(t.numpy() for t in g) for g in c.groups + c.side_groups]
    assert group_hashes(torch_groups) == golden["group_table_sha256"].tolist()


def test_package_torch_transform_matches_oracle(pkg_cqt_cpu, oracle):
    x, _ = inputs()
    with torch.no_grad():
        bl, sd = pkg_cqt_cpu.fwd(torch.from_numpy(x))
        y = pkg_cqt_cpu.bwd(bl, sd)
    obl, osd = oracle.fwd(x)
    got = torch.cat([c.reshape(2, -1) for c in list(bl) + list(sd)], -1).numpy()
    assert snr_db(oracle.flatten(obl, osd), got) > 125
    assert snr_db(oracle.bwd(obl, osd), y.numpy()) > 125


def test_task_table_covers_every_coefficient_once(factored_tables):
    t = factored_tables
    seen = np.zeros(t["ncoef"], dtype=np.int64)
    for M, first, nb, _ in t["tasks"].tolist():
        seen[first:first + nb * M] += 1
    assert (seen == 1).all()


def test_weights_and_band_descriptors(factored_tables, pkg_cqt_cpu):
    """Analysis weights are the fp32 window / M; the band descriptor rule
    reproduces every live gather index and conj flag of the reference tables;
    synthesis-adjoint weights are the dual window * 2/N, halved at bins 0, L."""
    from flash_cqt import tables as T
    t = factored_tables
    groups = pkg_cqt_cpu.np_groups + pkg_cqt_cpu.np_side_groups
    gv = np.concatenate([g[1].reshape(-1) for g in groups]).astype(np.float64)
    gd = np.concatenate([g[3].reshape(-1) for g in groups]).astype(np.float64)
    k = np.concatenate([g[0].reshape(-1) for g in groups])
    M = np.concatenate([np.full(g[0].size, g[0].shape[1]) for g in groups])
    assert np.array_equal(t["route_taps"].astype(np.float64) * M, gv)
    edge = (k == 0) | (k == N // 2)
    assert np.array_equal(t["route_b_taps"].astype(np.float64) * (N / 2.0) / (1 - 0.5 * edge), gd)
    T.check_band_taps(t["bands"], groups)
    # kernel-order records: every (task, slot, thread) names its natural tap
    # (gather bin, conjugation, weight / scatter record), padding is inert
    cf = np.concatenate([g[4].reshape(-1) for g in groups]).astype(bool)
    tin, tout = T.kernel_taps(t["tasks"]), T.kernel_taps(t["tasks"], out=True)
    for taps in (tin, tout):
        live = np.sort(taps[taps >= 0])
        assert np.array_equal(live, np.arange(t["ncoef"]))        # a permutation of all taps
    for name in ("route", "route_b"):
        rec = t[name].reshape(tin.shape + (2,))
        live = tin >= 0
        word = rec[..., 0]
        w = rec[..., 1].view(np.float32)
        assert np.array_equal(word[live], k[tin[live]])
        assert np.array_equal(np.signbit(w)[live], cf[tin[live]])            # conjugation in the sign bit
        assert np.array_equal(np.abs(w)[live], t[name + "_taps"][tin[live]])
        assert not np.any(rec[~live])
    for name in ("scat", "scat_a"):
        rec = t[name].reshape(tout.shape + (2,))
        live = tout >= 0
        assert np.array_equal(rec[live], t[name + "_taps"][tout[live]])
        assert not np.any(rec[~live])


def test_schedule_sim_analysis_and_synthesis(factored_tables, oracle):
    t = factored_tables
    x, _ = inputs()
    x = x[:1].astype(np.float64)
    X = ks.packed_fft_fwd(x)
    assert snr_db(np.fft.rfft(x), X) > 140
    C = ks.route_bands(X, t["route_taps"], t["bands"], t["tasks"], t["ncoef"])
    obl, osd = oracle.fwd(x)
    Cref = oracle.flatten(obl, osd)
    assert snr_db(Cref, C) > 140
    F = ks.scatter_bands(Cref, t["scat_taps"], t["tasks"], t["ncoef"])
    y = ks.packed_fft_inv(F, t["ovf_scat"])
    assert snr_db(oracle.bwd(obl, osd), y) > 140


def test_schedule_sim_adjoints(factored_tables, oracle):
    t = factored_tables
    rs = np.random.RandomState(12)
    G = rs.standard_normal((1, t["ncoef"])) + 1j * rs.standard_normal((1, t["ncoef"]))
    F = ks.scatter_bands(G, t["scat_a_taps"], t["tasks"], t["ncoef"])
    gx = ks.packed_fft_inv(F, t["ovf_scat_a"])
    assert snr_db(oracle.fwd_adjoint(*oracle.unflatten(G)), gx) > 140
    u = rs.standard_normal((1, N))
    Xu = ks.packed_fft_fwd(u)
    gC = ks.route_bands(Xu, t["route_b_taps"], t["bands"], t["tasks"], t["ncoef"])
    assert snr_db(oracle.flatten(*oracle.bwd_adjoint(u)), gC) > 140


def test_inverse_tail_drops_edge_imaginary_parts():
    """irfft semantics: Im F[0] and Im F[L] do not reach the output."""
    rs = np.random.RandomState(2)
    L = N // 2
    F = rs.standard_normal((1, L + 1)) + 1j * rs.standard_normal((1, L + 1))
    y = ks.packed_fft_inv(F)
    assert snr_db(np.fft.irfft(F, n=N), y) > 140


def test_scatter_slots_unique_and_fold_lists(factored_tables):
    """Every live tap owns one slot; the fold lists name every bin with
    overflow slots exactly once, in the workgroup that owns its column."""
    from flash_cqt import tables as T
    for name in ("scat", "scat_a"):
        rec = factored_tables[name + "_taps"]
        fold = factored_tables["ovf_" + name]
        live = rec[:, 1] != 0
        tgt = (rec[live, 0].view(np.uint32) & 0x3FFFFFFF).astype(np.int64)
        assert np.unique(tgt).size == tgt.size
        assert tgt.max() < T.FROW
        over = tgt[tgt >= 2 * T.FSTRIDE]
        ks = np.unique((over - 2 * T.FSTRIDE) // 2)
        ents = fold[fold >= 0]
        assert np.array_equal(np.sort(ents >> 16), ks)
        assert np.unique(ents & 0xFFFF).size == ents.size
        for w in range(T.INV_WGS):
            for e in fold[w * T.FOLD_PER_WG:(w + 1) * T.FOLD_PER_WG]:
                if e >= 0 and (e & 0xFFFF) != T.L:
                    assert T.inverse_column_wg(int(e) & 255) == w


def test_trainable_base_detection_cpu():
    """TrainableCQT.bwd reads the coefficient buffer in place only for fwd's
    own consecutive group views; anything else takes the concatenating path."""
    import torch
    from flash_cqt.trainable import TrainableCQT
    eng = TrainableCQT.__new__(TrainableCQT)           # host logic only, no GPU engine
    eng.dev = torch.device("cpu")
    eng.gspec = [(2, 4, 0), (3, 8, 8), (1, 16, 32)]
    eng.ncoef = 48
    B = 3
    kc = torch.zeros(B, eng.ncoef, dtype=torch.complex64)
    views = [kc.narrow(1, off, b * M).view(B, b, M) for b, M, off in eng.gspec]
    assert eng._base_of(views, B) is kc
    assert eng._base_of([v.clone() for v in views], B) is None           # copies
    assert eng._base_of([views[1], views[0], views[2]], B) is None        # order
    assert eng._base_of(views, B + 1) is None                             # batch
    other = torch.zeros(B, eng.ncoef, dtype=torch.complex64)
    mixed = [views[0], other.narrow(1, 8, 24).view(B, 3, 8), views[2]]
    assert eng._base_of(mixed, B) is None                                 # two buffers


def test_reference_named_window_helpers_cpu():
    """flash_cqt.ref_util.calcwinrange / nsdual (the reference's names and
    signatures, torch in and out) equal the pinned oracle's on the bank."""
    import torch
    from oracle import cqt_oracle as co
    from flash_cqt import ref_util as R
    b = co.FlexOctBank([3, 4, 2], [8, 16, 32], fs=44100, audio_len=65536)
    g = [torch.as_tensor(gi) for gi in b.g]
    wins, nn = R.calcwinrange(g, b.rfbas, 65536)
    assert nn == b.nn and all(np.array_equal(w.numpy(), ow) for w, ow in zip(wins, b.wins))
    gd = R.nsdual(g, wins, nn, torch.as_tensor(b.M))
    assert all(np.array_equal(d.numpy().view(np.uint32) if d.dtype == torch.float32 else d.numpy(),
                              od.view(np.uint32) if od.dtype == np.float32 else od)
               for d, od in zip(gd, b.gd))
    with pytest.raises(ValueError):
        R.nsdual(g, wins, nn)


def test_sliced_framing_index_math_cpu():
    """The sliced column pass's framing (whole signal, and one streamed slice
    from [previous chunk, chunk] with first = k, origin = hop (k - 1)) equals
    the reference framing: zero pad, 50% overlap, Tukey window, quarter roll."""
    from oracle.cqt_oracle import makewnd
    N, H = ks.N, ks.N // 4
    hop = 2 * H
    rs = np.random.RandomState(3)
    win = makewnd(N, N // 4).astype(np.float32)
    for length in (1, 1000, 3 * hop + 17, 5 * hop):
        x = rs.standard_normal((2, length)).astype(np.float32)
        quarters = -(-length // H)
        S = (quarters + 1) // 2 + 1
        xp = np.concatenate([np.zeros((2, 2 * H), np.float32), x,
                             np.zeros((2, quarters * H - length + 3 * H), np.float32)], axis=1)
        ref = np.stack([np.roll(xp[:, 2 * H * s:2 * H * s + N] * win, -H if s % 2 == 0 else H, axis=1)
                        for s in range(S)], axis=1).reshape(2 * S, N)
        assert np.array_equal(ks.sliced_frames(x, win, S), ref)
        if length % 2 == 0:          # the launcher's pair-load form
            assert np.array_equal(ks.sliced_frames(x, win, S, pairs=True), ref)
        # streamed: chunks of hop samples, zero padded, one call per slice
        xs = np.concatenate([x, np.zeros((2, (S - 1) * hop - length), np.float32)], axis=1)
        chunks = [xs[:, i * hop:(i + 1) * hop] for i in range(S - 1)]
        prev = np.zeros_like(chunks[0])
        for k, chunk in enumerate(chunks + [np.zeros_like(chunks[0])]):
            buf = np.concatenate([prev, chunk], axis=1)
            got = ks.sliced_frames(buf, win, 1, first=k, origin=hop * (k - 1))
            assert np.array_equal(got, ref.reshape(2, S, N)[:, k]), (length, k)
            got = ks.sliced_frames(buf, win, 1, first=k, origin=hop * (k - 1), pairs=True)
            assert np.array_equal(got, ref.reshape(2, S, N)[:, k]), (length, k)
            for pairs in (True, False):            # the two-buffer read of fcqt_stream_analysis
                got = ks.stream_frames(prev, chunk, win, k, pairs=pairs)
                assert np.array_equal(got, ref.reshape(2, S, N)[:, k]), (length, k, pairs)
            prev = chunk


def test_overlap_add_index_math_cpu():
    """Both overlap-add kernels' indexing (one sample per thread, and four
    for lengths divisible by 4) equals the reference's roll of each inverse
    slice by +H (even) / -H (odd), overlap-add at hop 2H and trim of 2H."""
    N, H = ks.N, ks.N // 4
    rs = np.random.RandomState(5)
    for length in (8, 1000, 3 * 2 * H + 12, 5 * 2 * H):
        quarters = -(-length // H)
        S = (quarters + 1) // 2 + 1
        y = rs.standard_normal((2 * S, N)).astype(np.float32)
        full = np.zeros((2, (S + 1) * 2 * H), np.float32)
        for s in range(S):
            full[:, 2 * H * s:2 * H * s + N] += np.roll(y.reshape(2, S, N)[:, s], H if s % 2 == 0 else -H, axis=1)
        ref = full[:, 2 * H:2 * H + length]
        assert np.array_equal(ks.overlap_add(y, 2, S, length), ref)
        if length % 4 == 0:
            assert np.array_equal(ks.overlap_add(y, 2, S, length, vec4=True), ref)


def test_fused_row_overlap_add_index_math_cpu():
    """The inverse row pass with the overlap-add in its store (even slices,
    then odd ones) writes every output sample once before adding to it, and
    gives k_overlap_add's bits, signed zeros included, for ragged lengths,
    one slice, and slices past the end of the signal."""
    N, H = ks.N, ks.N // 4
    rs = np.random.RandomState(6)
    cases = [(8, None), (1000, None), (3 * 2 * H + 12, None), (5 * 2 * H, None), (2 * H - 2, None),
             (1000, 1), (2 * H, 1), (2 * H + 1, 2), (7, 5)]
    for length, S in cases:
        if S is None:
            quarters = -(-length // H)
            S = (quarters + 1) // 2 + 1
        y = rs.standard_normal((2 * S, N)).astype(np.float32)
        y[:, ::97] = np.float32(-0.0)                 # exact zeros of both signs
        y[:, 1::89] = np.float32(0.0)
        ref = ks.overlap_add(y, 2, S, length)
        got = ks.row_inv_ola(y, 2, S, length)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (length, S)


def test_stream_overlap_index_math_cpu():
    """The streamed overlap-add kernel's indexing equals the reference's roll
    by +H (even slices) / -H (odd) and half-slice overlap-add."""
    import torch
    N, H = ks.N, ks.N // 4
    rs = np.random.RandomState(4)
    tail_ref, tail = None, np.zeros((3, 2 * H), np.float32)
    for k in range(4):
        y = rs.standard_normal((3, N)).astype(np.float32)
        yr = torch.roll(torch.from_numpy(y), H if k % 2 == 0 else -H, -1).numpy()
        out, tail = ks.stream_overlap(y, tail, k)
        if k > 0:
            assert np.array_equal(out, tail_ref + yr[:, :2 * H])
        tail_ref = yr[:, 2 * H:]
        assert np.array_equal(tail, tail_ref)


def test_sliced_block_buffer_detection_cpu():
    """SlicedCQT.bwd reads the fused forward's coefficient buffer in place only
    when handed that buffer's own group views; otherwise it assembles a copy
    (zeros for missing side blocks)."""
    import types
    import torch
    from flash_cqt.sliced import SlicedCQT
    s = SlicedCQT.__new__(SlicedCQT)                     # host logic only
    f = types.SimpleNamespace(gspec=[(2, 4, 0), (1, 8, 8), (1, 4, 16)], ncoef=20, dev=torch.device("cpu"))
    nsig, S = 3, 2
    coef = torch.arange(nsig * S * f.ncoef, dtype=torch.float32).to(torch.complex64)
    views = [coef[nsig * S * off:nsig * S * (off + b * M)].view(1, nsig, b, S * M) for b, M, off in f.gspec]
    blocks, side = views[:2], views[2:]
    assert s._block_buffer(f, blocks, side, nsig, S) is coef
    copy = s._block_buffer(f, [b.clone() for b in blocks], [c.clone() for c in side], nsig, S)
    assert copy is not coef and torch.equal(copy, coef)
    noside = s._block_buffer(f, blocks, None, nsig, S)
    tail = nsig * S * 16
    assert torch.equal(noside[:tail], coef[:tail]) and not noside[tail:].any()


def test_sliced_buffer_sets_kept_for_recorded_graphs_cpu(monkeypatch):
    """SlicedCQT's engine buffers: one set, grown to the largest call, smaller
    calls get leading rows. A set that served a call under stream capture is
    kept allocated when a larger set replaces it (recorded launches hold its
    addresses); an unrecorded set is dropped. X is sized to the chunked
    analysis's rows and only allocated when an analysis asks for it."""
    import types
    from flash_cqt import tables as T
    from flash_cqt.sliced import SlicedCQT
    s = SlicedCQT.__new__(SlicedCQT)                     # host logic only
    s.sl_len = T.N
    f = types.SimpleNamespace(dev=torch.device("cpu"))
    capturing = [False]
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: capturing[0])
    w = s._ws(f, 1, 2)
    assert w["X"].shape == (2, T.XSTRIDE, 2) and w["F"].shape == (2, T.FROW, 2) and not w["F"].any()
    assert "X" not in s._ws(f, 1, 2, x=False)                          # the synthesis needs no X
    first = s._fused_ws["rows"]
    s._ws(f, 1, 3)                                       # grows; the first set was never recorded
    assert s._fused_ws["rows"] is not first and "recorded" not in s._fused_ws
    second = s._fused_ws["rows"]
    assert s._ws(f, 1, 2)["W"].data_ptr() == second["W"].data_ptr()      # leading rows
    capturing[0] = True
    s._ws(f, 1, 2)                                       # served under capture: marked
    capturing[0] = False
    third_call = s._ws(f, 2, 2)                          # grows again
    assert s._fused_ws["recorded"] == [second] and s._fused_ws["rows"]["B"] == 4
    assert "Y" not in third_call and "Y" not in s._fused_ws["rows"]   # the whole-signal path needs no Y
    assert s._ws(f, 3, 1, y=True)["Y"].shape == (3, T.N)           # the streamed synthesis gets one
    y3 = s._fused_ws["rows"]["Y"]
    capturing[0] = True
    s._ws(f, 3, 1, y=True)
    capturing[0] = False
    s._ws(f, 4, 1, y=True)                               # a larger Y: the recorded one is kept
    assert s._fused_ws["recorded"][-1]["Y"] is y3 and s._fused_ws["rows"]["Y"].shape == (4, T.N)
    # from 256 slices on the chunked analysis uses 128 rows of X; W and F
    # keep every row (the synthesis runs the whole batch); a synthesis-only
    # engine allocates no X at all
    big = s._ws(f, 2, 150)
    assert big["X"].shape[0] == 128 and big["W"].shape[0] == 300 and big["F"].shape[0] == 300
    assert s._ws(f, 1, 200)["X"].shape[0] == 200 and s._ws(f, 1, 100)["X"].shape[0] == 100   # below 256: no chunks
    assert s._ws(f, 280, 1, x="full")["X"].shape[0] == 280         # the streamed analysis: one row per slice
    assert s._ws(f, 1, 300)["X"].shape[0] == 128
    s2 = SlicedCQT.__new__(SlicedCQT)
    s2.sl_len = T.N
    s2._ws(f, 2, 150, x=False)
    assert "X" not in s2._fused_ws["rows"]
    # the streamed path marks the set it hands out cached pointers for
    s._stream_ptrs = SlicedCQT._stream_ptrs.__get__(s)
    s._tw32 = lambda: torch.zeros(1)
    s._stream_ptrs(f, 1)
    capturing[0] = True
    s._stream_ptrs(f, 1)
    capturing[0] = False
    assert s._fused_ws["rows"]["captured"]


def test_product_sliced_host_framing_matches_reference_cpu(golden):
    """flash_cqt.SlicedCQT with the torch engine on the CPU (the host framing
    that autograd and the torch engine use) against the reference's own
    SlicedCQT vectors, and its stream against its whole-buffer transform."""
    import hashlib
    import torch
    from golden.golden_inputs import sliced_input
    from flash_cqt import SlicedCQT
    s = SlicedCQT(engine="torch")
    x = torch.from_numpy(sliced_input())
    with torch.no_grad():
        bl, sd = s.fwd(x)
        y = s.bwd(bl, sd, length=x.shape[-1])
    st = int(golden["meta_stride"][0])
    sts = int(golden["meta_stride"][1])
    assert [list(c.shape) for c in bl] == golden["sliced_shapes"].tolist()
    tw = s.tw.numpy().astype(np.float32)
    assert hashlib.sha256(np.ascontiguousarray(tw).tobytes()).hexdigest() == golden["sliced_tw_sha256"][0]
    cb = np.concatenate([c.numpy().reshape(1, 2, -1)[..., ::sts] for c in bl], -1)
    cs = np.concatenate([c.numpy().reshape(1, 2, -1)[..., ::st] for c in sd], -1)
    assert snr_db(golden["sliced_blocks_sub"], cb) > 120
    assert snr_db(golden["sliced_side_sub"], cs) > 120
    assert snr_db(golden["sliced_bwd_sub"], y.numpy()[..., ::st]) > 120
    # streamed (hop chunks, bounded state): each streamed slice is framed bit
    # for bit as the whole buffer frames it, and the stream reproduces the
    # whole-buffer transform (to the torch engine's batch-size rounding)
    n = x.shape[-1]
    S = s._num_slices(n)
    xp = torch.cat([x, torch.zeros(*x.shape[:2], (S - 1) * s.hop - n)], dim=-1)
    chunks = [xp[..., i * s.hop:(i + 1) * s.hop] for i in range(S - 1)]
    whole = s._slice(x)
    prev = torch.zeros_like(chunks[0])
    for k, chunk in enumerate(chunks + [torch.zeros_like(chunks[0])]):
        one = s._slice(torch.cat([prev, chunk], dim=-1), first=k, origin=s.hop * (k - 1), S=1)
        assert torch.equal(one, whole[:, :, k:k + 1])
        prev = chunk
    with torch.no_grad():
        out = list(s.stream_fwd(iter(chunks)))
        ys = torch.cat(list(s.stream_bwd(iter(out))), dim=-1)
        yfull = s.bwd(bl, sd)
    m = s.size_per_oct
    for k, (blk, side) in enumerate(out):
        for i, c in enumerate(blk):
            assert snr_db(bl[i][..., k * m[i]:(k + 1) * m[i]].numpy(), c.numpy()) > 120
    assert snr_db(yfull[..., :ys.shape[-1]].numpy(), ys.numpy()) > 125


def test_graphed_input_check_cpu():
    """Graphed refuses a call whose inputs differ in count or shape from the
    recorded ones (copy_ would otherwise broadcast a [1, N] input into a
    recorded [4, N] buffer)."""
    from flash_cqt.graphed import _check_inputs, _leaves
    rec = list(_leaves((torch.zeros(4, 8), [torch.zeros(3)])))
    _check_inputs(rec, list(_leaves((torch.ones(4, 8), [torch.ones(3)]))))
    with pytest.raises(ValueError, match="shape"):
        _check_inputs(rec, list(_leaves((torch.ones(1, 8), [torch.ones(3)]))))
    with pytest.raises(ValueError, match="input tensors"):
        _check_inputs(rec, list(_leaves((torch.ones(4, 8),))))


def test_narrow_pass_shapes_equal_wide_cpu(factored_tables):
    """The narrow tile shapes of the pass kernels (batches up to
    ks.NARROW_MAX_BATCH) replayed with their own index arithmetic: every
    output element written once, every fold-list entry consumed once by the
    narrow workgroup that owns its column, LDS positions in bounds, and the
    results equal the wide shapes' exactly (same per-column arithmetic)."""
    t = factored_tables
    rs = np.random.RandomState(21)
    x = rs.standard_normal((1, N))
    Xw = ks.packed_fft_fwd(x, ks.WIDE)
    Xn = ks.packed_fft_fwd(x, ks.NARROW)
    assert np.array_equal(Xw, Xn)
    assert snr_db(np.fft.rfft(x), Xn) > 140
    for table in ("scat", "scat_a"):
        G = rs.standard_normal((1, t["ncoef"])) + 1j * rs.standard_normal((1, t["ncoef"]))
        F = ks.scatter_bands(G, t[table + "_taps"], t["tasks"], t["ncoef"])
        yw = ks.packed_fft_inv(F, t["ovf_" + table], ks.WIDE)
        yn = ks.packed_fft_inv(F, t["ovf_" + table], ks.NARROW)
        assert np.array_equal(yw, yn)
        ref = np.fft.irfft(ks.staged_bins(F[0], t["ovf_" + table])[None, :], n=N)
        assert snr_db(ref, yn) > 140


def test_narrow_shape_constants_match_kernels_cpu():
    """The simulator's tile shapes and batch threshold are the kernels'."""
    src = (ROOT / "flash-cqt_amd" / "csrc" / "fcqt_passes.hpp").read_text()
    import re
    def const(name):
        return int(re.search(rf"\b{name}\s*=\s*(\d+)", src).group(1))
    assert const("kColsWide") == ks.WIDE["cols"] and const("kColsNarrow") == ks.NARROW["cols"]
    assert const("kRowsWide") == ks.WIDE["rows"] and const("kRowsNarrow") == ks.NARROW["rows"]
    assert const("kInvColsWide") == ks.WIDE["inv_cols"] and const("kInvColsNarrow") == ks.NARROW["inv_cols"]
    assert const("kNarrowMaxBatch") == ks.NARROW_MAX_BATCH


def test_xcd_remaps_are_bijections_with_shared_ranges_cpu():
    """Both workgroup maps cover every logical id once, and give each XCD
    the same contiguous range (the reverse map walks it from the end), for
    grids of 1 to 301 slices of the band kernels and odd sizes."""
    for G in (1, 7, 8, 9, 68, 1088, 4352, 68 * 301, 16 * 3 + 5):
        fwd = [ks.xcd_remap(l, G) for l in range(G)]
        rev = [ks.xcd_remap_reverse(l, G) for l in range(G)]
        assert sorted(fwd) == list(range(G)) and sorted(rev) == list(range(G))
        for x in range(8):
            a = [fwd[l] for l in range(x, G, 8)]
            b = [rev[l] for l in range(x, G, 8)]
            assert a == sorted(a) and b == sorted(b, reverse=True) and sorted(a) == sorted(b)
            assert not a or a == list(range(a[0], a[0] + len(a)))


def test_xcd_map_replicas_equal_the_kernels_maps_cpu(tmp_path):
    """The simulator's xcd_remap / xcd_remap_reverse replicas against the
    kernels' own functions, compiled for the host from fcqt_fft.hpp (no GPU
    needed), on grid sizes of every residue mod 8 and the engine's grids."""
    import shutil
    import subprocess
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not pathlib.Path(hipcc).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path / "xcd_maps"
    r = subprocess.run([hipcc, "-O1", "-std=c++17", "--offload-arch=gfx950", str(ROOT / "tests" / "c" / "xcd_maps.hip"),
                        "-o", str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    grids = [1, 2, 7, 8, 9, 13, 68, 130, 1088, 4352]
    out = subprocess.run([str(exe)] + [str(g) for g in grids], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.strip().splitlines()
    assert len(lines) == len(grids)
    for G, ln in zip(grids, lines):
        head, rev = ln.split("|")
        vals = [int(v) for v in head.split()]
        assert vals[0] == G
        assert vals[1:] == [ks.xcd_remap(l, G) for l in range(G)]
        assert [int(v) for v in rev.split()] == [ks.xcd_remap_reverse(l, G) for l in range(G)]


def test_band_orders_match_the_kernels_and_keep_slices_on_one_xcd_cpu(tmp_path):
    """band_place, compiled for the host from fcqt_fft.hpp, equals the
    simulator's replica under both orders; each order covers every (task,
    slice) once; and slice-major puts whole slices on each XCD of the band
    grid (xcd_remap ranges) at the batch sizes where the launchers use it,
    the same slices xcd_remap gives that XCD in the wide pass grids."""
    import shutil
    import subprocess
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not pathlib.Path(hipcc).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path / "xcd_maps"
    r = subprocess.run([hipcc, "-O1", "-std=c++17", "--offload-arch=gfx950", str(ROOT / "tests" / "c" / "xcd_maps.hip"),
                        "-o", str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    nt = 68
    for B in (1, 5, 16, 64, 128):
        out = subprocess.run([str(exe), "band", str(nt), str(B)], capture_output=True, text=True, timeout=120)
        assert out.returncode == 0, out.stderr
        lines = out.stdout.strip().splitlines()
        assert len(lines) == 2
        for order, ln in enumerate(lines):
            got = [tuple(int(v) for v in p.split(",")) for p in ln.split()]
            want = [ks.band_place(lg, nt, B, order == 1) for lg in range(nt * B)]
            assert got == want
            assert sorted(got) == sorted((t, b) for t in range(nt) for b in range(B))
    for B in (64, 128, 256):
        G = nt * B
        per_xcd = {}
        for lin in range(G):
            t, b = ks.band_place(ks.xcd_remap(lin, G), nt, B, True)
            per_xcd.setdefault(lin & 7, set()).add(b)
        pass_xcd = {}
        for lin in range(8 * B):           # wide row pass: 8 workgroups per slice
            pass_xcd.setdefault(lin & 7, set()).add(ks.xcd_remap(lin, 8 * B) // 8)
        for x in range(8):
            assert per_xcd[x] == pass_xcd[x] == set(range(x * B // 8, (x + 1) * B // 8))


def test_stream_fwd_fused_step_needs_matching_pieces_cpu(monkeypatch):
    """SlicedCQT.stream_fwd takes the fused step (which reads hop samples of
    every row of both the carried piece and the new chunk) only when both
    are [B, C, hop] with the same shape; a short piece, or a carried piece of
    another shape, goes to the host path. Host logic only: the engine and
    both step bodies are stand-ins that record which path ran."""
    import types
    from flash_cqt.sliced import SlicedCQT
    s = SlicedCQT.__new__(SlicedCQT)
    s.hop = 8
    taken = []
    monkeypatch.setattr(s, "_fused", lambda *t: types.SimpleNamespace(dev=torch.device("cpu")), raising=False)
    monkeypatch.setattr(s, "_stream_slice_fused", lambda f, prev, chunk, k: taken.append(("fused", k)),
                        raising=False)
    monkeypatch.setattr(s, "_stream_slice_host", lambda prev, chunk, k: taken.append(("host", k)), raising=False)
    full = torch.zeros(2, 1, 8)
    list(s.stream_fwd([full, full]))
    assert taken == [("fused", 0), ("fused", 1), ("fused", 2)]
    taken.clear()
    list(s.stream_fwd([full, torch.zeros(2, 1, 5), full]))     # a short piece, then a full chunk after it
    assert taken == [("fused", 0), ("host", 1), ("host", 2), ("fused", 3)]
    taken.clear()
    list(s.stream_fwd([torch.zeros(3, 1, 8), full]))           # the carried piece has other signals
    assert taken == [("fused", 0), ("host", 1), ("fused", 2)]


def test_stream_bwd_recognises_only_the_marked_views_cpu():
    """stream_bwd reads a streamed slice's coefficient buffer in place only
    when it is handed the very view objects stream_fwd marked, from the
    engine the object uses now: a replaced part, a part of another slice,
    another engine, or views that record a gradient take the checked path.
    Host logic only (CPU tensors, a stand-in engine)."""
    import types
    from flash_cqt.sliced import SlicedCQT
    class Engine:                      # stand-in engine object (weakly referenced)
        dev = torch.device("cpu")

    s = SlicedCQT.__new__(SlicedCQT)
    f = Engine()
    s.cqt = types.SimpleNamespace(f=f)
    s.fused_framing = True

    def one_slice():
        buf = torch.zeros(64)
        views = SlicedCQT._stream_mark(f, [buf.as_strided((2, 4), (4, 1), 8 * i) for i in range(5)])
        return buf, views[:3], views[3:]

    buf, blocks, side = one_slice()
    got = s._stream_buffer(blocks, side)
    assert got is not None and got[0] is f and got[1] is buf
    assert s._stream_buffer(blocks, [side[0], side[1].clone()]) is None          # a part replaced
    assert s._stream_buffer(list(blocks), side[:1]) is None                      # a part missing
    assert s._stream_buffer(blocks, None) is None
    buf2, blocks2, side2 = one_slice()
    assert s._stream_buffer(blocks, side2) is None                               # parts of two slices
    assert s._stream_buffer([b.clone() for b in blocks], side) is None          # unmarked blocks
    other = Engine()
    s.cqt = types.SimpleNamespace(f=other)
    assert s._stream_buffer(blocks, side) is None                                # another engine
    s.cqt = types.SimpleNamespace(f=f)
    s.fused_framing = False
    assert s._stream_buffer(blocks, side) is None
    s.fused_framing = True
    g = torch.zeros(64, requires_grad=True)
    gviews = SlicedCQT._stream_mark(f, [g.as_strided((2, 4), (4, 1), 8 * i) for i in range(5)])
    assert s._stream_buffer(gviews[:3], gviews[3:]) is None                      # records a gradient
    with torch.no_grad():
        assert s._stream_buffer(gviews[:3], gviews[3:]) is not None


def test_stream_view_arguments_follow_the_engine_cpu():
    """The streamed slice's view arguments are cached with the engine's
    other caches: another engine (another layout) gets its own, computed
    from its own group table. Host logic only (stand-in engines)."""
    from flash_cqt.sliced import SlicedCQT

    class Engine:
        def __init__(self, gspec):
            self.gspec = gspec

    s = SlicedCQT.__new__(SlicedCQT)
    a, b = Engine([(2, 4, 0), (1, 8, 8)]), Engine([(4, 2, 0)])
    va = s._stream_view_args(a, 1, 3)
    assert va == [((1, 3, 2, 4), (24, 8, 4, 1), 0), ((1, 3, 1, 8), (24, 8, 8, 1), 24)]
    assert s._stream_view_args(a, 1, 3) is va                       # cached
    assert s._stream_view_args(b, 1, 3) == [((1, 3, 4, 2), (24, 8, 2, 1), 0)]
    assert s._stream_view_args(a, 1, 3) == va and s._stream_view_args(a, 1, 3) is not va   # rebuilt for a
