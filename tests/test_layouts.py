"""Further OctCQT layouts (CPU): the oracle and the package's tables against
reference fixtures for four layouts other than [3,4,2]/[8,16,32], and the
kernels' index math replayed on the tables the builder makes for them.

The layouts (tests/golden/make_golden.py LAYOUTS) are ones the reference's
factored engine accepts (every band length 32..2048, fused.py:274-299),
picked for what they stress: layout 0 has more than 2048 bins with three or
four synthesis taps and about 300 of them in one inverse column workgroup,
layout 1 has bins with four taps, layout 2 runs at 48 kHz with two octave
groups, layout 3 at 22.05 kHz has an octave group of one band."""
import hashlib
import pathlib

import numpy as np
import pytest

import kernel_sim as ks
from golden.golden_inputs import inputs, sliced_input
from oracle import cqt_oracle as co
from sweep_layouts import SWEEP

N = 65536
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "golden_layouts.npz"
NLAYOUTS = 4


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def group_hashes(groups):
    return [[sha(idx.astype(np.int64)), sha(gv.astype(np.float32)), sha(pos.astype(np.int64)),
             sha(gdv.astype(np.float32)), sha(conj.astype(np.bool_))]
            for idx, gv, pos, gdv, conj in groups]


@pytest.fixture(scope="module")
def gl():
    return np.load(GOLDEN, allow_pickle=False)


def layout(gl, i):
    """(num_octs, bins_per_oct, fs) of fixture layout i."""
    v = gl[f"l{i}_layout"].tolist()
    a = v.index(-1)
    b = v.index(-1, a + 1)
    return v[:a], v[a + 1:b], v[b + 1]


_oracles, _tables = {}, {}


def oracle_for(gl, i):
    if i not in _oracles:
        octs, bpo, fs = layout(gl, i)
        _oracles[i] = co.OctCQT(octs, bpo, fs, N)
    return _oracles[i]


def tables_for(gl, i):
    if i not in _tables:
        from flash_cqt import OctCQT, tables
        octs, bpo, fs = layout(gl, i)
        c = OctCQT(octs, bpo, fs=fs, audio_len=N, device="cpu")
        _tables[i] = (c, tables.build(c.np_groups + c.np_side_groups))
    return _tables[i]


@pytest.mark.parametrize("i", range(NLAYOUTS))
def test_layout_tables_bit_exact(gl, i):
    """Oracle and package group tables equal the reference's bit for bit."""
    o = oracle_for(gl, i)
    ref = gl[f"l{i}_group_table_sha256"].tolist()
    assert group_hashes(o.all_groups) == ref
    c, _ = tables_for(gl, i)
    assert group_hashes(c.np_groups + c.np_side_groups) == ref
    assert [list(g[0].shape) for g in o.all_groups] == gl[f"l{i}_group_shapes"].tolist()


@pytest.mark.parametrize("i", range(NLAYOUTS))
def test_layout_fwd_bwd_match_reference(gl, i):
    o = oracle_for(gl, i)
    x = inputs()[0][:1]
    st = int(gl["meta_stride"][0])
    bl, sd = o.fwd(x)
    assert co.snr_db(gl[f"l{i}_fwd_sub"], o.flatten(bl, sd)[:, ::st]) > 125
    assert co.snr_db(gl[f"l{i}_bwd_sub"], o.bwd(bl, sd)[:, ::st]) > 125
    assert co.snr_db(x, o.bwd(bl, sd)) > 140


def test_layout_sliced_matches_reference(gl):
    i = int(gl["meta_stride"][2])
    octs, bpo, fs = layout(gl, i)
    s = co.SlicedCQT(octs, bpo, fs)
    x = sliced_input()[:, :1]
    bl, sd = s.fwd(x)
    st, sts = int(gl["meta_stride"][0]), int(gl["meta_stride"][1])
    assert [list(c.shape) for c in bl] == gl["sliced_shapes"].tolist()
    cb = np.concatenate([c.reshape(1, -1)[..., ::sts] for c in bl], -1)
    assert co.snr_db(gl["sliced_blocks_sub"], cb) > 120
    cs = np.concatenate([c.reshape(1, -1)[..., ::st] for c in sd], -1)
    assert co.snr_db(gl["sliced_side_sub"], cs) > 120
    y = s.bwd(bl, sd, length=x.shape[-1])
    assert co.snr_db(gl["sliced_bwd_sub"], y[..., ::st]) > 120


def test_layout0_needs_the_overflow_capacity(gl):
    """Layout 0 overflows more than 2048 bins, about 300 in one fold list:
    the synthesis slot buffer's overflow area and fold lists are sized for
    it (4096 bins, 512 entries per inverse column workgroup)."""
    from flash_cqt import tables as T
    _, t = tables_for(gl, 0)
    for key in ("ovf_scat", "ovf_scat_a"):
        per = (t[key].reshape(T.INV_WGS, T.FOLD_PER_WG) >= 0).sum(1)
        assert per.sum() <= T.OVF_CAP and per.max() <= T.FOLD_PER_WG
    per = (t["ovf_scat"].reshape(T.INV_WGS, T.FOLD_PER_WG) >= 0).sum(1)
    assert per.sum() > 2048 and per.max() > 256


@pytest.mark.parametrize("i", range(NLAYOUTS))
def test_layout_schedule_sim(gl, i):
    """The band and pass kernels' index math (tests/kernel_sim.py) on this
    layout's tables: analysis, synthesis (wide and narrow inverse tiles,
    every fold entry consumed once) and both adjoints against the oracle."""
    o = oracle_for(gl, i)
    _, t = tables_for(gl, i)
    x = inputs()[0][:1].astype(np.float64)
    X = ks.packed_fft_fwd(x)
    C = ks.route_bands(X, t["route_taps"], t["bands"], t["tasks"], t["ncoef"])
    obl, osd = o.fwd(x)
    Cref = o.flatten(obl, osd)
    assert co.snr_db(Cref, C) > 140
    F = ks.scatter_bands(Cref, t["scat_taps"], t["tasks"], t["ncoef"])
    ref = o.bwd(obl, osd)
    assert co.snr_db(ref, ks.packed_fft_inv(F, t["ovf_scat"], ks.WIDE)) > 140
    assert co.snr_db(ref, ks.packed_fft_inv(F, t["ovf_scat"], ks.NARROW)) > 140
    rs = np.random.RandomState(40 + i)
    G = rs.standard_normal((1, t["ncoef"])) + 1j * rs.standard_normal((1, t["ncoef"]))
    F = ks.scatter_bands(G, t["scat_a_taps"], t["tasks"], t["ncoef"])
    assert co.snr_db(o.fwd_adjoint(*o.unflatten(G)), ks.packed_fft_inv(F, t["ovf_scat_a"])) > 140
    u = rs.standard_normal((1, N))
    gC = ks.route_bands(ks.packed_fft_fwd(u), t["route_b_taps"], t["bands"], t["tasks"], t["ncoef"])
    assert co.snr_db(o.flatten(*o.bwd_adjoint(u)), gC) > 140


def test_unsupported_band_lengths_refused_and_auto_engine():
    """A layout with a band length outside 32..2048 (here 16: [3,3,3] /
    [16,32,64]) is refused by FusedOctCQT with a ValueError naming it, before
    any device work, as the reference's factored engine cannot build it
    either; SlicedCQT's 'auto' then keeps the torch engine, which takes any
    layout (float64 and other slice lengths likewise)."""
    import torch
    from flash_cqt import OctCQT, SlicedCQT
    from flash_cqt.fused import FusedOctCQT
    c = OctCQT([3, 3, 3], [16, 32, 64], fs=44100, audio_len=N, device="cpu")
    lengths = {g[0].shape[1] for g in c.np_groups + c.np_side_groups}
    assert min(lengths) < 32
    with pytest.raises(ValueError, match="band lengths"):
        FusedOctCQT(c, "cuda")
    pick = SlicedCQT.auto_picks_hip
    ok = {32, 64, 2048}
    assert pick("cuda", N, torch.float32, ok)
    assert pick("cuda:0", N, torch.float32, ok)
    assert not pick("cuda", N, torch.float32, lengths)
    assert not pick("cuda", N, torch.float64, ok)
    assert not pick("cpu", N, torch.float32, ok)
    assert not pick("cuda", N // 2, torch.float32, ok)
    s = SlicedCQT([3, 3, 3], [16, 32, 64], fs=44100, device="cpu")
    assert type(s.cqt).__name__ == "OctCQT"


@pytest.mark.parametrize("i", range(len(SWEEP)))
def test_sweep_layout_schedule_sim(i):
    """Index-math replay of the analysis and the synthesis (wide and narrow
    inverse tiles) on the tables of a sweep layout, against the oracle."""
    from flash_cqt import OctCQT, tables
    octs, bpo, fs = SWEEP[i]
    c = OctCQT(octs, bpo, fs=fs, audio_len=N, device="cpu")
    t = tables.build(c.np_groups + c.np_side_groups)
    o = co.OctCQT(octs, bpo, fs, N)
    x = inputs()[0][1:].astype(np.float64)
    C = ks.route_bands(ks.packed_fft_fwd(x), t["route_taps"], t["bands"], t["tasks"], t["ncoef"])
    obl, osd = o.fwd(x)
    Cref = o.flatten(obl, osd)
    assert co.snr_db(Cref, C) > 140
    F = ks.scatter_bands(Cref, t["scat_taps"], t["tasks"], t["ncoef"])
    ref = o.bwd(obl, osd)
    assert co.snr_db(ref, ks.packed_fft_inv(F, t["ovf_scat"], ks.WIDE)) > 140
    assert co.snr_db(ref, ks.packed_fft_inv(F, t["ovf_scat"], ks.NARROW)) > 140
