"""The package's float64 transform definition (CPU, no GPU).

OctCQT(dtype=torch.float64) builds its windows and frame diagonal in
float64, as the reference does (filterbank.py:114-117, ref_util.py:16-22,
43-52), so its round trip reconstructs to near machine precision; the
float32 bank is unchanged (its golden sha256 checks live in test_tables.py).
"""
import numpy as np
import torch

from golden.golden_inputs import inputs
from oracle import cqt_oracle as co

LAYOUT = ([3, 4, 2], [8, 16, 32])
N = 65536


def _pkg(dtype):
    from flash_cqt import OctCQT
    return OctCQT(*LAYOUT, fs=44100, audio_len=N, device="cpu", dtype=dtype)


def test_float64_tables_equal_oracle():
    pkg = _pkg(torch.float64)
    ora = co.OctCQT(*LAYOUT, 44100, N, dtype=np.float64)
    for (pi, pg, pp, pd, pc), (oi, og, op, od, oc) in zip(pkg.np_groups + pkg.np_side_groups, ora.all_groups):
        assert pg.dtype == np.float64 and pd.dtype == np.float64
        assert np.array_equal(pi, oi) and np.array_equal(pp, op) and np.array_equal(pc, oc)
        assert np.array_equal(pg, og) and np.array_equal(pd, od)
    for g in pkg.groups + pkg.side_groups:
        assert g[1].dtype == torch.float64 and g[3].dtype == torch.float64


def test_float32_tables_unchanged_by_dtype_path():
    """The float32 bank still rounds float64 windows once and accumulates
    its diagonal in float32 (equal to the oracle's float32 tables)."""
    pkg = _pkg(torch.float32)
    ora = co.OctCQT(*LAYOUT, 44100, N)
    for (pi, pg, pp, pd, pc), (oi, og, op, od, oc) in zip(pkg.np_groups + pkg.np_side_groups, ora.all_groups):
        assert pg.dtype == np.float32 and pd.dtype == np.float32
        assert np.array_equal(pg.view(np.uint32), og.view(np.uint32))
        assert np.array_equal(pd.view(np.uint32), od.view(np.uint32))


def test_float64_octcqt_round_trip():
    x, _ = inputs()
    x = x.astype(np.float64)
    c = _pkg(torch.float64)
    xt = torch.from_numpy(x)
    b, s = c.fwd(xt)
    assert b[0].dtype == torch.complex128
    assert co.snr_db(x, c.bwd(b, s).numpy()) >= 250
    # and the coefficients are the float64 oracle's
    ora = co.OctCQT(*LAYOUT, 44100, N, dtype=np.float64)
    ob, os_ = ora.fwd(x)
    got = np.concatenate([t.numpy().reshape(2, -1) for t in list(b) + list(s)], -1)
    assert co.snr_db(ora.flatten(ob, os_), got) >= 250


def test_float64_sliced_round_trip():
    """SlicedCQT(dtype=torch.float64) runs the float64 torch engine; its
    Tukey slices sum to one, so the whole-signal round trip is as exact as
    the per-slice transform."""
    from flash_cqt import SlicedCQT
    s = SlicedCQT(device="cpu", dtype=torch.float64)
    assert s.cqt.dtype == torch.float64
    rs = np.random.RandomState(11)
    x = torch.from_numpy(rs.standard_normal((1, 2, 100_000)))
    bl, sd = s.fwd(x)
    y = s.bwd(bl, sd, length=x.shape[-1])
    assert y.dtype == torch.float64
    assert co.snr_db(x.numpy(), y.numpy()) >= 250
