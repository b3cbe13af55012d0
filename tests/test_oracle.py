"""Pin the CPU oracle: golden vectors from the reference, exact identities, and
checks that a plausible mistake in the oracle would fail."""
import hashlib

import numpy as np
import pytest

from golden.golden_inputs import inputs, cotangents, sliced_input
from oracle import cqt_oracle as co

N = 65536


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def group_hashes(groups):
    return [[sha(idx.astype(np.int64)), sha(gv.astype(np.float32)), sha(pos.astype(np.int64)),
             sha(gdv.astype(np.float32)), sha(conj.astype(np.bool_))]
            for idx, gv, pos, gdv, conj in groups]


# ------------------------------------------------------------------ bank

def test_bank_layout_matches_reference(oracle, golden):
    b = oracle.bank
    assert np.array_equal(b.M, golden["bank_M"])
    assert np.array_equal(b.size_per_oct, golden["bank_size_per_oct"])
    assert np.array_equal(b.oct_bins, golden["bank_oct_bins"])
    assert [b.M0, b.Mnyq, b.fbins, b.nn] == golden["bank_M0_Mnyq_fbins_nn"].tolist()
    assert b.Mnyq == 2048  # the mirrored write one slot low
    assert np.array_equal(b.frqs_hz, golden["bank_frqs_hz"])
    assert np.array_equal([w[0] for w in b.wins], golden["bank_win_start"])
    assert np.array_equal([len(w) for w in b.wins], golden["bank_win_len"])


def test_windows_and_duals_bit_exact(oracle, golden):
    b = oracle.bank
    kept = b.fbins + 2
    g = np.concatenate([b.g[i] for i in range(kept)])
    gd = np.concatenate([b.gd[i] for i in range(kept)])
    assert np.array_equal(g.view(np.uint32), golden["bank_g_kept"].view(np.uint32))
    assert np.array_equal(gd.view(np.uint32), golden["bank_gd_kept"].view(np.uint32))


def test_group_tables_bit_exact(oracle, golden):
    assert group_hashes(oracle.all_groups) == golden["group_table_sha256"].tolist()
    assert sha(oracle.pos_flat.astype(np.int64)) == golden["pos_flat_sha256"][0]


def test_planted_bank_mistake_is_caught(golden):
    """Dropping the mirrored block-size quirk (the 'obvious fix') must break
    the golden tables: shows the table check has teeth."""
    orig = co.next_power_of_2
    bank = co.FlexOctBank([3, 4, 2], [8, 16, 32], 44100, N)
    M = bank.M.copy()
    # recompute M with the mirror written at the symmetric slot
    Mq = bank.M_raw.copy()
    idx = 1
    for b in bank.oct_bins:
        v = orig(bank.M_raw[idx:idx + b].max())
        Mq[idx:idx + b] = v
        Mq[len(Mq) - idx - b + 1:len(Mq) - idx + 1] = v
        idx += b
    assert not np.array_equal(Mq.astype(np.int64), golden["bank_M"])
    assert np.array_equal(M, golden["bank_M"])


def test_dual_frame_identity(oracle):
    """Painless frame: sum_i M_i g_i gd_i = 1 on every bin (to fp32 rounding
    of the duals). Checked on the natural-order supports."""
    b = oracle.bank
    acc = np.zeros(b.nn)
    for g, gd, m, rng in zip(b.g, b.gd, b.M, b.wins):
        acc[rng] += float(m) * np.fft.fftshift(g).astype(np.float64) * np.fft.fftshift(gd).astype(np.float64)
    assert np.max(np.abs(acc - 1.0)) < 1e-6


# ------------------------------------------------------- float64 bank

@pytest.fixture(scope="module")
def oracle64():
    return co.OctCQT([3, 4, 2], [8, 16, 32], 44100, N, dtype=np.float64)


def test_float64_bank_pins(oracle64, golden):
    """The float64 bank (reference OctCQT(dtype=torch.float64): windows and
    frame diagonal in float64, filterbank.py:114-117) is pinned three ways:
    its windows round to the reference's float32 windows bit for bit (the
    float32 bank is float32(float64 Hann)), its index tables are the
    reference's, and its frame identity sum_i M_i g_i gd_i = 1 holds to
    float64 rounding."""
    b = oracle64.bank
    kept = b.fbins + 2
    g = np.concatenate([b.g[i] for i in range(kept)])
    assert g.dtype == np.float64
    assert np.array_equal(g.astype(np.float32).view(np.uint32), golden["bank_g_kept"].view(np.uint32))
    ref = golden["group_table_sha256"].tolist()
    got = group_hashes(oracle64.all_groups)
    for r, h in zip(ref, got):
        assert (h[0], h[2], h[4]) == (r[0], r[2], r[4])   # idx, pos, conj
    acc = np.zeros(b.nn)
    for gi, gd, m, rng in zip(b.g, b.gd, b.M, b.wins):
        acc[rng] += float(m) * np.fft.fftshift(gi) * np.fft.fftshift(gd)
    assert np.max(np.abs(acc - 1.0)) < 1e-13


def test_float64_round_trip_exact(oracle64):
    """A painless frame reconstructs exactly in exact arithmetic, so the
    float64 bank's round trip reaches near machine precision (>= 250 dB);
    the float32 bank stops near 147 dB even in float64 arithmetic."""
    x, _ = inputs()
    assert co.snr_db(x, oracle64.bwd(*oracle64.fwd(x))) >= 250


def test_planted_float32_diagonal_fails_float64_bar(monkeypatch):
    """The slip of accumulating a float64 bank's frame diagonal in float32
    (float64 windows, float32 diagonal) must miss the float64 round-trip bar."""
    orig = co.nsdual
    monkeypatch.setattr(co, "nsdual", lambda g, wins, nn, M, dtype=np.float32: orig(g, wins, nn, M, np.float32))
    planted = co.OctCQT([3, 4, 2], [8, 16, 32], 44100, N, dtype=np.float64)
    x, _ = inputs()
    assert co.snr_db(x, planted.bwd(*planted.fwd(x))) < 200


# ------------------------------------------------------- forward / inverse

def test_fwd_matches_reference(oracle, golden):
    x, _ = inputs()
    bl, sd = oracle.fwd(x)
    flat = oracle.flatten(bl, sd)
    st = int(golden["meta_stride"][0])
    assert co.snr_db(golden["fwd_sub"], flat[:, ::st]) > 125
    en = np.concatenate([(np.abs(c) ** 2).sum(-1).reshape(2, -1) for c in list(bl) + list(sd)], -1)
    assert np.allclose(en, golden["fwd_band_energy"], rtol=2e-5)


def test_bwd_matches_reference(oracle, golden):
    x, _ = inputs()
    bl, sd = oracle.fwd(x)
    st = int(golden["meta_stride"][0])
    assert co.snr_db(golden["bwd_sub"], oracle.bwd(bl, sd)[:, ::st]) > 125
    assert co.snr_db(golden["bwd_noside_sub"], oracle.bwd(bl)[:, ::st]) > 125
    assert co.snr_db(x, oracle.bwd(bl, sd)) > 140


def test_linearity(oracle):
    rs = np.random.RandomState(3)
    a, b = rs.standard_normal((2, N))
    fa = oracle.flatten(*oracle.fwd(a))
    fb = oracle.flatten(*oracle.fwd(b))
    fab = oracle.flatten(*oracle.fwd(2.5 * a - 0.75 * b))
    assert co.snr_db(fab, 2.5 * fa - 0.75 * fb) > 250


def test_band_tap_is_windowed_rfft_bin(oracle):
    """Closed form: for a pure tone the forward equals the gather of the DFT
    at the window's bins times the window, inverse-DFT'd (spot-check one band)."""
    n = np.arange(N)
    x = np.cos(2 * np.pi * 1234.5 * n / N)
    bl, _ = oracle.fwd(x)
    idx, gv = oracle.groups[4][0], oracle.groups[4][1]
    X = np.array([np.sum(x * np.exp(-2j * np.pi * k * n / N)) for k in np.unique(idx[3])])
    lut = dict(zip(np.unique(idx[3]).tolist(), X))
    taps = np.array([lut[k] for k in idx[3]]) * gv[3]
    assert co.snr_db(np.fft.ifft(taps), bl[4][3]) > 200


# ------------------------------------------------------------- adjoints

def test_adjoint_dot_products(oracle):
    rs = np.random.RandomState(5)
    x = rs.standard_normal((2, N))
    G = rs.standard_normal((2, oracle.ncoef)) + 1j * rs.standard_normal((2, oracle.ncoef))
    C = oracle.flatten(*oracle.fwd(x))
    gx = oracle.fwd_adjoint(*oracle.unflatten(G))
    lhs = np.sum(C.real * G.real + C.imag * G.imag)
    rhs = np.sum(x * gx)
    assert abs(lhs - rhs) < 1e-10 * abs(lhs)
    u = rs.standard_normal((2, N))
    y = oracle.bwd(*oracle.unflatten(G))
    gC = oracle.flatten(*oracle.bwd_adjoint(u))
    lhs2 = np.sum(y * u)
    rhs2 = np.sum(G.real * gC.real + G.imag * gC.imag)
    assert abs(lhs2 - rhs2) < 1e-10 * abs(lhs2)


def test_planted_adjoint_mistake_fails_dot_product(oracle):
    """Forgetting the doubled DC/Nyquist rows (a real-FFT transpose slip)
    must fail the dot-product identity."""
    rs = np.random.RandomState(6)
    x = rs.standard_normal((1, N))
    G = rs.standard_normal((1, oracle.ncoef)) + 1j * rs.standard_normal((1, oracle.ncoef))
    C = oracle.flatten(*oracle.fwd(x))
    lhs = np.sum(C.real * G.real + C.imag * G.imag)
    gx_good = oracle.fwd_adjoint(*oracle.unflatten(G))
    # bad variant: plain (N/2) irfft without the edge doubling
    L = N // 2
    Y = np.zeros((1, L + 1), dtype=np.complex128)
    for Gb, (idx, gv, _, _, conj) in zip(oracle.unflatten(G)[0] + oracle.unflatten(G)[1], oracle.all_groups):
        M = idx.shape[1]
        ab = np.fft.fft(Gb, axis=-1) / M
        ab = np.where(conj, np.conj(ab), ab) * gv
        np.add.at(Y[0], idx.reshape(-1), ab.reshape(-1))
    gx_bad = (N / 2.0) * np.fft.irfft(Y, n=N)
    assert abs(lhs - np.sum(x * gx_good)) < 1e-10 * abs(lhs)
    assert abs(lhs - np.sum(x * gx_bad)) > 1e-8 * abs(lhs)


def test_adjoints_match_reference_autograd(oracle, golden):
    x, u = inputs()
    st = int(golden["meta_stride"][0])
    ys = cotangents(oracle.ncoef)
    G = ys[..., 0].astype(np.float64) + 1j * ys[..., 1].astype(np.float64)
    gx = oracle.fwd_adjoint(*oracle.unflatten(G))
    assert co.snr_db(golden["grad_fwd_sub"], gx[:, ::st]) > 120
    gC = oracle.flatten(*oracle.bwd_adjoint(u))
    assert co.snr_db(golden["grad_bwd_sub"], gC[:, ::st]) > 120


# ------------------------------------------------------ packed real FFT

def test_untangle_identity():
    rs = np.random.RandomState(8)
    x = rs.standard_normal((2, N))
    Z = co.packed_spectrum(x)
    k = np.arange(N // 2 + 1)
    assert co.snr_db(np.fft.rfft(x), co.untangle(Z, k)) > 280
    assert co.snr_db(np.fft.fft(x[:, 0::2] + 1j * x[:, 1::2]), Z) > 280


# ------------------------------------------------------------ sliced

def test_sliced_matches_reference(golden):
    s = co.SlicedCQT()
    x = sliced_input()
    bl, sd = s.fwd(x)
    st = int(golden["meta_stride"][0])
    sts = int(golden["meta_stride"][1])
    assert [list(c.shape) for c in bl] == golden["sliced_shapes"].tolist()
    assert sha(co.makewnd(65536, 16384)) == golden["sliced_tw_sha256"][0]
    cb = np.concatenate([c.reshape(1, 2, -1)[..., ::sts] for c in bl], -1)
    assert co.snr_db(golden["sliced_blocks_sub"], cb) > 120
    cs = np.concatenate([c.reshape(1, 2, -1)[..., ::st] for c in sd], -1)
    assert co.snr_db(golden["sliced_side_sub"], cs) > 120
    y = s.bwd(bl, sd, length=x.shape[-1])
    assert co.snr_db(golden["sliced_bwd_sub"], y[..., ::st]) > 120
    assert co.snr_db(x, y) > 135


# ------------------------------------------------------- host-core baseline

def test_torch_port_matches_oracle_and_reference(oracle, golden):
    """oracle/torch_port.py is what bench.py times as the host-core
    baseline: it must compute the same transform. Forward coefficients and
    the inverse (with and without the side bands) against the float64
    oracle at >= 120 dB, and against the reference's golden vectors."""
    import torch
    from oracle.torch_port import TorchPortOctCQT
    port = TorchPortOctCQT()
    x, _ = inputs()
    with torch.no_grad():
        pb, ps = port.fwd(torch.from_numpy(x))
        got = np.concatenate([c.numpy().reshape(x.shape[0], -1) for c in list(pb) + list(ps)], -1)
        bl, sd = oracle.fwd(x)
        ref = oracle.flatten(bl, sd)
        assert co.snr_db(ref, got) >= 120
        st = int(golden["meta_stride"][0])
        assert co.snr_db(golden["fwd_sub"], got[:, ::st]) >= 120
        # the inverse on the oracle's coefficients (rounded to complex64)
        c64 = [torch.from_numpy(c.astype(np.complex64)) for c in list(bl) + list(sd)]
        y = port.bwd(c64[:len(bl)], c64[len(bl):]).numpy()
        assert co.snr_db(oracle.bwd(bl, sd), y) >= 120
        assert co.snr_db(golden["bwd_sub"], y[:, ::st]) >= 120
        # round trip of the port alone
        assert co.snr_db(x, port.bwd(pb, ps).numpy()) >= 125


def test_planted_port_mistake_is_caught(oracle):
    """A plausible slip in the port (the dual window of one group left out of
    the inverse) must fail the comparison above."""
    import torch
    from oracle.torch_port import TorchPortOctCQT
    port = TorchPortOctCQT()
    idx, gv, pos, gdv, conj = port.groups[3]
    port.groups[3] = (idx, gv, pos, torch.ones_like(gdv), conj)
    x, _ = inputs()
    bl, sd = oracle.fwd(x)
    c64 = [torch.from_numpy(c.astype(np.complex64)) for c in list(bl) + list(sd)]
    with torch.no_grad():
        y = port.bwd(c64[:len(bl)], c64[len(bl):]).numpy()
    assert co.snr_db(oracle.bwd(bl, sd), y) < 60
