"""Write the golden fixtures that pin the oracle to the reference.

Runs ONCE, in the build container, on CPU:  python tests/golden/make_golden.py
(golden_ref.npz, the headline layout) and python tests/golden/make_golden.py
layouts (golden_layouts.npz, four further layouts).

Why an import: the reference holds no golden vectors, and the bank numerics
(np.round ties in filterbank.py:74-76 and 85-94, the mirrored block-size
write one slot low at filterbank.py:110 that makes Mnyq 2048, the float32
frame diagonal of ref_util.py:43-52) and the SlicedCQT roll/overlap-add
conventions (sliced.py:106-167) are fixed by no closed form. So this script
imports the reference's pure-torch modules from /root/reference and records
their outputs on closed-form inputs. The reference never travels: only the
numbers below are committed (tests/golden/*.npz).

Inputs come from golden_inputs.py (numpy's legacy RandomState, a frozen
stream), so the tests regenerate them bit-for-bit without storing them.
"""
import hashlib
import pathlib
import sys

import numpy as np
import torch

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))
from golden_inputs import inputs, cotangents, sliced_input  # noqa: E402

REF = pathlib.Path("/root/reference")
OUT = pathlib.Path(__file__).resolve().parent

N = 65536
FS = 44100
LAYOUT = ([3, 4, 2], [8, 16, 32])
STRIDE = 7  # coefficient / sample subsampling stride of the stored vectors
STRIDE_SLICED = 31  # subsampling stride of the sliced coefficient vectors


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    sys.path.insert(0, str(REF))
    from flash_cqt import OctCQT, SlicedCQT  # noqa: E402  (reference, CPU only)

    torch.set_num_threads(8)
    cqt = OctCQT(*LAYOUT, fs=FS, audio_len=N, device="cpu")
    bank = cqt.bank
    kept = bank.fbins + 2

    fx = {}
    # ---- bank tables
    fx["bank_M"] = bank.M.numpy().astype(np.int64)
    fx["bank_size_per_oct"] = np.array(bank.size_per_oct, dtype=np.int64)
    fx["bank_oct_bins"] = np.array(bank.oct_bins, dtype=np.int64)
    fx["bank_M0_Mnyq_fbins_nn"] = np.array([bank.M0, bank.Mnyq, bank.fbins, bank.nn], dtype=np.int64)
    fx["bank_frqs_hz"] = np.asarray(bank.frqs_hz, dtype=np.float64)
    fx["bank_win_start"] = np.array([int(w[0]) for w in bank.wins], dtype=np.int64)
    fx["bank_win_len"] = np.array([int(w.shape[0]) for w in bank.wins], dtype=np.int64)
    fx["bank_g_kept"] = np.concatenate([bank.g[i].numpy() for i in range(kept)]).astype(np.float32)
    fx["bank_gd_kept"] = np.concatenate([bank.gd[i].numpy() for i in range(kept)]).astype(np.float32)

    # ---- OctCQT group tables, hashed in canonical dtypes
    hashes = []
    for idx, gv, pos, gdv, conj in list(cqt.groups) + list(cqt.side_groups):
        hashes.append([sha(idx.numpy().astype(np.int64)), sha(gv.numpy().astype(np.float32)),
                       sha(pos.numpy().astype(np.int64)), sha(gdv.numpy().astype(np.float32)),
                       sha(conj.numpy().astype(np.bool_))])
    fx["group_table_sha256"] = np.array(hashes)
    fx["pos_flat_sha256"] = np.array([sha(cqt.pos_flat.numpy().astype(np.int64))])

    # ---- forward / inverse on closed-form inputs
    x, u = inputs()
    xt = torch.from_numpy(x)
    with torch.no_grad():
        blocks, side = cqt.fwd(xt)
        flat = torch.cat([c.reshape(2, -1) for c in list(blocks) + list(side)], dim=-1)
        y = cqt.bwd(blocks, side)
        y_noside = cqt.bwd(blocks)
    ncoef = flat.shape[-1]
    fx["fwd_sub"] = flat[:, ::STRIDE].numpy().astype(np.complex64)
    fx["fwd_band_energy"] = np.stack(
        [np.concatenate([(c.abs().double() ** 2).sum(-1).reshape(2, -1).numpy()
                         for c in list(blocks) + list(side)], axis=-1)])[0]
    fx["bwd_sub"] = y[:, ::STRIDE].numpy().astype(np.float32)
    fx["bwd_noside_sub"] = y_noside[:, ::STRIDE].numpy().astype(np.float32)

    # ---- gradients through reference autograd
    ys = cotangents(ncoef)
    xg = xt.clone().requires_grad_(True)
    bl, sd = cqt.fwd(xg)
    fl = torch.cat([c.reshape(2, -1) for c in list(bl) + list(sd)], dim=-1)
    (torch.view_as_real(fl) * torch.from_numpy(ys)).sum().backward()
    fx["grad_fwd_sub"] = xg.grad[:, ::STRIDE].numpy().astype(np.float32)

    leaves = [c.detach().clone().requires_grad_(True) for c in list(blocks) + list(side)]
    ng = len(cqt.groups)
    (cqt.bwd(leaves[:ng], leaves[ng:]) * torch.from_numpy(u)).sum().backward()
    gfl = torch.cat([lv.grad.reshape(2, -1) for lv in leaves], dim=-1)
    fx["grad_bwd_sub"] = gfl[:, ::STRIDE].numpy().astype(np.complex64)

    # ---- sliced
    s = SlicedCQT(*LAYOUT, fs=FS, sl_len=N, device="cpu")
    xs = torch.from_numpy(sliced_input())
    with torch.no_grad():
        sb, ss = s.fwd(xs)
        ys_ = s.bwd(sb, ss, length=xs.shape[-1])
        fx["sliced_tw_sha256"] = np.array([sha(s.tw.numpy().astype(np.float32))])
        fx["sliced_blocks_sub"] = np.concatenate(
            [c.reshape(1, 2, -1)[..., ::STRIDE_SLICED].numpy() for c in sb], axis=-1).astype(np.complex64)
        fx["sliced_side_sub"] = np.concatenate(
            [c.reshape(1, 2, -1)[..., ::STRIDE].numpy() for c in ss], axis=-1).astype(np.complex64)
        fx["sliced_bwd_sub"] = ys_[..., ::STRIDE].numpy().astype(np.float32)
        fx["sliced_shapes"] = np.array([list(c.shape) for c in sb], dtype=np.int64)

    fx["meta_versions"] = np.array([torch.__version__, np.__version__])
    fx["meta_stride"] = np.array([STRIDE, STRIDE_SLICED])
    np.savez_compressed(OUT / "golden_ref.npz", **fx)
    print("wrote", OUT / "golden_ref.npz", (OUT / "golden_ref.npz").stat().st_size, "bytes")


# Further layouts the reference's factored engine accepts (band lengths
# 32-2048), chosen for what they stress: the most bins with three or four
# taps found over ~1000 random layouts (more than 2048 overflow bins, ~300 in
# one inverse column workgroup), four taps on one bin, two octave groups at
# another rate, and an octave group of a single band.
LAYOUTS = (
    (([6, 2, 1], [4, 12, 24]), 16000),
    (([2, 5, 2], [4, 8, 64]), 44100),
    (([4, 3], [12, 48]), 48000),
    (([1, 2, 2], [4, 16, 96]), 22050),
)
STRIDE_LAYOUTS = 13
SLICED_LAYOUT = 1           # index into LAYOUTS of the layout also run sliced


def layouts():
    """golden_layouts.npz: for each of LAYOUTS, the group table hashes, the
    block shapes, and forward / inverse vectors of the reference on the
    closed-form inputs (first row only), plus one sliced run."""
    sys.path.insert(0, str(REF))
    from flash_cqt import OctCQT, SlicedCQT  # noqa: E402  (reference, CPU only)

    torch.set_num_threads(8)
    fx = {}
    x, _ = inputs()
    xt = torch.from_numpy(x[:1])
    for li, ((octs, bpo), fs) in enumerate(LAYOUTS):
        cqt = OctCQT(octs, bpo, fs=fs, audio_len=N, device="cpu")
        groups = list(cqt.groups) + list(cqt.side_groups)
        fx[f"l{li}_layout"] = np.array(octs + [-1] + bpo + [-1, fs], dtype=np.int64)
        fx[f"l{li}_group_shapes"] = np.array([list(g[0].shape) for g in groups], dtype=np.int64)
        fx[f"l{li}_group_table_sha256"] = np.array(
            [[sha(idx.numpy().astype(np.int64)), sha(gv.numpy().astype(np.float32)),
              sha(pos.numpy().astype(np.int64)), sha(gdv.numpy().astype(np.float32)),
              sha(conj.numpy().astype(np.bool_))] for idx, gv, pos, gdv, conj in groups])
        with torch.no_grad():
            blocks, side = cqt.fwd(xt)
            flat = torch.cat([c.reshape(1, -1) for c in list(blocks) + list(side)], dim=-1)
            y = cqt.bwd(blocks, side)
        fx[f"l{li}_fwd_sub"] = flat[:, ::STRIDE_LAYOUTS].numpy().astype(np.complex64)
        fx[f"l{li}_bwd_sub"] = y[:, ::STRIDE_LAYOUTS].numpy().astype(np.float32)
    (octs, bpo), fs = LAYOUTS[SLICED_LAYOUT]
    s = SlicedCQT(octs, bpo, fs=fs, sl_len=N, device="cpu")
    xs = torch.from_numpy(sliced_input()[:, :1])
    with torch.no_grad():
        sb, ss = s.fwd(xs)
        ys_ = s.bwd(sb, ss, length=xs.shape[-1])
    fx["sliced_shapes"] = np.array([list(c.shape) for c in sb], dtype=np.int64)
    fx["sliced_blocks_sub"] = torch.cat(
        [c.reshape(1, -1)[..., ::STRIDE_SLICED] for c in sb], dim=-1).numpy().astype(np.complex64)
    fx["sliced_side_sub"] = torch.cat(
        [c.reshape(1, -1)[..., ::STRIDE_LAYOUTS] for c in ss], dim=-1).numpy().astype(np.complex64)
    fx["sliced_bwd_sub"] = ys_[..., ::STRIDE_LAYOUTS].numpy().astype(np.float32)
    fx["meta_versions"] = np.array([torch.__version__, np.__version__])
    fx["meta_stride"] = np.array([STRIDE_LAYOUTS, STRIDE_SLICED, SLICED_LAYOUT])
    np.savez_compressed(OUT / "golden_layouts.npz", **fx)
    print("wrote", OUT / "golden_layouts.npz", (OUT / "golden_layouts.npz").stat().st_size, "bytes")


if __name__ == "__main__":
    if sys.argv[1:] == ["layouts"]:
        layouts()
    else:
        main()
