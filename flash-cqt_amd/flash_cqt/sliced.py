"""Streamable sliced octave CQT (reference surface: sliced.py:26-209).

The signal is cut into 50%-overlapped slices of sl_len samples under a Tukey
window (flat top, Hann transitions) whose overlapped copies sum to one, each
slice goes through the per-slice engine `self.cqt`, and the inverse
overlap-adds the per-slice inverses. Slices are rolled by a quarter (even
slices left, odd slices right) so the window plateau alternates, and the
octave coefficients are rolled back by a quarter of each block.

The per-slice engine is any object with fwd(x[..., sl_len]) -> (blocks, side)
and bwd(blocks, side) -> x. engine="auto" uses the fused HIP engine
(TrainableCQT, differentiable) for fp32 on a GPU device with sl_len 65536 and
band lengths 32..2048, and the pure-torch OctCQT otherwise; "hip" forces the fused engine, "torch" the
pure-torch one. Assigning self.cqt swaps engines as in the reference.

With the HIP engine and no gradient to record, fwd and bwd run the framing
inside the engine's kernels (fcqt_sliced_analysis, which frames, transforms
and routes, in chunks of about 128 slices from 256 slices on;
fcqt_scatter_bands_sliced, the inverse passes and fcqt_overlap_add, or from
256 slices on fcqt_sliced_synthesis, which overlap-adds in the inverse row
pass's store): slices are read straight from the signal, coefficients are
written and read in the block layout with the quarter roll applied, and the
inverse slices are rolled and overlap-added in one pass. Blocks returned by that path are views of one buffer; passing
them back to bwd reads that buffer without a copy. The bounded-state stream
(stream_fwd / stream_bwd) runs each step as one C-ABI call per direction
(fcqt_stream_analysis reads the carried half slice and the new chunk in place,
fcqt_stream_synthesis scatters, inverts and overlap-adds).
"""
import math
import weakref

import torch

from . import _native

from .ref_util import hann_fft_order
from .oct_cqt import OctCQT


# From this many slices on the whole-signal synthesis overlap-adds in the
# inverse row pass (fcqt_sliced_synthesis); below, the slices go through a
# slice buffer and one overlap-add kernel, which measured faster there
# (SlicedCQT.bwd, fused against buffered): 53 against 49 us at 64 slices;
# at configs[4]'s 120 slices the two row-pass launches took 8.4 + 12.7 us
# against 11.3 + 8.2 us for the row pass and the overlap-add; 170 against
# 179 us at 256 slices and 327-336 against 353-364 us at 512. Same bits
# either way.
FUSED_OLA_MIN_SLICES = 256


def makewnd(sl_len, tr_area, device="cpu", dtype=torch.float32):
    """Tukey window of one slice, transitions centred at sl_len/4 and 3 sl_len/4."""
    q = sl_len // 4
    h = tr_area // 2
    hann = torch.as_tensor(hann_fft_order(2 * tr_area), device=torch.device(device)).to(dtype)
    w = torch.zeros(sl_len, dtype=dtype, device=torch.device(device))
    w[q - h:q + h] = hann[tr_area:]
    w[q + h:3 * q - h] = 1
    w[3 * q - h:3 * q + h] = hann[:tr_area]
    return w


class SlicedCQT:
    def __init__(self, num_octs=(3, 4, 2), bins_per_oct=(8, 16, 32), fs=44100,
                 sl_len=65536, tr_area=None, device="cpu", dtype=torch.float32,
                 engine="auto"):
        assert sl_len % 4 == 0
        if tr_area is None:
            tr_area = sl_len // 4
        assert tr_area % 2 == 0 and 0 < tr_area * 2 <= sl_len
        self.fs = fs
        self.sl_len = sl_len
        self.tr_area = tr_area
        self.H = sl_len // 4
        self.hop = sl_len // 2
        self.device = torch.device(device)
        self.dtype = dtype

        oct_ = OctCQT(list(num_octs), list(bins_per_oct), fs=fs, audio_len=sl_len,
                      device=device, dtype=dtype)
        self.oct = oct_
        self.oct_bins = oct_.oct_bins
        self.size_per_oct = oct_.size_per_oct
        self.frqs_hz = oct_.frqs_hz
        if engine not in ("auto", "hip", "torch"):
            raise ValueError("engine must be 'auto', 'hip' or 'torch'")
        lengths = {g[0].shape[1] for g in oct_.np_groups + oct_.np_side_groups}
        if engine == "hip" or (engine == "auto" and self.auto_picks_hip(self.device, sl_len, dtype, lengths)):
            from .trainable import TrainableCQT
            self.cqt = TrainableCQT(oct_, device)
        else:
            self.cqt = oct_
        self.tw = makewnd(sl_len, tr_area, device=device, dtype=dtype)
        # run the framing inside the HIP engine's kernels when it can (False:
        # always frame on the host around self.cqt, as the reference does)
        self.fused_framing = True

    @staticmethod
    def auto_picks_hip(device, sl_len, dtype, lengths):
        """engine='auto' takes the fp32 HIP engine for fp32 on a GPU at the
        fused slice length when every band length is one the engine runs
        (32..2048, as the reference's factored engine); otherwise the torch
        engine, which computes in the requested precision and takes any
        layout, as the reference's OctCQT does."""
        from .tables import BAND_LENGTHS
        return (torch.device(device).type == "cuda" and sl_len == 65536 and dtype == torch.float32
                and all(M in BAND_LENGTHS for M in lengths))

    # ------------------------------------------------------------ latency

    def latency_ms(self, sl_len=None):
        """Algorithmic latency of the scheme: one full slice."""
        return 1000.0 * (sl_len if sl_len is not None else self.sl_len) / self.fs

    def lowest_fmin(self, sl_len=None):
        """Lowest analysis frequency a slice of sl_len samples still holds a
        full window for. A window at frequency f spans 8 fs Q / f samples, so
        f >= 8 fs Q / sl_len, where Q is the quality factor of the lowest bin
        group: that group spans its n octaves plus the dropped one below in
        (n + 1) b - 1 geometric steps of ratio r, and Q = sqrt(r) / (r - 1) / 2."""
        sl = self.sl_len if sl_len is None else sl_len
        b = self.oct_bins[0]
        n = next((i for i, v in enumerate(self.oct_bins) if v != b), len(self.oct_bins))
        r = 2.0 ** ((n + 1) / ((n + 1) * b - 1))
        return 8.0 * self.fs * (math.sqrt(r) / (r - 1.0) / 2.0) / sl

    def latency_table(self, sl_lens=(8192, 16384, 32768, 65536, 131072)):
        need = float(self.frqs_hz[0])
        lines = [f"{'sl_len':>8} {'latency_ms':>11} {'lowest_fmin_hz':>15}   covers fmin {need:.1f} hz"]
        for sl in sl_lens:
            fmin = self.lowest_fmin(sl)
            lines.append(f"{sl:>8} {self.latency_ms(sl):>11.1f} {fmin:>15.1f}   "
                         f"{'yes' if fmin <= need else 'no'}")
        return "\n".join(lines)

    # ------------------------------------------------------------ slicing
    # Host framing, written the way the sliced kernels read: index maps, not
    # pad / unfold / roll. Slice g of a signal holds x[2H (g - 1) + jj] tw[jj]
    # at position j, with jj = (j + H) mod N for even g and (j - H) mod N for
    # odd g and zero outside the signal; the inverse un-rolls with the same
    # maps and overlap-adds half slices. The values are the reference
    # framing's bit for bit (sliced.py:106-166): every sample is one product
    # x * tw, every overlap one sum of two half slices.

    def _num_slices(self, L):
        quarters = -(-L // self.H)
        return (quarters + 1) // 2 + 1

    def _frame_maps(self, L, S, first, origin, device):
        """(signal index clamped into [0, L), in-signal mask, window index jj),
        each [S, N], for slices first .. first + S - 1 of a signal held from
        sample `origin` on. Cached by what they depend on (the parity of
        first and the start of slice `first` relative to the buffer)."""
        N, H = self.sl_len, self.H
        c0 = 2 * H * (first - 1) - origin
        key = (L, S, first & 1, c0, str(device))
        cache = self.__dict__.setdefault("_frame_cache", {})
        if key not in cache:
            if len(cache) >= 8:                 # a few signal lengths at a time (24 B per map entry)
                cache.pop(next(iter(cache)))
            g = torch.arange(first & 1, (first & 1) + S, device=device).view(-1, 1)
            j = torch.arange(N, device=device).view(1, -1)
            jj = (j + torch.where(g % 2 == 0, H, N - H)) % N
            i = c0 + 2 * H * (g - (first & 1)) + jj
            cache[key] = (i.clamp(0, L - 1), (i >= 0) & (i < L), jj)
        return cache[key]

    def _slice(self, x, first=0, origin=0, S=None):
        """[B, C, L] -> windowed, rolled slices [B, C, S, sl_len] (slices
        first .. first + S - 1; x starts at signal sample `origin`)."""
        L = x.shape[-1]
        S = self._num_slices(L) if S is None else S
        idx, inside, jj = self._frame_maps(L, S, first, origin, x.device)
        taps = torch.where(inside, x[..., idx], x.new_zeros(()))
        return taps * self.tw[jj]

    def _quarter_roll(self, blocks, first, fwd):
        """Octave blocks [..., S, bins, M] between transform order and the
        layout fwd returns: transform output m of slice g sits at
        (m + M/4) mod M for even g and (m - M/4) mod M for odd g (fwd=True
        applies that, fwd=False undoes it). Side blocks are not rolled."""
        out = []
        for c in blocks:
            S, M = c.shape[-3], c.shape[-1]
            g = torch.arange(first, first + S, device=c.device).view(-1, 1, 1)
            shift = torch.where(g % 2 == 0, M // 4, M - M // 4)
            m = torch.arange(M, device=c.device).view(1, 1, -1)
            src = (m - shift) % M if fwd else (m + shift) % M
            out.append(torch.take_along_dim(c, src.view((1,) * (c.dim() - 3) + tuple(src.shape)), dim=-1))
        return out

    def _unroll_slices(self, y, first):
        """Inverse slices [..., S, N] back from the quarter roll: even g by +H,
        odd g by -H (position j takes y[(j -+ H) mod N])."""
        N, H = self.sl_len, self.H
        S = y.shape[-2]
        g = torch.arange(first, first + S, device=y.device).view(-1, 1)
        j = torch.arange(N, device=y.device).view(1, -1)
        src = (j + torch.where(g % 2 == 0, N - H, H)) % N
        return torch.take_along_dim(y, src.view((1,) * (y.dim() - 2) + tuple(src.shape)), dim=-1)

    # ------------------------------------------- fused framing (HIP engine)

    def _fused(self, *tensors):
        """The HIP engine when the framing can run inside it: enabled, engine
        is TrainableCQT, inputs on its GPU, and no gradient is being recorded."""
        if not self.fused_framing:
            return None
        f = getattr(self.cqt, "f", None)
        if type(self.cqt).__name__ != "TrainableCQT" or f is None:
            return None
        ts = [t for t in tensors if t is not None]
        if any(t.device != f.dev for t in ts):
            return None
        if torch.is_grad_enabled() and any(t.requires_grad for t in ts):
            return None
        return f

    def _caches(self, f):
        """Caches of engine f (its buffer set; raw pointers and streamed view
        arguments); swapping self.cqt drops the old ones (the slot buffer F
        belongs to one engine's scatter table, view arguments to its layout)."""
        if self.__dict__.get("_cache_owner") is not f:
            self.__dict__.update(_cache_owner=f, _fused_ws={}, _stream_ptr_cache={})
        return self.__dict__["_fused_ws"], self.__dict__["_stream_ptr_cache"]

    def _ws(self, f, nsig, S, y=False, x="chunk"):
        """Engine buffers for nsig * S slice rows: W and F, the spectrum X
        (x="chunk": the whole-signal analysis, which from 256 slices on runs
        in chunks of 128 slices through the same leading rows, so X holds
        sliced_analysis_rows rows; x="full": one row per slice, the streamed
        analysis; x=False: none), and with y=True (the streamed synthesis) a
        slice buffer Y; the whole-signal synthesis overlap-adds inside its
        row pass and needs neither X nor Y. There is one
        buffer set per engine, sized to the largest row count seen so far
        (X and Y to the largest that asked for them); a smaller call uses
        leading rows. Rows are independent, and F is only ever used with the
        synthesis scatter table, so the slots that table never writes stay
        zero in every row (F is zeroed when allocated). Memory is therefore
        bounded by the largest call, whatever the signal lengths.

        A set (or an X or Y) that served a call under stream capture
        (hipGraph) stays allocated after a larger one replaces it: the
        recorded launches hold its addresses and write into it on every
        replay."""
        from .fused import sliced_analysis_rows
        cache, ptrs = self._caches(f)
        B = nsig * S
        full = cache.get("rows")
        if full is None or full["B"] < B:
            from . import tables as T
            from .fused import slot_buffer
            dev = f.dev
            if full is not None and full["captured"]:
                cache.setdefault("recorded", []).append(full)
            ptrs.clear()                 # cached raw pointers refer to the old buffers
            cache["rows"] = full = dict(B=B, captured=False, W=torch.empty(B, T.L, 2, device=dev),
                                        F=slot_buffer(B, dev))
        xr = B if x == "full" else sliced_analysis_rows(B)
        if x and ("X" not in full or full["X"].shape[0] < xr):
            from . import tables as T
            if "X" in full and full["captured"]:
                cache.setdefault("recorded", []).append({"X": full["X"]})
            ptrs.clear()
            full["X"] = torch.empty(xr, T.XSTRIDE, 2, device=f.dev)
        if y and ("Y" not in full or full["Y"].shape[0] < B):
            if "Y" in full and full["captured"]:
                cache.setdefault("recorded", []).append({"Y": full["Y"]})
            ptrs.clear()
            full["Y"] = torch.empty(B, self.sl_len, device=f.dev)
        if torch.cuda.is_current_stream_capturing():
            full["captured"] = True
        out = {"W": full["W"][:B], "F": full["F"][:B]}
        if x:
            out["X"] = full["X"][:xr]
        if y:
            out["Y"] = full["Y"][:B]
        return out

    def _tw32(self):
        tw = self.__dict__.get("_tw32_cache")
        if tw is None:
            tw = self.__dict__["_tw32_cache"] = self.tw.to(torch.float32).contiguous()
        return tw

    def _fwd_fused(self, f, x):
        B, C, L = x.shape
        S = self._num_slices(L)
        nsig = B * C
        sig = x.reshape(nsig, L).to(torch.float32).contiguous()
        ws = self._ws(f, nsig, S)
        coef = torch.empty(nsig * S * f.ncoef, dtype=torch.complex64, device=f.dev)
        f.sliced_analysis(sig, self._tw32(), S, coef, ws["X"], ws["W"])
        ng = len(self.oct_bins)
        blocks, side = [], []
        for gi, (b, M, off) in enumerate(f.gspec):
            v = coef[nsig * S * off:nsig * S * (off + b * M)]
            if gi < ng:
                blocks.append(v.view(B, C, b, S * M))
            else:
                side.append(v.view(B, C, S, b, M))
        return blocks, side

    def _block_buffer(self, f, blocks, side, nsig, S):
        """One complex64 buffer in the fused block layout: the blocks' own
        storage when they are the views the fused forward returned (views of
        one buffer at the group offsets), else a copy."""
        parts = list(blocks) + (list(side) if side is not None else [])
        base = parts[0]._base
        if side is not None and base is not None and base.dim() == 1 and base.dtype == torch.complex64 \
                and base.numel() == nsig * S * f.ncoef and base.device == f.dev and base.is_contiguous():
            ptr = base.data_ptr()
            if all(p._base is base and p.is_contiguous() and p.data_ptr() == ptr + 8 * nsig * S * off
                   for p, (_, _, off) in zip(parts, f.gspec)):
                return base
        coef = torch.zeros(nsig * S * f.ncoef, dtype=torch.complex64, device=f.dev)
        for p, (b, M, off) in zip(parts, f.gspec):
            coef[nsig * S * off:nsig * S * (off + b * M)] = p.reshape(-1).to(torch.complex64)
        return coef

    def _bwd_fused(self, f, blocks, side, length):
        B, C = blocks[0].shape[:2]
        S = blocks[0].shape[-1] // self.size_per_oct[0]
        nsig = B * C
        coef = self._block_buffer(f, blocks, side, nsig, S)
        n = S * 2 * self.H if length is None else min(int(length), S * 2 * self.H)
        out = torch.empty(B, C, n, dtype=torch.float32, device=f.dev)
        if nsig * S >= FUSED_OLA_MIN_SLICES:
            # scatter, inverse passes and the overlap-add (in the row pass's
            # store) in one call; no slice buffer
            ws = self._ws(f, nsig, S, x=False)
            f.sliced_synthesis(coef, ws["F"], ws["W"], out, nsig, S, n)
        else:
            ws = self._ws(f, nsig, S, y=True, x=False)
            f.scatter_bands_sliced(coef, ws["F"], nsig, S)
            f.packed_ifft(ws["F"], ws["Y"], ws["W"])
            f.overlap_add(ws["Y"], out, nsig, S, n)
        return out

    # --------------------------------------------------- whole buffer api

    def fwd(self, x):
        """x [B, C, L] -> (blocks, side): blocks[i] [B, C, oct_bins[i], S*size_per_oct[i]]
        in time order along the last axis, side (dc, nyq) per slice [B, C, S, 1, M]."""
        f = self._fused(x)
        if f is not None:
            return self._fwd_fused(f, x)
        B, C, _ = x.shape
        sl = self._slice(x)
        S = sl.shape[2]
        blocks, side = self.cqt.fwd(sl)
        blocks = self._quarter_roll(blocks, 0, fwd=True)
        # [B, C, S, bins, M] -> [B, C, bins, S M]: slices in time order per band
        blocks = [c.transpose(2, 3).reshape(B, C, b, S * m)
                  for c, b, m in zip(blocks, self.oct_bins, self.size_per_oct)]
        return blocks, side

    def bwd(self, blocks, side=None, length=None):
        """Inverse of fwd; length trims the tail padding."""
        f = self._fused(*blocks, *(side if side is not None else []))
        if f is not None:
            return self._bwd_fused(f, blocks, side, length)
        B, C = blocks[0].shape[:2]
        S = blocks[0].shape[-1] // self.size_per_oct[0]
        blocks = [c.reshape(B, C, b, S, m).transpose(2, 3)
                  for c, b, m in zip(blocks, self.oct_bins, self.size_per_oct)]
        blocks = self._quarter_roll(blocks, 0, fwd=False)
        y = self._unroll_slices(self.cqt.bwd(blocks, side), 0)
        # output hop t (2H samples, from signal sample 2H (t - 1)) is the first
        # half of slice t plus the second half of slice t - 1; hop 0 lies in
        # the leading padding and is dropped
        hops = y.reshape(B, C, S, 2, 2 * self.H)
        pad = torch.nn.functional.pad
        out = (pad(hops[..., 0, :], (0, 0, 0, 1)) + pad(hops[..., 1, :], (0, 0, 1, 0)))[..., 1:, :]
        out = out.reshape(B, C, S * 2 * self.H)
        return out[..., :length] if length is not None else out

    # --------------------------------------------- streaming, bounded state
    # With the HIP engine each streamed slice k is one fused call: the slice
    # is framed from [previous chunk, chunk] by the column pass (first = k,
    # origin = hop (k - 1)), its coefficients are stored straight into the
    # per-slice block layout, and the inverse rolls and overlap-adds in one
    # kernel that carries the half-slice tail. Same values as the host
    # framing below, which runs when the engine cannot (autograd, torch engine).

    def _stream_ptrs(self, f, nsig):
        """Raw pointers of the one-slice buffers for nsig signals (the engine's
        own, sized at allocation), so a streamed step is two C-ABI calls."""
        bufs, cache = self._caches(f)
        st = cache.get(nsig)
        if st is None:
            st = {k: v.data_ptr() for k, v in self._ws(f, nsig, 1, y=True, x="full").items()}
            st["tw"] = self._tw32().data_ptr()
            cache[nsig] = st
        elif torch.cuda.is_current_stream_capturing():
            bufs["rows"]["captured"] = True      # recorded launches keep these addresses
        return st

    @staticmethod
    def _rows(t):
        """A [B, C, n] chunk as nsig = B C fp32 rows with one row stride: the
        tensor itself when it already is (e.g. a view into a longer signal),
        else a contiguous fp32 copy. Returns (tensor, row stride in floats)."""
        if t.dtype != torch.float32:
            t = t.float()
        B, C, n = t.shape
        s0, s1, s2 = t.stride()
        if s2 == 1:
            if B * C == 1:
                return t, n
            rs = s0 if C == 1 else s1
            if (B == 1 or s0 == C * s1) and rs >= n:
                return t, rs
        return t.contiguous(), n

    def _stream_slice_fused(self, f, prev, chunk, k):
        B, C, hop = chunk.shape
        nsig = B * C
        # the slice's samples are [prev row, chunk row]: one call reads both
        # halves in place (no concatenated copy), frames, transforms and routes
        pv, ps = self._rows(prev)
        cv, cs = self._rows(chunk)
        st = self._stream_ptrs(f, nsig)
        coef = torch.empty(nsig * f.ncoef, dtype=torch.complex64, device=f.dev)
        _native.check(f.lib.fcqt_stream_analysis(f._ct, f._tp["route"], f._tp["slice_groups"], pv.data_ptr(), ps,
                                                 cv.data_ptr(), cs, st["tw"], nsig, k, coef.data_ptr(), st["X"],
                                                 st["W"], _native.stream_handle(f.dev.index)), "stream_analysis")
        views = self._stream_mark(f, [coef.as_strided(*a) for a in self._stream_view_args(f, B, C)])
        ng = len(self.oct_bins)
        return views[:ng], views[ng:]

    @staticmethod
    def _stream_mark(f, views):
        """Mark one streamed slice's views so that stream_bwd recognises
        these exact objects (weak references to the engine and to every view:
        a freed object's address reused by another never matches) and reads
        their buffer in place without re-checking them."""
        views[0]._fcqt_stream = (weakref.ref(f), tuple(weakref.ref(v) for v in views))
        return views

    def _stream_view_args(self, f, B, C):
        """as_strided arguments of one streamed slice's group views
        [B, C, bins, M] into its coefficient buffer (cached per B, C with the
        engine's other per-engine caches, which a new engine replaces)."""
        cache = self._caches(f)[1]
        key = ("views", B, C)
        args = cache.get(key)
        if args is None:
            nsig = B * C
            args = cache[key] = [((B, C, b, M), (C * b * M, b * M, M, 1), nsig * off) for b, M, off in f.gspec]
        return args

    def _stream_buffer(self, blocks, side):
        """(engine, coefficient buffer) when blocks + side are exactly the
        views the fused stream_fwd returned for one slice (same objects, no
        gradient to record), else None."""
        rec = getattr(blocks[0], "_fcqt_stream", None)
        if rec is None or side is None:
            return None
        f = getattr(self.cqt, "f", None)
        if f is None or rec[0]() is not f or not self.fused_framing:
            return None
        parts = tuple(blocks) + tuple(side)
        if len(parts) != len(rec[1]) or any(r() is not p for p, r in zip(parts, rec[1])):
            return None
        if torch.is_grad_enabled() and blocks[0].requires_grad:
            return None
        return f, blocks[0]._base

    def _stream_slice_host(self, prev, chunk, k):
        hop = chunk.shape[-1]
        sl = self._slice(torch.cat([prev, chunk], dim=-1), first=k, origin=hop * (k - 1), S=1)
        blocks, side = self.cqt.fwd(sl)
        blocks = self._quarter_roll(blocks, k, fwd=True)
        return [c[:, :, 0] for c in blocks], [c[:, :, 0] for c in side]

    def stream_fwd(self, chunks):
        """chunks yields [B, C, hop] pieces (pad the last one); yields one
        (blocks, side) per slice, blocks[i] [B, C, oct_bins[i], M_i].
        State: one half slice of input."""
        prev = None
        k = 0

        def one(prev, chunk, k):
            # the fused step reads hop samples of every row of both pieces:
            # only when the carried piece has the chunk's own [B, C, hop]
            # shape (a short or differently shaped piece takes the host path)
            f = self._fused(prev, chunk)
            if f is not None and chunk.dim() == 3 and chunk.shape[-1] == self.hop and prev.shape == chunk.shape:
                return self._stream_slice_fused(f, prev, chunk, k)
            return self._stream_slice_host(prev, chunk, k)

        for chunk in chunks:
            if prev is None:
                prev = torch.zeros_like(chunk)
            yield one(prev, chunk, k)
            prev = chunk
            k += 1
        yield one(prev, torch.zeros_like(prev), k)

    def stream_bwd(self, slice_coeffs):
        """slice_coeffs yields (blocks, side) as stream_fwd emits; yields
        [B, C, hop] output pieces one slice behind. State: one half slice
        (the rolled second half of the last inverse slice)."""
        tail = None
        k = 0
        for blocks, side in slice_coeffs:
            own = self._stream_buffer(blocks, side)
            f = own[0] if own is not None else self._fused(*blocks, *(side if side is not None else []))
            B, C = blocks[0].shape[:2]
            if f is not None:
                nsig = B * C
                if tail is None:
                    tail = torch.zeros(B, C, self.hop, dtype=torch.float32, device=f.dev)
                elif tail.shape != (B, C, self.hop):
                    raise ValueError(f"stream_bwd: slice {k} has {B} x {C} signals, the stream started with "
                                     f"{tail.shape[0]} x {tail.shape[1]}")
                elif not (tail.is_contiguous() and tail.dtype == torch.float32 and tail.device == f.dev):
                    tail = tail.to(device=f.dev, dtype=torch.float32).contiguous()
                coef = own[1] if own is not None else self._block_buffer(f, blocks, side, nsig, 1)
                st = self._stream_ptrs(f, nsig)
                out = torch.empty(B, C, self.hop, dtype=torch.float32, device=f.dev) if k > 0 else None
                # scatter, inverse passes and the half-slice overlap-add in one call
                _native.check(f.lib.fcqt_stream_synthesis(f._ct, f._tp["scat"], f._tp["slice_groups"],
                                                          f._tp["ovf_scat"], coef.data_ptr(), st["F"], st["W"],
                                                          st["Y"], tail.data_ptr(),
                                                          out.data_ptr() if out is not None else None, nsig, k,
                                                          _native.stream_handle(f.dev.index)), "stream_synthesis")
                if out is not None:
                    yield out
                k += 1
                continue
            blocks = self._quarter_roll([c.unsqueeze(2) for c in blocks], k, fwd=False)
            side = [c.unsqueeze(2) for c in side] if side is not None else None
            y = self._unroll_slices(self.cqt.bwd(blocks, side), k)[:, :, 0]
            if k > 0:
                yield tail + y[..., :self.hop]
            tail = y[..., self.hop:]
            k += 1
