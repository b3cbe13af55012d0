"""FusedOctCQT: the factored CQT engine on hand-written HIP kernels (gfx950).

Same surface as the reference's FusedOctCQT (fused.py:226-243, 787-801,
918-1080): construct from an OctCQT, then
    KR, KI = f.fwd(x)      # x [B, 65536] fp32 -> coefficient planes [B, ncoef]
    XO     = f.bwd(KR, KI) # -> [B, 65536]
Outputs are views of the engine's workspace, reused by the next call (the
reference reuses them per batch size); clone them to keep results. Graph capture (Graphed or
torch.cuda.graph, i.e. hipGraph) records the launches as they are.

Pipeline (all launches on the current stream, no host sync, no allocation
after the first call at the largest batch size so far):
  analysis   column pass -> row pass (untangle: X = rfft(x))
             -> windowed band gathers + band IDFT              (3 kernels)
  synthesis  band DFT + slot scatter -> column pass (slot sum, retangle)
             -> row pass (unpack)                              (3 kernels)
No result is accumulated with atomics (every output value has one writer):
every result is bitwise reproducible.
Table semantics follow fused.py:303-476; see flash_cqt/tables.py.
"""
import numpy as np
import torch

from . import _native
from . import tables as T

N = T.N
HALF = N // 2
L = T.L


def _np_groups(cqt):
    """numpy (idx, gv, pos, gdv, conj) per group, octave groups then side."""
    if hasattr(cqt, "np_groups"):
        return list(cqt.np_groups) + list(cqt.np_side_groups)
    out = []
    for idx, gv, pos, gdv, conj in list(cqt.groups) + list(cqt.side_groups):
        out.append((idx.cpu().numpy(), gv.cpu().float().numpy(), pos.cpu().numpy(),
                    gdv.cpu().float().numpy(), conj.cpu().numpy()))
    return out


SKEW = 4096      # floats (16 KiB): KR-to-KI plane gap, and offset of F into its allocation

ANALYSIS_CHUNK, ANALYSIS_CHUNK_MIN_BATCH = 128, 256     # FCQT_ANALYSIS_CHUNK, FCQT_ANALYSIS_CHUNK_MIN_BATCH


def sliced_analysis_rows(batch):
    """FCQT_SLICED_ANALYSIS_ROWS: the rows of xs and work a whole-signal
    sliced analysis of `batch` slices uses (its chunks reuse the leading
    128 rows from 256 slices on)."""
    return batch if batch < ANALYSIS_CHUNK_MIN_BATCH else ANALYSIS_CHUNK


def slot_buffer(B, dev):
    """A zeroed F buffer [B, FROW, 2] that starts SKEW floats into its
    allocation. Large allocations start 2 MiB-aligned, and an F there
    measured slower: the scatter's stores and the inverse column pass's
    paired plane loads (F[bin], F[FSTRIDE + bin]) took 0.5-1.5 us longer at
    batch 64 than with any base offset from 512 bytes on."""
    n = B * T.FROW * 2
    return torch.zeros(n + SKEW, dtype=torch.float32, device=dev)[SKEW:].view(B, T.FROW, 2)


class FusedOctCQT:
    """Kernel tables, workspaces and launchers for one OctCQT at audio_len 65536."""

    def __init__(self, cqt, device=None):
        assert cqt.nn == N, "fused path is built for sl_len 65536"
        groups = _np_groups(cqt)
        bad = sorted({g[0].shape[1] for g in groups} - set(T.BAND_LENGTHS))
        if bad:
            # the reference's factored engine has no stages for them either
            # (fused.py:274-299: roots rmr[::M // 32], radix factors up to 2048)
            raise ValueError(f"band lengths {bad} of this layout are outside the engine's "
                             f"{T.BAND_LENGTHS[0]}..{T.BAND_LENGTHS[-1]}")
        dev = torch.device(device) if device is not None else torch.device(cqt.device)
        if dev.type != "cuda":
            raise ValueError("FusedOctCQT runs on a GPU (device 'cuda')")
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.dev = dev
        self.cqt = cqt
        self.lib = _native.load()

        built = T.build(groups, noct=len(cqt.groups))
        self.gspec = built["gspec"]
        self.ncoef = built["ncoef"]
        # the tables go to the device as one table image through the C ABI's
        # checked upload (fcqt_tables_upload validates every record against
        # the kernels' bounds on the host first), into one device buffer
        image = T.image_bytes(built)
        info = _native.ImageInfo()
        _native.check(self.lib.fcqt_image_check(image, len(image), info), "image_check")
        with torch.cuda.device(dev):
            self._table_mem = torch.empty(info.device_bytes, dtype=torch.uint8, device=dev)
            up = _native.EngineTables()
            _native.check(self.lib.fcqt_tables_upload(image, len(image), self._table_mem.data_ptr(), info.device_bytes,
                                                      _native.stream_handle(dev.index), up), "tables_upload")
        self._up = up
        self._ct = up.tab
        assert self._ct.ncoef == self.ncoef and self._ct.coef_span == built["coef_span"]
        # per-table tensor views of the uploaded image (same device memory)
        self.tables = {}
        for _, (name, dt) in T.IMAGE_SECTIONS.items():
            if name == "ncoef":
                continue
            ptr = getattr(up, name) if hasattr(up, name) else getattr(up.tab, name)
            a = np.asarray(built[name], dtype=dt)
            off = ptr - self._table_mem.data_ptr()
            tdt = torch.float32 if dt == np.float32 else torch.int32
            self.tables[name] = self._table_mem[off:off + a.nbytes].view(tdt).view(a.shape)
        # table bytes per direction (batch invariant, L2/MALL resident at batch)
        self.table_bytes = {k: v.numel() * v.element_size() for k, v in self.tables.items()}
        self._tp = {k: v.data_ptr() for k, v in self.tables.items()}
        # the reference exposes its band-engine tables as .radix (fused.py:430);
        # here the same name holds this engine's tables (formats in tables.py)
        self.radix = self.tables
        self._full = None      # the one buffer set (see _workspace)
        self._recorded = []    # sets a captured graph still uses
        self._ws = {}          # batch size -> views of the set's leading rows
        self._wp = {}          # batch size -> their raw pointers

    # ------------------------------------------------------------ buffers

    def _workspace(self, B):
        """The buffers of fwd/bwd for batch B: X, W, F (the synthesis scatter
        buffer, zeroed once: the slots its table never writes must stay
        zero), the coefficient planes KR / KI and the output XO, plus FA
        (fa_buffer) and SYNC (sync_buffer) once those have been asked for.

        There is one buffer set per engine, sized to the largest batch seen
        so far; a smaller call gets views of its leading rows. Rows are
        independent and each F buffer is only ever used with its own scatter
        table, so the slots that table never writes stay zero in every row,
        and a successful single-launch call leaves its sync words at zero:
        the leading rows are valid for every smaller batch. Memory is
        therefore bounded by the largest call (the reference keeps one set
        per batch size, trainable.py:65-73). The returned views are
        overwritten by the next call of any batch size.

        A set that served a call under stream capture (hipGraph) stays
        allocated when a larger one replaces it: the recorded launches hold
        its addresses and use them on every replay."""
        full = self._full
        if full is None or full["B"] < B:
            if full is not None and full["captured"]:
                self._recorded.append(full)
            self._ws.clear()
            self._wp.clear()
            self._full = full = None       # release the old set before allocating the new one
            with torch.cuda.device(self.dev):
                e = lambda *s: torch.empty(*s, dtype=torch.float32, device=self.dev)
                z = lambda *s: torch.zeros(*s, dtype=torch.float32, device=self.dev)
                # both coefficient planes in one allocation, KI starting
                # SKEW floats past the end of KR: the band kernels
                # store (load) KR[i] and KI[i] together, and with KI right at
                # the end of a 2 MiB-aligned KR (how the caching allocator can
                # split one freed block between two plane tensors) both
                # streams met in the same memory channels and the route
                # kernel ran 10-12% slower
                n = B * self.ncoef
                planes = z(2 * n + SKEW)
                self._full = full = dict(B=B, captured=False, X=e(B, T.XSTRIDE, 2), W=e(B, L, 2),
                                         F=slot_buffer(B, self.dev), KR=planes[:n], KI=planes[n + SKEW:],
                                         XO=z(B, N))
        if B not in self._ws:
            nc = B * self.ncoef
            w = dict(X=full["X"][:B], W=full["W"][:B], F=full["F"][:B],
                     KR=full["KR"][:nc].view(B, self.ncoef), KI=full["KI"][:nc].view(B, self.ncoef),
                     XO=full["XO"][:B])
            if "FA" in full:
                w["FA"] = full["FA"][:B]
            if "SYNC" in full:
                w["SYNC"] = full["SYNC"][:_native.sync_words(B)]
            self._ws[B] = w
            self._wp[B] = {k: v.data_ptr() for k, v in w.items()}
        if torch.cuda.is_current_stream_capturing():
            full["captured"] = True
        return self._ws[B]

    def release_workspace(self):
        """Drop the engine's buffer set (a set recorded by a graph capture
        stays with the graph's engine); the next call allocates afresh."""
        if self._full is not None and self._full["captured"]:
            self._recorded.append(self._full)
        self._full = None
        self._ws.clear()
        self._wp.clear()

    def _add_full(self, name, make):
        """Add a lazily allocated buffer (FA, SYNC) to the current set and to
        every batch size's views of it."""
        full = self._full
        if name not in full:
            with torch.cuda.device(self.dev):
                full[name] = make(full["B"])
            for B, w in self._ws.items():
                w[name] = full[name][:B] if name != "SYNC" else full[name][:_native.sync_words(B)]
                self._wp[B][name] = w[name].data_ptr()

    def fa_buffer(self, B):
        """The analysis-adjoint scatter buffer for batch B, allocated and
        zeroed on first use (it belongs to the scat_a table only)."""
        self._workspace(B)
        self._add_full("FA", lambda n: slot_buffer(n, self.dev))
        return self._ws[B]["FA"]

    def sync_buffer(self, B):
        """Counters of the single-launch directions for batch B
        (FCQT_SYNC_WORDS(B) uint32: per-slice stage counts, then the error
        word, the exit count and the per-XCD queue claims), zeroed on first
        use; a call that succeeds returns every word to zero."""
        self._workspace(B)
        self._add_full("SYNC", lambda n: torch.zeros(_native.sync_words(n), dtype=torch.int32, device=self.dev))
        return self._ws[B]["SYNC"]

    def sync_error(self, B):
        """The single-launch error word for batch B: 0 when every call so far
        completed; bit 1: a stage wait outlasted its bound; bit 4: a queue
        was served by no workgroup (no workgroup ran on one of the XCDs).
        Reads device memory: synchronizes."""
        return int(self.sync_buffer(B)[B * _native.SYNC_PER_SLICE].item())

    def sync_reset(self, B):
        """After a nonzero error word: wait for the device, then zero the
        whole sync buffer (a failed call leaves its counters as they were)."""
        torch.cuda.synchronize(self.dev)
        self.sync_buffer(B)
        self._full["SYNC"].zero_()
        torch.cuda.synchronize(self.dev)

    def _persist_checked(self, B, what):
        err = self.sync_error(B)
        if err:
            self.sync_reset(B)
            raise _native.NativeError(f"{what}: single-launch error word {err} (1: a stage wait timed out, "
                                      f"4: an XCD's queue was not served); the results are not valid")

    def _fbuf(self, table, B):
        return self._workspace(B)["F"] if table == "scat" else self.fa_buffer(B)

    def _check_x(self, x):
        if x.dim() != 2 or x.shape[1] != N or x.shape[0] < 1:
            raise ValueError(f"x must be [B, {N}] with B >= 1, got {tuple(x.shape)}")
        _native.require_device(x, "x")
        if x.device != self.dev:
            raise ValueError(f"x is on {x.device}, engine on {self.dev}")

    # ------------------------------------------------- raw engine launches
    # Every launch validates its buffers first: device, contiguity, dtype and
    # byte size must match what the kernels index, so a wrong tensor raises
    # here instead of reaching the GPU.

    def _need(self, t, nbytes, name):
        if not torch.is_tensor(t):
            raise ValueError(f"{name} must be a tensor")
        if t.device != self.dev:
            raise ValueError(f"{name} is on {t.device}, engine on {self.dev}")
        if t.dtype not in (torch.float32, torch.complex64) or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous float32/complex64")
        if t.numel() * t.element_size() != nbytes:
            raise ValueError(f"{name} has {t.numel() * t.element_size()} bytes, expected {nbytes}")

    def _need_rows(self, t, rows, row_bytes, name):
        """As _need for a buffer of at least `rows` rows of row_bytes (the
        kernels use its leading rows)."""
        if not torch.is_tensor(t):
            raise ValueError(f"{name} must be a tensor")
        nb = t.numel() * t.element_size()
        if nb < rows * row_bytes or nb % row_bytes:
            raise ValueError(f"{name} has {nb} bytes, expected whole rows of {row_bytes} bytes, at least {rows}")
        self._need(t, nb, name)

    def _need_coef(self, re, im, layout, B, name):
        if layout == _native.PLANAR:
            self._need(re, B * self.ncoef * 4, name + "_re")
            self._need(im, B * self.ncoef * 4, name + "_im")
        elif layout == _native.INTERLEAVED:
            self._need(re, B * self.ncoef * 8, name)
        else:
            raise ValueError("layout must be PLANAR or INTERLEAVED")

    def _batch(self, t, per_row_bytes, name):
        B = t.shape[0] if t.dim() >= 1 else 0
        if B < 1:
            raise ValueError(f"{name} needs a leading batch dimension")
        self._need(t, B * per_row_bytes, name)
        return B

    def packed_fft(self, x, xs, work):
        """X = rfft(x) (bins 0..L) into xs [B, XSTRIDE, 2]."""
        B = self._batch(x, N * 4, "x")
        self._need(xs, B * T.XSTRIDE * 8, "xs")
        self._need(work, B * L * 8, "work")
        _native.check(self.lib.fcqt_packed_fft_fwd(self._ct, _native.ptr(x), _native.ptr(xs),
                                                   _native.ptr(work), B, _native.stream_handle(self.dev.index)),
                      "packed_fft_fwd")

    def route_bands(self, xs, out_re, out_im, layout, table="route"):
        B = self._batch(xs, T.XSTRIDE * 8, "xs")
        self._need_coef(out_re, out_im, layout, B, "out")
        _native.check(self.lib.fcqt_route_bands(self._ct, _native.ptr(self.tables[table]), _native.ptr(xs),
                                                _native.ptr(out_re), _native.ptr(out_im), layout, B,
                                                _native.stream_handle(self.dev.index)), "route_bands")

    def scatter_bands(self, c_re, c_im, layout, f, table="scat"):
        B = self._batch(f, T.FROW * 8, "f")
        self._need_coef(c_re, c_im, layout, B, "coef")
        _native.check(self.lib.fcqt_scatter_bands(self._ct, _native.ptr(self.tables[table]), _native.ptr(c_re),
                                                  _native.ptr(c_im), layout, _native.ptr(f), B,
                                                  _native.stream_handle(self.dev.index)), "scatter_bands")

    def packed_ifft(self, f, y, work, table="scat"):
        """y = irfft of the half spectrum held in f's slots (filled with `table`)."""
        B = self._batch(f, T.FROW * 8, "f")
        self._need(y, B * N * 4, "y")
        self._need(work, B * L * 8, "work")
        _native.check(self.lib.fcqt_packed_fft_inv(self._ct, _native.ptr(self.tables["ovf_" + table]),
                                                   _native.ptr(f), _native.ptr(y), _native.ptr(work),
                                                   B, _native.stream_handle(self.dev.index)), "packed_fft_inv")

    def analysis(self, x, out_re, out_im, layout, table="route"):
        """x [B, N] -> coefficients (planar planes or one interleaved buffer)."""
        B = self._batch(x, N * 4, "x")
        self._need_coef(out_re, out_im, layout, B, "out")
        w = self._workspace(B)
        _native.check(self.lib.fcqt_analysis(self._ct, _native.ptr(self.tables[table]), _native.ptr(x),
                                             _native.ptr(out_re), _native.ptr(out_im), layout,
                                             _native.ptr(w["X"]), _native.ptr(w["W"]), B,
                                             _native.stream_handle(self.dev.index)), "analysis")

    def synthesis(self, c_re, c_im, layout, y, table="scat"):
        """coefficients -> y [B, N] (table 'scat' synthesis, 'scat_a' analysis adjoint)."""
        B = self._batch(y, N * 4, "y")
        self._need_coef(c_re, c_im, layout, B, "coef")
        w = self._workspace(B)
        _native.check(self.lib.fcqt_synthesis(self._ct, _native.ptr(self.tables[table]),
                                              _native.ptr(self.tables["ovf_" + table]), _native.ptr(c_re),
                                              _native.ptr(c_im), layout, _native.ptr(self._fbuf(table, B)),
                                              _native.ptr(w["W"]), _native.ptr(y), B,
                                              _native.stream_handle(self.dev.index)), "synthesis")

    # ------------------------------------------- SlicedCQT framing

    def slice_fft(self, sig, window, nslices, xs, work, first=0, origin=0):
        """X of slices first .. first + nslices - 1 of the signals sig [nsig, len]
        (SlicedCQT framing: zero pad, 50% overlap, window, quarter roll);
        sig[:, 0] is signal sample `origin` (0 for a whole signal)."""
        if sig.dim() != 2 or sig.shape[1] < 1:
            raise ValueError("sig must be [nsig, len]")
        nsig, length = sig.shape
        self._need(sig, nsig * length * 4, "sig")
        self._need(window, N * 4, "window")
        B = nsig * nslices
        self._need(xs, B * T.XSTRIDE * 8, "xs")
        self._need(work, B * L * 8, "work")
        _native.check(self.lib.fcqt_slice_fft_fwd(self._ct, _native.ptr(sig), length, _native.ptr(window), nsig,
                                                  nslices, first, origin, _native.ptr(xs), _native.ptr(work),
                                                  _native.stream_handle(self.dev.index)), "slice_fft_fwd")

    def route_bands_sliced(self, xs, coef, nsig, nslices, table="route", first=0):
        """Coefficients of every slice into the SlicedCQT block layout
        (complex64, nsig * nslices * ncoef values); `first` is the signal
        index of the call's first slice (its parity sets the quarter roll)."""
        B = nsig * nslices
        self._need(xs, B * T.XSTRIDE * 8, "xs")
        self._need(coef, B * self.ncoef * 8, "coef")
        _native.check(self.lib.fcqt_route_bands_sliced(self._ct, _native.ptr(self.tables[table]),
                                                       _native.ptr(self.tables["slice_groups"]), _native.ptr(xs),
                                                       _native.ptr(coef), nsig, nslices, first,
                                                       _native.stream_handle(self.dev.index)), "route_bands_sliced")

    def sliced_analysis(self, sig, window, nslices, coef, xs, work, table="route"):
        """slice_fft then route_bands_sliced of whole signals sig [nsig, len]
        in one call (fcqt_sliced_analysis: from 256 slices on in chunks of
        about 128 slices, same bits). xs and work hold at least
        sliced_analysis_rows(nsig * nslices) rows: every row below 256
        slices, the 128 rows of one chunk from 256 on."""
        if sig.dim() != 2 or sig.shape[1] < 1:
            raise ValueError("sig must be [nsig, len]")
        nsig, length = sig.shape
        self._need(sig, nsig * length * 4, "sig")
        self._need(window, N * 4, "window")
        B = nsig * nslices
        rows = sliced_analysis_rows(B)
        self._need_rows(xs, rows, T.XSTRIDE * 8, "xs")
        self._need_rows(work, rows, L * 8, "work")
        self._need(coef, B * self.ncoef * 8, "coef")
        _native.check(self.lib.fcqt_sliced_analysis(self._ct, _native.ptr(self.tables[table]),
                                                    _native.ptr(self.tables["slice_groups"]), _native.ptr(sig), length,
                                                    _native.ptr(window), nsig, nslices, _native.ptr(coef),
                                                    _native.ptr(xs), _native.ptr(work),
                                                    _native.stream_handle(self.dev.index)), "sliced_analysis")

    def sliced_synthesis(self, coef, f, work, out, nsig, nslices, length, table="scat"):
        """scatter_bands_sliced, the inverse passes and overlap_add of whole
        signals in one call (fcqt_sliced_synthesis: the overlap-add happens
        in the inverse row pass's store, same bits): out [nsig, length]."""
        B = nsig * nslices
        self._need(coef, B * self.ncoef * 8, "coef")
        self._need(f, B * T.FROW * 8, "f")
        self._need(work, B * L * 8, "work")
        self._need(out, nsig * length * 4, "out")
        _native.check(self.lib.fcqt_sliced_synthesis(self._ct, _native.ptr(self.tables[table]),
                                                     _native.ptr(self.tables["slice_groups"]),
                                                     _native.ptr(self.tables["ovf_" + table]), _native.ptr(coef),
                                                     _native.ptr(f), _native.ptr(work), _native.ptr(out), nsig,
                                                     nslices, length, _native.stream_handle(self.dev.index)),
                      "sliced_synthesis")

    def scatter_bands_sliced(self, coef, f, nsig, nslices, table="scat", first=0):
        B = nsig * nslices
        self._need(coef, B * self.ncoef * 8, "coef")
        self._need(f, B * T.FROW * 8, "f")
        _native.check(self.lib.fcqt_scatter_bands_sliced(self._ct, _native.ptr(self.tables[table]),
                                                         _native.ptr(self.tables["slice_groups"]),
                                                         _native.ptr(coef), _native.ptr(f), nsig, nslices, first,
                                                         _native.stream_handle(self.dev.index)), "scatter_bands_sliced")

    def stream_overlap(self, y, tail, out, nsig, slice_index):
        """One streamed slice's half-slice overlap-add: out = tail + y rolled
        back (first half), tail = its second half; out unused for slice 0."""
        self._need(y, nsig * N * 4, "y")
        self._need(tail, nsig * HALF * 4, "tail")
        if slice_index > 0:
            self._need(out, nsig * HALF * 4, "out")
        _native.check(self.lib.fcqt_stream_overlap(_native.ptr(y), _native.ptr(tail),
                                                   _native.ptr(out if slice_index > 0 else None), nsig, slice_index,
                                                   _native.stream_handle(self.dev.index)), "stream_overlap")

    def overlap_add(self, y, out, nsig, nslices, length):
        self._need(y, nsig * nslices * N * 4, "y")
        self._need(out, nsig * length * 4, "out")
        _native.check(self.lib.fcqt_overlap_add(_native.ptr(y), _native.ptr(out), nsig, nslices, length,
                                                _native.stream_handle(self.dev.index)), "overlap_add")

    # ------------------------------------------------- reference surface

    # fwd/bwd check only the caller's tensors: the workspace buffers and
    # tables are the engine's own, sized at allocation, so the pointers of
    # each batch size's views are cached and passed as they are (host cost
    # per call is then about that of the kernel launches themselves).

    def fwd(self, x):
        """x [B, 65536] fp32 -> (KR, KI) [B, ncoef], workspace views."""
        self._check_x(x)
        B = x.shape[0]
        w = self._workspace(B)
        p = self._wp[B]
        _native.check(self.lib.fcqt_analysis(self._ct, self._tp["route"], x.data_ptr(), p["KR"], p["KI"],
                                             _native.PLANAR, p["X"], p["W"], B,
                                             _native.stream_handle(self.dev.index)), "analysis")
        return w["KR"], w["KI"]

    def bwd(self, KR, KI):
        """(KR, KI) [B, ncoef] -> XO [B, 65536], a workspace view."""
        B = KR.shape[0] if KR.dim() else 0
        if B < 1 or KR.shape != (B, self.ncoef) or KI.shape != (B, self.ncoef):
            raise ValueError(f"KR, KI must be [B, {self.ncoef}]")
        _native.require_device(KR, "KR")
        _native.require_device(KI, "KI")
        if KR.device != self.dev or KI.device != self.dev:
            raise ValueError(f"KR, KI must be on {self.dev}")
        w = self._workspace(B)
        p = self._wp[B]
        _native.check(self.lib.fcqt_synthesis(self._ct, self._tp["scat"], self._tp["ovf_scat"], KR.data_ptr(),
                                              KI.data_ptr(), _native.PLANAR, p["F"], p["W"], p["XO"], B,
                                              _native.stream_handle(self.dev.index)), "synthesis")
        return w["XO"]

    def blocks_view(self, KR, KI):
        """Complex per-group blocks [B, bins, M] built from the planes."""
        return [torch.complex(KR[:, off:off + b * M], KI[:, off:off + b * M]).view(-1, b, M)
                for b, M, off in self.gspec]

    # --------------------------------------- reference entry points kept

    def persist_fwd(self, x, check=True):
        """The reference's single-launch forward (fused.py:748-762,
        persist2.cu:140-161): the whole analysis as one launch
        (fcqt_persist_analysis: persistent workgroups take the column tiles,
        row tiles and band tasks of the slices of their own XCD from a
        queue, each task waiting for its slice's previous stage). Same
        outputs as fwd, bit for bit (workspace views).

        check=True reads the call's error word (one device synchronization)
        and raises NativeError, after zeroing the sync buffer, when it is
        nonzero. check=False leaves that to the caller (graph capture, or
        timing without host synchronizations): call sync_error(B) after the
        calls or replays and sync_reset(B) if it is nonzero."""
        self._check_x(x)
        B = x.shape[0]
        w = self._workspace(B)
        self.sync_buffer(B)
        p = self._wp[B]
        _native.check(self.lib.fcqt_persist_analysis(self._ct, self._tp["route"], x.data_ptr(), p["KR"], p["KI"],
                                                     _native.PLANAR, p["X"], p["W"], p["SYNC"], B,
                                                     _native.stream_handle(self.dev.index)), "persist_analysis")
        if check:
            self._persist_checked(B, "persist_analysis")
        return w["KR"], w["KI"]

    def persist_inv(self, KR, KI, check=True):
        """The reference's single-launch inverse (fused.py:764-778,
        persist2.cu:163-222): the whole synthesis as one launch
        (fcqt_persist_synthesis: band scatter tasks, inverse column tiles
        and inverse row tiles, as persist_fwd). Same output as bwd, bit for
        bit (a workspace view). check: as persist_fwd."""
        B = KR.shape[0] if KR.dim() else 0
        if B < 1 or KR.shape != (B, self.ncoef) or KI.shape != (B, self.ncoef):
            raise ValueError(f"KR, KI must be [B, {self.ncoef}]")
        _native.require_device(KR, "KR")
        _native.require_device(KI, "KI")
        if KR.device != self.dev or KI.device != self.dev:
            raise ValueError(f"KR, KI must be on {self.dev}")
        w = self._workspace(B)
        self.sync_buffer(B)
        p = self._wp[B]
        _native.check(self.lib.fcqt_persist_synthesis(self._ct, self._tp["scat"], self._tp["ovf_scat"],
                                                      KR.data_ptr(), KI.data_ptr(), _native.PLANAR, p["F"], p["W"],
                                                      p["XO"], p["SYNC"], B, _native.stream_handle(self.dev.index)),
                      "persist_synthesis")
        if check:
            self._persist_checked(B, "persist_synthesis")
        return w["XO"]

    def bench_parts(self, x, reps=50):
        """Median ms per engine part for input x [B, 65536], each part
        graph-captured and replayed (diagnosis, as the reference's
        bench_parts, fused.py:1082): the two forward FFT passes, the route
        + band IDFT kernel, the band DFT + scatter kernel, the two inverse
        FFT passes."""
        self._check_x(x)
        B = x.shape[0]
        w = self._workspace(B)
        self.bwd(*self.fwd(x))

        def med(fn):
            s = torch.cuda.Stream(self.dev)
            s.wait_stream(torch.cuda.current_stream(self.dev))
            with torch.cuda.stream(s):
                for _ in range(3):
                    fn()
            torch.cuda.current_stream(self.dev).wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn()
            ts = []
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            for _ in range(reps):
                a.record()
                g.replay()
                b.record()
                b.synchronize()
                ts.append(a.elapsed_time(b))
            ts.sort()
            return ts[len(ts) // 2]

        return [("fwd packed fft", med(lambda: self.packed_fft(x, w["X"], w["W"]))),
                ("fwd route + band idft", med(lambda: self.route_bands(w["X"], w["KR"], w["KI"], _native.PLANAR))),
                ("inv band dft + scatter", med(lambda: self.scatter_bands(w["KR"], w["KI"], _native.PLANAR, w["F"]))),
                ("inv packed ifft", med(lambda: self.packed_ifft(w["F"], w["XO"], w["W"])))]
