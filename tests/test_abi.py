"""C-ABI checks that need no GPU: the library loads, exports exactly what
include/flashcqt.h declares, and rejects bad arguments before any HIP call."""
import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "flashcqt.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(fcqt_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from flash_cqt import _native
    return _native.load()


def test_header_and_python_agree():
    from flash_cqt import _native
    assert declared() == sorted(_native.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared():
        assert hasattr(lib, name), name


def test_variant_library_exports_the_same_abi():
    """The cross-lane variant library (same sources, band units of M <= 256
    exchanging across lanes) loads with the library's C ABI: every declared
    symbol and the same ABI version (no GPU call)."""
    from flash_cqt import _native
    xl = _native.load_variant("xlane")
    for name in declared():
        assert hasattr(xl, name), name
    assert xl.fcqt_abi_version() == _native.ABI_VERSION
    with pytest.raises(_native.NativeError):
        _native.load_variant("nope")


def test_trace_build_exports_the_same_abi(lib):
    """The trace build (libflashcqt_flowtrace.so) loads with the library's C
    ABI; only it accepts a stage-trace buffer (host calls, no GPU): the
    library refuses one, the trace build refuses one too small and accepts
    one large enough and a null buffer (recording off)."""
    from flash_cqt import _native
    tr = _native.load_variant("flowtrace")
    for name in declared():
        assert hasattr(tr, name), name
    assert tr.fcqt_abi_version() == _native.ABI_VERSION
    need = 8 * 256 * 32 * 6 * 8
    assert lib.fcqt_persist_trace(ctypes.c_void_p(4096), need) == 1           # FCQT_EARG: no trace here
    assert tr.fcqt_persist_trace(ctypes.c_void_p(4096), need - 8) == 1        # too small
    assert tr.fcqt_persist_trace(ctypes.c_void_p(4096), need) == 0
    assert tr.fcqt_persist_trace(None, 0) == 0


def test_abi_version(lib):
    from flash_cqt import _native
    assert lib.fcqt_abi_version() == _native.ABI_VERSION == 13


def test_header_constants_match_tables_and_kernels():
    """The layout macros of flashcqt.h, the device constants of fcqt_fft.hpp
    and the table builder's constants are one set of numbers."""
    from flash_cqt import tables as T
    h = dict(re.findall(r"#define (FCQT_[A-Z_]+) (\d+)", HEADER.read_text()))
    k = dict(re.findall(r"constexpr int (k\w+) = ([^;]+);",
                        (ROOT / "flash-cqt_amd" / "csrc" / "fcqt_fft.hpp").read_text()))
    want = {"FCQT_N": T.N, "FCQT_L": T.L, "FCQT_FSTRIDE": T.FSTRIDE, "FCQT_OVF_CAP": T.OVF_CAP,
            "FCQT_FROW": T.FROW, "FCQT_OVF_LEN": T.INV_WGS * T.FOLD_PER_WG, "FCQT_XSTRIDE": T.XSTRIDE,
            "FCQT_TW_STAGE_LEN": T.TW_STAGE_LEN}
    for name, v in want.items():
        assert int(h[name]) == v, name
    assert int(k["kOvfCap"]) == T.OVF_CAP and int(k["kFoldPerWg"]) == T.FOLD_PER_WG
    assert k["kFRow"].replace(" ", "") == "2*kFStride+2*kOvfCap" and k["kFStride"].startswith("kL + ")
    assert T.FROW % 32 == 0          # F rows stay 256-byte aligned


def test_status_strings(lib):
    assert lib.fcqt_status_string(0) == b"ok"
    assert b"argument" in lib.fcqt_status_string(1)


def test_argument_errors_detected_before_any_launch(lib):
    from flash_cqt._native import Tables
    tab = Tables(tw_pass=16, tw_half=16, tw_stage=16, tasks=16, ntasks=1, ncoef=1, coef_span=1)
    bad = Tables(tw_pass=0, tw_half=0, tw_stage=0, tasks=0, ntasks=0, ncoef=0, coef_span=0)
    s = ctypes.c_void_p(0)
    p = ctypes.c_void_p(4096)
    odd = ctypes.c_void_p(4100)
    null = ctypes.c_void_p(0)
    EARG, EALIGN = 1, 2
    # null table descriptor / buffers / batch 0
    assert lib.fcqt_packed_fft_fwd(None, p, p, p, 1, s) == EARG
    assert lib.fcqt_packed_fft_fwd(ctypes.byref(tab), null, p, p, 1, s) == EARG
    assert lib.fcqt_packed_fft_fwd(ctypes.byref(tab), p, p, p, 0, s) == EARG
    assert lib.fcqt_packed_fft_fwd(ctypes.byref(bad), p, p, p, 1, s) == EARG
    # misaligned complex buffer
    assert lib.fcqt_packed_fft_fwd(ctypes.byref(tab), odd, p, p, 1, s) == EALIGN
    # bad layout, null im plane for planar
    assert lib.fcqt_route_bands(ctypes.byref(tab), p, p, p, p, 7, 1, s) == EARG
    assert lib.fcqt_route_bands(ctypes.byref(tab), p, p, p, null, 0, 1, s) == EARG
    assert lib.fcqt_route_bands(ctypes.byref(tab), ctypes.c_void_p(4098), p, p, p, 0, 1, s) == EALIGN
    assert lib.fcqt_route_bands(ctypes.byref(bad), p, p, p, p, 0, 1, s) == EARG
    assert lib.fcqt_scatter_bands(ctypes.byref(tab), p, p, p, 0, null, 1, s) == EARG
    assert lib.fcqt_packed_fft_inv(ctypes.byref(tab), p, p, p, p, -3, s) == EARG
    assert lib.fcqt_packed_fft_inv(ctypes.byref(tab), null, p, p, p, 1, s) == EARG
    assert lib.fcqt_analysis(ctypes.byref(tab), null, p, p, p, 0, p, p, 1, s) == EARG
    assert lib.fcqt_synthesis(ctypes.byref(tab), p, p, p, p, 0, odd, p, p, 1, s) == EALIGN
    assert lib.fcqt_synthesis(ctypes.byref(tab), p, null, p, p, 0, p, p, p, 1, s) == EARG
    assert lib.fcqt_fill_zero(null, 10, s) == EARG
    # sliced framing entry points
    assert lib.fcqt_slice_fft_fwd(ctypes.byref(tab), null, 100, p, 1, 1, 0, 0, p, p, s) == EARG
    assert lib.fcqt_slice_fft_fwd(ctypes.byref(tab), p, 100, p, 1, 0, 0, 0, p, p, s) == EARG
    assert lib.fcqt_slice_fft_fwd(ctypes.byref(tab), p, 100, p, 1, 1, -1, 0, p, p, s) == EARG   # negative first
    assert lib.fcqt_route_bands_sliced(ctypes.byref(tab), p, null, p, p, 1, 1, 0, s) == EARG
    assert lib.fcqt_route_bands_sliced(ctypes.byref(tab), p, p, p, p, 1, 1, -3, s) == EARG
    assert lib.fcqt_route_bands_sliced(ctypes.byref(tab), p, ctypes.c_void_p(4104), p, p, 1, 1, 0, s) == EALIGN
    assert lib.fcqt_scatter_bands_sliced(ctypes.byref(tab), p, p, p, null, 1, 1, 0, s) == EARG
    assert lib.fcqt_stream_overlap(p, null, p, 1, 1, s) == EARG                 # no tail
    assert lib.fcqt_stream_overlap(p, p, null, 1, 2, s) == EARG                 # output needed after slice 0
    assert lib.fcqt_stream_overlap(p, p, p, 0, 1, s) == EARG
    assert lib.fcqt_stream_overlap(p, p, p, 1, -1, s) == EARG
    # streamed composites: (tab, route, groups, prev, prev_stride, next, next_stride, window, nsig, slice,
    # coef, xs, work, stream) and (tab, scat, groups, ovf, coef, f, work, y, tail, out, nsig, slice, stream)
    T = ctypes.byref(tab)
    H2 = 32768
    assert lib.fcqt_stream_analysis(T, p, p, null, H2, p, H2, p, 1, 0, p, p, p, s) == EARG      # no prev
    assert lib.fcqt_stream_analysis(T, p, p, p, H2, p, H2, p, 0, 0, p, p, p, s) == EARG         # no signals
    assert lib.fcqt_stream_analysis(T, p, p, p, H2, p, H2, p, 1, -1, p, p, p, s) == EARG        # negative slice
    assert lib.fcqt_stream_analysis(T, p, p, p, 100, p, H2, p, 2, 0, p, p, p, s) == EARG        # rows overlap
    assert lib.fcqt_stream_analysis(T, p, ctypes.c_void_p(4104), p, H2, p, H2, p, 1, 0, p, p, p, s) == EALIGN
    assert lib.fcqt_stream_synthesis(T, p, p, p, p, p, p, p, null, p, 1, 1, s) == EARG   # no tail
    assert lib.fcqt_stream_synthesis(T, p, p, p, p, p, p, p, p, null, 1, 2, s) == EARG   # output needed
    assert lib.fcqt_stream_synthesis(T, p, p, p, p, p, p, p, p, p, 65536, 1, s) == EARG  # too many signals
    assert lib.fcqt_stream_synthesis(T, p, p, p, p, odd, p, p, p, p, 1, 1, s) == EALIGN  # F alignment
    # whole-signal sliced analysis: (tab, route, groups, sig, sig_len, window, nsig, nslices, coef, xs, work, stream)
    assert lib.fcqt_sliced_analysis(T, p, p, null, 100, p, 1, 1, p, p, p, s) == EARG           # no signal
    assert lib.fcqt_sliced_analysis(T, p, p, p, 0, p, 1, 1, p, p, p, s) == EARG                # empty signal
    assert lib.fcqt_sliced_analysis(T, p, p, p, 100, p, 1, 0, p, p, p, s) == EARG              # no slices
    assert lib.fcqt_sliced_analysis(T, p, p, p, 100, p, 1 << 12, 1 << 12, p, p, p, s) == EARG  # too many rows
    assert lib.fcqt_sliced_analysis(T, p, p, p, 100, p, 1, 1, p, p, null, s) == EARG           # no work buffer
    assert lib.fcqt_sliced_analysis(T, p, ctypes.c_void_p(4104), p, 100, p, 1, 1, p, p, p, s) == EALIGN
    # whole-signal sliced synthesis: (tab, scat, groups, ovf, coef, f, work, out, nsig, nslices, length, stream)
    assert lib.fcqt_sliced_synthesis(T, p, p, p, p, p, p, null, 1, 1, 100, s) == EARG          # no output
    assert lib.fcqt_sliced_synthesis(T, p, p, p, p, p, p, p, 1, 1, 32769, s) == EARG           # longer than 2H
    assert lib.fcqt_sliced_synthesis(T, p, p, p, p, p, p, p, 1, 1, 0, s) == EARG               # empty output
    assert lib.fcqt_sliced_synthesis(T, p, p, p, p, p, p, p, 0, 1, 100, s) == EARG             # no signals
    assert lib.fcqt_sliced_synthesis(T, p, p, p, p, odd, p, p, 1, 1, 100, s) == EALIGN         # F alignment
    assert lib.fcqt_sliced_synthesis(T, p, p, p, p, p, p, ctypes.c_void_p(4098), 1, 1, 100, s) == EALIGN
    assert lib.fcqt_overlap_add(p, p, 1, 1, 2 * 32768 + 1, s) == EARG      # longer than nslices * 2H
    assert lib.fcqt_overlap_add(p, null, 1, 1, 10, s) == EARG
    assert lib.fcqt_fill_zero(p, 0, s) == 0  # nothing to do, no launch


def test_coefficient_span_beyond_ncoef_is_refused(lib):
    """A descriptor whose task table reaches past the coefficient row (ncoef
    below the tasks' coverage), or that declares no coverage, is refused by
    every band entry point before any launch (the compositions included:
    fcqt_analysis checks its band half before launching its FFT half)."""
    from flash_cqt._native import Tables
    p = ctypes.c_void_p(4096)
    s = ctypes.c_void_p(0)
    for span, ncoef in ((132992, 132991), (0, 132992), (-5, 10)):
        tab = ctypes.byref(Tables(tw_pass=16, tw_half=16, tw_stage=16, tasks=16, ntasks=68, ncoef=ncoef,
                                  coef_span=span))
        assert lib.fcqt_route_bands(tab, p, p, p, p, 0, 1, s) == 1
        assert lib.fcqt_route_bands_sliced(tab, p, p, p, p, 1, 1, 0, s) == 1
        assert lib.fcqt_scatter_bands(tab, p, p, p, 0, p, 1, s) == 1
        assert lib.fcqt_scatter_bands_sliced(tab, p, p, p, p, 1, 1, 0, s) == 1
        assert lib.fcqt_analysis(tab, p, p, p, p, 0, p, p, 1, s) == 1
        assert lib.fcqt_synthesis(tab, p, p, p, p, 0, p, p, p, 1, s) == 1
        assert lib.fcqt_sliced_analysis(tab, p, p, p, 100, p, 1, 1, p, p, p, s) == 1
        assert lib.fcqt_sliced_synthesis(tab, p, p, p, p, p, p, p, 1, 1, 100, s) == 1


def test_static_analysis_argument_errors_before_any_launch(lib):
    """fcqt_analysis_static checks its arguments, and its batch against the
    static scratch capacity (FCQT_ECAPACITY), before any HIP call."""
    from flash_cqt._native import Tables
    p = ctypes.c_void_p(4096)
    s = ctypes.c_void_p(0)
    tab = ctypes.byref(Tables(tw_pass=16, tw_half=16, tw_stage=16, tasks=16, ntasks=68, ncoef=132992,
                              coef_span=132992))
    assert lib.fcqt_analysis_static(tab, p, p, p, p, 0, 17, s) == 4
    assert b"capacity" in lib.fcqt_status_string(4)
    assert lib.fcqt_analysis_static(tab, None, p, p, p, 0, 1, s) == 1
    assert lib.fcqt_analysis_static(tab, p, None, p, p, 0, 1, s) == 1
    assert lib.fcqt_analysis_static(tab, p, p, p, p, 0, 0, s) == 1
    assert lib.fcqt_analysis_static(tab, p, ctypes.c_void_p(4100), p, p, 0, 1, s) == 2
    bad = ctypes.byref(Tables(tw_pass=16, tw_half=16, tw_stage=16, tasks=16, ntasks=68, ncoef=10, coef_span=132992))
    assert lib.fcqt_analysis_static(bad, p, p, p, p, 0, 1, s) == 1


def test_package_descriptor_declares_the_task_coverage(factored_tables):
    """The table builder's coef_span is the task table's coverage, equal to
    ncoef for the [3,4,2]/[8,16,32] layout."""
    t = factored_tables
    cov = max(int(f) + int(nb) * int(M) for M, f, nb, _ in t["tasks"].tolist())
    assert t["coef_span"] == cov == t["ncoef"]


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from flash_cqt import _native
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(_native.NativeError):
        _native.load()


def test_stream_of_another_device_is_refused(monkeypatch):
    """An engine on a device other than the current one gets an error, not
    the current device's stream (the default stream launches there)."""
    from flash_cqt import _native
    monkeypatch.setattr(_native, "_get_device", lambda: 1)
    monkeypatch.setattr(_native, "_raw_stream", lambda i: 1000 + i)
    assert _native.stream_handle(1) == 1001
    assert _native.stream_handle() == 1001
    with pytest.raises(_native.NativeError, match="current device is cuda:1"):
        _native.stream_handle(0)


def test_engine_refuses_cpu_device(pkg_cqt_cpu):
    from flash_cqt.fused import FusedOctCQT
    with pytest.raises(ValueError):
        FusedOctCQT(pkg_cqt_cpu, "cpu")
