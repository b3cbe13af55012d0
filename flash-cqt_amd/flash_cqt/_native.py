"""ctypes boundary to libflashcqt.so (the C ABI declared in include/flashcqt.h).

The library is built in-tree by __graft_entry__.build() (hipcc, gfx950) into
flash_cqt/_lib/. It is loaded after torch so that it binds to the HIP runtime
torch already loaded (same SONAME), which makes torch's streams and hipGraph
capture valid for its launches. There is no fallback: if the library is
missing or does not load, every engine entry point raises.
"""
import ctypes
import pathlib

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libflashcqt.so"
ABI_VERSION = 13
SYNC_PER_SLICE = 64       # FCQT_SYNC_PER_SLICE: uint32 per slice in a single-launch counter buffer
SYNC_HEAD_WORDS = 320     # FCQT_SYNC_HEAD_WORDS: the error word, exit count and per-XCD queue claims


def sync_words(batch):
    """FCQT_SYNC_WORDS(batch): uint32 words of a single-launch sync buffer;
    word batch * SYNC_PER_SLICE is the error word."""
    return batch * SYNC_PER_SLICE + SYNC_HEAD_WORDS
PLANAR = 0
INTERLEAVED = 1

#: every symbol include/flashcqt.h declares
EXPORTS = ("fcqt_abi_version", "fcqt_status_string", "fcqt_last_hip_error",
           "fcqt_packed_fft_fwd", "fcqt_route_bands", "fcqt_scatter_bands",
           "fcqt_packed_fft_inv", "fcqt_analysis", "fcqt_synthesis", "fcqt_fill_zero",
           "fcqt_slice_fft_fwd", "fcqt_route_bands_sliced", "fcqt_scatter_bands_sliced",
           "fcqt_overlap_add", "fcqt_stream_overlap", "fcqt_image_check", "fcqt_tables_upload",
           "fcqt_workspace_sizes", "fcqt_analysis_static", "fcqt_persist_analysis", "fcqt_persist_synthesis",
           "fcqt_stream_analysis", "fcqt_stream_synthesis", "fcqt_sliced_analysis",
           "fcqt_sliced_synthesis", "fcqt_persist_tune", "fcqt_persist_trace")


class Tables(ctypes.Structure):
    """Mirror of struct fcqt_tables."""
    _fields_ = [("tw_pass", ctypes.c_void_p), ("tw_half", ctypes.c_void_p),
                ("tw_stage", ctypes.c_void_p), ("tasks", ctypes.c_void_p),
                ("ntasks", ctypes.c_int32), ("ncoef", ctypes.c_int64), ("coef_span", ctypes.c_int64)]


class ImageInfo(ctypes.Structure):
    """Mirror of struct fcqt_image_info."""
    _fields_ = [("device_bytes", ctypes.c_int64), ("ncoef", ctypes.c_int64), ("coef_span", ctypes.c_int64),
                ("ntasks", ctypes.c_int32), ("format", ctypes.c_int32)]


class EngineTables(ctypes.Structure):
    """Mirror of struct fcqt_engine_tables."""
    _fields_ = [("tab", Tables)] + [(n, ctypes.c_void_p) for n in
                                    ("route", "route_b", "scat", "scat_a", "ovf_scat", "ovf_scat_a",
                                     "slice_groups")]


class Sizes(ctypes.Structure):
    """Mirror of struct fcqt_sizes."""
    _fields_ = [(n, ctypes.c_int64) for n in ("signal", "spectrum", "work", "scatter", "coef_plane", "tail", "sync")]


class NativeError(RuntimeError):
    pass


_lib = None
_variants = {}
#: variant libraries (same C ABI, other kernel builds): name -> file in _lib/
VARIANTS = {"xlane": "libflashcqt_xlane.so", "flowtrace": "libflashcqt_flowtrace.so"}


def load():
    """Load and type the library once; raise NativeError if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    _lib = _open(LIB_PATH)
    return _lib


def load_variant(name):
    """Load and type a variant library built beside the library (its C ABI
    is the library's): "xlane" runs the band units of M <= 256 with the
    cross-lane exchange between their first two stages; "flowtrace" records
    the single-launch kernels' stage trace (fcqt_persist_trace). Raises
    NativeError if it is not built."""
    if name not in _variants:
        if name not in VARIANTS:
            raise NativeError(f"unknown library variant {name!r}")
        _variants[name] = _open(LIB_PATH.with_name(VARIANTS[name]))
    return _variants[name]


def _open(path):
    if not path.exists():
        raise NativeError(f"flash_cqt HIP library not built ({path}); "
                          "run __graft_entry__.build()")
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as e:
        raise NativeError(f"cannot load {path}: {e}") from e
    P, I32, I64, S = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    T = ctypes.POINTER(Tables)
    sig = {
        "fcqt_abi_version": ([], ctypes.c_int),
        "fcqt_status_string": ([ctypes.c_int], ctypes.c_char_p),
        "fcqt_last_hip_error": ([], ctypes.c_char_p),
        "fcqt_packed_fft_fwd": ([T, P, P, P, I64, S], ctypes.c_int),
        "fcqt_route_bands": ([T, P, P, P, P, ctypes.c_int, I64, S], ctypes.c_int),
        "fcqt_scatter_bands": ([T, P, P, P, ctypes.c_int, P, I64, S], ctypes.c_int),
        "fcqt_packed_fft_inv": ([T, P, P, P, P, I64, S], ctypes.c_int),
        "fcqt_analysis": ([T, P, P, P, P, ctypes.c_int, P, P, I64, S], ctypes.c_int),
        "fcqt_synthesis": ([T, P, P, P, P, ctypes.c_int, P, P, P, I64, S], ctypes.c_int),
        "fcqt_fill_zero": ([P, I64, S], ctypes.c_int),
        "fcqt_slice_fft_fwd": ([T, P, I64, P, I64, I64, I64, I64, P, P, S], ctypes.c_int),
        "fcqt_route_bands_sliced": ([T, P, P, P, P, I64, I64, I64, S], ctypes.c_int),
        "fcqt_sliced_analysis": ([T, P, P, P, I64, P, I64, I64, P, P, P, S], ctypes.c_int),
        "fcqt_sliced_synthesis": ([T, P, P, P, P, P, P, P, I64, I64, I64, S], ctypes.c_int),
        "fcqt_scatter_bands_sliced": ([T, P, P, P, P, I64, I64, I64, S], ctypes.c_int),
        "fcqt_overlap_add": ([P, P, I64, I64, I64, S], ctypes.c_int),
        "fcqt_stream_overlap": ([P, P, P, I64, I64, S], ctypes.c_int),
        "fcqt_stream_analysis": ([T, P, P, P, I64, P, I64, P, I64, I64, P, P, P, S], ctypes.c_int),
        "fcqt_stream_synthesis": ([T, P, P, P, P, P, P, P, P, P, I64, I64, S], ctypes.c_int),
        "fcqt_image_check": ([ctypes.c_char_p, I64, ctypes.POINTER(ImageInfo)], ctypes.c_int),
        "fcqt_tables_upload": ([ctypes.c_char_p, I64, P, I64, S, ctypes.POINTER(EngineTables)], ctypes.c_int),
        "fcqt_workspace_sizes": ([T, I64, ctypes.POINTER(Sizes)], ctypes.c_int),
        "fcqt_analysis_static": ([T, P, P, P, P, ctypes.c_int, I64, S], ctypes.c_int),
        "fcqt_persist_analysis": ([T, P, P, P, P, ctypes.c_int, P, P, P, I64, S], ctypes.c_int),
        "fcqt_persist_synthesis": ([T, P, P, P, P, ctypes.c_int, P, P, P, P, I64, S], ctypes.c_int),
        "fcqt_persist_tune": ([ctypes.c_int, ctypes.c_int, ctypes.c_int, I64], ctypes.c_int),
        "fcqt_persist_trace": ([P, I64], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    ver = lib.fcqt_abi_version()
    if ver != ABI_VERSION:
        raise NativeError(f"libflashcqt ABI {ver}, expected {ABI_VERSION}; rebuild")
    return lib


def check(status, what):
    if status != 0:
        lib = load()
        msg = lib.fcqt_status_string(status).decode()
        hip = lib.fcqt_last_hip_error().decode()
        raise NativeError(f"{what}: {msg}" + (f" [{hip}]" if hip else ""))


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)


def stream_handle(device_index=None):
    """hipStream_t (as an int) of the current torch stream of a device
    (default: the current device).

    The device must be the current one: a launch on the default stream
    (handle 0) goes to the current device, so an engine on another device
    would otherwise be handed the wrong device's stream. Like a torch op
    without a device guard, the caller selects the device
    (torch.cuda.device / set_device); this raises instead of launching."""
    cur = _get_device() if _get_device is not None else torch.cuda.current_device()
    if device_index is None:
        device_index = cur
    elif device_index != cur:
        raise NativeError(f"engine is on cuda:{device_index} but the current device is cuda:{cur}; "
                          f"launch under torch.cuda.device({device_index})")
    if _raw_stream is not None:
        return _raw_stream(device_index)
    return torch.cuda.current_stream(device_index).cuda_stream


def require_device(t, name, dtype=torch.float32):
    if not (torch.is_tensor(t) and t.is_cuda and t.dtype == dtype and t.is_contiguous()):
        raise ValueError(f"{name} must be a contiguous {dtype} tensor on a GPU")
