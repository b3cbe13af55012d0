"""The table image and the C ABI's host-side checks (no GPU): the Python
builder's image passes fcqt_image_check with the expected contents, every
kind of corrupted image is refused with FCQT_EARG, and fcqt_workspace_sizes
gives the buffer sizes the package allocates."""
import ctypes
import struct

import numpy as np
import pytest

EARG = 1


@pytest.fixture(scope="module")
def lib():
    from flash_cqt import _native
    return _native.load()


@pytest.fixture(scope="module")
def image(factored_tables):
    from flash_cqt import tables as T
    return T.image_bytes(factored_tables)


def sections(img):
    nsec = struct.unpack_from("<I", img, 8)[0]
    out = {}
    for k in range(nsec):
        sid, elem, count, off = struct.unpack_from("<IIQQ", img, 16 + 24 * k)
        out[sid] = (elem, count, off, 16 + 24 * k)
    return out


def check(lib, img):
    from flash_cqt import _native
    info = _native.ImageInfo()
    return lib.fcqt_image_check(bytes(img), len(img), ctypes.byref(info)), info


def test_builder_image_passes_with_its_contents(lib, image, factored_tables):
    from flash_cqt import tables as T
    rc, info = check(lib, image)
    assert rc == 0
    t = factored_tables
    assert info.ncoef == t["ncoef"] == info.coef_span and info.ntasks == t["tasks"].shape[0]
    assert info.device_bytes == len(image) and info.format == T.IMAGE_VERSION
    secs = sections(image)
    assert set(secs) == set(T.IMAGE_SECTIONS)
    for sid, (name, dt) in T.IMAGE_SECTIONS.items():
        elem, count, off, _ = secs[sid]
        assert off % T.IMAGE_ALIGN == 0
        got = np.frombuffer(image, dtype=dt, count=count, offset=off)
        assert np.array_equal(got, np.asarray(t[name], dtype=dt).reshape(-1)), name


def _patched(image, sid, index, value, dtype=np.int32):
    img = bytearray(image)
    elem, count, off, _ = sections(image)[sid]
    np.frombuffer(img, dtype=dtype, count=count, offset=off)[index] = value
    return img


def test_corrupted_images_are_refused(lib, image, factored_tables):
    """Each corruption names a bound a kernel relies on."""
    from flash_cqt import tables as T
    t = factored_tables
    nt = t["tasks"].shape[0]
    bad = {}
    img = bytearray(image)
    img[0:4] = b"XCQT"
    bad["magic"] = img
    img = bytearray(image)
    img[4:8] = struct.pack("<I", 99)
    bad["format version"] = img
    bad["truncated"] = image[:len(image) // 2]
    bad["header only"] = image[:40]
    img = bytearray(image)
    img[8:12] = struct.pack("<I", 11)                          # one section missing
    bad["missing section"] = img
    img = bytearray(image)
    h = sections(image)[5][3]
    img[h:h + 4] = struct.pack("<I", 4)                        # route section claims to be tasks
    bad["repeated section"] = img
    img = bytearray(image)
    h = sections(image)[7][3]
    struct.pack_into("<Q", img, h + 16, sections(image)[7][2] + 4)
    bad["misaligned section"] = img
    bad["band length"] = _patched(image, 4, 4 * 3, 100)
    bad["band count"] = _patched(image, 4, 4 * 0 + 2, 2048 // t["tasks"][0, 0] + 1)
    last = 4 * (nt - 1)
    bad["task past ncoef"] = _patched(image, 4, last + 1, int(t["tasks"][-1, 1]) + 1)
    bad["negative first"] = _patched(image, 4, 1, -5)
    bad["ncoef below coverage"] = _patched(image, 12, 0, int(t["ncoef"]) - 1, np.int64)
    bad["route bin"] = _patched(image, 5, 2 * 777, 32769)
    bad["route bin with a high bit"] = _patched(image, 5, 2 * 778, np.int32(np.uint32(5 | (1 << 31)).view(np.int32)))
    bad["adjoint route bin"] = _patched(image, 6, 2 * 1234, 40000)
    bad["scatter slot"] = _patched(image, 7, 2 * 99, T.FROW)
    bad["scatter mode"] = _patched(image, 8, 2 * 5, np.int32(np.uint32(3 << 30).view(np.int32)))
    bad["fold bin"] = _patched(image, 9, 0, 32769)
    bad["fold index"] = _patched(image, 10, 1, 5 | (T.OVF_CAP << 16))
    bad["slice roll"] = _patched(image, 11, 2, 2)
    bad["slice group past ncoef"] = _patched(image, 11, 4 * (nt - 1) + 1, 10 ** 6)
    for name, img in bad.items():
        rc, _ = check(lib, img)
        assert rc == EARG, name
    assert check(lib, image)[0] == 0


def test_null_and_short_arguments(lib):
    from flash_cqt import _native
    assert lib.fcqt_image_check(None, 100, None) == EARG
    assert lib.fcqt_image_check(b"FCQT", 4, None) == EARG
    up = _native.EngineTables()
    assert lib.fcqt_tables_upload(b"nope", 4, ctypes.c_void_p(4096), 4096, ctypes.c_void_p(0),
                                  ctypes.byref(up)) == EARG


def test_upload_refuses_short_or_misaligned_device_memory_before_any_copy(lib, image):
    from flash_cqt import _native
    up = _native.EngineTables()
    s = ctypes.c_void_p(0)
    assert lib.fcqt_tables_upload(image, len(image), ctypes.c_void_p(4096), len(image) - 1, s,
                                  ctypes.byref(up)) == EARG
    assert lib.fcqt_tables_upload(image, len(image), None, len(image), s, ctypes.byref(up)) == EARG
    assert lib.fcqt_tables_upload(image, len(image), ctypes.c_void_p(4096 + 64), len(image), s,
                                  ctypes.byref(up)) == 2


def test_workspace_sizes(lib, factored_tables):
    from flash_cqt import _native, tables as T
    tab = _native.Tables(tw_pass=16, tw_half=16, tw_stage=16, tasks=16, ntasks=68, ncoef=factored_tables["ncoef"],
                         coef_span=factored_tables["ncoef"])
    sz = _native.Sizes()
    assert lib.fcqt_workspace_sizes(ctypes.byref(tab), 64, ctypes.byref(sz)) == 0
    assert sz.signal == 64 * T.N * 4 and sz.spectrum == 64 * T.XSTRIDE * 8 and sz.work == 64 * T.L * 8
    assert sz.scatter == 64 * T.FROW * 8 and sz.coef_plane == 64 * factored_tables["ncoef"] * 4
    assert sz.tail == 64 * (T.N // 2) * 4
    assert sz.sync == (64 * 64 + 320) * 4   # FCQT_SYNC_WORDS(64): slice records, then the head block
    assert lib.fcqt_workspace_sizes(ctypes.byref(tab), 0, ctypes.byref(sz)) == EARG
    assert lib.fcqt_workspace_sizes(None, 1, ctypes.byref(sz)) == EARG
