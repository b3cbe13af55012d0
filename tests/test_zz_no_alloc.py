"""fcqt_analysis_static, the allocation-free analysis, through the C ABI: its
coefficients equal fcqt_analysis's (same kernels, workspace in the library's
static device array instead of caller buffers) bit for bit, on two calls in a
row with the second smaller, in both coefficient layouts; a batch beyond
FCQT_STATIC_MAX_BATCH is refused with FCQT_ECAPACITY before any launch."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

N = 65536
ECAPACITY = 4
STATIC_MAX_BATCH = 16


@pytest.fixture(scope="module")
def engine():
    from flash_cqt import OctCQT
    from flash_cqt.fused import FusedOctCQT
    cqt = OctCQT([3, 4, 2], [8, 16, 32], fs=44100, audio_len=N, device="cuda:0")
    return FusedOctCQT(cqt, "cuda:0")


def _static(f, x, kr, ki, layout):
    from flash_cqt import _native
    B = x.shape[0]
    return f.lib.fcqt_analysis_static(f._ct, f._tp["route"], x.data_ptr(), kr.data_ptr(),
                                      ki.data_ptr() if ki is not None else None, layout, B,
                                      _native.stream_handle(f.dev.index))


@pytest.mark.parametrize("layout", [0, 1])
def test_static_analysis_equals_analysis_twice_second_smaller(engine, layout):
    from flash_cqt import _native
    f = engine
    rs = np.random.RandomState(5 + layout)
    for B in (STATIC_MAX_BATCH, 3):
        print(f"static analysis: layout {layout}, batch {B}", flush=True)
        x = torch.from_numpy(rs.standard_normal((B, N)).astype(np.float32)).cuda()
        if layout == _native.PLANAR:
            ref_r, ref_i = torch.empty(B, f.ncoef, device="cuda"), torch.empty(B, f.ncoef, device="cuda")
            got_r, got_i = torch.full_like(ref_r, float("nan")), torch.full_like(ref_i, float("nan"))
            f.analysis(x, ref_r, ref_i, layout)
            assert _static(f, x, got_r, got_i, layout) == 0
            torch.cuda.synchronize()
            assert torch.equal(got_r, ref_r) and torch.equal(got_i, ref_i)
        else:
            ref = torch.empty(B, f.ncoef, dtype=torch.complex64, device="cuda")
            got = torch.full_like(ref, complex(float("nan"), 0.0))
            f.analysis(x, ref, None, layout)
            assert _static(f, x, got, None, layout) == 0
            torch.cuda.synchronize()
            assert torch.equal(got, ref)


def test_static_analysis_refuses_batch_beyond_capacity(engine):
    f = engine
    B = STATIC_MAX_BATCH + 1
    x = torch.zeros(B, N, device="cuda")
    kr = torch.full((B, f.ncoef), 7.0, device="cuda")
    ki = torch.full_like(kr, 7.0)
    assert _static(f, x, kr, ki, 0) == ECAPACITY
    torch.cuda.synchronize()
    assert bool((kr == 7.0).all()) and bool((ki == 7.0).all())        # nothing was launched
    assert b"capacity" in f.lib.fcqt_status_string(ECAPACITY)
