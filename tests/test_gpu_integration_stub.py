"""The reference-side ctypes stub printed in INTEGRATION.md, run as written
(with the library path and the table-builder import filled in): its analysis,
synthesis and sliced forward must equal the package's own launches bit for
bit, so the documented binding is a working one."""
import pathlib
import re
import types

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]
N = 65536


def _stub_module():
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = [b for b in re.findall(r"```python\n(.*?)```", text, re.S) if "_lib" in b]
    assert len(blocks) == 2, "expected the engine stub and the sliced stub"
    from flash_cqt import _native
    src = "\n".join(blocks)
    src = src.replace('"/path/to/libflashcqt.so"', repr(str(_native.LIB_PATH)))
    src = src.replace("from flash_cqt_amd_tables import build", "from flash_cqt.tables import build")
    mod = types.ModuleType("flash_cqt_amd_stub")
    exec(compile(src, "INTEGRATION.md", "exec"), mod.__dict__)
    return mod


@pytest.fixture(scope="module")
def stub():
    return _stub_module()


@pytest.fixture(scope="module")
def cqt_gpu():
    from flash_cqt import OctCQT
    return OctCQT([3, 4, 2], [8, 16, 32], fs=44100, audio_len=N, device="cuda")


def test_stub_engine_equals_package(stub, cqt_gpu):
    from flash_cqt.fused import FusedOctCQT
    f = FusedOctCQT(cqt_gpu, "cuda")
    eng = stub.AmdEngine(cqt_gpu)
    assert eng.ncoef == f.ncoef
    rs = np.random.RandomState(77)
    x = torch.from_numpy(rs.standard_normal((3, N)).astype(np.float32)).cuda()
    kr = torch.empty(3, eng.ncoef, device="cuda")
    ki = torch.empty_like(kr)
    eng.analysis(x, kr, ki)
    KR, KI = f.fwd(x)
    assert torch.equal(kr, KR) and torch.equal(ki, KI)
    y = torch.empty(3, N, device="cuda")
    eng.synthesis(kr, ki, y)
    assert torch.equal(y, f.bwd(KR, KI))


def test_stub_sliced_forward_equals_package(stub, cqt_gpu):
    from flash_cqt import SlicedCQT
    s = SlicedCQT(device="cuda")
    rs = np.random.RandomState(78)
    x = torch.from_numpy(rs.standard_normal((1, 2, 100000)).astype(np.float32)).cuda()
    with torch.no_grad():
        blocks, side = s.fwd(x)
    eng = stub.AmdEngine(cqt_gpu)
    S = s._num_slices(x.shape[-1])
    coef = stub.sliced_fwd(eng, x.reshape(2, -1).contiguous(), s.tw.float().contiguous(), S)
    assert torch.equal(coef, blocks[0]._base)


def test_stub_reports_errors(stub, cqt_gpu):
    """A bad call through the stub raises with the library's message."""
    eng = stub.AmdEngine(cqt_gpu)
    with pytest.raises(RuntimeError, match="argument"):
        stub._ok(stub._lib.fcqt_packed_fft_fwd(eng.ct, 0, 0, 0, 1, stub._stream()), "fft")
