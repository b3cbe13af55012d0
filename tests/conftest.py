import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (str(ROOT), str(ROOT / "flash-cqt_amd"), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = ROOT / "tests" / "golden" / "golden_ref.npz"
LAYOUT = ([3, 4, 2], [8, 16, 32])
FS = 44100
N = 65536


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


def pytest_sessionstart(session):
    """Build the HIP library once if this checkout has none yet (a fresh
    clone); a built library is used as it is."""
    lib = ROOT / "flash-cqt_amd" / "flash_cqt" / "_lib" / "libflashcqt.so"
    if not lib.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location("flashcqt_build", ROOT / "flash-cqt_amd" / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build(verbose=False)


@pytest.fixture(scope="session")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.fixture(scope="session")
def oracle():
    from oracle.cqt_oracle import OctCQT
    return OctCQT(*LAYOUT, FS, N)


@pytest.fixture(scope="session")
def pkg_cqt_cpu():
    from flash_cqt import OctCQT
    return OctCQT(*LAYOUT, fs=FS, audio_len=N, device="cpu")


@pytest.fixture(scope="session")
def factored_tables(pkg_cqt_cpu):
    from flash_cqt import tables
    return tables.build(pkg_cqt_cpu.np_groups + pkg_cqt_cpu.np_side_groups)
