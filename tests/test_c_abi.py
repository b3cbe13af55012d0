"""include/flashcqt.h from C: tests/c/abi_check.c compiles as C99 with
warnings on, links libflashcqt.so and runs the calls that need no GPU,
including loading a table image file and sizing the buffers without Python."""
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIBDIR = ROOT / "flash-cqt_amd" / "flash_cqt" / "_lib"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_header_from_c(tmp_path, factored_tables):
    exe = tmp_path / "abi_check"
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROOT / 'include'}", "-I/opt/rocm/include", str(ROOT / "tests" / "c" / "abi_check.c"),
           f"-L{LIBDIR}", "-lflashcqt", f"-Wl,-rpath,{LIBDIR}", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    from flash_cqt import tables as T
    img = tmp_path / "cqt_tables.img"
    T.save_image(factored_tables, img)
    r = subprocess.run([str(exe), str(img)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "c abi check ok (ABI 13)" in r.stdout
    assert f"ncoef {factored_tables['ncoef']}, {factored_tables['tasks'].shape[0]} tasks" in r.stdout
    B = 64
    assert (f"signal {B * T.N * 4} spectrum {B * T.XSTRIDE * 8} work {B * T.L * 8} scatter {B * T.FROW * 8} "
            f"coef_plane {B * factored_tables['ncoef'] * 4} tail {B * T.N // 2 * 4} sync {(B * 64 + 320) * 4}") in r.stdout


@pytest.mark.gpu
def test_c_consumer_round_trip_on_gpu(tmp_path):
    """tests/c/roundtrip.c (built by __graft_entry__.build) runs the whole
    round trip from C: table image file, checked upload, buffer sizes from
    the library, hipMalloc, analysis, synthesis. Every row reconstructs at
    >= 125 dB and its coefficients equal the package's bit for bit; the
    single-launch entry points give the same bits and leave their stage
    counters clear."""
    import numpy as np
    import torch
    from flash_cqt import OctCQT, tables as T
    from flash_cqt.fused import FusedOctCQT
    exe = ROOT / "tests" / "c" / "_build" / "roundtrip"
    assert exe.exists(), "the C consumer is built by __graft_entry__.build()"
    dev = torch.device("cuda:0")
    cqt = OctCQT([3, 4, 2], [8, 16, 32], fs=44100, audio_len=T.N, device=dev)
    img = tmp_path / "cqt_tables.img"
    T.save_image(T.build(cqt.np_groups + cqt.np_side_groups, noct=len(cqt.groups)), img)
    B = 3
    x = np.random.RandomState(41).standard_normal((B, T.N)).astype(np.float32)
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    r = subprocess.run([str(exe), str(img), str(B), str(tmp_path / "x.bin"), str(tmp_path / "k.bin")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    snrs = [float(line.split()[3]) for line in r.stdout.splitlines() if line.startswith("row ")]
    assert len(snrs) == B and min(snrs) >= 125, r.stdout
    assert "single launch: same bits 1, counters and error word clear 1" in r.stdout, r.stdout
    eng = FusedOctCQT(cqt, dev)
    KR, KI = eng.fwd(torch.from_numpy(x).to(dev))
    k = np.frombuffer((tmp_path / "k.bin").read_bytes(), dtype=np.float32).reshape(2, B, eng.ncoef)
    assert np.array_equal(k[0], KR.cpu().numpy()) and np.array_equal(k[1], KI.cpu().numpy())
