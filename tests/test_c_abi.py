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
    assert "c abi check ok (ABI 7)" in r.stdout
    assert f"ncoef {factored_tables['ncoef']}, {factored_tables['tasks'].shape[0]} tasks" in r.stdout
    B = 64
    assert (f"signal {B * T.N * 4} spectrum {B * T.XSTRIDE * 8} work {B * T.L * 8} scatter {B * T.FROW * 8} "
            f"coef_plane {B * factored_tables['ncoef'] * 4} tail {B * T.N // 2 * 4}") in r.stdout
