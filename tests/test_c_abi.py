"""include/flashcqt.h from C: tests/c/abi_check.c compiles as C99 with
warnings on, links libflashcqt.so and runs the calls that need no GPU."""
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIBDIR = ROOT / "flash-cqt_amd" / "flash_cqt" / "_lib"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_header_from_c(tmp_path):
    exe = tmp_path / "abi_check"
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROOT / 'include'}", "-I/opt/rocm/include", str(ROOT / "tests" / "c" / "abi_check.c"),
           f"-L{LIBDIR}", "-lflashcqt", f"-Wl,-rpath,{LIBDIR}", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "c abi check ok (ABI 7)" in r.stdout
