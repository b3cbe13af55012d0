"""Build libflashcqt.so (gfx950) in-tree with hipcc.

    python flash-cqt_amd/build.py [--verbose]

Output: flash-cqt_amd/flash_cqt/_lib/libflashcqt.so. Flags: -O3 for gfx950,
packed fp32 instructions disabled (-Xclang -target-feature -Xclang
-packed-fp32-ops), hardware fp32 atomics (-munsafe-fp-atomics; every atomic
target is ordinary device memory). The host pass warns that it does not know
the packed-fp32 feature; that warning is harmless.
"""
import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "flash_cqt" / "_lib" / "libflashcqt.so"
SOURCES = ("abi.hip", "bands.hip", "packed_fft.hip")
ARCH = "gfx950"


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def command(out=OUT):
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-munsafe-fp-atomics", "-Wall", "-Wno-unused-command-line-argument",
            *[str(CSRC / s) for s in SOURCES], "-o", str(out)]


def build(verbose=False):
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = command(tmp)
    res = subprocess.run(cmd, capture_output=True, text=True)
    lines = [ln for ln in (res.stdout + res.stderr).splitlines()
             if "packed-fp32-ops' is not a recognized feature" not in ln]
    if verbose or res.returncode != 0:
        print(" ".join(cmd))
        print("\n".join(lines))
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode})")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
