"""Build libflashcqt.so (gfx950) in-tree with hipcc.

    python flash-cqt_amd/build.py [--verbose]

Output: flash-cqt_amd/flash_cqt/_lib/libflashcqt.so, and beside it two
variant libraries of the same sources: libflashcqt_xlane.so (the band units of
M <= 256 exchanging across lanes instead of through LDS; the benchmark and the
GPU tests compare the two) and libflashcqt_flowtrace.so (the single-launch
kernels stamping a stage trace, fcqt_persist_trace). All compile in parallel. Flags: -O3 for gfx950,
packed fp32 instructions disabled (-Xclang -target-feature -Xclang
-packed-fp32-ops). The host pass warns that it does not know the packed-fp32
feature; that warning is harmless.

The compiler's kernel resource report (-Rpass-analysis=kernel-resource-usage)
is parsed on every build: a kernel that uses scratch memory (register spills
or a private array the compiler could not keep in registers) fails the
build, since every kernel here is meant to run out of registers and LDS.
"""
import re
import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "flash_cqt" / "_lib" / "libflashcqt.so"
SOURCES = ("abi.hip", "bands.hip", "packed_fft.hip", "image.hip", "persist.hip")
ARCH = "gfx950"


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


# variant name -> (output, extra defines)
VARIANTS = {"": (OUT, ()), "xlane": (OUT.with_name("libflashcqt_xlane.so"), ("-DFCQT_XLANE_MAX_M=256",)),
            "flowtrace": (OUT.with_name("libflashcqt_flowtrace.so"), ("-DFCQT_FLOW_TRACE",))}


def command(out=OUT, defines=()):
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Rpass-analysis=kernel-resource-usage", "-Wall", "-Wno-unused-command-line-argument",
            *defines, *[str(CSRC / s) for s in SOURCES], "-o", str(out)]


_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|LDS Size \[bytes/block\]|"
                     r"Occupancy \[waves/SIMD\]):\s+(\S+)")


def resource_usage(text):
    """{kernel: {field: value}} from the kernel-resource-usage remarks."""
    out, cur = {}, None
    for m in _REMARK.finditer(text):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[key.split(" [")[0]] = int(val)
    return out


def build(verbose=False):
    """Compile the library and its variants (in parallel); returns the
    library's path. Fails on a compile error or on any kernel that uses
    scratch memory; writes the library's resource report to
    _lib/resources.txt."""
    OUT.parent.mkdir(parents=True, exist_ok=True)
    procs = {}
    for name, (out, defines) in VARIANTS.items():
        tmp = out.with_suffix(".so.tmp")
        cmd = command(tmp, defines)
        procs[name] = (out, tmp, cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                                       text=True))
    failed = []
    for name, (out, tmp, cmd, proc) in procs.items():
        text, _ = proc.communicate()
        lines = [ln for ln in text.splitlines()
                 if "packed-fp32-ops' is not a recognized feature" not in ln and "remark:" not in ln]
        if verbose or proc.returncode != 0:
            print(" ".join(cmd))
            print("\n".join(lines))
        if proc.returncode != 0:
            failed.append(f"{name or 'library'}: hipcc failed ({proc.returncode})")
            continue
        usage = resource_usage(text)
        if not usage:
            failed.append(f"{name or 'library'}: hipcc printed no kernel resource report")
            continue
        spilled = {k: v for k, v in usage.items() if v.get("ScratchSize", 0) > 0}
        if spilled:
            failed.append(f"{name or 'library'}: kernels use scratch memory: {spilled}")
            continue
        if not name:
            with open(OUT.parent / "resources.txt", "w") as f:
                for k, v in sorted(usage.items()):
                    f.write(k + " " + " ".join(f"{a}={b}" for a, b in v.items()) + "\n")
        os.replace(tmp, out)
    if failed:
        raise RuntimeError("; ".join(failed))
    return OUT


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
