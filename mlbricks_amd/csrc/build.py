"""Build libelasticbit_hip.so for gfx950 with hipcc / amdclang++.

    python -m mlbricks_amd.csrc.build        # from the repository root

The kernels (eb_kernels.hip, eb_prefill.hip, eb_analyze.hip) are compiled for
gfx950 only; the host runtime (eb_host.cpp) is plain C++17 compiled with
-ffp-contract=off so the host analyzer rounds exactly as written.  The four
translation units compile in parallel.  Outputs go to mlbricks_amd/lib/.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
ROOT = PKG.parent
BUILD_DIR = HERE / "_build"
LIB_DIR = PKG / "lib"
LIB_NAME = "libelasticbit_hip.so"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"
DEVICE_SOURCES = ("eb_kernels.hip", "eb_prefill.hip", "eb_decode_rows.hip", "eb_analyze.hip")
HOST_SOURCES = ("eb_host.cpp",)

# Packed-fp32 VALU forms are disabled for every device compile on this target.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]
HOST_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
    "-D__HIP_PLATFORM_AMD__", "-Wall", "-Wextra", "-Wno-unused-parameter",
]
_NOISE = "is not a recognized feature for this target"


def _check(cmd: list[str], res: subprocess.CompletedProcess, verbose: bool) -> None:
    err = "\n".join(line for line in res.stderr.splitlines() if _NOISE not in line)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def _run_all(cmds: list[list[str]], verbose: bool) -> None:
    """Run the commands concurrently; raise on the first that failed."""
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    failures = []
    for cmd, proc in procs:
        out, err = proc.communicate()
        res = subprocess.CompletedProcess(cmd, proc.returncode, out, err)
        try:
            _check(cmd, res, verbose)
        except RuntimeError as exc:
            failures.append(exc)
    if failures:
        raise failures[0]


def build(verbose: bool = False) -> Path:
    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    clangxx = str(ROCM / "llvm" / "bin" / "clang++")
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    inc = [f"-I{ROOT / 'include'}", f"-I{HERE}", f"-I{ROCM / 'include'}"]
    objs = []
    cmds = []
    for src in DEVICE_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc, *DEVICE_FLAGS, *inc, "-c", str(HERE / src), "-o", str(obj)])
    for src in HOST_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([clangxx, *HOST_FLAGS, *inc, "-c", str(HERE / src), "-o", str(obj)])
    _run_all(cmds, verbose)
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
            f"-L{ROCM / 'lib'}", "-lamdhip64", "-lpthread"]
    _run_all([link], verbose)
    out = LIB_DIR / LIB_NAME
    os.replace(tmp, out)
    stale = LIB_DIR / "libeb_probe_read.so"     # the bench's probe no longer lives in the package
    if stale.exists():
        stale.unlink()
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
