"""Build libelasticbit_hip.so for gfx950 with hipcc / amdclang++.

    python -m mlbricks_amd.csrc.build        # from the repository root

The kernels (eb_kernels.hip) are compiled for gfx950 only; the host runtime
(eb_host.cpp) is plain C++17 compiled with -ffp-contract=off so the host
analyzer rounds exactly as written.  Outputs go to mlbricks_amd/lib/.
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
PROBE_LIB_NAME = "libeb_probe_read.so"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

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


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    clangxx = str(ROCM / "llvm" / "bin" / "clang++")
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    inc = [f"-I{ROOT / 'include'}", f"-I{HERE}", f"-I{ROCM / 'include'}"]
    kobj = BUILD_DIR / "eb_kernels.o"
    aobj = BUILD_DIR / "eb_analyze.o"
    hobj = BUILD_DIR / "eb_host.o"
    _run([hipcc, *DEVICE_FLAGS, *inc, "-c", str(HERE / "eb_kernels.hip"), "-o", str(kobj)], verbose)
    _run([hipcc, *DEVICE_FLAGS, *inc, "-c", str(HERE / "eb_analyze.hip"), "-o", str(aobj)], verbose)
    _run([clangxx, *HOST_FLAGS, *inc, "-c", str(HERE / "eb_host.cpp"), "-o", str(hobj)], verbose)
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), str(kobj), str(aobj), str(hobj),
          f"-L{ROCM / 'lib'}", "-lamdhip64", "-lpthread"], verbose)
    out = LIB_DIR / LIB_NAME
    os.replace(tmp, out)
    # bench.py's read-bandwidth probe, a library of its own
    ptmp = LIB_DIR / (PROBE_LIB_NAME + ".tmp")
    _run([hipcc, *DEVICE_FLAGS, "-shared", str(HERE / "probe_read.hip"), "-o", str(ptmp)], verbose)
    os.replace(ptmp, LIB_DIR / PROBE_LIB_NAME)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
