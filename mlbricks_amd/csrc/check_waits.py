"""Developer check of the activation-staging waits in the decode kernels.

linear_gemv_kernel and linear_decode_kernel stage the activations into LDS
with global_load_lds and then issue the first weight loads; before reading
the LDS copy they wait with an explicit `s_waitcnt vmcnt(N)`, N = the weight
loads issued after the staging.  That is correct only if the compiled code
keeps the staging loads ahead of exactly those N loads (a scheduling barrier
in the source pins the order).  This script reads the assembly hipcc writes
for eb_kernels.hip and checks, in every instantiation, that the first
explicit wait after the staging leaves no more loads outstanding than were
issued after the last staging load.

    python mlbricks_amd/csrc/check_waits.py            # compiles to a temporary directory
    python mlbricks_amd/csrc/check_waits.py FILE.s     # checks an existing gfx950 assembly file
"""
from __future__ import annotations

import re
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
KERNELS = ("linear_gemv_kernel", "linear_decode_kernel")


def assembly() -> str:
    with tempfile.TemporaryDirectory() as tmp:
        cmd = ["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang",
               "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{HERE}",
               "--cuda-device-only", "-S", str(HERE / "eb_kernels.hip"), "-o", str(Path(tmp) / "k.s")]
        subprocess.run(cmd, check=True)
        return (Path(tmp) / "k.s").read_text()


def check(text: str) -> int:
    pattern = r"^(_ZN3ebk12_GLOBAL__N_1\d+(?:%s)\S*):[^\n]*\n(.*?)s_endpgm" % "|".join(KERNELS)
    problems = 0
    funcs = re.findall(pattern, text, re.M | re.S)
    for name, body in funcs:
        lines = [line.strip() for line in body.splitlines()]
        staged = [i for i, line in enumerate(lines) if line.startswith("global_load_lds")]
        if not staged:
            continue
        wait = next((i for i in range(staged[0], len(lines)) if lines[i].startswith("s_waitcnt vmcnt(")), None)
        if wait is None:
            print(f"no wait after the staging: {name}")
            problems += 1
            continue
        allowed = int(re.search(r"vmcnt\((\d+)\)", lines[wait]).group(1))
        last = max(i for i in staged if i < wait)
        after = [line for line in lines[last + 1:wait] if re.match(r"(global_load|buffer_load)", line)]
        if allowed > len(after):
            print(f"wait vmcnt({allowed}) with {len(after)} loads after the staging: {name}")
            problems += 1
    print(f"checked {len(funcs)} kernels, {problems} problems")
    return problems


if __name__ == "__main__":
    text = Path(sys.argv[1]).read_text() if len(sys.argv) > 1 else assembly()
    sys.exit(1 if check(text) else 0)
