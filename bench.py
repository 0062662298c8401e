"""ElasticBit linear benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-prefill] [--no-cpu]

Headline: decode GEMV, ElasticBit linear 4096->4096,
fp16 activations M=1, weights N(0,0.02) with 1% x8 outlier columns, compressed
by ElasticBit.compress at threshold 0.01 (the GPU width search picks b).  One
step is one fused unpack+dequant+GEMV launch over one weight copy; the copies
rotate over >= 512 MB so the 256 MB MALL cannot hold them, and the K steps are
queued behind a spin kernel and timed with HIP events on the stream the
kernels run on.  value = algorithmic bytes per step / time per step, with
bytes counted at the storage width: ceil(N*K*b/8) + 4N + 2MK + 2MN.

Also reported (not the headline): the prefill GEMM of configs[3] (4096->14336,
M=2048) in TFLOP/s, and the oracle's OpenMP CPU GEMV on the host's cores.

Every configuration beside the reference's execution format (markdown table):

    python bench.py --all-configs

The forward over activation row counts 1..2048 on several shapes:

    python bench.py --m-sweep

configs[4]'s compressed Linears, one decode token at a time:

    python bench.py --bolt-decode

The read ceiling (a kernel that only reads) over a range of sizes, timed the
same way (markdown table):

    python bench.py --ceiling-curve

Profiling helpers (same file, so the committed summaries name committed code):

    python bench.py --traffic-probe      # eager launches for rocprofv3 --pmc passes
    python bench.py --summarize-pmc FETCH.csv WRITE.csv    # -> profiles/*_traffic.md
    python bench.py --summarize-trace KERNEL_STATS.csv     # -> kernel table (markdown)
    python bench.py --counter-probe      # eager decode / prefill / hipBLASLt launches for counter passes
    python bench.py --summarize-counters A.csv B.csv C.csv  # -> per-kernel counter table (markdown)
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_PEAK_TFLOPS = 2516.6      # MI355X dense fp16 MFMA
MALL_BYTES = 256 << 20
# Calibration copy for the PMC byte counters: an fp16 -> fp32 conversion copy of
# this many elements reads exactly 2x and writes exactly 4x that many bytes.
COPY_CAL_ELEMS = 64 << 20
COPY_CAL_KERNEL = "float16tofloat32_copy_kernel"
DECODE_KERNEL = "linear_gemv_kernel"
PREFILL_KERNEL = "linear_prefill"          # the 256 x 256 and the 128 x 256 tile kernels
TRAFFIC_FILE = "decode_gemv_4096x4096_b10_m1_traffic.md"
PROBE_SRC = ROOT / "probe_read.hip"
PROBE_LIB = ROOT / "_build" / "libeb_probe_read.so"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--prefill-steps", type=int, default=20)
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-reference-route", action="store_true",
                   help="skip the timings of the reference's own execution formats on this GPU")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--traffic-probe", action="store_true",
                   help="run eager GEMV/prefill launches and a calibration copy for rocprofv3 --pmc")
    p.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    p.add_argument("--summarize-trace", metavar="KERNEL_STATS_CSV")
    p.add_argument("--counter-probe", action="store_true",
                   help="eager launches for rocprofv3 --pmc counter passes: the configs[1] GEMV, configs[3] "
                        "through both 256 x 256 prefill kernels, and hipBLASLt on resident fp16 weights")
    p.add_argument("--summarize-counters", nargs="+", metavar="COUNTER_CSV")
    p.add_argument("--bolt-decode", action="store_true",
                   help="configs[4]'s compressed Linears: one greedy decode token's 96 M = 1 forwards "
                        "(12 layers) plus the tied fp16 LM head, timed per token")
    p.add_argument("--m-sweep", action="store_true",
                   help="time the forward over activation row counts 1..2048 on several shapes; "
                        "prints a markdown table")
    p.add_argument("--ceiling-curve", action="store_true",
                   help="time the pure-read probe over 21 MB .. 1 GiB with the headline's timing; "
                        "prints a markdown table")
    p.add_argument("--build-probe", action="store_true", help="compile probe_read.hip and exit")
    p.add_argument("--all-configs", action="store_true",
                   help="time every BASELINE configuration (0-3) beside the reference's execution format; "
                        "prints a markdown table")
    return p.parse_args()


def make_weight(rows: int, cols: int):
    """configs[1..3] weights: randn*0.02 (seed 0), round(0.01*K) columns x8 (seed 3), fp16."""
    import torch

    w = torch.randn(rows, cols, generator=torch.Generator().manual_seed(0)) * 0.02
    idx = torch.randperm(cols, generator=torch.Generator().manual_seed(3))[: round(0.01 * cols)]
    w[:, idx] *= 8
    return w.half()


def compressed_layer(rows: int, cols: int, threshold: float, calib_rows: int):
    """Run the real ElasticBit.compress pipeline on one Linear (wrapped, as the
    root module cannot be replaced) and return the compressed layer."""
    import torch

    from mlbricks_amd import ElasticBit

    lin = torch.nn.Linear(cols, rows, bias=False)
    with torch.no_grad():
        lin.weight.copy_(make_weight(rows, cols).float())
    model = torch.nn.Sequential(lin).cuda().half().eval()
    calib = torch.randn(calib_rows, cols, generator=torch.Generator().manual_seed(2)).half()
    ElasticBit.compress(model, calib, threshold)
    return model[0]


def algorithmic_bytes(rows: int, cols: int, bits: int, M: int) -> int:
    payload = (rows * cols * bits + 7) // 8 if bits < 16 else 2 * rows * cols
    scales = 4 * rows if bits < 16 else 0
    return payload + scales + 2 * M * cols + 2 * M * rows


def copies_of(layer, count: int):
    """`count` independent RuntimeMatrix copies of the layer's canonical storage."""
    from mlbricks_amd.elasticbit import _native as native

    nm = layer.matrix._native
    scales, _ = nm._canonical()
    codes = nm._unpackCodesTorch().cpu().numpy()
    return [native.RuntimeMatrix._compressSelectedCodes(codes, scales, nm.storageBits, nm.threshold, nm.error)
            for _ in range(count)]


_SPIN_CYCLES_PER_MS = None
# Untimed work right before every timed run.  After seconds of host-side
# set-up the GPU starts below its working clock; with 2 ms of warm launches
# the first shape timed after a compression still measured ~10% slow.
WARM_MS = 25.0
LEAD_LAUNCHES = 200
CHUNK_LAUNCHES = 800


def _spin_cycles_per_ms() -> float:
    """Clock cycles per millisecond of torch's spin kernel (torch.cuda._sleep),
    measured once with HIP events."""
    global _SPIN_CYCLES_PER_MS
    if _SPIN_CYCLES_PER_MS is None:
        import torch

        probe = 2_000_000
        torch.cuda._sleep(probe)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        torch.cuda._sleep(probe)
        stop.record()
        stop.synchronize()
        _SPIN_CYCLES_PER_MS = probe / max(float(start.elapsed_time(stop)), 1e-3)
    return _SPIN_CYCLES_PER_MS


def time_launches(launches, steps: int, warmup: int, kernels_per_launch: int = 1) -> float:
    """Time exactly `steps` launches (cycling over `launches`) with HIP events
    on the launch stream.  Returns ms.  A launch may issue several kernels
    (`kernels_per_launch`); the limits below count kernels.

    First WARM_MS (and at least `warmup`) of untimed launches run as fast as
    the host issues them, so the GPU is at its working clock.  The timed
    launches then go in chunks of at most CHUNK_LAUNCHES: for each, a spin
    kernel holds the stream while the host queues behind it LEAD_LAUNCHES
    untimed launches, the start event, the chunk and the stop event, so the
    events bracket launches running back to back and the host's enqueue cost
    stays outside them.  The result is the sum over the chunks.  A chunk
    plus its lead stays within what the host can queue ahead of a held
    stream: measured on MI355X, 1000 to 2000 of this library's decode
    launches (their kernel arguments are ~400 bytes), beyond which the host
    waits for the spin to end.  A captured graph replay was measured to add
    ~4 us of device-side start-up per replay, which a short run would charge
    to its few steps; eager launches behind the spin do not."""
    import torch

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    n = len(launches)
    total = 0.0
    with torch.cuda.stream(stream):
        launches[0]()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        done = 0
        while (time.perf_counter() - t0) * 1e3 < WARM_MS or done < warmup:
            launches[done % n]()
            done += 1
        per_launch_ms = (time.perf_counter() - t0) * 1e3 / done
        lead = max(1, LEAD_LAUNCHES // kernels_per_launch)
        chunk = max(1, CHUNK_LAUNCHES // kernels_per_launch)
        first = 0
        while first < steps:
            count = min(chunk, steps - first)
            hold_ms = 1.5 * (lead + count) * per_launch_ms + 1.0
            for _ in range(6):
                start = torch.cuda.Event(enable_timing=True)
                stop = torch.cuda.Event(enable_timing=True)
                t_host = time.perf_counter()
                torch.cuda._sleep(int(_spin_cycles_per_ms() * hold_ms))
                for i in range(first - lead, first):
                    launches[i % n]()
                start.record(stream)
                for i in range(first, first + count):
                    launches[i % n]()
                stop.record(stream)
                enqueue_ms = (time.perf_counter() - t_host) * 1e3
                stop.synchronize()
                if enqueue_ms < 0.8 * hold_ms:
                    break
                hold_ms = 2.0 * enqueue_ms  # the host was slower than the spin: hold longer
            else:
                raise RuntimeError("could not queue the timed launches ahead of the GPU")
            total += float(start.elapsed_time(stop))
            first += count
    return total


def bench_gemv(args) -> dict:
    import torch

    rows = cols = 4096
    layer = compressed_layer(rows, cols, 0.01, 512)
    bits = layer.matrix.storageBits
    per_copy = layer.matrix.executionBytes
    n_copies = max(2, -(-2 * MALL_BYTES // per_copy) + 1)
    log(f"gemv 4096x4096: selected b={bits}, {n_copies} copies x {per_copy / 1e6:.1f} MB")
    mats = copies_of(layer, n_copies)
    x = torch.randn(1, cols, generator=torch.Generator().manual_seed(1)).half().cuda()
    outs = [torch.empty(1, rows, dtype=torch.float16, device="cuda") for _ in mats]
    launches = [lambda m=m, y=y: m.forwardTorch(x, out=y) for m, y in zip(mats, outs)]
    ms = time_launches(launches, args.steps, args.warmup)
    per_step_ms = ms / args.steps
    nbytes = algorithmic_bytes(rows, cols, bits, 1)
    gbs = nbytes / (per_step_ms * 1e-3) / 1e9
    log(f"gemv: {per_step_ms * 1e3:.3f} us/step, {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% HBM)")
    return {"bits": bits, "ms": ms, "per_step_ms": per_step_ms, "bytes": nbytes, "gbs": gbs,
            "copies": n_copies, "layer": layer}


def bench_prefill(args) -> dict:
    import torch

    rows, cols, M = 14336, 4096, 2048
    layer = compressed_layer(rows, cols, 0.01, 512)
    bits = layer.matrix.storageBits
    x = torch.randn(M, cols, generator=torch.Generator().manual_seed(1)).half().cuda()
    y = torch.empty(M, rows, dtype=torch.float16, device="cuda")
    nm = layer.matrix._native
    ms = time_launches([lambda: nm.forwardTorch(x, out=y)], args.prefill_steps, 3)
    per = ms / args.prefill_steps
    flops = 2.0 * M * rows * cols
    tflops = flops / (per * 1e-3) / 1e12
    log(f"prefill 4096->14336 M=2048 b={bits}: {per * 1e3:.1f} us, {tflops:.1f} TFLOP/s "
        f"({100 * tflops / FP16_PEAK_TFLOPS:.1f}% fp16 MFMA)")
    return {"workload": "ElasticBit linear 4096->14336, fp16 x M=2048, threshold 0.01 (configs[3])",
            "bits": bits, "us_per_launch": round(per * 1e3, 2), "tflops": round(tflops, 2),
            "frac_fp16_mfma_peak": round(tflops / FP16_PEAK_TFLOPS, 4)}


def build_probe(force: bool = False) -> Path:
    """Compile probe_read.hip (bench.py's own read probe) for gfx950."""
    import shutil
    import subprocess

    if PROBE_LIB.exists() and not force and PROBE_LIB.stat().st_mtime >= PROBE_SRC.stat().st_mtime:
        return PROBE_LIB
    PROBE_LIB.parent.mkdir(exist_ok=True)
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", str(PROBE_SRC), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"probe build failed: {res.stderr[-2000:]}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


# Launch shapes of the read probe's sweep: workgroups x threads, plain and
# nontemporal loads (the probe rejects shapes needing > 512 B per thread).
PROBE_SHAPES = tuple((b, t, nt) for nt in (0, 1)
                     for b, t in ((256, 1024), (512, 1024), (512, 512), (1024, 256), (1024, 512), (1024, 1024),
                                  (2048, 256), (2048, 512), (4096, 256)))


def read_ceiling(nbytes: int, copies: int, steps: int, warmup: int) -> dict:
    """Best per-launch time of a kernel that only reads `nbytes` (the GEMV's
    algorithmic bytes), over `copies` rotated buffers, launched and timed
    exactly as the GEMV: the most any one-launch-per-step kernel over those
    bytes reaches here.  Sweeps workgroup count and size, with plain and
    nontemporal loads."""
    import ctypes

    import torch

    lib = ctypes.CDLL(str(build_probe()))
    lib.eb_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_void_p, ctypes.c_void_p]
    size = -(-nbytes // 16) * 16
    bufs = [torch.empty(size, dtype=torch.uint8, device="cuda").random_(0, 255) for _ in range(copies)]
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    best = None
    for blocks, threads, nt in PROBE_SHAPES:
        def mk(buf, blocks=blocks, threads=threads, nt=nt):
            def launch():
                rc = lib.eb_probe_read(buf.data_ptr(), size, blocks, threads, nt, sink.data_ptr(),
                                       torch.cuda.current_stream().cuda_stream)
                if rc != 0:
                    raise RuntimeError(f"eb_probe_read: {rc}")
            return launch
        try:
            ms = time_launches([mk(b) for b in bufs], steps, warmup)
        except RuntimeError:
            continue
        us = ms / steps * 1e3
        if best is None or us < best[0]:
            best = (us, blocks, threads, nt)
    us, blocks, threads, nt = best
    gbs = nbytes / (us * 1e-6) / 1e9
    kind = "nontemporal" if nt else "plain"
    log(f"read ceiling: {us:.3f} us per {nbytes / 1e6:.1f} MB read ({gbs:.1f} GB/s, {blocks} x {threads}, {kind})")
    del bufs
    return {"us_per_launch": round(us, 3), "gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "launch": f"{blocks} workgroups x {threads} threads, {kind} loads",
            "what": "pure-read kernel (probe_read.hip) over the GEMV's algorithmic bytes, "
                    "same copy rotation and timing"}


def ceiling_curve(args) -> int:
    """The read probe's best time over a range of sizes, each rotated over at
    least twice the MALL and timed like the headline: how much of a launch is
    fixed cost and how close a read of a given size gets to the HBM peak."""
    sizes = (4 << 20, 8 << 20, 21_004_288, 56_435_200, 128 << 20, 256 << 20, 1 << 30)
    lines = ["| bytes per launch | us per launch | GB/s | % of 8 TB/s | best launch |", "|---|---|---|---|---|"]
    for nbytes in sizes:
        copies = max(2, -(-2 * MALL_BYTES // nbytes) + 1)
        steps = max(20, min(args.steps, int(2e6 // max(nbytes >> 10, 1))))
        r = read_ceiling(nbytes, copies, steps, max(3, steps // 10))
        lines.append(f"| {nbytes:,} | {r['us_per_launch']:.3f} | {r['gbs']:.0f} | {100 * r['frac_hbm_peak']:.1f} | "
                     f"{r['launch']} |")
    print("\n".join(lines), flush=True)
    print("\n" + vendor_reads(args), flush=True)
    return 0


def vendor_reads(args) -> str:
    """Kernels this build did not write, reading about the same bytes per
    launch, timed the same way over rotated copies: torch's sum over an fp16
    tensor (a reduction) and torch.matmul of one fp16 row by an fp16 matrix
    (hipBLASLt's M = 1 GEMM).  Independent points beside the probe for what
    one launch of that size reaches."""
    import torch

    lines = ["| kernel | bytes per launch | us per launch | GB/s | % of 8 TB/s |", "|---|---|---|---|---|"]
    for rows, cols in ((4096, 2560), (11008, 2560), (16384, 16384)):
        nbytes = 2 * rows * cols
        copies = max(2, -(-2 * MALL_BYTES // nbytes) + 1)
        steps = max(20, min(args.steps, int(2e6 // max(nbytes >> 10, 1))))
        ws = [torch.randn(rows, cols, device="cuda").half() for _ in range(copies)]
        x = torch.randn(1, cols, device="cuda").half()
        ys = [torch.empty(1, rows, dtype=torch.float16, device="cuda") for _ in ws]
        outs = [torch.empty((), dtype=torch.float16, device="cuda") for _ in ws]
        for label, fns in (("torch.sum (fp16)", [lambda w=w, o=o: torch.sum(w, dim=(0, 1), out=o) for w, o in zip(ws, outs)]),
                           ("torch.matmul, M = 1 (hipBLASLt)",
                            [lambda w=w, y=y: torch.matmul(x, w.t(), out=y) for w, y in zip(ws, ys)])):
            us = time_launches(fns, steps, max(3, steps // 10)) / steps * 1e3
            lines.append(f"| {label} | {nbytes:,} | {us:.3f} | {nbytes / us / 1e3:.0f} | "
                         f"{nbytes / us / 1e3 / HBM_PEAK_GBS * 100:.1f} |")
            log(f"vendor read: {label} {nbytes / 1e6:.1f} MB: {us:.3f} us")
        del ws, ys, outs
    return "\n".join(lines)


def reference_route(args) -> dict:
    """The reference's own execution formats, timed on this GPU with the same
    methods (informational; never `value`).  Decode: at b = 9..15 the
    reference executes W16A16 (elasticbit_runtime.cu:240-244,1174-1178), a
    GEMV over fp16 weights, 2 bytes per weight; here that is this build's
    GEMV kernel over b = 16 storage of the same weights.  Prefill: at
    b = 9..15 the reference keeps the fp16 weights resident and hands
    F.linear a zero-copy view of them (runtime.cu:989-999, core.py:462-471);
    here torch.matmul (hipBLASLt) on an fp16 copy decoded once, outside the
    timed region."""
    import torch

    from mlbricks_amd.elasticbit import _native as native

    out = {}
    rows = cols = 4096
    w = make_weight(rows, cols).float().numpy()
    per = 2 * rows * cols
    n_copies = max(2, -(-2 * MALL_BYTES // per) + 1)
    mats = [native.RuntimeMatrix._compressSelected(w, 16, 0.01, 0.0) for _ in range(n_copies)]
    x = torch.randn(1, cols, generator=torch.Generator().manual_seed(1)).half().cuda()
    ys = [torch.empty(1, rows, dtype=torch.float16, device="cuda") for _ in mats]
    ms = time_launches([lambda m=m, y=y: m.forwardTorch(x, out=y) for m, y in zip(mats, ys)], args.steps, args.warmup)
    us = ms / args.steps * 1e3
    nbytes = algorithmic_bytes(rows, cols, 16, 1)
    out["decode_w16"] = {"us_per_launch": round(us, 3), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                         "bytes_per_launch": nbytes,
                         "what": "configs[1] as W16A16 (fp16 weights, the reference's format at b = 9..15), "
                                 f"{n_copies} rotated copies"}
    log(f"reference route, decode W16: {us:.3f} us/launch ({out['decode_w16']['gbs']} GB/s on 2 B/weight)")
    del mats, ys
    prows, pcols, M = 14336, 4096, 2048
    layer = compressed_layer(prows, pcols, 0.01, 512)
    nm = layer.matrix._native
    xp = torch.randn(M, pcols, generator=torch.Generator().manual_seed(1)).half().cuda()
    yp = torch.empty(M, prows, dtype=torch.float16, device="cuda")
    if nm.storageBits >= 9:
        resident = nm._materializeTorch()          # decoded once, outside the timed region
        ms = time_launches([lambda: torch.matmul(xp, resident.t(), out=yp)], args.prefill_steps, 3)
        what = ("configs[3] as the reference runs it at b = 9..15: torch.matmul (hipBLASLt) on resident fp16 "
                "weights (runtime.cu:989-999)")
    else:
        wbuf = torch.empty(prows, pcols, dtype=torch.float16, device="cuda")

        def materialize_then_linear():
            native.check(native.lib().eb_materialize_fp16(nm._h, wbuf.data_ptr(), native.stream_handle(wbuf.device)))
            torch.matmul(xp, wbuf.t(), out=yp)

        ms = time_launches([materialize_then_linear], args.prefill_steps, 3)
        what = "configs[3] as the reference runs it at b <= 8: materialize to fp16, then torch.matmul"
    us = ms / args.prefill_steps * 1e3
    flops = 2.0 * M * prows * pcols
    out["prefill"] = {"us_per_launch": round(us, 2), "tflops": round(flops / (us * 1e-6) / 1e12, 1), "what": what}
    log(f"reference route, prefill: {us:.1f} us/launch ({what})")
    return out


def all_configs(args) -> int:
    """Every BASELINE configuration that runs on one GPU, compressed by the
    real ElasticBit.compress, timed like the headline (spin-held launches, events on
    the launch stream, weight copies rotated past the MALL for M <= 16),
    beside the reference's execution format on the same weights: W16A16
    decode for M = 1 at b = 9..15 (this build's GEMV over fp16 storage), and
    for M > 1 F.linear (core.py:462-471) on resident fp16 weights at
    b = 9..15 (runtime.cu:989-999) or on weights materialized per call at
    b <= 8 (runtime.cu:1001-1021).  Where our launches rotate over weight
    copies, so do the reference's (fp16 copies)."""
    import torch

    from mlbricks_amd.elasticbit import _native as native

    def weight0(rows, cols):
        # N(0, 0.02) from seed 0, no outlier columns
        return (torch.randn(rows, cols, generator=torch.Generator().manual_seed(0)) * 0.02).half()

    def compress(rows, cols, thr, calib_rows, outliers=True):
        from mlbricks_amd import ElasticBit

        lin = torch.nn.Linear(cols, rows, bias=False)
        with torch.no_grad():
            lin.weight.copy_((make_weight(rows, cols) if outliers else weight0(rows, cols)).float())
        model = torch.nn.Sequential(lin).cuda().half().eval()
        calib = torch.randn(calib_rows, cols, generator=torch.Generator().manual_seed(2)).half()
        ElasticBit.compress(model, calib, thr)
        return model[0]

    def ours(mats, M, steps):
        cols, rows = mats[0].cols, mats[0].rows
        x = torch.randn(M, cols, generator=torch.Generator().manual_seed(1)).half().cuda()
        ys = [torch.empty(M, rows, dtype=torch.float16, device="cuda") for _ in mats]
        ms = time_launches([lambda m=m, y=y: m.forwardTorch(x, out=y) for m, y in zip(mats, ys)], steps, steps // 10)
        return ms / steps * 1e3

    def reference(mats, M, steps):
        nm = mats[0]
        cols, rows = nm.cols, nm.rows
        x = torch.randn(M, cols, generator=torch.Generator().manual_seed(1)).half().cuda()
        if M == 1 and nm.storageBits >= 9:
            w16 = [native.RuntimeMatrix._compressSelected(m._materializeTorch().float().cpu().numpy(), 16, 0.01, 0.0)
                   for m in mats[: max(2, -(-2 * MALL_BYTES // (2 * rows * cols)) + 1)]]
            ys = [torch.empty(1, rows, dtype=torch.float16, device="cuda") for _ in w16]
            ms = time_launches([lambda m=m, y=y: m.forwardTorch(x, out=y) for m, y in zip(w16, ys)], steps, steps // 10)
            return ms / steps * 1e3, "W16A16 GEMV"
        if M == 1:
            return None, "W4/W8 GEMV (not timed)"
        y = torch.empty(M, rows, dtype=torch.float16, device="cuda")
        if nm.storageBits >= 9:
            keep = mats[: max(1, min(len(mats), -(-2 * MALL_BYTES // (2 * rows * cols)) + 1))]
            w16s = [m._materializeTorch() for m in keep]      # resident, decoded outside the timing
            ms = time_launches([lambda w=w: torch.matmul(x, w.t(), out=y) for w in w16s], steps, steps // 10)
            return ms / steps * 1e3, "resident fp16 + F.linear"
        wbuf = torch.empty(rows, cols, dtype=torch.float16, device="cuda")

        def mk(m):
            def run():
                native.check(native.lib().eb_materialize_fp16(m._h, wbuf.data_ptr(), native.stream_handle(wbuf.device)))
                torch.matmul(x, wbuf.t(), out=y)
            return run
        ms = time_launches([mk(m) for m in mats], steps, steps // 10)
        return ms / steps * 1e3, "materialize + F.linear"

    lines = ["| config | N x K | thr | b | M | ours us | GB/s (% HBM) | TFLOP/s (% fp16) | reference route | ref us |",
             "|---|---|---|---|---|---|---|---|---|---|"]

    def row(cfg, layer, thr, Ms, rotate):
        nm = layer.matrix._native
        rows, cols, bits = nm.rows, nm.cols, nm.storageBits
        n_copies = max(2, -(-2 * MALL_BYTES // nm.executionBytes) + 1) if rotate else 1
        mats = copies_of(layer, n_copies) if n_copies > 1 else [nm]
        for M in Ms:
            steps = 1000 if M <= 16 else 50
            us = ours(mats, M, steps)
            nbytes = algorithmic_bytes(rows, cols, bits, M)
            gbs = nbytes / (us * 1e-6) / 1e9
            tf = 2.0 * M * rows * cols / (us * 1e-6) / 1e12
            ref_us, ref_what = reference(mats, M, 200 if M <= 16 else 20)
            ref_txt = f"{ref_us:.2f}" if ref_us is not None else "-"
            lines.append(f"| {cfg} | {rows} x {cols} | {thr} | {bits} | {M} | {us:.2f} | {gbs:.0f} "
                         f"({100 * gbs / HBM_PEAK_GBS:.1f}%) | {tf:.1f} ({100 * tf / FP16_PEAK_TFLOPS:.1f}%) | "
                         f"{ref_what} | {ref_txt} |")
            log(lines[-1])
        del mats

    row("configs[0]", compress(1536, 384, 0.01, 256, outliers=False), 0.01, (256,), rotate=False)
    row("configs[1]", compress(4096, 4096, 0.01, 512), 0.01, (1,), rotate=True)
    for thr in (0.005, 0.01, 0.02):
        for rows, cols in ((11008, 4096), (4096, 11008)):
            row("configs[2]", compress(rows, cols, thr, 512), thr, (1, 4, 16), rotate=True)
    row("configs[3]", compress(14336, 4096, 0.01, 512), 0.01, (2048,), rotate=False)
    print("\n".join(lines), flush=True)
    return 0


# configs[4]'s per-layer compressed Linears (out, in, bias), in block order:
# avq.project, q/k/v/out_proj, head_gate (zero-initialised), fc, proj
# (bolt/presets.py:93,155; bolt/enhanced_mqa.py:128-135; components.py:209-220).
BOLT_LINEARS = (("avq.project", 2048, 1024, True), ("q_proj", 1024, 1024, False), ("k_proj", 64, 1024, False),
                ("v_proj", 64, 1024, False), ("out_proj", 1024, 1024, False), ("head_gate", 16, 1024, True),
                ("fc", 4096, 1024, False), ("proj", 1024, 4096, False))


def bolt_decode(args) -> int:
    """The compressed-Linear share of one configs[4] greedy decode token
    (bolt/model.py:416-431): 12 layers x 8 ElasticBit Linears at M = 1, each
    through the public module forward, plus the tied fp16 LM head
    (32000 x 1024, F.linear).  The attention, retention and norm kernels
    between them are not part of this build, so the tokens/s printed is a
    ceiling set by the Linears alone.  Weights: nn.Linear's default init
    under seed 0 (head_gate zero), compressed by ElasticBit.compress at
    threshold 0.01 with 32 seeded N(0,1) calibration rows per Linear.  The
    timed launches run whole tokens back to back, as a decode loop does, so
    whatever of the model fits in the MALL stays there as it would in a real
    run."""
    import torch
    import torch.nn.functional as F

    from mlbricks_amd import ElasticBit
    from mlbricks_amd.elasticbit.core import RuntimeMatrix

    torch.manual_seed(0)
    layers = []
    for li in range(12):
        block = []
        for name, out_f, in_f, bias in BOLT_LINEARS:
            lin = torch.nn.Linear(in_f, out_f, bias=bias)
            if name == "head_gate":
                torch.nn.init.zeros_(lin.weight)
            model = torch.nn.Sequential(lin).cuda().half().eval()
            calib = torch.randn(32, in_f, generator=torch.Generator().manual_seed(2 + 100 * li + len(block))).half()
            ElasticBit.compress(model, calib, 0.01)
            block.append(model[0])
        layers.append(block)
    emb = (torch.randn(32000, 1024, generator=torch.Generator().manual_seed(0)) * 0.02).half().cuda()
    xs = {w: torch.randn(1, w, generator=torch.Generator().manual_seed(1)).half().cuda() for w in (1024, 4096)}
    widths = {}
    nbytes = 0
    for block in layers:
        for (name, out_f, in_f, _), lin in zip(BOLT_LINEARS, block):
            b = lin.matrix.storageBits
            widths[b] = widths.get(b, 0) + 1
            nbytes += algorithmic_bytes(out_f, in_f, b, 1)
    head_bytes = 2 * 32000 * 1024 + 2 * 1024 + 2 * 32000
    log(f"bolt decode: widths {dict(sorted(widths.items()))}, {nbytes / 1e6:.1f} MB of compressed Linears per token")

    def token_separate():
        for block in layers:
            for (name, _, in_f, _), lin in zip(BOLT_LINEARS, block):
                lin(xs[in_f])
        F.linear(xs[1024], emb)

    def token_fused():
        # q, k, v and head_gate read the same activations: one multi-matrix
        # launch per run of equal widths
        for block in layers:
            block[0](xs[1024])
            group = [block[1], block[2], block[3], block[5]]
            RuntimeMatrix.forwardTorchMulti([l.matrix for l in group], xs[1024], [l.bias for l in group])
            block[4](xs[1024])
            block[6](xs[1024])
            block[7](xs[4096])
        F.linear(xs[1024], emb)

    def head_only():
        F.linear(xs[1024], emb)

    tokens = 20
    rows = []
    for label, fn, kernels in (("96 Linears + LM head", token_separate, 97),
                               ("q/k/v/head_gate fused + LM head", token_fused, 97),
                               ("LM head alone", head_only, 1)):
        us = time_launches([fn], tokens, 3, kernels) / tokens * 1e3
        rows.append((label, us))
        log(f"  {label}: {us:.1f} us per token")
    head_us = rows[2][1]
    lines = ["| per token | us | tokens/s ceiling | Linears' GB/s |", "|---|---|---|---|"]
    for label, us in rows[:2]:
        lin_us = us - head_us
        lines.append(f"| {label} | {us:.1f} | {1e6 / us:.0f} | {nbytes / lin_us / 1e3:.0f} over {lin_us:.1f} us |")
    lines.append(f"| {rows[2][0]} | {head_us:.1f} | - | {head_bytes / head_us / 1e3:.0f} (fp16 head) |")
    # As a decode loop would run the fused token: issued from Python with
    # nothing holding the GPU (the host's per-launch cost shows), and as one
    # captured HIP graph replayed per token.
    with torch.inference_mode():
        for _ in range(3):
            token_fused()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(200):
            token_fused()
        torch.cuda.synchronize()
        eager_us = (time.perf_counter() - t0) / 200 * 1e6
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            token_fused()
        graph_us = time_launches([graph.replay], tokens, 3, 97) / tokens * 1e3
    log(f"  fused token issued from Python: {eager_us:.1f} us; as one HIP graph: {graph_us:.1f} us")
    lines.append(f"| fused token issued from Python, GPU not held (wall clock) | {eager_us:.1f} | {1e6 / eager_us:.0f} | - |")
    lines.append(f"| fused token as one captured HIP graph per token | {graph_us:.1f} | {1e6 / graph_us:.0f} | - |")
    print(f"configs[4] compressed Linears: widths {dict(sorted(widths.items()))}; "
          f"{nbytes:,} B of compressed Linears + {head_bytes:,} B fp16 head per token", flush=True)
    print("\n".join(lines), flush=True)
    return 0


def m_sweep(args) -> int:
    """The forward over activation row counts on several shapes (b = 10,
    synthetic codes), timed like the headline: every launch reads a weight
    copy other than the last ones read (>= 512 MB of rotated copies, twice
    the MALL), so no M is helped by a warm cache.  Shows where the launcher
    moves between its kernels (GEMV, decode with 1/2/4 activation blocks,
    row-blocked decode, prefill tiles)."""
    import numpy as np
    import torch

    from mlbricks_amd.elasticbit import _native as native

    shapes = ((4096, 4096), (11008, 4096), (4096, 11008), (14336, 4096), (1024, 1024), (1536, 384))
    Ms = (1, 4, 8, 12, 16, 17, 32, 64, 96, 128, 256, 512, 1024, 2048)
    lines = ["| N x K | " + " | ".join(f"M={M}" for M in Ms) + " |", "|---" * (len(Ms) + 1) + "|"]
    for rows, cols in shapes:
        rng = np.random.default_rng(rows + cols)
        qm = 511
        mats = []
        per = None
        while per is None or len(mats) * per < 2 * MALL_BYTES + per:
            q = rng.integers(-qm, qm + 1, size=(rows, cols)).astype(np.int16)
            s = rng.uniform(1e-4, 1e-3, size=rows).astype(np.float32)
            mats.append(native.RuntimeMatrix._compressSelectedCodes(q, s, 10, 0.01, 0.0))
            per = mats[0].executionBytes
        cells = []
        for M in Ms:
            x = torch.randn(M, cols, generator=torch.Generator().manual_seed(1)).half().cuda()
            ys = [torch.empty(M, rows, dtype=torch.float16, device="cuda") for _ in mats]
            steps = 400 if M <= 64 else max(40, len(mats))
            ms = time_launches([lambda m=m, y=y: m.forwardTorch(x, out=y) for m, y in zip(mats, ys)], steps, 3)
            cells.append(f"{ms / steps * 1e3:.1f}")
        lines.append(f"| {rows} x {cols} | " + " | ".join(cells) + " |")
        log(lines[-1])
        del mats
    print("\n".join(lines), flush=True)
    return 0


def cpu_baseline(layer, seconds: float) -> dict:
    """The oracle's OpenMP GEMV (fp32 accumulate) over the same matrix and the
    same algorithmic bytes, on every core this process may use (bounded to
    ~`seconds`); beside it torch's fp32 F.linear on the CPU over the decoded
    weights, the secondary CPU baseline of the benchmark definition."""
    import numpy as np
    import torch

    from oracle import oracle as ora

    nm = layer.matrix._native
    rows, cols, bits = nm.rows, nm.cols, nm.storageBits
    scales, payload = nm._canonical()
    x16 = torch.randn(1, cols, generator=torch.Generator().manual_seed(1)).half().numpy().view(np.uint16)
    cores = len(os.sched_getaffinity(0))
    threads = cores
    ora.gemv_f32_baseline(payload, scales, rows, cols, bits, x16, threads=threads)   # warm-up
    reps = 0
    t0 = time.perf_counter()
    while True:
        _, used = ora.gemv_f32_baseline(payload, scales, rows, cols, bits, x16, threads=threads)
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    per = elapsed / reps
    nbytes = algorithmic_bytes(rows, cols, bits, 1)
    gbs = nbytes / per / 1e9
    log(f"cpu baseline: {per * 1e3:.2f} ms/GEMV on {used} threads ({cores} cores visible): {gbs:.2f} GB/s")
    # torch's fp32 F.linear over the decoded weights (the bytes are still
    # counted at the storage width, as for every line of this benchmark)
    wf = torch.from_numpy(np.asarray(ora.dequantize(payload, scales, rows, cols, bits)[0]))
    xf = torch.from_numpy(x16.view(np.float16).astype(np.float32))
    torch.nn.functional.linear(xf, wf)
    treps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds / 2:
        torch.nn.functional.linear(xf, wf)
        treps += 1
    tper = (time.perf_counter() - t0) / treps
    log(f"cpu torch fp32 F.linear: {tper * 1e3:.2f} ms on {torch.get_num_threads()} threads")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": int(used), "kind": "port",
            "sample": f"{reps} full 4096x4096 b={bits} M=1 GEMVs ({elapsed:.1f} s), oracle/eb_oracle.c "
                      f"ebo_gemv_f32_baseline, OpenMP over rows; {cores} cores visible",
            "torch_fp32_linear": {"value": round(nbytes / tper / 1e9, 3), "unit": "GB/s",
                                  "threads": int(torch.get_num_threads()), "ms_per_call": round(tper * 1e3, 3),
                                  "sample": f"{treps} calls of torch.nn.functional.linear(x.float(), W_decoded_f32) "
                                            "on the CPU"}}


def traffic_probe(args) -> int:
    """Eager launches to be counted by `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE`: the
    headline GEMV over its rotated copies, the prefill GEMM, and COPY_CAL_ELEMS-element
    fp16 -> fp32 copies whose true read and write bytes are known."""
    import torch

    rows = cols = 4096
    layer = compressed_layer(rows, cols, 0.01, 512)
    mats = copies_of(layer, max(2, -(-2 * MALL_BYTES // layer.matrix.executionBytes) + 1))
    x = torch.randn(1, cols, generator=torch.Generator().manual_seed(1)).half().cuda()
    y = torch.empty(1, rows, dtype=torch.float16, device="cuda")
    for i in range(args.steps):
        mats[i % len(mats)].forwardTorch(x, out=y)
    torch.cuda.synchronize()
    log(f"probe: {args.steps} GEMV launches, b={layer.matrix.storageBits}")
    src = torch.randn(COPY_CAL_ELEMS, device="cuda").half()
    dst = torch.empty(COPY_CAL_ELEMS, dtype=torch.float32, device="cuda")
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"probe: 4 calibration copies of {COPY_CAL_ELEMS} fp16 -> fp32 elements")
    if not args.no_prefill:
        big = compressed_layer(14336, 4096, 0.01, 512)
        xp = torch.randn(2048, 4096, generator=torch.Generator().manual_seed(1)).half().cuda()
        yp = torch.empty(2048, 14336, dtype=torch.float16, device="cuda")
        for _ in range(4):
            big.matrix._native.forwardTorch(xp, out=yp)
        torch.cuda.synchronize()
        log(f"probe: 4 prefill launches, b={big.matrix.storageBits}")
    return 0


def counter_probe(args) -> int:
    """Eager launches whose counters `--summarize-counters` compares: the
    headline GEMV, configs[3] through the eight-wave and the
    four-wave 256 x 256 prefill kernels, and torch.matmul (hipBLASLt) on
    the same weights decoded to resident fp16 (the reference's route)."""
    import torch

    from mlbricks_amd.elasticbit import _native as native

    layer = compressed_layer(4096, 4096, 0.01, 512)
    mats = copies_of(layer, max(2, -(-2 * MALL_BYTES // layer.matrix.executionBytes) + 1))
    x = torch.randn(1, 4096, generator=torch.Generator().manual_seed(1)).half().cuda()
    y = torch.empty(1, 4096, dtype=torch.float16, device="cuda")
    for i in range(args.steps):
        mats[i % len(mats)].forwardTorch(x, out=y)
    torch.cuda.synchronize()
    log(f"probe: {args.steps} GEMV launches")
    big = compressed_layer(14336, 4096, 0.01, 512).matrix._native
    xp = torch.randn(2048, 4096, generator=torch.Generator().manual_seed(1)).half().cuda()
    yp = torch.empty(2048, 14336, dtype=torch.float16, device="cuda")
    for mode in ("wide8", "wide"):
        native.set_prefill_tiles(mode)
        for _ in range(4):
            big.forwardTorch(xp, out=yp)
        torch.cuda.synchronize()
        log(f"probe: 4 prefill launches, {mode} tiles, b={big.storageBits}")
    native.set_prefill_tiles("auto")
    resident = big._materializeTorch()
    for _ in range(4):
        torch.matmul(xp, resident.t(), out=yp)
    torch.cuda.synchronize()
    log("probe: 4 torch.matmul launches on resident fp16")
    return 0


def summarize_counters(paths: list[str]) -> int:
    """Per-kernel averages of counter passes over `--counter-probe`, with the
    clock (GRBM_GUI_ACTIVE per XCD over the dispatch's duration) and the
    MFMA-busy fraction of the SIMDs over those cycles.  Of each kernel only
    the launch shape (name, grid) that ran most often counts, without its
    first dispatch (warm-up): the calibration forwards of the compression
    run hipBLASLt GEMMs of other shapes.  Clock and MFMA-busy are left out
    for kernels under 20 us, where the counter's window around the dispatch
    is not small beside it."""
    import collections
    import csv
    import statistics

    wanted = ("linear_gemv_kernel", "linear_prefill_pp_kernel", "linear_prefill_wide_kernel", "Cijk")
    table: dict[str, dict[str, list[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for path in paths:
        per: dict[int, dict] = collections.defaultdict(dict)
        for r in csv.DictReader(open(path, newline="")):
            d = per[int(r["Dispatch_Id"])]
            d["name"] = r["Kernel_Name"]
            d["shape"] = (r["Kernel_Name"], r["Grid_Size"])
            d[r["Counter_Name"]] = float(r["Counter_Value"])
            d["duration_us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        runs: dict[str, dict[tuple, list[dict]]] = collections.defaultdict(lambda: collections.defaultdict(list))
        for did in sorted(per):
            key = next((w for w in wanted if w in per[did]["name"]), None)
            if key is not None:
                runs[key][per[did]["shape"]].append(per[did])
        for key, shapes in runs.items():
            for d in max(shapes.values(), key=len)[1:]:      # first dispatch: warm-up
                for k, v in d.items():
                    if k not in ("name", "shape"):
                        table[key][k].append(v)
    cols = sorted({k for t in table.values() for k in t if k not in ("duration_us",)})
    lines = ["| kernel | dispatches | us | clock GHz | MFMA busy | " + " | ".join(cols) + " |",
             "|---" * (len(cols) + 5) + "|"]
    for key in wanted:
        if key not in table:
            continue
        t = table[key]
        avg = {k: statistics.mean(v) for k, v in t.items()}
        n = max(len(v) for v in t.values())
        grbm = avg.get("GRBM_GUI_ACTIVE", 0.0) / 8 if avg["duration_us"] >= 20 else 0.0   # eight XCDs
        ghz = grbm / (avg["duration_us"] * 1e3) if grbm else float("nan")
        busy = avg["SQ_VALU_MFMA_BUSY_CYCLES"] / (grbm * 1024) if grbm and "SQ_VALU_MFMA_BUSY_CYCLES" in avg \
            else float("nan")
        name = "hipBLASLt fp16 GEMM (resident weights)" if key == "Cijk" else key
        lines.append(f"| `{name}` | {n} | {avg['duration_us']:.2f} | {ghz:.3f} | {busy:.3f} | "
                     + " | ".join(f"{avg[c]:.4g}" if c in avg else "-" for c in cols) + " |")
    print("\n".join(lines))
    return 0


def _pmc_rows(path: str, counter: str) -> dict:
    """{kernel name: [per-dispatch counter values]} from a rocprofv3 counter_collection.csv."""
    import collections
    import csv

    out = collections.defaultdict(list)
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                out[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return out


def _pick(rows: dict, needle: str) -> list:
    vals = [v for name, vs in rows.items() if needle in name for v in vs]
    if not vals:
        raise SystemExit(f"no dispatch of a kernel named *{needle}* in the counter file")
    return vals


def summarize_pmc(fetch_csv: str, write_csv: str) -> int:
    """Markdown summary of the FETCH_SIZE and WRITE_SIZE passes (KiB per dispatch),
    each counter scaled by the factor that maps the calibration copy's reading onto
    its known bytes.  Prints the GEMV's `traffic_bytes_per_launch` for bench.py."""
    import statistics

    fetch = _pmc_rows(fetch_csv, "FETCH_SIZE")
    write = _pmc_rows(write_csv, "WRITE_SIZE")
    # The calibration copies are the largest fp16->fp32 copies in the run.
    cf = _pick(fetch, COPY_CAL_KERNEL)
    cw = _pick(write, COPY_CAL_KERNEL)
    cf = [v for v in cf if v >= 0.5 * max(cf)]
    cw = [v for v in cw if v >= 0.5 * max(cw)]
    true_read, true_write = 2 * COPY_CAL_ELEMS, 4 * COPY_CAL_ELEMS
    f_fetch = true_read / (statistics.mean(cf) * 1024)
    f_write = true_write / (statistics.mean(cw) * 1024)
    lines = [
        "# HBM traffic per launch: decode GEMV and prefill GEMM (rocprofv3 PMC)",
        "",
        "Workloads: decode GEMV 4096x4096, M=1 (BASELINE configs[1], the bench headline); "
        "prefill GEMM 4096->14336, M=2048 (configs[3]). Weights compressed by ElasticBit.compress "
        "at threshold 0.01, b selected by the width search.",
        "",
        "Commands (one MI355X, repository root):",
        "",
        "    timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE -f csv -d gpurun_out/pmc_fetch -o fetch -- python -u bench.py --traffic-probe --steps 200",
        "    timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE -f csv -d gpurun_out/pmc_write -o write -- python -u bench.py --traffic-probe --steps 200",
        "    python bench.py --summarize-pmc gpurun_out/pmc_fetch/fetch_counter_collection.csv gpurun_out/pmc_write/write_counter_collection.csv",
        "",
        f"Calibration: `{COPY_CAL_KERNEL}` over {COPY_CAL_ELEMS} elements reads {true_read} B and "
        f"writes {true_write} B. It reads FETCH_SIZE {statistics.mean(cf):.1f} KiB and WRITE_SIZE "
        f"{statistics.mean(cw):.1f} KiB per dispatch ({len(cf)} dispatches), so bytes = "
        f"FETCH_SIZE x 1024 x {f_fetch:.4f} and WRITE_SIZE x 1024 x {f_write:.4f}.",
        "",
        "| kernel | dispatches | FETCH_SIZE KiB (avg) | WRITE_SIZE KiB (avg) | scaled read B | scaled write B | traffic B |",
        "|---|---|---|---|---|---|---|",
    ]
    # One launch of the path may be several dispatches (the prefill runs its
    # full tiles and its half tiles as two kernels): per-launch traffic sums
    # the per-dispatch averages of each distinct kernel.
    result = {}
    for needle in (DECODE_KERNEL, PREFILL_KERNEL):
        names = sorted(n for n in fetch if needle in n)
        if not names:
            continue
        total = 0.0
        for name in names:
            fv, wv = fetch[name], write.get(name, [0.0])
            rd = statistics.mean(fv) * 1024 * f_fetch
            wr = statistics.mean(wv) * 1024 * f_write
            total += rd + wr
            short = name.replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]
            lines.append(f"| `{short}` | {len(fv)} | {statistics.mean(fv):.1f} | {statistics.mean(wv):.1f} | "
                         f"{rd:.0f} | {wr:.0f} | {rd + wr:.0f} |")
        result[needle] = int(round(total))
    lines.append("")
    if DECODE_KERNEL in result:
        lines.append(f"traffic_bytes_per_launch: {result[DECODE_KERNEL]}")
    if PREFILL_KERNEL in result:
        lines.append(f"prefill_traffic_bytes_per_launch: {result[PREFILL_KERNEL]}")
    print("\n".join(lines))
    return 0


def summarize_trace(stats_csv: str) -> int:
    """Markdown table of the ElasticBit kernels in a rocprofv3 kernel_stats.csv."""
    import csv

    print("| kernel | calls | avg us | min us | max us |")
    print("|---|---|---|---|---|")
    with open(stats_csv, newline="") as f:
        for r in csv.DictReader(f):
            name = r["Name"]
            if "ebk::" not in name:
                continue
            short = name.replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]
            print(f"| `{short}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.3f} | "
                  f"{float(r['MinNs']) / 1e3:.3f} | {float(r['MaxNs']) / 1e3:.3f} |")
    return 0


def measured_traffic() -> int | None:
    """HBM bytes per GEMV launch from the committed rocprofv3 PMC summary, if present."""
    path = ROOT / "profiles" / TRAFFIC_FILE
    if not path.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", path.read_text())
    return int(m.group(1)) if m else None


def main() -> int:
    args = parse_args()
    if args.summarize_pmc:
        return summarize_pmc(*args.summarize_pmc)
    if args.summarize_trace:
        return summarize_trace(args.summarize_trace)
    if args.build_probe:
        print(build_probe(force=True))
        return 0
    if args.summarize_counters:
        return summarize_counters(args.summarize_counters)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the ElasticBit path is "
              "benchmarked on a single MI355X.", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    import mlbricks_amd.elasticbit._native  # noqa: F401  fail loudly if the HIP library is missing

    if args.traffic_probe:
        return traffic_probe(args)
    if args.counter_probe:
        return counter_probe(args)
    if args.all_configs:
        return all_configs(args)
    if args.ceiling_curve:
        return ceiling_curve(args)
    if args.m_sweep:
        return m_sweep(args)
    if args.bolt_decode:
        return bolt_decode(args)

    g = bench_gemv(args)
    ceiling = read_ceiling(g["bytes"], g["copies"], args.steps, args.warmup)
    prefill = None if args.no_prefill else bench_prefill(args)
    reference = None if args.no_reference_route else reference_route(args)
    cpu = None if args.no_cpu else cpu_baseline(g["layer"], args.cpu_seconds)
    achieved = g["bytes"] / (g["per_step_ms"] * 1e-3) / 1e9
    line = {
        "metric": "ElasticBit linear GB/s (%HBM peak) at M=1; TFLOP/s (%MFMA peak) at M=2048",
        "value": round(g["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["per_step_ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: BASELINE seeds, weights N(0,0.02) with 1% x8 outlier columns, x N(0,1)",
        "config": {
            "workload": "decode GEMV: ElasticBit linear 4096->4096, fp16 x M=1, threshold 0.01 (configs[1])",
            "storage_bits": g["bits"],
            "weight_copies_rotated": g["copies"],
            "bytes_per_step": g["bytes"],
            "timing": "HIP events on the launch stream around exactly `steps` launches, after >= 25 ms of "
                      "untimed warm launches, in chunks of <= 800 launches each queued behind its own spin "
                      "kernel and 200 untimed launches; the sum over the chunks",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "read_ceiling": ceiling,
            "frac_of_read_ceiling": round(ceiling["us_per_launch"] / (g["per_step_ms"] * 1e3), 4),
        },
        "cpu_baseline": cpu,
        "prefill": prefill,
        "reference_route": reference,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
