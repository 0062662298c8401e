"""Write the ElasticBit golden fixtures from numpy / pure-Python closed forms.

The MLBricks reference ships no golden vectors or known-answer tests for the
ElasticBit path and cannot run here (CUDA-only).  These fixtures are computed
from the mathematical definitions in ``mlbricks/elasticbit/csrc/
elasticbit_runtime.cu`` using code that shares nothing with the C oracle:

* scales  s_r = f32(max|w_r|) / f32(qmax), 1 when the row is zero   (:83-101)
* codes   q = clip(rint_even(f32(w) / s), -qmax, qmax)               (:77-81)
* payload the little-endian integer sum_i (q_i + qmax) << (i*b)      (:150-186)
* decoded numpy.float16(f32(q) * s) bit patterns                     (:208-238)
* outputs float64 matrix products of the decoded semantics           (:538-647)
* MLB4    struct-packed header + FNV-1a-64 written in Python         (:682-712)
* legacy  group-scale op with offset 2^(b-1), flat groups             (bolt/ops_cuda.cu:2708-2750)
* analyzer errors from a pure-Python float32 sequential restatement   (:280-392)

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import math
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent
F32 = np.float32


def qmax(b: int) -> int:
    return (1 << (b - 1)) - 1


def scales_closed_form(w32: np.ndarray, b: int) -> np.ndarray:
    mx = np.abs(w32).max(axis=1).astype(F32)
    s = (mx / F32(qmax(b))).astype(F32)
    return np.where(mx > 0, s, F32(1.0)).astype(F32)


def codes_closed_form(w32: np.ndarray, s: np.ndarray, b: int) -> np.ndarray:
    ratio = (w32 / s[:, None]).astype(F32)
    return np.clip(np.rint(ratio), -qmax(b), qmax(b)).astype(np.int16)


def payload_closed_form(codes: np.ndarray, b: int) -> np.ndarray:
    total = 0
    for i, q in enumerate(codes.reshape(-1).tolist()):
        total |= (q + qmax(b)) << (i * b)
    nbytes = (codes.size * b + 7) // 8
    return np.frombuffer(total.to_bytes(nbytes, "little"), dtype=np.uint8).copy()


def decoded_f16(codes: np.ndarray, s: np.ndarray) -> np.ndarray:
    return (codes.astype(F32) * s[:, None]).astype(F32).astype(np.float16)


def fnv1a64_py(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for byte in data:
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def mlb4_py(rows, cols, b, scales, payload: bytes, threshold, err) -> bytes:
    sc = b"" if b == 16 else np.asarray(scales, F32).tobytes()
    header = struct.pack(
        "<4sHHIIB3sIQQQQQdd",
        b"MLB4", 4, 80, rows, cols, b, b"\0\0\0",
        0 if b == 16 else rows, len(sc), len(payload), rows * cols * 2,
        fnv1a64_py(sc), fnv1a64_py(payload), float(threshold), float(err),
    )
    assert len(header) == 80
    return header + sc + payload


def f16_round(v: np.float32) -> np.float32:
    return F32(np.float16(v))


def analyzer_py(w: np.ndarray, calib: np.ndarray) -> list[tuple[int, float, float]]:
    """Pure-Python float32 sequential restatement of runtime.cu:280-392.

    The long-double sums of squares are taken exactly with Fractions, so the
    errors agree with the 80-bit accumulation to ~1e-15 relative."""
    rows, cols = w.shape
    samples = calib.shape[0]
    xh = [[f16_round(F32(v)) for v in row] for row in calib]
    refs = []
    for s in range(samples):
        line = []
        for r in range(rows):
            acc = F32(0.0)
            for c in range(cols):
                acc = F32(acc + F32(f16_round(F32(w[r, c])) * xh[s][c]))
            line.append(acc)
        refs.append(line)
    results = []
    for b in range(3, 17):
        if b != 16:
            sc = scales_closed_form(w, b)
        hw_num = Fraction(0)
        full_num = Fraction(0)
        denom = Fraction(0)
        for s in range(samples):
            for r in range(rows):
                hw = F32(0.0)
                full = F32(0.0)
                if b == 16:
                    for c in range(cols):
                        hw = F32(hw + F32(f16_round(F32(w[r, c])) * xh[s][c]))
                    full = hw
                else:
                    scale = sc[r]
                    idot = F32(0.0)
                    for c in range(cols):
                        q = int(np.clip(np.rint(F32(F32(w[r, c]) / scale)), -qmax(b), qmax(b)))
                        deq = f16_round(F32(F32(q) * scale))
                        if b <= 8:
                            idot = F32(idot + F32(F32(q) * xh[s][c]))
                            full = F32(full + F32(deq * xh[s][c]))
                        else:
                            hw = F32(hw + F32(deq * xh[s][c]))
                    if b <= 8:
                        hw = F32(idot * scale)
                    else:
                        full = hw
                ref = float(refs[s][r])
                hd = float(hw) - ref
                fd = float(full) - ref
                hw_num += Fraction(hd) * Fraction(hd)
                full_num += Fraction(fd) * Fraction(fd)
                denom += Fraction(ref) * Fraction(ref)
        den = max(denom, Fraction(1, 10**30))
        hwe = math.sqrt(float(hw_num / den))
        fe = math.sqrt(float(full_num / den))
        results.append((b, hwe, fe))
    return results


def legacy_pack(u: np.ndarray, b: int) -> np.ndarray:
    total = 0
    for i, v in enumerate(u.reshape(-1).tolist()):
        total |= int(v) << (i * b)
    nbytes = (u.size * b + 7) // 8
    return np.frombuffer(total.to_bytes(nbytes, "little"), dtype=np.uint8).copy()


def main() -> None:
    rng = np.random.default_rng(20261201)
    rows, cols = 8, 32
    w16 = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float16)
    w16[0, :] = 0                         # all-zero row: s = 1, q = 0
    w16[2, 5] = np.float16(-0.125)        # the row max is negative
    w = w16.astype(F32)
    x16 = {M: rng.standard_normal((M, cols)).astype(np.float16) for M in (1, 4)}

    fixtures: dict[str, np.ndarray] = {"w": w, "x16_m1": x16[1].view(np.uint16),
                                       "x16_m4": x16[4].view(np.uint16)}
    for b in range(3, 16):
        s = scales_closed_form(w, b)
        q = codes_closed_form(w, s, b)
        payload = payload_closed_form(q, b)
        dec = decoded_f16(q, s)
        fixtures[f"scales_b{b}"] = s
        fixtures[f"codes_b{b}"] = q
        fixtures[f"payload_b{b}"] = payload
        fixtures[f"dec16_b{b}"] = dec.view(np.uint16)
        for M in (1, 4):
            xf = x16[M].astype(np.float64)
            fixtures[f"y_intdot_m{M}_b{b}"] = (xf @ q.astype(np.float64).T) * s.astype(np.float64)[None, :]
            fixtures[f"y_w16_m{M}_b{b}"] = xf @ dec.astype(np.float64).T
    # b = 16: raw fp16 storage
    fixtures["payload_b16"] = np.frombuffer(w16.tobytes(), dtype=np.uint8).copy()
    for M in (1, 4):
        fixtures[f"y_w16_m{M}_b16"] = x16[M].astype(np.float64) @ w16.astype(np.float64).T

    # MLB4 files (little-endian packed header, FNV-1a-64 checksums)
    for b in (3, 8, 10, 16):
        payload = fixtures[f"payload_b{b}"].tobytes()
        data = mlb4_py(rows, cols, b, fixtures.get(f"scales_b{b}"), payload, 0.01, 0.005 if b != 16 else 0.0)
        (OUT / f"mlb4_b{b}.mlb").write_bytes(data)
        bad = bytearray(data)
        bad[80 + (4 * rows if b != 16 else 0) + 3] ^= 0x10    # flip one payload bit
        (OUT / f"mlb4_b{b}_corrupt.mlb").write_bytes(bytes(bad))
    fixtures["fnv_vectors"] = np.array(
        [fnv1a64_py(b""), fnv1a64_py(b"a"), fnv1a64_py(b"foobar")], dtype=np.uint64)

    # Legacy group-scale op vectors
    lx = rng.standard_normal((3, 13)).astype(np.float32)
    for b in (2, 4, 8):
        u = rng.integers(0, 1 << b, size=(5, 13))
        packed = legacy_pack(u, b)
        fixtures[f"legacy_u_b{b}"] = u.astype(np.int32)
        fixtures[f"legacy_packed_b{b}"] = packed
        for g in (13, 32, 7):
            n_groups = (5 * 13 + g - 1) // g
            sc = rng.uniform(0.01, 0.1, size=n_groups).astype(np.float32)
            bias = rng.standard_normal(5).astype(np.float32)
            flat = np.arange(5 * 13)
            wmat = ((u.reshape(-1) - (1 << (b - 1))).astype(np.float64) * sc[flat // g].astype(np.float64)).reshape(5, 13)
            fixtures[f"legacy_scales_b{b}_g{g}"] = sc
            fixtures[f"legacy_bias_b{b}_g{g}"] = bias
            fixtures[f"legacy_y_b{b}_g{g}"] = lx.astype(np.float64) @ wmat.T + bias.astype(np.float64)
    fixtures["legacy_x"] = lx

    # Host analyzer on a tiny case
    aw = (rng.standard_normal((4, 8)) * 0.05).astype(np.float16).astype(F32)
    ac = rng.standard_normal((3, 8)).astype(F32)
    fixtures["analyze_w"] = aw
    fixtures["analyze_calib"] = ac
    fixtures["analyze_errors"] = np.array(analyzer_py(aw, ac), dtype=np.float64)

    np.savez(OUT / "eb_golden.npz", **fixtures)
    print(f"wrote {len(fixtures)} arrays to {OUT / 'eb_golden.npz'}")


if __name__ == "__main__":
    main()
