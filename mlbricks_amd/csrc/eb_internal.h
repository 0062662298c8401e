// Internal interface between the host runtime (eb_host.cpp) and the gfx950
// kernels (eb_kernels.hip).  Not installed; the public ABI is include/elasticbit.h.
//
// Device execution layout ("bit planes")
// --------------------------------------
// Canonical ElasticBit storage is one dense LSB-first bitstream of b-bit codes
// u = q + qmax over the row-major weight index (elasticbit_runtime.cu:150-186).
// At load time the device re-lays it out, still at b bits per weight, as:
//
//  * rows padded to a multiple of 32 columns with u = qmax (q = 0);
//  * groups of 32 consecutive codes of one row, gpr = ceil(cols/32) per row,
//    flat group index g = row * gpr + col / 32;
//  * one array per binary digit of b, "planes" of width 8, 4, 2 and 1 bits.
//    The widest plane holds the lowest bits of u, the next plane the next
//    bits, and so on (b = 10: plane8 = u & 0xff, plane2 = u >> 8).  A plane of
//    width w stores a group in 4*w bytes (8 / 4 / 2 / 1 dwords);
//  * inside a group, code i (0..31) of plane w sits in dword i / (32/w),
//    byte i % 4, bit field (i / 4) % (8/w).  Every plane therefore yields the
//    four codes 4d..4d+3 of a "quad" with one shift and one byte-lane mask,
//    already aligned to the byte lanes a v_perm_b32 consumes.
//  * b = 16 keeps raw fp16 weights in the same padded group order.
//
// All planes are separate arrays, so each lane's share is a naturally aligned
// 32/16/8/4-byte chunk and a wave reads every plane fully coalesced.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ebk {

constexpr int kGroup = 32;

struct DevMatrix {
    const uint8_t* p8 = nullptr;    // [G][32] bytes
    const uint8_t* p4 = nullptr;    // [G][16]
    const uint8_t* p2 = nullptr;    // [G][8]
    const uint8_t* p1 = nullptr;    // [G][4]
    const uint16_t* w16 = nullptr;  // [G][32] fp16, b = 16 only
    const float* scales = nullptr;  // [rows], b <= 15
    int rows = 0;
    int cols = 0;
    int gpr = 0;                    // groups per row
    int bits = 0;
};

struct DevMatrixOut {
    uint8_t* p8 = nullptr;
    uint8_t* p4 = nullptr;
    uint8_t* p2 = nullptr;
    uint8_t* p1 = nullptr;
    uint16_t* w16 = nullptr;
    int rows = 0;
    int cols = 0;
    int gpr = 0;
    int bits = 0;
};

// Bytes of the plane of width `width` (8, 4, 2, 1; 16 = raw fp16) for
// `groups` groups; 0 when b has no such plane.
inline size_t plane_bytes(int bits, int width, size_t groups) {
    if (bits == 16) return width == 16 ? groups * 64u : 0u;
    if (width == 16 || (bits & width) == 0) return 0u;
    return groups * 4u * static_cast<size_t>(width);
}

// Canonical bitstream (device copy) -> bit planes.
hipError_t launch_repack(const uint8_t* canon, uint64_t canon_bytes, const DevMatrixOut& out,
                         hipStream_t stream);

// Planes -> int16 codes q = u - qmax, [rows][cols].
hipError_t launch_unpack(const DevMatrix& m, int16_t* out, hipStream_t stream);

// Planes -> fp16 fp16_rn(q * s), [rows][cols].
hipError_t launch_materialize(const DevMatrix& m, uint16_t* out, hipStream_t stream);

// y[M][rows] = x[M][cols] . W^T (+ bias).  exact_w16 selects the decoded-fp16
// (W16A16) arithmetic; otherwise b <= 10 uses the integer-code dot product with
// the row scale applied once.  Requires cols % 8 == 0 and 16-byte aligned x
// for the vector path; other shapes take the guarded scalar path.
hipError_t launch_linear(const DevMatrix& m, bool exact_w16, const uint16_t* x, int64_t M,
                         uint16_t* y, const uint16_t* bias, hipStream_t stream);

// Legacy flat-group op (bolt/ops_cuda.cu:2708-2795).
hipError_t launch_packed_linear(const void* x, int x_dtype, int64_t M, const uint8_t* packed,
                                const void* scales, int scale_dtype, const void* bias, int bits,
                                int64_t group_size, int64_t N, int64_t K, void* y,
                                hipStream_t stream);

}  // namespace ebk
