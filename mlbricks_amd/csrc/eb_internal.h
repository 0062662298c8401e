// Internal interface between the host runtime (eb_host.cpp) and the gfx950
// kernels (eb_kernels.hip, eb_prefill.hip, eb_analyze.hip).  Not installed; the public ABI is include/elasticbit.h.
//
// Device execution layout ("bit planes" in lane-ordered tiles)
// -------------------------------------------------------------
// Canonical ElasticBit storage is one dense LSB-first bitstream of b-bit codes
// u = q + qmax over the row-major weight index (elasticbit_runtime.cu:150-186).
// At load time the device re-lays it out, still at b bits per weight, as:
//
//  * groups of 32 consecutive codes of one row, gpr = ceil(cols/32) per row;
//  * tiles of 16 rows x 4 groups (16 x 128 codes).  The matrix is padded to
//    whole tiles with u = qmax (q = 0): rtiles = ceil(rows/16) row tiles,
//    spr = ceil(gpr/4) tiles per row tile.  Tile (rt, st) is stored at tile
//    index rt * spr + st, so a row tile's tiles are contiguous along K;
//  * inside a tile the 64 groups sit in MFMA lane order, slot l = 16*q + n
//    for the group q (0..3) of row n (0..15): the slot a wave64 lane loads
//    for the B operand of v_mfma_f32_16x16x32_f16.  A wave reading one tile
//    therefore reads one contiguous block (2 KB of the 8-bit plane);
//  * one array per binary digit of b, "planes" of width 8, 4, 2 and 1 bits.
//    The widest plane holds the lowest bits of u, the next plane the next
//    bits, and so on (b = 10: plane8 = u & 0xff, plane2 = u >> 8).  A plane of
//    width w stores a group in 4*w bytes (8 / 4 / 2 / 1 dwords);
//  * inside a group, code i (0..31) of plane w sits in dword i / (32/w),
//    byte i % 4, bit field (i / 4) % (8/w).  Every plane therefore yields the
//    four codes 4d..4d+3 of a "quad" with one shift and one byte-lane mask,
//    already aligned to the byte lanes a v_perm_b32 consumes.
//  * b = 16 keeps raw fp16 weights (64 bytes per group) in the same slots.
//
// All planes are separate arrays, so each lane's share is a naturally aligned
// 32/16/8/4-byte chunk and a wave reads every plane fully coalesced.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ebk {

constexpr int kGroup = 32;      // codes per group
constexpr int kTileRows = 16;   // rows per tile
constexpr int kTileGroups = 4;  // groups per tile along a row
constexpr int kTileSlots = kTileRows * kTileGroups;

// Slot (flat group index in the planes) of group `grp` of row `row`.
__host__ __device__ inline size_t group_slot(int row, int grp, int spr) {
    return (static_cast<size_t>(row >> 4) * spr + (grp >> 2)) * kTileSlots + (grp & 3) * kTileRows + (row & 15);
}

struct DevMatrix {
    const uint8_t* p8 = nullptr;    // [G][32] bytes
    const uint8_t* p4 = nullptr;    // [G][16]
    const uint8_t* p2 = nullptr;    // [G][8], or [G][12] with the 1-bit word (merged tail)
    const uint8_t* p1 = nullptr;    // [G][4], unused with a merged tail
    const uint16_t* w16 = nullptr;  // [G][32] fp16, b = 16 only
    const float* scales = nullptr;  // [rows], b <= 15
    int rows = 0;
    int cols = 0;
    int gpr = 0;                    // groups per row
    int spr = 0;                    // tiles per row tile, ceil(gpr / 4)
    int rtiles = 0;                 // row tiles, ceil(rows / 16)
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
    int spr = 0;
    int rtiles = 0;
    int bits = 0;
};

// Widths with a wide plane and both a 2-bit and a 1-bit plane (b = 7, 11,
// 15) keep the two small ones together: per group 12 bytes in the width-2
// array (the two 2-bit words, then the 1-bit word), so a lane reads them
// with one load instead of two.  Measured on MI355X at M = 1 and 4:
// 11008 x 4096 b = 11 13.66 -> 13.23 us, b = 15 0.4-2% faster; b = 3 (whose
// only planes these are) was no faster and keeps them apart.
constexpr bool merged_tail(int bits) { return bits >= 7 && bits != 16 && (bits & 3) == 3; }

// Bytes of the plane of width `width` (8, 4, 2, 1; 16 = raw fp16) for
// `groups` slots (rtiles * spr * 64); 0 when b has no such plane (or keeps
// it in the merged tail).
inline size_t plane_bytes(int bits, int width, size_t groups) {
    if (bits == 16) return width == 16 ? groups * 64u : 0u;
    if (width == 16 || (bits & width) == 0) return 0u;
    if (merged_tail(bits)) return width == 1 ? 0u : width == 2 ? groups * 12u : groups * 4u * width;
    return groups * 4u * static_cast<size_t>(width);
}

// int16 codes (device) -> canonical bitstream (device), b = 3..15; *bad
// (device, zeroed by the caller) becomes nonzero for a code outside
// [-qmax, qmax].
hipError_t launch_pack_codes(const int16_t* codes, uint64_t count, int bits, uint8_t* out, uint64_t out_bytes,
                             int* bad, hipStream_t stream);

// Canonical bitstream (device copy) -> bit planes.
hipError_t launch_repack(const uint8_t* canon, uint64_t canon_bytes, const DevMatrixOut& out,
                         hipStream_t stream);

// Planes -> int16 codes q = u - qmax, [rows][cols] row-major.
hipError_t launch_unpack(const DevMatrix& m, int16_t* out, hipStream_t stream);

// Planes -> fp16 fp16_rn(q * s), [rows][cols] row-major.
hipError_t launch_materialize(const DevMatrix& m, uint16_t* out, hipStream_t stream);

// y[M][rows] = x[M][cols] . W^T (+ bias).  exact_w16 selects the decoded-fp16
// (W16A16) arithmetic; otherwise b <= 12 uses the integer-code dot product with
// the row scale applied once.  Requires cols % 8 == 0 and 16-byte aligned x
// for the vector path; other shapes take the guarded scalar path.
hipError_t launch_linear(const DevMatrix& m, bool exact_w16, const uint16_t* x, int64_t M,
                         uint16_t* y, const uint16_t* bias, hipStream_t stream);

// Several matrices that read the same x in one decode launch (M <= 16):
// matrix j owns the grid's row tiles [tile0[j-1], tile0[j]) and writes its
// own y.  Matrix 0 is the launch's own argument; this holds the others.
constexpr int kMultiMax = 4;
struct MultiTail {
    DevMatrix m[kMultiMax - 1];               // matrices 1 .. count - 1
    uint16_t* y[kMultiMax - 1] = {};
    const uint16_t* bias[kMultiMax - 1] = {};
    int tile0[kMultiMax - 1] = {};            // first grid row tile of matrix j + 1
    int count = 1;                            // matrices in the launch
};

// ys[j][M][ms[j].rows] = x[M][cols] . W_j^T (+ biases[j]) for count <= kMultiMax
// matrices with the same cols, bits and arithmetic: one launch when
// M <= 16, one launch per matrix otherwise.  biases may be null.
hipError_t launch_linear_multi(const DevMatrix* ms, int count, bool exact_w16, const uint16_t* x, int64_t M,
                               uint16_t* const* ys, const uint16_t* const* biases, hipStream_t stream);

// Fused width search (eb_analyze.hip): per tile of kAnalyzeTileRows weight
// rows, kAnalyzeSums partial sums (|ref|^2, then |full_b - ref|^2 for
// b = 3..15, then |hw_b - ref|^2 for b = 3..12) over up to
// kAnalyzeMaxSamples calibration rows.
constexpr int kAnalyzeTileRows = 16;
constexpr int kAnalyzeMaxSamples = 32;
constexpr int kAnalyzeSums = 24;
hipError_t launch_analyze_widths(const uint16_t* w, int N, int K, const uint16_t* x, int S, const float* max_abs,
                                 float* partials, hipStream_t stream);

// The same width search with the per-tile partials in a static device array
// (allocates nothing), reduced on the device into totals[kAnalyzeSums]
// (double, device).  At most kAnalyzeScratchTiles tiles; calls that overlap
// on one device share the array and race.
constexpr int kAnalyzeScratchTiles = 16384;
hipError_t launch_analyze_widths_totals(const uint16_t* w, int N, int K, const uint16_t* x, int S,
                                        const float* max_abs, double* totals, hipStream_t stream);

// Prefill tile shape: 0 auto, 1 128 x 256, 2 256 x 256 with four waves,
// 3 256 x 256 with eight waves, a partial last round balanced with 192 x 256
// tiles where that is estimated faster, 4 the same without the balancing,
// 5 192 x 256 tiles with eight waves throughout (process-wide).
constexpr int kPrefillTilesWide = 2;
constexpr int kPrefillTilesWide8 = 3;
constexpr int kPrefillTilesWide8Plain = 4;
constexpr int kPrefillTilesWide8Short = 5;
constexpr int kPrefillTilesWidePlain = 6;
constexpr int kPrefillTilesWideShort = 7;
void set_prefill_tiles(int mode);

// The tiles of one launch of a 256 x 256 prefill kernel (four or eight
// waves): up to two rectangles of tiles, each walked four activation blocks
// at a time along its weight-row blocks.
struct PrefillRect {
    int m0;         // first activation row
    int mblocks;    // activation blocks (of the launch's tile height)
    int nb0;        // first 256-row weight block
    int nblocks;
};
struct PrefillGrid {
    PrefillRect r[2];
    int jobs0;      // tiles of r[0]; later jobs are r[1]'s
    int njobs;
    int per_xcd;    // jobs per XCD (workgroup i runs on XCD i % 8)
};
// 256 x 256 tiles (full) and 192 x 256 tiles (short), each one launch,
// either possibly empty; cost in full rounds of 256 x 256 tiles.
struct PrefillPlan {
    PrefillGrid full;
    PrefillGrid short_tiles;
    double cost;
};
// The plan for M x rows on `cus` CUs under a set_prefill_tiles mode
// (eb_prefill.hip; cached per host thread).
PrefillPlan prefill_plan(int64_t M, int rows, int cus, int tiles_mode);

// 256 x 256 (and 192 x 256) prefill tiles with eight waves (eb_prefill.hip).
// mode: 0 integer-code dot product (b <= 12), 1 decoded fp16 weights, 2 raw
// fp16 weights (b = 16).  cus: the device's compute units; tiles_mode: the
// set_prefill_tiles mode.  Requires M >= 1, cols % 8 == 0, a 16-byte
// aligned x, M * cols * 2 below 4 GiB and planes below 4 GiB.
hipError_t launch_prefill_pp(const DevMatrix& m, int mode, const uint16_t* x, int64_t M, uint16_t* y,
                             const uint16_t* bias, hipStream_t stream, int cus, int tiles_mode);
// Estimated time of launch_prefill_pp's launches for M x rows, in full
// rounds of 256 x 256 tiles over `cus` CUs.
double prefill_pp_rounds(int64_t M, int rows, int cus, int tiles_mode);
// The same plan as rectangles of tiles (eb_prefill_plan's layout); returns
// its estimated cost.
double prefill_pp_plan_rects(int64_t M, int rows, int cus, int tiles_mode, int32_t* out);
// The current set_prefill_tiles mode.
int prefill_tiles_mode();

// Batched decode with several row tiles per workgroup (eb_decode_rows.hip).
// decode_rows_per_workgroup: the row tiles per workgroup it takes for this
// call (2..4), or 0 where linear_decode_kernel is used: 8 <= M <= 16, b <=
// kDecodeRowsMaxBits (not raw fp16), cols <= 4096, and more row tiles than
// CUs (two per CU from M = 12).  mode as for launch_prefill_pp.
constexpr int kDecodeRowsMaxBits = 12;
int decode_rows_per_workgroup(int64_t M, const DevMatrix& m, int mode, int cus);
hipError_t launch_decode_rows(const DevMatrix& m, int mode, int rt, const uint16_t* x, int64_t M, uint16_t* y,
                              const uint16_t* bias, int xvec, hipStream_t stream);

// Legacy flat-group op (bolt/ops_cuda.cu:2708-2795).
hipError_t launch_packed_linear(const void* x, int x_dtype, int64_t M, const uint8_t* packed,
                                const void* scales, int scale_dtype, const void* bias, int bits,
                                int64_t group_size, int64_t N, int64_t K, void* y,
                                hipStream_t stream);

}  // namespace ebk
