// Batched decode, 8 <= M <= 16, on matrices with more than two row tiles
// per CU: each workgroup owns RT consecutive row tiles and reads the
// activations once for all of them.
//
// y[M][rows] = x[M][cols] . W^T (+ bias), W in the bit-plane layout of
// eb_internal.h, one v_mfma_f32_16x16x32_f16 per group and row tile: A = 16
// activation rows (rows M .. 15 zero), B = 16 weight rows decoded in
// registers.
//
// Why.  linear_decode_kernel gives every row tile its own workgroup, which
// stages the whole of x (M x cols fp16, 128 KB at M = 16, cols = 4096) in
// LDS.  At M = 16 that staging is more data per row tile than the weights
// (80 KB at b = 10), and the 128 KB of LDS leaves one workgroup per CU.
// Measured on MI355X at 11008 x 4096 b = 10 its time grows with M: M = 4
// 12.6 us, 8 13.9, 12 16.3, 16 17.1; the activation rows a CU takes in cost
// ~15 ns per KB beyond the weights.  Here a workgroup covers RT = ceil(row
// tiles / CUs) row tiles (one round of workgroups), so a CU takes in x once
// for RT row tiles, and x goes straight from L2 into the A operands held in
// registers (no LDS copy): M = 12 14.2 us, M = 16 15.2 us at that shape.
//
// Wave w takes steps w and w + 16 of every row tile of the workgroup
// (cols <= 4096, 32 steps of 128 columns), so each wave holds two steps of
// A operands and 2 RT tiles of weight bits, all requested before it waits
// for any.  The activations of a step are requested ahead of its weight
// bits: vector loads retire in issue order, and the MFMAs of step w need
// both.  At the end the sixteen waves' 16 x 16 partial sums of each row
// tile are added through LDS in wave order.
//
// Tried and slower: splitting K over workgroups, with the partial sums
// combined by the last workgroup to finish (agent-scope release / acquire
// fences around a counter; 4-10x slower) or by a second kernel (4096 x
// 11008 M = 16: 17.8-22.4 us against 16.4 for linear_decode_kernel); two
// row tiles per workgroup where three or more fit one round.
#include "eb_device.h"

namespace ebk {
namespace {

constexpr int kRowsWaves = 16;               // waves per workgroup
constexpr int kRowsSteps = 2;                // K steps per wave: cols <= 16 * 2 * 128

template <int B, int MODE, int RT>
__global__ __launch_bounds__(64 * kRowsWaves) void linear_decode_rows_kernel(
    DevMatrix m, const uint16_t* __restrict__ x, int M, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ bias, int xvec) {
    static_assert(MODE != kModeRaw, "raw fp16 weights keep linear_decode_kernel");
    using Bits = GroupBits<B, MODE>;
    constexpr int kThreads = 64 * kRowsWaves;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nl = lane & 15;
    const int quarter = lane >> 4;
    const int steps = m.spr;
    const int tile0 = blockIdx.x * RT;
    int rtile[RT];                                // past the last row tile: re-read the last one
#pragma unroll
    for (int r = 0; r < RT; ++r) rtile[r] = min(tile0 + r, m.rtiles - 1);
    const bool xok = nl < M;
    const uint16_t* xr = x + static_cast<size_t>(xok ? nl : 0) * m.cols;

    Bits bits[kRowsSteps][RT];
    half8 a[kRowsSteps][4];
#pragma unroll
    for (int i = 0; i < kRowsSteps; ++i) {
        const int st = wave + kRowsWaves * i;
        if (xok && st < steps) {
            load_x32(xr, (st * kTileGroups + quarter) * kGroup, m.cols, xvec != 0, a[i]);
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) a[i][t] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        const int stc = min(st, steps - 1);       // zero activations meet the re-read step
#pragma unroll
        for (int r = 0; r < RT; ++r)
            bits[i][r].load(m, (static_cast<size_t>(rtile[r]) * steps + stc) * kTileSlots + lane);
    }
    float s[RT];                                  // decoded-fp16 arithmetic scales the B operand
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int row = rtile[r] * kTileRows + nl;
        s[r] = (MODE == kModeW && row < m.rows) ? m.scales[row] : 0.0f;
    }
    floatx4 acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < kRowsSteps; ++i) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int r = 0; r < RT; ++r)
                acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][t], bits[i][r].operand(t, s[r]), acc[r], 0, 0, 0);
        }
    }

    // D[4 (l / 16) + e][l % 16] of row tile r sits in lane l, element e, of
    // every wave; output element o = 256 r + 64 e + l is summed in wave order.
    __shared__ floatx4 red[kRowsWaves][RT][64];
#pragma unroll
    for (int r = 0; r < RT; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    constexpr int kPasses = (RT * 256 + kThreads - 1) / kThreads;
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
        const int o = threadIdx.x + kThreads * ps;
        if (o >= RT * 256) break;
        const int r = o >> 8;
        const int e = (o >> 6) & 3;
        const int src = o & 63;
        const int mi = 4 * (src >> 4) + e;
        const int n = (tile0 + r) * kTileRows + (src & 15);
        if (tile0 + r >= m.rtiles || n >= m.rows || mi >= M) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kRowsWaves; ++w) v += red[w][r][src][e];
        const float sc = MODE == kModeQ ? m.scales[n] : 1.0f;
        store_out(y + static_cast<size_t>(mi) * m.rows + n, epilogue<MODE>(v, sc, bias != nullptr, bias ? bias[n] : 0));
    }
}

// Sixteen waves leave 128 VGPRs per lane.  Four row tiles per workgroup
// fit them without scratch for the integer-code arithmetic at b <= 12
// except b = 11; the decoded-fp16 arithmetic (one more operand conversion
// per tile) spills there from b = 9 (hipcc -Rpass-analysis=kernel-resource-usage).
template <int B, int MODE>
constexpr bool rows_fit_four() {
    return MODE == kModeQ && B != 11;
}

template <int B, int MODE>
hipError_t launch_rows(const DevMatrix& m, int rt, const uint16_t* x, int M, uint16_t* y, const uint16_t* bias,
                       int xvec, hipStream_t s) {
    const dim3 grid((m.rtiles + rt - 1) / rt);
    switch (rt) {
        case 2:
            hipLaunchKernelGGL((linear_decode_rows_kernel<B, MODE, 2>), grid, dim3(64 * kRowsWaves), 0, s, m, x, M, y,
                               bias, xvec);
            break;
        case 3:
            hipLaunchKernelGGL((linear_decode_rows_kernel<B, MODE, 3>), grid, dim3(64 * kRowsWaves), 0, s, m, x, M, y,
                               bias, xvec);
            break;
        case 4:
            if constexpr (rows_fit_four<B, MODE>()) {
                hipLaunchKernelGGL((linear_decode_rows_kernel<B, MODE, 4>), grid, dim3(64 * kRowsWaves), 0, s, m, x, M,
                                   y, bias, xvec);
                break;
            }
            return hipErrorInvalidValue;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int B>
hipError_t launch_rows_bits(const DevMatrix& m, int mode, int rt, const uint16_t* x, int M, uint16_t* y,
                            const uint16_t* bias, int xvec, hipStream_t s) {
    if (mode == kModeQ) return launch_rows<B, kModeQ>(m, rt, x, M, y, bias, xvec, s);
    if (mode == kModeW) return launch_rows<B, kModeW>(m, rt, x, M, y, bias, xvec, s);
    return hipErrorInvalidValue;
}

}  // namespace

int decode_rows_per_workgroup(int64_t M, const DevMatrix& m, int mode, int cus) {
    if (M < 8 || M > 16 || mode == kModeRaw || m.bits > kDecodeRowsMaxBits || cus <= 0) return 0;
    if (m.spr > kRowsWaves * kRowsSteps) return 0;
    const int rt = (m.rtiles + cus - 1) / cus;
    if (rt < 2 || rt > 4) return 0;
    if (rt == 4 && (mode != kModeQ || m.bits == 11)) return 0;   // as rows_fit_four
    if (rt == 2 && M < 12) return 0;   // 8192 x 4096: M = 8 measured no faster
    return rt;
}

hipError_t launch_decode_rows(const DevMatrix& m, int mode, int rt, const uint16_t* x, int64_t M, uint16_t* y,
                              const uint16_t* bias, int xvec, hipStream_t s) {
    if (M < 1 || M > 16 || m.spr > kRowsWaves * kRowsSteps) return hipErrorInvalidValue;
    const int Mi = static_cast<int>(M);
    switch (m.bits) {
        case 3: return launch_rows_bits<3>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 4: return launch_rows_bits<4>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 5: return launch_rows_bits<5>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 6: return launch_rows_bits<6>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 7: return launch_rows_bits<7>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 8: return launch_rows_bits<8>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 9: return launch_rows_bits<9>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 10: return launch_rows_bits<10>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 11: return launch_rows_bits<11>(m, mode, rt, x, Mi, y, bias, xvec, s);
        case 12: return launch_rows_bits<12>(m, mode, rt, x, Mi, y, bias, xvec, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ebk
