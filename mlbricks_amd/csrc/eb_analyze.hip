// Fused width search on the device: the errors the reference's GPU analyzer
// (_selectBitsTorch, mlbricks/elasticbit/core.py:112-195) measures for every
// storage width b = 3..15, in one pass over the weights.
//
// For calibration rows x (fp16 [S][K]) and weights W (fp16 [N][K]), with the
// row scale s_b = max|w_r| * fp32(1 / qmax_b) (1 for an all-zero row,
// core.py:145-149, as torch evaluates it; see width_scale) and codes
// q_b = clamp(rint(w / s_b), -qmax_b, qmax_b) (core.py:151-153):
//   ref    = fp16(x . W^T)                           (core.py:140)
//   full_b = fp16(x . fp16(q_b * s_b)^T)             (core.py:154-158)
//   hw_b   = fp16(fp32(x . q_b^T) * s_b), b <= 12    (core.py:160-169)
// and the squared distances |full_b - ref|^2, |hw_b - ref|^2 and |ref|^2,
// summed per tile of 16 weight rows.  The caller adds the tiles and forms
// relL2 = sqrt(sum |c - ref|^2) / max(sqrt(sum |ref|^2), 1e-30)
// (core.py:_relativeL2Torch).
//
// Products run on v_mfma_f32_16x16x32_f16 with fp32 accumulation, as the
// vendor GEMM does; every fp16 operand is exact (fp16(q*s) is the decoded
// weight, and |q| <= 2047 is an fp16 integer for the b <= 12 codes).  The
// division w / s_b is IEEE fp32 (no fast-math), as torch's.
//
// The reference measures hw_b only for b <= 8: above that its
// hardwareNative policy executes W16A16, whose output is full_b.  This
// runtime's hardwareNative executes the integer-code product up to b = 12
// (the codes stay exact fp16 integers), so hw_b is measured up to b = 12
// and the width search checks the arithmetic that will run.
#include "eb_internal.h"

#include <hip/hip_runtime.h>

#include <mutex>

namespace ebk {

// Per-tile partial sums of the width search that allocates nothing
// (launch_analyze_widths_totals): one copy per device, as many tiles as
// kAnalyzeScratchTiles.  Host code must not pass this name to a kernel (it is
// a host-side stand-in); analyze_scratch() looks up its device address.
static __device__ __align__(256) float scratch[kAnalyzeScratchTiles * kAnalyzeSums];

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kAnRows = kAnalyzeTileRows;     // weight rows per workgroup (MFMA n)
constexpr int kAnWaves = 4;                   // waves split the 32-column chunks
constexpr int kAnBlocks = kAnalyzeMaxSamples / 16;   // 16-row calibration blocks (MFMA m)
constexpr int kLo = 3;                        // widths kLo .. kLo + kWidths - 1
constexpr int kWidths = 13;
constexpr int kHw = 10;                       // b = 3..12 also run the integer-code product
constexpr int kSets = 1 + kWidths + kHw;      // ref, full_b, hw_b
static_assert(kSets == kAnalyzeSums, "partial sums per tile");

__device__ __forceinline__ float mul_rn(float a, float b) {
    float p = a * b;            // rounded to fp32 before any fp16 rounding
    __asm__("" : "+v"(p));
    return p;
}

__device__ __forceinline__ uint16_t to_f16(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }
__device__ __forceinline__ float from_f16(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

// Eight fp16 values of row `row` from column k0 (zero outside the matrix).
__device__ __forceinline__ half8 load_row8(const uint16_t* __restrict__ p, int row, int rows, int k0, int K,
                                           bool vec) {
    half8 v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (row >= rows || k0 >= K) return v;
    const uint16_t* q = p + static_cast<size_t>(row) * K + k0;
    if (vec) return *reinterpret_cast<const half8*>(q);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (k0 + i < K) v[i] = __builtin_bit_cast(_Float16, q[i]);
    }
    return v;
}

// torch.where(maxAbs > 0, maxAbs / qmax, 1) (core.py:145-149).  torch's
// CUDA and HIP kernels divide a tensor by a Python scalar as a product with
// the fp32 reciprocal of the scalar (BinaryDivTrueKernel), so the
// reference's scales are maxAbs * fp32(1 / qmax), not the IEEE quotient.
__device__ __forceinline__ float width_scale(float mx, int b) {
    const float inv = 1.0f / static_cast<float>((1 << (b - 1)) - 1);
    return mx > 0.0f ? mx * inv : 1.0f;
}

// One workgroup: weight rows n0 .. n0 + 15 against up to 32 calibration
// rows.  Lane l holds, per 32-column chunk, columns 8*(l/16) .. +7 of weight
// row n0 + l%16 (the B operand) and of calibration rows l%16 and 16 + l%16
// (the A operands); D[4*(l/16) + e][l%16] is element e of its result.
__global__ __launch_bounds__(64 * kAnWaves) void analyze_widths_kernel(
    const uint16_t* __restrict__ w, int N, int K, const uint16_t* __restrict__ x, int S,
    const float* __restrict__ max_abs, float* __restrict__ partials, int wvec, int xvec) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nl = lane & 15;
    const int quarter = lane >> 4;
    const int n0 = blockIdx.x * kAnRows;
    const int n = n0 + nl;
    const float mx = n < N ? max_abs[n] : 0.0f;
    float sc[kWidths];
#pragma unroll
    for (int i = 0; i < kWidths; ++i) sc[i] = width_scale(mx, kLo + i);

    floatx4 acc[kSets][kAnBlocks];
#pragma unroll
    for (int j = 0; j < kSets; ++j)
#pragma unroll
        for (int sb = 0; sb < kAnBlocks; ++sb) acc[j][sb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    const int chunks = (K + 31) / 32;
    for (int c = wave; c < chunks; c += kAnWaves) {
        const int k0 = c * 32 + 8 * quarter;
        const half8 wv = load_row8(w, n, N, k0, K, wvec != 0);
        half8 xa[kAnBlocks];
#pragma unroll
        for (int sb = 0; sb < kAnBlocks; ++sb) xa[sb] = load_row8(x, 16 * sb + nl, S, k0, K, xvec != 0);
#pragma unroll
        for (int sb = 0; sb < kAnBlocks; ++sb)
            acc[0][sb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[sb], wv, acc[0][sb], 0, 0, 0);
        float wf[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) wf[e] = static_cast<float>(wv[e]);
#pragma unroll
        for (int i = 0; i < kWidths; ++i) {
            const float qmax = static_cast<float>((1 << (kLo + i - 1)) - 1);
            half8 dq, qh;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float q = fminf(fmaxf(rintf(wf[e] / sc[i]), -qmax), qmax);
                dq[e] = static_cast<_Float16>(mul_rn(q, sc[i]));
                qh[e] = static_cast<_Float16>(q);
            }
#pragma unroll
            for (int sb = 0; sb < kAnBlocks; ++sb) {
                acc[1 + i][sb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[sb], dq, acc[1 + i][sb], 0, 0, 0);
                if (i < kHw) {
                    acc[1 + kWidths + i][sb] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[sb], qh, acc[1 + kWidths + i][sb], 0, 0, 0);
                }
            }
        }
    }

    // Add the four waves' K parts one set at a time through LDS (in wave
    // order), round each output to fp16 and square its distance to ref.
    // Thread t owns element e = t / 64 of lane t % 64 in both blocks.
    __shared__ floatx4 red[kAnWaves][kAnBlocks][64];
    const int tl = threadIdx.x & 63;
    const int te = threadIdx.x >> 6;
    const int on = n0 + (tl & 15);
    const float omx = on < N ? max_abs[on] : 0.0f;
    bool ok[kAnBlocks];
#pragma unroll
    for (int sb = 0; sb < kAnBlocks; ++sb) ok[sb] = on < N && 16 * sb + 4 * (tl >> 4) + te < S;
    float ref[kAnBlocks];
    float sq[kSets];
#pragma unroll
    for (int j = 0; j < kSets; ++j) sq[j] = 0.0f;
#pragma unroll
    for (int j = 0; j < kSets; ++j) {
        if (j > 0) __syncthreads();
#pragma unroll
        for (int sb = 0; sb < kAnBlocks; ++sb) red[wave][sb][lane] = acc[j][sb];
        __syncthreads();
#pragma unroll
        for (int sb = 0; sb < kAnBlocks; ++sb) {
            float v = 0.0f;
#pragma unroll
            for (int wv = 0; wv < kAnWaves; ++wv) v += red[wv][sb][tl][te];
            if (j == 0) {
                ref[sb] = from_f16(to_f16(v));
                if (ok[sb]) sq[0] += ref[sb] * ref[sb];
            } else {
                if (j > kWidths) v = mul_rn(v, width_scale(omx, kLo + j - 1 - kWidths));
                const float d = from_f16(to_f16(v)) - ref[sb];
                if (ok[sb]) sq[j] += d * d;
            }
        }
    }

    // Workgroup sums of the kSets sets, in a fixed order: lanes by a shuffle
    // tree, then the waves through LDS.
    __shared__ float wsum[kAnWaves][kSets];
#pragma unroll
    for (int j = 0; j < kSets; ++j) {
        float v = sq[j];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0) wsum[wave][j] = v;
    }
    __syncthreads();
    if (threadIdx.x < kSets) {
        float v = 0.0f;
#pragma unroll
        for (int wv = 0; wv < kAnWaves; ++wv) v += wsum[wv][threadIdx.x];
        partials[static_cast<size_t>(blockIdx.x) * kSets + threadIdx.x] = v;
    }
}

// totals[j] = sum over tiles of partials[t][j] in double, in a fixed order
// (lane l takes tiles l, l + 64, ...; then a shuffle tree): one wave per sum.
__global__ __launch_bounds__(64) void analyze_total_kernel(const float* __restrict__ partials, int tiles,
                                                           double* __restrict__ totals) {
    const int lane = threadIdx.x;
    const int j = blockIdx.x;
    double v = 0.0;
    for (int t = lane; t < tiles; t += 64) v += static_cast<double>(partials[static_cast<size_t>(t) * kAnalyzeSums + j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) totals[j] = v;
}

// Device address of `scratch` on the current device, looked up once per
// device with that device current and kept.
hipError_t analyze_scratch(float** out) {
    static std::mutex mu;
    static float* per_device[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (per_device[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        per_device[dev] = static_cast<float*>(p);
    }
    *out = per_device[dev];
    return hipSuccess;
}

}  // namespace

hipError_t launch_analyze_widths_totals(const uint16_t* w, int N, int K, const uint16_t* x, int S,
                                        const float* max_abs, double* totals, hipStream_t stream) {
    const int tiles = (N + kAnRows - 1) / kAnRows;
    if (N < 1 || tiles > kAnalyzeScratchTiles) return hipErrorInvalidValue;
    float* partials = nullptr;
    const hipError_t e = analyze_scratch(&partials);
    if (e != hipSuccess) return e;
    // every tile's sums are written by the first kernel before the second
    // reads them, so nothing left by an earlier call needs clearing
    const hipError_t e1 = launch_analyze_widths(w, N, K, x, S, max_abs, partials, stream);
    if (e1 != hipSuccess) return e1;
    hipLaunchKernelGGL(analyze_total_kernel, dim3(kAnalyzeSums), dim3(64), 0, stream, partials, tiles, totals);
    return hipGetLastError();
}

hipError_t launch_analyze_widths(const uint16_t* w, int N, int K, const uint16_t* x, int S, const float* max_abs,
                                 float* partials, hipStream_t stream) {
    if (N < 1 || K < 1 || S < 1 || S > kAnalyzeMaxSamples) return hipErrorInvalidValue;
    const int wvec = (K % 8 == 0) && (reinterpret_cast<uintptr_t>(w) % 16 == 0);
    const int xvec = (K % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    const unsigned tiles = static_cast<unsigned>((N + kAnRows - 1) / kAnRows);
    hipLaunchKernelGGL(analyze_widths_kernel, dim3(tiles), dim3(64 * kAnWaves), 0, stream, w, N, K, x, S, max_abs,
                       partials, wvec, xvec);
    return hipGetLastError();
}

}  // namespace ebk
