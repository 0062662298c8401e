// Read-bandwidth probe for bench.py (not part of the ElasticBit library).
//
// Measures what a kernel that only reads a buffer of a given size achieves
// when launched the way bench.py launches the GEMV: the same bytes, the same
// rotation over weight copies, the same graph replay.  That bounds what any
// one-launch-per-step kernel over those bytes can reach on this GPU, which
// the GEMV's HBM fraction is then read against.
//
// Each workgroup reads one contiguous chunk; every thread issues all of its
// 16-byte loads before it uses any.  The XOR of the data is written only if
// it equals a value it never takes, so the loads stay live and nothing is
// stored.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

template <int T, int L>
__global__ __launch_bounds__(T) void read_chunks(const uint4* __restrict__ src, uint64_t n16, uint64_t chunk16,
                                                  uint32_t* __restrict__ sink) {
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * chunk16;
    uint4 v[L];
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const uint64_t idx = threadIdx.x + static_cast<uint64_t>(i) * T;
        v[i] = (idx < chunk16 && base + idx < n16) ? src[base + idx] : make_uint4(0, 0, 0, 0);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < L; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (acc == 0x9E3779B9u && threadIdx.x == 0) sink[blockIdx.x & 1023] = acc;
}

template <int T>
int launch(const uint4* src, uint64_t n16, int blocks, uint32_t* sink, hipStream_t s) {
    const uint64_t chunk16 = (n16 + blocks - 1) / blocks;
    if (chunk16 <= static_cast<uint64_t>(T) * 2) {
        hipLaunchKernelGGL((read_chunks<T, 2>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    } else if (chunk16 <= static_cast<uint64_t>(T) * 4) {
        hipLaunchKernelGGL((read_chunks<T, 4>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    } else if (chunk16 <= static_cast<uint64_t>(T) * 8) {
        hipLaunchKernelGGL((read_chunks<T, 8>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    } else if (chunk16 <= static_cast<uint64_t>(T) * 16) {
        hipLaunchKernelGGL((read_chunks<T, 16>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    } else {
        return -1;   // too many bytes per thread for this launch shape
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace

// Read `bytes` (a multiple of 16) from `src` with `blocks` workgroups of
// `threads` (256, 512 or 1024) threads; `sink` is a device buffer of 1024
// uint32.  0 on success, -1 for an unsupported shape, -2 on a launch error.
extern "C" int eb_probe_read(const void* src, uint64_t bytes, int blocks, int threads, void* sink, void* stream) {
    if (!src || !sink || bytes % 16 != 0 || blocks <= 0) return -1;
    const auto* s16 = static_cast<const uint4*>(src);
    auto* out = static_cast<uint32_t*>(sink);
    const auto st = static_cast<hipStream_t>(stream);
    switch (threads) {
        case 256: return launch<256>(s16, bytes / 16, blocks, out, st);
        case 512: return launch<512>(s16, bytes / 16, blocks, out, st);
        case 1024: return launch<1024>(s16, bytes / 16, blocks, out, st);
        default: return -1;
    }
}
