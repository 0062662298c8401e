// Read-bandwidth probe for bench.py (not part of the ElasticBit library;
// bench.py builds it on first use into _build/libeb_probe_read.so).
//
// Measures what a kernel that only reads a buffer of a given size achieves
// when launched the way bench.py launches the GEMV: the same bytes, the same
// rotation over weight copies, the same graph replay.  That bounds what any
// one-launch-per-step kernel over those bytes can reach on this GPU, which
// the GEMV's HBM fraction is then read against.
//
// Each workgroup reads one contiguous chunk; every thread issues up to 32
// 16-byte loads (512 bytes in flight) before it uses any, in as many passes
// as its share needs, optionally as nontemporal loads.  The XOR of the data is written
// only if it equals a value it never takes, so the loads stay live and
// nothing is stored.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int T, int L, bool NT>
__global__ __launch_bounds__(T) void read_chunks(const uint4* __restrict__ src, uint64_t n16, uint64_t chunk16,
                                                  uint32_t* __restrict__ sink) {
    const uint64_t first = static_cast<uint64_t>(blockIdx.x) * chunk16;
    uint32_t acc = 0;
    // passes of L loads per thread over the workgroup's chunk
    for (uint64_t pass = 0; pass < chunk16; pass += static_cast<uint64_t>(L) * T) {
        uint4 v[L];
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const uint64_t idx = pass + threadIdx.x + static_cast<uint64_t>(i) * T;
            if (idx < chunk16 && first + idx < n16) {
                if constexpr (NT) {
                    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + first + idx);
                    v[i] = make_uint4(w.x, w.y, w.z, w.w);
                } else {
                    v[i] = src[first + idx];
                }
            } else {
                v[i] = make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < L; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (acc == 0x9E3779B9u && threadIdx.x == 0) sink[blockIdx.x & 1023] = acc;
}

template <int T, bool NT>
int launch(const uint4* src, uint64_t n16, int blocks, uint32_t* sink, hipStream_t s) {
    const uint64_t chunk16 = (n16 + blocks - 1) / blocks;
    const uint64_t per = (chunk16 + T - 1) / T;     // 16-byte loads per thread
    if (per <= 2) {
        hipLaunchKernelGGL((read_chunks<T, 2, NT>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    } else if (per <= 4) {
        hipLaunchKernelGGL((read_chunks<T, 4, NT>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    } else if (per <= 8) {
        hipLaunchKernelGGL((read_chunks<T, 8, NT>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    } else if (per <= 16) {
        hipLaunchKernelGGL((read_chunks<T, 16, NT>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    } else {
        // 32 loads per thread per pass, as many passes as the chunk needs
        hipLaunchKernelGGL((read_chunks<T, 32, NT>), dim3(blocks), dim3(T), 0, s, src, n16, chunk16, sink);
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

template <bool NT>
int launch_threads(const uint4* src, uint64_t n16, int blocks, int threads, uint32_t* sink, hipStream_t s) {
    switch (threads) {
        case 256: return launch<256, NT>(src, n16, blocks, sink, s);
        case 512: return launch<512, NT>(src, n16, blocks, sink, s);
        case 1024: return launch<1024, NT>(src, n16, blocks, sink, s);
        default: return -1;
    }
}

}  // namespace

// Read `bytes` (a multiple of 16) from `src` with `blocks` workgroups of
// `threads` (256, 512 or 1024) threads, with nontemporal loads when
// `nontemporal` is nonzero; `sink` is a device buffer of 1024 uint32.  0 on
// success, -1 for an unsupported thread count, -2 on a launch error.
extern "C" int eb_probe_read(const void* src, uint64_t bytes, int blocks, int threads, int nontemporal, void* sink,
                             void* stream) {
    if (!src || !sink || bytes % 16 != 0 || blocks <= 0) return -1;
    const auto* s16 = static_cast<const uint4*>(src);
    auto* out = static_cast<uint32_t*>(sink);
    const auto st = static_cast<hipStream_t>(stream);
    return nontemporal ? launch_threads<true>(s16, bytes / 16, blocks, threads, out, st)
                       : launch_threads<false>(s16, bytes / 16, blocks, threads, out, st);
}
