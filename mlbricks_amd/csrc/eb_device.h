// Device-side pieces shared by the gfx950 kernel files (eb_kernels.hip,
// eb_prefill.hip): plane geometry, in-register decode of a 32-code group
// into MFMA operands, the output epilogue and the wait / barrier helpers.
// Not installed; the layout itself is described in eb_internal.h.
#pragma once

#include "eb_internal.h"

#include <hip/hip_runtime.h>

namespace ebk {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// plane geometry
// ---------------------------------------------------------------------------

template <int B>
struct Planes {
    static_assert(B >= 3 && B <= 15, "compressed widths only");
    static constexpr bool h8 = (B & 8) != 0;
    static constexpr bool h4 = (B & 4) != 0;
    static constexpr bool h2 = (B & 2) != 0;
    static constexpr bool h1 = (B & 1) != 0;
    static constexpr bool h21 = merged_tail(B);        // 2- and 1-bit words in one 12-byte slot
    static constexpr int off4 = h8 ? 8 : 0;           // bit offset of each plane in u
    static constexpr int off2 = off4 + (h4 ? 4 : 0);
    static constexpr int off1 = off2 + (h2 ? 2 : 0);
    static constexpr int qmax = (1 << (B - 1)) - 1;
};

// Raw plane words of one 32-code group.
template <int B>
struct Raw {
    uint32_t d8[8];
    uint32_t d4[4];
    uint32_t d2[2];
    uint32_t d1;
};

template <int B>
__device__ __forceinline__ void raw_zero(Raw<B>& r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) r.d8[i] = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.d4[i] = 0u;
    r.d2[0] = r.d2[1] = 0u;
    r.d1 = 0u;
}

template <int B>
__device__ __forceinline__ void raw_load(const DevMatrix& m, size_t g, Raw<B>& r) {
    using P = Planes<B>;
    if constexpr (P::h8) {
        const uint4* p = reinterpret_cast<const uint4*>(m.p8) + 2 * g;
        const uint4 a = p[0];
        const uint4 b = p[1];
        r.d8[0] = a.x; r.d8[1] = a.y; r.d8[2] = a.z; r.d8[3] = a.w;
        r.d8[4] = b.x; r.d8[5] = b.y; r.d8[6] = b.z; r.d8[7] = b.w;
    }
    if constexpr (P::h4) {
        const uint4 a = reinterpret_cast<const uint4*>(m.p4)[g];
        r.d4[0] = a.x; r.d4[1] = a.y; r.d4[2] = a.z; r.d4[3] = a.w;
    }
    if constexpr (P::h21) {
        const uint3 a = *reinterpret_cast<const uint3*>(m.p2 + g * 12);
        r.d2[0] = a.x; r.d2[1] = a.y; r.d1 = a.z;
    } else {
        if constexpr (P::h2) {
            const uint2 a = reinterpret_cast<const uint2*>(m.p2)[g];
            r.d2[0] = a.x; r.d2[1] = a.y;
        }
        if constexpr (P::h1) {
            r.d1 = reinterpret_cast<const uint32_t*>(m.p1)[g];
        }
    }
}

// raw_load with a 32-bit slot index: the planes of one matrix stay below
// 4 GiB, so each address is a scalar base plus a 32-bit vector byte offset
// (the saddr form of global_load) instead of 64-bit vector arithmetic.
template <int B>
__device__ __forceinline__ void raw_load32(const DevMatrix& m, uint32_t g, Raw<B>& r) {
    using P = Planes<B>;
    if constexpr (P::h8) {
        const uint8_t* p = m.p8 + g * 32u;
        const uint4 a = *reinterpret_cast<const uint4*>(p);
        const uint4 b = *reinterpret_cast<const uint4*>(p + 16);
        r.d8[0] = a.x; r.d8[1] = a.y; r.d8[2] = a.z; r.d8[3] = a.w;
        r.d8[4] = b.x; r.d8[5] = b.y; r.d8[6] = b.z; r.d8[7] = b.w;
    }
    if constexpr (P::h4) {
        const uint4 a = *reinterpret_cast<const uint4*>(m.p4 + g * 16u);
        r.d4[0] = a.x; r.d4[1] = a.y; r.d4[2] = a.z; r.d4[3] = a.w;
    }
    if constexpr (P::h21) {
        const uint3 a = *reinterpret_cast<const uint3*>(m.p2 + g * 12u);
        r.d2[0] = a.x; r.d2[1] = a.y; r.d1 = a.z;
    } else {
        if constexpr (P::h2) {
            const uint2 a = *reinterpret_cast<const uint2*>(m.p2 + g * 8u);
            r.d2[0] = a.x; r.d2[1] = a.y;
        }
        if constexpr (P::h1) {
            r.d1 = *reinterpret_cast<const uint32_t*>(m.p1 + g * 4u);
        }
    }
}

// Quad d (codes 4d..4d+3) as byte lanes: lo = bits 0..7 of each u, hi = bits 8+.
template <int B>
__device__ __forceinline__ void quad_bytes(const Raw<B>& r, int d, uint32_t& lo, uint32_t& hi) {
    using P = Planes<B>;
    constexpr int base = P::h8 ? 8 : 0;
    uint32_t small = 0u;
    if constexpr (P::h4) small |= ((r.d4[d >> 1] >> (4 * (d & 1))) & 0x0F0F0F0Fu) << (P::off4 - base);
    if constexpr (P::h2) small |= ((r.d2[d >> 2] >> (2 * (d & 3))) & 0x03030303u) << (P::off2 - base);
    if constexpr (P::h1) small |= ((r.d1 >> d) & 0x01010101u) << (P::off1 - base);
    if constexpr (P::h8) {
        lo = r.d8[d];
        hi = small;
    } else {
        lo = small;
        hi = 0u;
    }
}

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
    half2v v = {a, b};
    return __builtin_bit_cast(uint32_t, v);
}

// Exact fp16 codes q for one quad, b <= 12 (every |q| <= 2047 is an fp16
// integer).  The low ten bits of u become the mantissa of 1024 + u_lo
// (fp16 0x6400 | u_lo).  For b <= 10 that is all of u, and 1024 + qmax is
// subtracted.  For b = 11, 12 the subtraction is 2047 = 1024 + 1023, and the
// top bits t = u >> 10 add 1024 t + 1023 - qmax, looked up with one
// v_perm_b32 as fp16 high bytes (the low bytes are zero): b = 11, t in
// {0, 1}: {0, 1024}; b = 12, t in {0..3}: {-1024, 0, 1024, 2048}.  Every
// partial result is an integer of magnitude at most 2048, so each fp16 step
// is exact.
template <int B>
__device__ __forceinline__ void quad_q(uint32_t lo, uint32_t hi, uint32_t& w0, uint32_t& w1) {
    static_assert(B <= 12, "fp16 holds the codes exactly only up to 12 bits");
    // the low two bits of each hi byte are bits 8..9 of u; OR-ing in the
    // exponent byte 0x64 is then a bit-field insert
    const uint32_t H = (B <= 10 ? hi : (hi & 0x03030303u)) | 0x64646464u;
    const uint32_t a = __builtin_amdgcn_perm(H, lo, 0x05010400u);  // [lo0 H0 lo1 H1]
    const uint32_t b = __builtin_amdgcn_perm(H, lo, 0x07030602u);  // [lo2 H2 lo3 H3]
    constexpr _Float16 off = static_cast<_Float16>(B <= 10 ? 1024 + Planes<B>::qmax : 2047);
    const half2v o = {off, off};
    half2v q01 = __builtin_bit_cast(half2v, a) - o;
    half2v q23 = __builtin_bit_cast(half2v, b) - o;
    if constexpr (B > 10) {
        // fp16 high bytes of 1024 t + 1023 - qmax for t = 0..3
        constexpr uint32_t lut = B == 11 ? 0x00006400u : 0x686400E4u;
        const uint32_t t = (hi >> 2) & (B == 11 ? 0x01010101u : 0x03030303u);
        const uint32_t tb = __builtin_amdgcn_perm(0u, lut, t);                   // [L(t0) L(t1) L(t2) L(t3)]
        const uint32_t h01 = __builtin_amdgcn_perm(0u, tb, 0x01040004u);         // [0 L(t0) 0 L(t1)]
        const uint32_t h23 = __builtin_amdgcn_perm(0u, tb, 0x03040204u);         // [0 L(t2) 0 L(t3)]
        q01 = q01 + __builtin_bit_cast(half2v, h01);
        q23 = q23 + __builtin_bit_cast(half2v, h23);
    }
    w0 = __builtin_bit_cast(uint32_t, q01);
    w1 = __builtin_bit_cast(uint32_t, q23);
}

// a * b rounded to fp32.  The reference rounds products to fp32 before the
// fp16 rounding (__float2half_rn(q * s)); left alone the compiler fuses
// fmul + fptrunc into one v_fma_mix with a single rounding, which differs on
// rare double-rounding ties.  The empty asm hides the product from that
// combine and emits no instruction.
__device__ __forceinline__ float mul_f32(float a, float b) {
    float p = a * b;
    __asm__("" : "+v"(p));
    return p;
}

// Exact decoded weights fp16_rn(f32(q) * s) for one quad (any b <= 15).
template <int B>
__device__ __forceinline__ void quad_w(uint32_t lo, uint32_t hi, float s, uint32_t& w0, uint32_t& w1) {
    _Float16 h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = static_cast<int>(((lo >> (8 * j)) & 0xFFu) | (((hi >> (8 * j)) & 0xFFu) << 8));
        const float q = static_cast<float>(u - Planes<B>::qmax);
        h[j] = static_cast<_Float16>(mul_f32(q, s));
    }
    w0 = pack_h2(h[0], h[1]);
    w1 = pack_h2(h[2], h[3]);
}

enum Mode { kModeQ = 0, kModeW = 1, kModeRaw = 2 };

// Decode the 8 codes [8t, 8t+8) of a group into an MFMA operand.
template <int B, int MODE>
__device__ __forceinline__ half8 decode8(const Raw<B>& r, int t, float s) {
    uint32_t w[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t lo, hi;
        quad_bytes<B>(r, 2 * t + h, lo, hi);
        if constexpr (MODE == kModeQ) {
            quad_q<B>(lo, hi, w[2 * h], w[2 * h + 1]);
        } else {
            quad_w<B>(lo, hi, s, w[2 * h], w[2 * h + 1]);
        }
    }
    uint4 v = {w[0], w[1], w[2], w[3]};
    return __builtin_bit_cast(half8, v);
}

// ---------------------------------------------------------------------------
// shared pieces of the linear kernels
// ---------------------------------------------------------------------------

// fp16 bits -> float and float -> fp16 bits (round to nearest even).
__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

// Output epilogue: integer-dot scale, fp16 rounding, then torch-style bias add.
template <int MODE>
__device__ __forceinline__ uint16_t epilogue(float acc, float s, bool has_bias, uint16_t bias_bits) {
    uint16_t y = f2h(MODE == kModeQ ? mul_f32(acc, s) : acc);
    if (has_bias) y = f2h(h2f(y) + h2f(bias_bits));
    return y;
}

// Output store of the decode-shaped kernels: agent scope, so the store writes
// through this XCD's L2 (global_store_short ... sc1) and leaves no dirty line
// for the end-of-kernel L2 write-back.  Measured on MI355X (us, plain store
// -> this): 4096^2 b = 10 M = 1 5.695 -> 5.590, b = 9 5.397 -> 5.310,
// 4096 x 3072 5.143 -> 5.056; results bit-identical.
__device__ __forceinline__ void store_out(uint16_t* p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte output store of the prefill-shaped kernels: nontemporal
// (global_store_dwordx4 ... nt).  The output is written once and not read
// back by the kernel, so it streams past the L2 instead of displacing the
// activation and weight blocks that the workgroups of an XCD share there.
// Measured on MI355X (eight-wave kernel, b = 10, us, plain store -> this):
// 14336 x 4096 M = 2048 211-212 -> 203.5, 4096^2 M = 8192 229-231 -> 220.0;
// results bit-identical.  (For the decode kernels' few output lines a
// nontemporal store gained nothing: 5.695 -> 5.695 us.)
__device__ __forceinline__ void store_out16(uint16_t* p, const uint4& v) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(p));
}

// Load the 32 activations x[row][k0 .. k0+32) as four 8-half MFMA operands,
// zero beyond `cols`.  vec: cols % 8 == 0 and x 16-byte aligned.
__device__ __forceinline__ void load_x32(const uint16_t* __restrict__ xrow, int k0, int cols, bool vec,
                                         half8 (&a)[4]) {
    if (vec && k0 + kGroup <= cols) {
        const uint4* p = reinterpret_cast<const uint4*>(xrow + k0);
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t] = __builtin_bit_cast(half8, p[t]);
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int k = k0 + 8 * t + i;
                a[t][i] = k < cols ? __builtin_bit_cast(_Float16, xrow[k]) : static_cast<_Float16>(0.0f);
            }
        }
    }
}

// An LDS address as the address-space-3 pointer global_load_lds takes.  The
// explicit cast at the call matters: without it hipcc's host pass silently
// drops the launch stub of a kernel template that passes an LDS array
// expression of dependent type to the builtin (and a __device__ helper doing
// the cast has the same effect).
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// Workgroup barrier for the direct-to-LDS pipeline.  __syncthreads() opens
// with a release fence, which waits for every outstanding vector load --
// including the prefetch that should stay in flight across the barrier.
// The caller waits for the loads the next step reads (wait_vmcnt) and the
// barrier keeps only the acquire side.  Prior LDS reads have all returned:
// their MFMAs consumed them.
__device__ __forceinline__ void barrier_after_wait() {
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// s_waitcnt with only the LDS / scalar-memory counter constrained.
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
    static_assert(N >= 0 && N < 16, "lgkmcnt is a 4-bit counter");
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (N << 8));
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One group's weight bits as held in registers between load and decode.
template <int B, int MODE>
struct GroupBits {
    Raw<B> r;
    __device__ __forceinline__ void load(const DevMatrix& m, size_t g) { raw_load<B>(m, g, r); }
    // Copy of the planes width B has (the others are never written).
    __device__ __forceinline__ void copy_from(const GroupBits& o) {
        using P = Planes<B>;
        if constexpr (P::h8) {
#pragma unroll
            for (int i = 0; i < 8; ++i) r.d8[i] = o.r.d8[i];
        }
        if constexpr (P::h4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) r.d4[i] = o.r.d4[i];
        }
        if constexpr (P::h2) {
            r.d2[0] = o.r.d2[0];
            r.d2[1] = o.r.d2[1];
        }
        if constexpr (P::h1) r.d1 = o.r.d1;
    }
    __device__ __forceinline__ void load32(const DevMatrix& m, uint32_t g) { raw_load32<B>(m, g, r); }
    __device__ __forceinline__ half8 operand(int t, float s) const { return decode8<B, MODE>(r, t, s); }
};

template <int B>
struct GroupBits<B, kModeRaw> {
    uint4 w[4];
    __device__ __forceinline__ void load(const DevMatrix& m, size_t g) {
        const uint4* p = reinterpret_cast<const uint4*>(m.w16 + g * kGroup);
#pragma unroll
        for (int t = 0; t < 4; ++t) w[t] = p[t];
    }
    __device__ __forceinline__ void load32(const DevMatrix& m, uint32_t g) { load(m, g); }
    __device__ __forceinline__ void copy_from(const GroupBits& o) {
#pragma unroll
        for (int t = 0; t < 4; ++t) w[t] = o.w[t];
    }
    __device__ __forceinline__ half8 operand(int t, float) const { return __builtin_bit_cast(half8, w[t]); }
};

// Vector-memory instructions one GroupBits::load issues.
template <int B, int MODE>
struct GroupLoads {
    static constexpr int value =
        MODE == kModeRaw ? 4
                         : (Planes<B>::h8 ? 2 : 0) + (Planes<B>::h4 ? 1 : 0) +
                               (Planes<B>::h21 ? 1 : (Planes<B>::h2 ? 1 : 0) + (Planes<B>::h1 ? 1 : 0));
};


typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kPK = kTileGroups * kGroup;  // 128 columns per prefill step (one tile)
constexpr int kPRow = kPK * 2;             // bytes per staged activation row of a step

}  // namespace
}  // namespace ebk
