// ElasticBit gfx950 kernels: bit-plane repack, unpack, materialize, the fused
// unpack + dequant + MFMA linear (decode and prefill), and the legacy
// flat-group packed op.  The execution layout is described in eb_internal.h.
//
// Arithmetic contracts (elasticbit_runtime.cu line numbers):
//   decoded weight      w = fp16_rn(f32(q) * s_r)                   (:233-234, :665, :679)
//   integer-dot output  y = fp16_rn(s_r * sum_c q_rc * x_c)         (:538-558, :594-608)
//   W16A16 output       y = fp16_rn(sum_c w_rc * x_c)               (:635-647)
//   bias                y = fp16_rn(y + bias), as torch adds it     (core.py:457-459)
// All sums accumulate in fp32 on the matrix cores.
#include "eb_device.h"

#include <atomic>
#include <type_traits>

#include <hip/hip_runtime.h>

namespace ebk {
namespace {

// ---------------------------------------------------------------------------
// bit-exact canonical extraction (elasticbit_runtime.cu:188-206)
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t extract_canon(const uint8_t* p, uint64_t nbytes, uint64_t index, int bits) {
    const uint64_t bit = index * static_cast<uint64_t>(bits);
    const uint64_t byte = bit >> 3;
    uint32_t word = 0u;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (byte + k < nbytes) word |= static_cast<uint32_t>(p[byte + k]) << (8 * k);
    }
    return (word >> (bit & 7u)) & ((1u << bits) - 1u);
}

// Row and group of slot `slot` of the tiled layout (inverse of group_slot).
__device__ __forceinline__ void slot_coords(uint64_t slot, int spr, int& row, int& grp) {
    const uint64_t tile = slot / kTileSlots;
    const int l = static_cast<int>(slot % kTileSlots);
    const int rt = static_cast<int>(tile / static_cast<uint64_t>(spr));
    const int st = static_cast<int>(tile - static_cast<uint64_t>(rt) * spr);
    row = rt * kTileRows + (l & (kTileRows - 1));
    grp = st * kTileGroups + l / kTileRows;
}

// One thread per slot: gathers the slot's 32 codes from the canonical stream
// (padding rows / columns get u = qmax, i.e. q = 0) and writes every plane.
template <int B>
__global__ void repack_kernel(const uint8_t* __restrict__ canon, uint64_t canon_bytes, DevMatrixOut out,
                              uint64_t slots) {
    using P = Planes<B>;
    const uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= slots) return;
    int row, grp;
    slot_coords(g, out.spr, row, grp);
    const int col0 = grp * kGroup;
    const bool row_ok = row < out.rows;
    uint32_t d8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t d4[4] = {0, 0, 0, 0};
    uint32_t d2[2] = {0, 0};
    uint32_t d1 = 0u;
#pragma unroll 4
    for (int i = 0; i < kGroup; ++i) {
        const int col = col0 + i;
        const uint32_t u = row_ok && col < out.cols
            ? extract_canon(canon, canon_bytes, static_cast<uint64_t>(row) * out.cols + col, B)
            : static_cast<uint32_t>(P::qmax);
        const int j = i & 3;
        const int d = i >> 2;
        if constexpr (P::h8) d8[d] |= (u & 0xFFu) << (8 * j);
        if constexpr (P::h4) d4[d >> 1] |= ((u >> P::off4) & 0xFu) << (8 * j + 4 * (d & 1));
        if constexpr (P::h2) d2[d >> 2] |= ((u >> P::off2) & 0x3u) << (8 * j + 2 * (d & 3));
        if constexpr (P::h1) d1 |= ((u >> P::off1) & 0x1u) << (8 * j + d);
    }
    if constexpr (P::h8) {
        uint4* p = reinterpret_cast<uint4*>(out.p8) + 2 * g;
        p[0] = make_uint4(d8[0], d8[1], d8[2], d8[3]);
        p[1] = make_uint4(d8[4], d8[5], d8[6], d8[7]);
    }
    if constexpr (P::h4) reinterpret_cast<uint4*>(out.p4)[g] = make_uint4(d4[0], d4[1], d4[2], d4[3]);
    if constexpr (P::h21) {
        *reinterpret_cast<uint3*>(out.p2 + g * 12) = make_uint3(d2[0], d2[1], d1);
    } else {
        if constexpr (P::h2) reinterpret_cast<uint2*>(out.p2)[g] = make_uint2(d2[0], d2[1]);
        if constexpr (P::h1) reinterpret_cast<uint32_t*>(out.p1)[g] = d1;
    }
}

// Codes q (int16, row-major) -> the canonical LSB-first bitstream of
// u = q + qmax (pack_exact_codes, runtime.cu:150-186).  Eight codes of B
// bits fill exactly B bytes, so thread t writes bytes B t .. B t + B - 1
// from codes 8t .. 8t + 7 (past the last code: u = 0, and no byte past the
// stream).  A code outside [-qmax, qmax] sets *bad.
template <int B>
__global__ void pack_codes_kernel(const int16_t* __restrict__ codes, uint64_t count, uint8_t* __restrict__ out,
                                  uint64_t out_bytes, int* __restrict__ bad) {
    constexpr int kQmax = (1 << (B - 1)) - 1;
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t i0 = 8 * t;
    if (i0 >= count) return;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t u = 0u;
        if (i0 + j < count) {
            const int q = codes[i0 + j];
            ok = ok && q >= -kQmax && q <= kQmax;
            u = static_cast<uint32_t>(q + kQmax) & ((1u << B) - 1u);
        }
        const int p = j * B;                      // bit offset within the B bytes
        w[p >> 5] |= u << (p & 31);
        if ((p & 31) + B > 32) w[(p >> 5) + 1] |= u >> (32 - (p & 31));
    }
    if (!ok) atomicOr(bad, 1);
    const uint64_t o = t * B;
#pragma unroll
    for (int k = 0; k < B; ++k) {
        if (o + k < out_bytes) out[o + k] = static_cast<uint8_t>(w[k >> 2] >> (8 * (k & 3)));
    }
}

__global__ void repack16_kernel(const uint16_t* __restrict__ canon, DevMatrixOut out, uint64_t slots) {
    const uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= slots) return;
    int row, grp;
    slot_coords(g, out.spr, row, grp);
    const int col0 = grp * kGroup;
    const bool row_ok = row < out.rows;
    uint16_t* dst = out.w16 + g * kGroup;
    for (int i = 0; i < kGroup; ++i) {
        const int col = col0 + i;
        dst[i] = row_ok && col < out.cols ? canon[static_cast<uint64_t>(row) * out.cols + col] : uint16_t(0);
    }
}

// ---------------------------------------------------------------------------
// unpack / materialize (one thread per group)
// ---------------------------------------------------------------------------

// A group's 32 outputs (2 bytes each) as four 16-byte stores when the group
// lies inside the row and the row start is 16-byte aligned (cols % 8 == 0);
// element by element otherwise.
__device__ __forceinline__ void store_group(uint16_t* __restrict__ dst, int col0, int cols, const uint32_t (&w)[16]) {
    if (col0 + kGroup <= cols && cols % 8 == 0) {
        uint4* d = reinterpret_cast<uint4*>(dst + col0);
#pragma unroll
        for (int v = 0; v < 4; ++v) d[v] = make_uint4(w[4 * v], w[4 * v + 1], w[4 * v + 2], w[4 * v + 3]);
    } else {
#pragma unroll
        for (int i = 0; i < kGroup; ++i) {
            if (col0 + i < cols) dst[col0 + i] = static_cast<uint16_t>(w[i >> 1] >> (16 * (i & 1)));
        }
    }
}

template <int B>
__global__ void unpack_kernel(DevMatrix m, int16_t* __restrict__ out, uint64_t slots) {
    const uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= slots) return;
    int row, grp;
    slot_coords(g, m.spr, row, grp);
    const int col0 = grp * kGroup;
    if (row >= m.rows || col0 >= m.cols) return;
    Raw<B> r;
    raw_load<B>(m, g, r);
    uint32_t w[16];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        uint32_t lo, hi;
        quad_bytes<B>(r, d, lo, hi);
        uint32_t q[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int u = static_cast<int>(((lo >> (8 * j)) & 0xFFu) | (((hi >> (8 * j)) & 0xFFu) << 8));
            q[j] = static_cast<uint16_t>(static_cast<int16_t>(u - Planes<B>::qmax));
        }
        w[2 * d] = q[0] | (q[1] << 16);
        w[2 * d + 1] = q[2] | (q[3] << 16);
    }
    store_group(reinterpret_cast<uint16_t*>(out) + static_cast<uint64_t>(row) * m.cols, col0, m.cols, w);
}

template <int B>
__global__ void materialize_kernel(DevMatrix m, uint16_t* __restrict__ out, uint64_t slots) {
    const uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= slots) return;
    int row, grp;
    slot_coords(g, m.spr, row, grp);
    const int col0 = grp * kGroup;
    if (row >= m.rows || col0 >= m.cols) return;
    uint32_t w[16];
    if constexpr (B == 16) {
        const uint4* src = reinterpret_cast<const uint4*>(m.w16 + g * kGroup);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 t = src[v];
            w[4 * v] = t.x;
            w[4 * v + 1] = t.y;
            w[4 * v + 2] = t.z;
            w[4 * v + 3] = t.w;
        }
    } else {
        Raw<B> r;
        raw_load<B>(m, g, r);
        const float s = m.scales[row];
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            uint32_t lo, hi;
            quad_bytes<B>(r, d, lo, hi);
            quad_w<B>(lo, hi, s, w[2 * d], w[2 * d + 1]);
        }
    }
    store_group(out + static_cast<uint64_t>(row) * m.cols, col0, m.cols, w);
}


// ---------------------------------------------------------------------------
// decode kernel, M <= 64: one workgroup owns one row tile (16 weight rows);
// its WAVES waves split the row tile's K tiles.  In step `st` lane l loads
// slot l of tile (row tile, st) -- group 4*st + l/16 of row l%16 -- so a
// wave's load is one contiguous block and one step feeds four
// v_mfma_f32_16x16x32_f16 with 16 rows x 128 columns per block of 16
// activation rows (MB blocks: each decoded operand feeds MB MFMAs).  The K
// order inside a group is the same for the A (activation) and B (weight)
// operands, so any order is a valid dot product.
//
// At small M the kernel is bound by HBM latency as much as by bandwidth: a
// CU's share of a 4096 x 4096 b=10 matrix is ~80 KB, about what it must keep
// in flight to cover the loaded DRAM latency.  Each wave therefore issues the
// loads of GPL steps at once and, while it decodes and multiplies one batch,
// already has the next batch's loads in flight.  Vector loads retire in
// issue order, so every activation load is issued before the weight loads
// it must not wait behind.
//
// XL: the activations (M x K, zero-padded to whole tiles) are staged once
// per workgroup in LDS.  XL = 1: up to kXLdsBytes, global -> LDS directly
// when x's rows are whole tiles and 16-byte aligned, through registers
// (zero-padded) otherwise.  XL = 2: up to kXLdsDirectBytes, direct only, so
// no registers are held for it.  XL = 3: longer rows (whole tiles, M <= 32)
// in double-buffered K chunks, direct.  XL = 0: each lane with an
// activation row loads its A operand from global memory per step.
// ---------------------------------------------------------------------------

constexpr int kXLdsBytes = 32768;
constexpr int kXLdsDirectBytes = 147456;   // 16 rows of 4608 halves

// Eight activations x[r][k .. k+8) as one uint4, zero at and beyond `cols`.
__device__ __forceinline__ uint4 load_x8(const uint16_t* __restrict__ x, int r, int k, int cols, bool vec) {
    const uint16_t* p = x + static_cast<size_t>(r) * cols + k;
    if (vec && k + 8 <= cols) return *reinterpret_cast<const uint4*>(p);
    uint32_t v[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (k + i < cols) v[i >> 1] |= static_cast<uint32_t>(p[i]) << (16 * (i & 1));
    }
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Load tiles first .. first+GPL-1 of this lane's row tile (clamped to the
// last tile) into `bits`.
template <int GPL, typename Bits>
__device__ __forceinline__ void decode_load_batch(const DevMatrix& m, Bits (&bits)[GPL], size_t slot0, int first,
                                                  int steps) {
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
        bits[j].load(m, slot0 + static_cast<size_t>(min(first + j, steps - 1)) * kTileSlots);
    }
}

// Activation operands of one workgroup batch (steps base + wave*GPL + j):
// from the LDS copy, or from global memory, zero past the last step.
// Block mb holds activation rows 16 mb .. 16 mb + 15.
// kshift: the column the LDS copy starts at (a chunk's first column, XL = 3).
template <int GPL, int XL, int MB>
__device__ __forceinline__ void decode_activations(half8 (&a)[MB][GPL][4], const DevMatrix& m, int base, int wave,
                                                   int quarter, const bool (&m_ok)[MB], int steps,
                                                   const uint16_t* const (&xrow)[MB],
                                                   const uint16_t* const (&xsrow)[MB], int xvec, int kshift = 0) {
    const int first = base + wave * GPL;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int j = 0; j < GPL; ++j) {
            const int k0 = ((first + j) * kTileGroups + quarter) * kGroup;
            const bool ok = m_ok[mb] && first + j < steps;
            if constexpr (XL != 0) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    a[mb][j][t] = ok ? *reinterpret_cast<const half8*>(xsrow[mb] + (k0 - kshift) + 8 * t)
                                     : half8{0, 0, 0, 0, 0, 0, 0, 0};
                }
            } else if (ok) {
                load_x32(xrow[mb], k0, m.cols, xvec != 0, a[mb][j]);
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) a[mb][j][t] = half8{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
    }
}

// Decode the batch held in `cur` and accumulate it against `a`.
// Decode the batch held in `cur` once and accumulate it against every
// activation block.
template <int B, int MODE, int GPL, int MB, typename Bits>
__device__ __forceinline__ void decode_mul_batch(const Bits (&cur)[GPL], const half8 (&a)[MB][GPL][4], int first,
                                                 int steps, float s, floatx4 (&acc)[MB]) {
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
        const bool st_ok = first + j < steps;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            half8 b = cur[j].operand(t, s);
            if constexpr (MODE == kModeRaw) {
                if (!st_ok) b = half8{0, 0, 0, 0, 0, 0, 0, 0};
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mb][j][t], b, acc[mb], 0, 0, 0);
        }
    }
}

// The matrix, row tile, output and bias of this workgroup in a launch over
// several matrices (MultiTail); a single-matrix launch keeps its arguments.
__device__ __forceinline__ int select_matrix(const MultiTail& mt, DevMatrix& m, uint16_t* __restrict__& y,
                                             const uint16_t* __restrict__& bias) {
    int tile = blockIdx.x;
    if (mt.count > 1) {
        int base = 0;
#pragma unroll
        for (int j = 0; j < kMultiMax - 1; ++j) {
            if (j + 1 < mt.count && tile >= mt.tile0[j]) {
                m = mt.m[j];
                y = mt.y[j];
                bias = mt.bias[j];
                base = mt.tile0[j];
            }
        }
        tile -= base;
    }
    return tile;
}

template <int B, int MODE, int WAVES, int GPL, int XL, int MB>
__global__ __launch_bounds__(64 * WAVES) void linear_decode_kernel(
    DevMatrix m, const uint16_t* __restrict__ x, int M, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ bias, int xvec, const MultiTail mt) {
    using Bits = GroupBits<B, MODE>;
    constexpr int kThreads = 64 * WAVES;
    constexpr int kBatch = WAVES * GPL;              // steps per workgroup batch
    constexpr int kXVecs = kXLdsBytes / 16 / kThreads;                              // XL = 1
    constexpr int kXDirect = (XL == 2 ? kXLdsDirectBytes : kXLdsBytes) / 16 / kThreads;
    static_assert(kXVecs >= 1, "LDS activation staging needs one uint4 per thread");
    static_assert(kThreads >= 256, "the epilogue stores the 16x16 tile with one thread per element");
    static_assert(XL != 3 || MB <= 2, "chunked staging holds at most 32 activation rows");
    // XL = 3: K chunks of CT tiles, double-buffered; kBpc workgroup batches per chunk
    constexpr int CT = MB == 1 ? 16 : 8;
    constexpr int kBpc = CT / kBatch;
    static_assert(XL != 3 || (kBpc >= 1 && CT % kBatch == 0), "a chunk holds whole workgroup batches");
    static_assert(XL != 3 || WAVES == 8, "stage_chunk issues Mp * CT / 32 loads per wave: eight waves per chunk");
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // XL = 1, 2: [M][spr * 128]; XL = 3: two chunks

    const int tile = select_matrix(mt, m, y, bias);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nl = lane & 15;
    const int quarter = lane >> 4;
    const int row = tile * kTileRows + nl;
    bool m_ok[MB];                                   // activation row 16 mb + nl of the A operand
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) m_ok[mb] = 16 * mb + nl < M;
    const int steps = m.spr;
    const int kpad = steps * kTileGroups * kGroup;
    float s = 0.0f;
    if constexpr (MODE == kModeW) s = row < m.rows ? m.scales[row] : 0.0f;
    // Thread o < 256 stores output (4*(o%64/16) + o/64, n0 + o%16) at the end;
    // its row scale and bias are loaded now, ahead of the weights, so that
    // the epilogue does not wait for another memory round trip.
    const int on = tile * kTileRows + (threadIdx.x & 15);
    float out_scale = 1.0f;
    uint16_t out_bias = 0;
    if (threadIdx.x < 256 && on < m.rows) {
        if constexpr (MODE == kModeQ) out_scale = m.scales[on];
        if (bias) out_bias = bias[on];
    }
    // Slot of this lane in the row tile's first tile; step st adds st * 64.
    const size_t slot0 = static_cast<size_t>(tile) * steps * kTileSlots + lane;

    uint4 xv[XL == 1 ? kXVecs : 1];
    const int vpr = kpad / 8;                        // uint4 vectors per staged row
    // xvec == 2: rows are whole tiles wide (cols == kpad) and x is 16-byte
    // aligned, so the staged copy is x itself and goes global -> LDS
    // directly, without registers; otherwise through registers, zero-padded.
    // XL = 2 is launched for xvec == 2 only.
    const bool xdirect = XL >= 2 || xvec == 2;
    // XL = 3 (launched for xvec == 2): chunk c, columns c*CT*128 .. +CT*128,
    // of Mp rows (M rounded up so that every wave issues Mp*CT/32 1 KB loads
    // per chunk, which keeps the vector-memory counts uniform; padding rows
    // repeat row M-1 and past the last column the source is clamped, neither
    // is read) goes global -> LDS into buffer c % 2.
    const int Mp = XL == 3 ? (M + 32 / CT - 1) / (32 / CT) * (32 / CT) : M;
    const int chunk_halves = Mp * CT * kTileGroups * kGroup;
    const int chunks = (steps + CT - 1) / CT;
    auto stage_chunk = [&](int c) {
        uint16_t* buf = xs + (c & 1) * chunk_halves;
        const int per_wave = Mp * CT / 32;
        for (int r = 0; r < per_wave; ++r) {
            const int v = (r * WAVES + wave) * 64 + lane;          // 16-byte vector of the chunk
            const int mi = v / (CT * 16);
            const int j = v - mi * (CT * 16);
            const int src_row = min(mi, M - 1);
            const int src_col = min(c * CT * kTileGroups * kGroup + 8 * j, m.cols - 8);
            __builtin_amdgcn_global_load_lds(x + static_cast<size_t>(src_row) * m.cols + src_col,
                                             (lds_void_ptr)(buf + 8 * (v - lane)), 16, 0, 0);
        }
    };
    if constexpr (XL == 3) {
        stage_chunk(0);
    } else if constexpr (XL != 0) {
        if (xdirect) {
#pragma unroll
            for (int r = 0; r < kXDirect; ++r) {
                const int i = threadIdx.x + r * kThreads;
                if (i < M * vpr) {
                    __builtin_amdgcn_global_load_lds(x + 8 * i,
                                                     (lds_void_ptr)(xs + 8 * (r * kThreads + (threadIdx.x & ~63))),
                                                     16, 0, 0);
                }
            }
        } else if constexpr (XL == 1) {
#pragma unroll
            for (int r = 0; r < kXVecs; ++r) {
                const int i = threadIdx.x + r * kThreads;
                xv[r] = make_uint4(0, 0, 0, 0);
                if (i < M * vpr) {
                    const int mi = i / vpr;
                    xv[r] = load_x8(x, mi, (i - mi * vpr) * 8, m.cols, xvec != 0);
                }
            }
        }
    }

    // The waits after the first weight batch count the loads issued after
    // the activation staging: keep the scheduler from moving any above it.
    __builtin_amdgcn_sched_barrier(0);

    // Steps past the end (steps % kBatch != 0) reload the last tile; they
    // meet zero activations, and raw fp16 weights, which could hold Inf or
    // NaN, are zeroed there.
    floatx4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    Bits buf0[GPL], buf1[GPL];
    const int nb = (steps + kBatch - 1) / kBatch;    // workgroup batches
    const uint16_t* xrow[MB];
    const uint16_t* xsrow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int r = m_ok[mb] ? 16 * mb + nl : 0;
        xrow[mb] = x + static_cast<size_t>(r) * m.cols;
        xsrow[mb] = xs + static_cast<size_t>(r) * kpad;
    }
    half8 a[MB][GPL][4];

    // One batch is prefetched while the previous one is multiplied (two
    // register buffers alternate, so no register copy waits on loads in
    // flight; every branch is uniform).  The activations of a batch are read
    // before the next batch's weights are issued, so that waiting for them
    // (global loads when they are not staged in LDS) does not wait for those
    // weights.  Keeping more batches in flight per wave measured slower on
    // MI355X: one tile per wave plus the prefetch keeps ~40 KB per CU in
    // flight, which already covers the loaded HBM latency.
    decode_load_batch<GPL>(m, buf0, slot0, wave * GPL, steps);
    if constexpr (XL == 3) {
        // chunk 0 precedes the weight loads just issued
        wait_vmcnt<GPL * GroupLoads<B, MODE>::value>();
        barrier_after_wait();
        if (chunks > 1) stage_chunk(1);
    } else if constexpr (XL != 0) {
        if (xdirect) {
            // the activation loads precede the weight loads just issued
            wait_vmcnt<GPL * GroupLoads<B, MODE>::value>();
            barrier_after_wait();
        } else if constexpr (XL == 1) {
#pragma unroll
            for (int r = 0; r < kXVecs; ++r) {
                const int i = threadIdx.x + r * kThreads;
                if (i < M * vpr) *reinterpret_cast<uint4*>(xs + 8 * i) = xv[r];
            }
            __syncthreads();
        }
    }
    auto batch = [&](const Bits (&cur)[GPL], Bits (&nxt)[GPL], bool prefetch, int bi) {
        int kshift = 0;
        if constexpr (XL == 3) {
            const int c = bi / kBpc;
            if (bi > 0 && bi == c * kBpc) {
                // First batch of chunk c: chunk c's loads are older than
                // this batch's weights (issued during the previous batch),
                // the only loads allowed to stay in flight.  The barrier
                // also retires every wave's reads of chunk c - 1, whose
                // buffer chunk c + 1 then refills.
                wait_vmcnt<GPL * GroupLoads<B, MODE>::value>();
                barrier_after_wait();
                if (c + 1 < chunks) stage_chunk(c + 1);
            }
            kshift = c * CT * kTileGroups * kGroup;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                xsrow[mb] = xs + (c & 1) * chunk_halves + (m_ok[mb] ? 16 * mb + nl : 0) * (CT * kTileGroups * kGroup);
            }
        }
        decode_activations<GPL, XL, MB>(a, m, bi * kBatch, wave, quarter, m_ok, steps, xrow, xsrow, xvec, kshift);
        if (prefetch) decode_load_batch<GPL>(m, nxt, slot0, (bi + 1) * kBatch + wave * GPL, steps);
        decode_mul_batch<B, MODE, GPL, MB>(cur, a, bi * kBatch + wave * GPL, steps, s, acc);
    };
    for (int bi = 0;; bi += 2) {
        if (bi + 1 >= nb) {
            batch(buf0, buf1, false, bi);
            break;
        }
        batch(buf0, buf1, true, bi);
        if (bi + 2 >= nb) {
            batch(buf1, buf0, false, bi + 1);
            break;
        }
        batch(buf1, buf0, true, bi + 1);
    }

    // cross-wave reduction of each 16x16 fp32 block, one block at a time
    __shared__ floatx4 red[WAVES][64];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        if (mb > 0) __syncthreads();
        red[wave][lane] = acc[mb];
        __syncthreads();
        if (threadIdx.x < 256) {
            const int src = threadIdx.x & 63;
            const int e = threadIdx.x >> 6;
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) v += red[w][src][e];
            const int mi = 16 * mb + 4 * (src >> 4) + e;   // D[4*(l/16)+e][l%16] of block mb
            if (mi < M && on < m.rows) {
                store_out(y + static_cast<size_t>(mi) * m.rows + on,
                          epilogue<MODE>(v, out_scale, bias != nullptr, out_bias));
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV, M <= 16, K at most 32 tiles (4096 columns): one workgroup of 16 waves
// owns one row tile and wave w takes its tiles w and w + 16, so every
// weight tile of the workgroup is requested at once, before the wave waits
// for anything.  On MI355X a 4096 x 4096 b = 10 matrix spreads as 16 waves
// per CU with 5 KB each in flight; the linear_decode_kernel organisation
// (8 waves, one tile in flight plus one prefetched) takes 7% longer there.
// For longer rows the all-in-flight form measured slower (more bytes in
// flight per CU than the memory system serves well), so those keep
// linear_decode_kernel.
//
// Only activation rows 0 .. M-1 of the A operand are non-zero, so D[e][n]
// (lane n, element e) holds row n's partial sum for activation row e; the
// 16 partials are added in wave order, so results are deterministic.
//
// Each wave stages only the activations of its own two tiles (256 columns
// of M rows, 512 B of LDS per row, one 32-lane global_load_lds per row) and
// waits on its own loads, so no workgroup barrier stands between the loads
// and the MFMAs.
// Per-wave clock stamps of the earlier form, where the workgroup staged all
// of x and passed a barrier first, showed the waves spending ~1.2 us of a
// ~3.7 us life until that barrier; measured on MI355X (us, that form ->
// this): 4096^2 b = 10 5.668 -> 5.643, b = 9 5.404 -> 5.358, 11008 x 4096
// 11.6 -> 11.33, 14336 x 4096 14.43 -> 13.99, 4096 x 3072 5.26 -> 5.11.
// ---------------------------------------------------------------------------

constexpr int kGemvWaves = 16;
constexpr int kGemvMaxSteps = 2 * kGemvWaves;
constexpr int kGemvMaxM = 4;                 // M up to this: lanes 0-15 hold all of D

// MR: 1 (M = 1, every row count a compile-time 1), kGemvMaxM (M = 2..4,
// outputs in lanes 0-15) or 16 (M = 5..16, outputs in every lane).
template <int B, int MODE, int MR>
__global__ __launch_bounds__(64 * kGemvWaves) void linear_gemv_kernel(
    DevMatrix m, const uint16_t* __restrict__ x, int m_rows, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ bias, const MultiTail mt) {
    using Bits = GroupBits<B, MODE>;
    constexpr int kXRow = 2 * kTileGroups * kGroup;                  // halves of one row's two steps
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // [kGemvWaves][M][2][128]
    __shared__ float red[kGemvWaves][MR][kTileRows];
    const int M = MR == 1 ? 1 : m_rows;

    const int tile = select_matrix(mt, m, y, bias);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nl = lane & 15;
    const int quarter = lane >> 4;
    const int steps = m.spr;
    const int row = tile * kTileRows + nl;
    float s = 0.0f;
    if constexpr (MODE == kModeW) s = row < m.rows ? m.scales[row] : 0.0f;
    // thread o < 16 M stores output (o / 16, row of n = o % 16) at the end
    const int on = tile * kTileRows + (threadIdx.x & 15);
    float out_scale = 1.0f;
    uint16_t out_bias = 0;
    if (static_cast<int>(threadIdx.x) < kTileRows * M && on < m.rows) {
        if constexpr (MODE == kModeQ) out_scale = m.scales[on];
        if (bias) out_bias = bias[on];
    }
    // The x of this wave's steps goes global -> LDS into this wave's M x 512
    // bytes: vector v (row v / 32, step wave + 16 ((v / 16) % 2), 16-byte
    // vector v % 16 of that step; cols == spr * 128).  A step past the last
    // is staged as the last one and multiplied by zero.
    uint16_t* xw = xs + wave * M * kXRow;
    for (int k = 0; 32 * M > 64 * k; ++k) {
        const int v = 64 * k + lane;
        if (v < 32 * M) {
            const int st = min(wave + kGemvWaves * ((v >> 4) & 1), steps - 1);
            __builtin_amdgcn_global_load_lds(x + static_cast<size_t>(v >> 5) * m.cols + 8 * (st * 16 + (v & 15)),
                                             (lds_void_ptr)(xw + 512 * k), 16, 0, 0);
        }
    }
    // The wait below counts the weight loads issued after these: keep the
    // scheduler from moving any of them above.
    __builtin_amdgcn_sched_barrier(0);
    const size_t slot0 = static_cast<size_t>(tile) * steps * kTileSlots + lane;
    Bits b0, b1;
    b0.load(m, slot0 + static_cast<size_t>(min(wave, steps - 1)) * kTileSlots);
    b1.load(m, slot0 + static_cast<size_t>(min(wave + kGemvWaves, steps - 1)) * kTileSlots);
    // everything but the two weight tiles (scales, bias, this wave's x) has
    // landed; no other wave's x is read
    wait_vmcnt<2 * GroupLoads<B, MODE>::value>();

    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool xok = nl < M;
    const uint16_t* xr = xw + (xok ? nl : 0) * kXRow;
    auto mul = [&](const Bits& bits, int st) {
        const bool ok = st < steps;
        const int k0 = (st >= kGemvWaves ? kTileGroups * kGroup : 0) + quarter * kGroup;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const half8 xa = *reinterpret_cast<const half8*>(xr + k0 + 8 * t);   // broadcast per quarter and row
            const half8 a = (ok && xok) ? xa : half8{0, 0, 0, 0, 0, 0, 0, 0};
            half8 b = bits.operand(t, s);
            if constexpr (MODE == kModeRaw) {
                // past the last tile the reloaded raw weights may hold Inf or NaN
                if (!ok) b = half8{0, 0, 0, 0, 0, 0, 0, 0};
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
        }
    };
    mul(b0, wave);
    mul(b1, wave + kGemvWaves);

    // D[i][n] of activation row i sits in lane 16 (i / 4) + n, element i % 4
    if constexpr (MR <= 4) {
        if (lane < kTileRows) {
#pragma unroll
            for (int e = 0; e < MR; ++e) {
                if (e < M) red[wave][e][lane] = acc[e];
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * quarter + e;
            if (i < M) red[wave][i][nl] = acc[e];
        }
    }
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < kTileRows * M && on < m.rows) {
        const int e = threadIdx.x >> 4;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kGemvWaves; ++w) v += red[w][e][threadIdx.x & 15];
        store_out(y + static_cast<size_t>(e) * m.rows + on, epilogue<MODE>(v, out_scale, bias != nullptr, out_bias));
    }
}

// ---------------------------------------------------------------------------
// general GEMM, M > 16, for what linear_prefill_kernel does not take: raw
// fp16 weights (b = 16) and activations that are not 16-byte aligned or
// whose K is not a multiple of 8.  128 x 128 output tiles, K steps of 64
// (two groups).  Four waves in a 2 x 2 grid each own 64 x 64.  Every K step
// the workgroup stages the activation tile and the decoded fp16 weight tile
// in LDS (double buffered) and feeds v_mfma_f32_16x16x32_f16.
// ---------------------------------------------------------------------------

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLDK = kBK + 8;  // padded row (halves) to stagger LDS banks

template <int B, int MODE>
__global__ __launch_bounds__(256) void linear_gemm_kernel(
    DevMatrix m, const uint16_t* __restrict__ x, int M, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ bias, int xvec) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][kBM * kLDK];
    __shared__ __attribute__((aligned(16))) _Float16 ws[2][kBN * kLDK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int m0 = blockIdx.y * kBM;
    const int n0 = blockIdx.x * kBN;
    const int ktiles = (m.gpr + 1) >> 1;

    // activation loader: rows tid/8 + 32j, 8 halves at column 8*(tid%8)
    const int xr = tid >> 3;
    const int xc = (tid & 7) * 8;
    // weight loader: row tid/2, group 2*kt + (tid & 1)
    const int wr = tid >> 1;
    const int wh = tid & 1;
    const int wrow = n0 + wr;
    const bool wrow_ok = wrow < m.rows;
    float ws_scale = 0.0f;
    if constexpr (MODE == kModeW) ws_scale = wrow_ok ? m.scales[wrow] : 0.0f;

    uint4 xreg[4];
    Raw<(B == 16 ? 8 : B)> wraw;
    uint4 w16reg[4];

    auto load_tile = [&](int kt) {
        const int k0 = kt * kBK;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = m0 + xr + 32 * j;
            const int k = k0 + xc;
            if (r < M && xvec && k + 8 <= m.cols) {
                xreg[j] = *reinterpret_cast<const uint4*>(x + static_cast<size_t>(r) * m.cols + k);
            } else {
                uint32_t v[4] = {0, 0, 0, 0};
                if (r < M) {
                    for (int i = 0; i < 8; ++i) {
                        if (k + i < m.cols) {
                            v[i >> 1] |= static_cast<uint32_t>(x[static_cast<size_t>(r) * m.cols + k + i]) << (16 * (i & 1));
                        }
                    }
                }
                xreg[j] = make_uint4(v[0], v[1], v[2], v[3]);
            }
        }
        const int grp = 2 * kt + wh;
        const bool ok = wrow_ok && grp < m.gpr;
        const size_t g = group_slot(wrow, grp, m.spr);
        if constexpr (MODE == kModeRaw) {
            if (ok) {
                const uint4* p = reinterpret_cast<const uint4*>(m.w16 + g * kGroup);
#pragma unroll
                for (int t = 0; t < 4; ++t) w16reg[t] = p[t];
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) w16reg[t] = make_uint4(0, 0, 0, 0);
            }
        } else {
            if (ok) raw_load<B>(m, g, wraw); else raw_zero<B>(wraw);
        }
    };

    auto store_tile = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            *reinterpret_cast<uint4*>(&xs[buf][(xr + 32 * j) * kLDK + xc]) = xreg[j];
        }
        _Float16* wdst = &ws[buf][wr * kLDK + wh * kGroup];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if constexpr (MODE == kModeRaw) {
                *reinterpret_cast<uint4*>(wdst + 8 * t) = w16reg[t];
            } else {
                *reinterpret_cast<half8*>(wdst + 8 * t) = decode8<B, MODE>(wraw, t, ws_scale);
            }
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    load_tile(0);
    store_tile(0);
    __syncthreads();

    const int fr = lane & 15;          // operand row inside a 16-row block
    const int fk = (lane >> 4) * 8;    // operand K offset inside a 32-wide step
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ktiles) load_tile(kt + 1);
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 32) {
            half8 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                af[i] = *reinterpret_cast<const half8*>(&xs[buf][(wm * 64 + 16 * i + fr) * kLDK + kk + fk]);
                bf[i] = *reinterpret_cast<const half8*>(&ws[buf][(wn * 64 + 16 * i + fr) * kLDK + kk + fk]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < ktiles) store_tile(buf ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds D[4*(lane/16)+e][lane%16] of each 16x16 block
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 64 + 16 * j + (lane & 15);
        if (n >= m.rows) continue;
        float sn = 1.0f;
        if constexpr (MODE == kModeQ) sn = m.scales[n];
        const uint16_t bn = bias ? bias[n] : uint16_t(0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = m0 + wm * 64 + 16 * i + 4 * (lane >> 4) + e;
                if (r < M) y[static_cast<size_t>(r) * m.rows + n] = epilogue<MODE>(acc[i][j][e], sn, bias != nullptr, bn);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// prefill kernel (tiled planes), M > 16, integer-dot and decoded-fp16 modes.
//
// Workgroup tile: 128 activation rows x 128*NB weight rows, K steps of 128
// columns (one plane tile).  Four column groups of waves each own 32*NB
// weight rows for all 128 activation rows: a 128 x 32*NB accumulator tile,
// 4 x NB blocks of v_mfma_f32_32x32x16_f16 (the 32x32 shape sustains
// near-peak rate with few independent accumulators; the 16x16x32 shape
// needs many more).  With KS = 2 each column group is two waves (eight
// waves, two per SIMD) that take the two group pairs of every step and
// add their partial sums through LDS at the end.  The launcher runs NB = 2
// (128 x 256) tiles and covers a partial last round of the machine with
// NB = 1 half tiles.
//
//  * B (weights) never goes through LDS.  For weight block nb2 (32 rows =
//    two row tiles) and group pair p, lane l = 32h + n loads slot
//    16*(2p+h) + n%16 of row tile 2*nb2 + n/16 -- the B operand rows of
//    v_mfma_f32_32x32x16_f16 -- and decodes it in registers.  Each decoded
//    operand feeds four MFMAs (one per 32 activation rows).  B of step k+1
//    (k+2 for codes of at most 10 bits) is loaded into a register buffer
//    while step k is multiplied.
//  * A (activations) goes global -> LDS directly (global_load_lds_dwordx4,
//    no registers), into a ring of three stages so that step k+2 is in
//    flight while step k is multiplied.  A stage row is 256 bytes with its
//    16-byte chunks XOR-swizzled by (row & 15), so a wave's operand reads
//    (16 consecutive rows, one chunk per half wave) hit every bank once.
//  * The K order inside a step is the same for both operands: MFMA (p, t)
//    takes codes 8t..8t+8 of group 2p+h in lane half h, i.e. columns
//    32*(2p+h) + 8t + i.
//  * Loads are unconditional: past the last step the clamped address
//    re-reads the last step (L2 hits), so no wait covers loads behind a
//    branch.  Rows past M read the last row; their outputs are not stored.
//  * Workgroup -> tile: dispatch places workgroup i on XCD i % 8, so each
//    XCD is given a contiguous range of tiles, walked four activation blocks
//    at a time, and the ~32 workgroups an XCD runs at once share their
//    activation and weight blocks in that XCD's L2.
// ---------------------------------------------------------------------------


constexpr int kPN = 256;                   // weight rows per workgroup (4 waves x 64)
constexpr int kPGroupM = 4;                // activation blocks per tile-order group

// Vector-memory instructions one GroupBits::load32 issues (kModeQ / kModeW).
template <int B>
constexpr int group_loads() {
    return (Planes<B>::h8 ? 2 : 0) + (Planes<B>::h4 ? 1 : 0) +
           (Planes<B>::h21 ? 1 : (Planes<B>::h2 ? 1 : 0) + (Planes<B>::h1 ? 1 : 0));
}

// Prefill tile geometry for MI 32-row activation blocks per wave.
template <int MI>
struct PrefillShape {
    // 256 rows (MI = 8) needs 256 accumulator registers per lane; that build
    // spilled and did not reproduce the oracle, so only 128 rows is enabled.
    static_assert(MI == 4 || MI == 2, "the prefill kernel is built for 128 or 64 activation rows per workgroup");
    static constexpr int kRows = 32 * MI;            // activation rows per workgroup
    static constexpr int kStage = kRows * kPRow;     // bytes per activation stage
    static constexpr int kStages = MI <= 4 ? 3 : 2;  // 48 KB, 96 KB or 128 KB of LDS
    static constexpr int kLds = kStages * kStage;
    static constexpr int kALoads = kRows / 16;       // A loads per step per wave (1 KB each)
    static constexpr int kADist = kStages - 1;       // activation prefetch distance
};

template <int B, int MODE, int MI, int NB, int KS>
__global__ __launch_bounds__(256 * KS) void linear_prefill_kernel(
    DevMatrix m, const uint16_t* __restrict__ x, int M, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ bias, int mblocks, int nblocks, int tile0, int njobs, int per_xcd) {
    using Bits = GroupBits<B, MODE>;
    using Shape = PrefillShape<MI>;
    __shared__ __attribute__((aligned(16))) uint8_t xs[Shape::kLds];

    static_assert(NB == 1 || NB == 2, "32 or 64 weight rows per wave");
    static_assert(KS == 1 || KS == 2, "one or two waves per weight column group");
    constexpr int kPL = 2 / KS;                     // group pairs (of a step's 4 groups) per wave
    // ---- tile of this workgroup (uniform early exit, before any barrier) ----
    // Jobs j = 0 .. njobs-1 cover the full tiles tile0, tile0+1, ... of the
    // grouped order (128 x 256); with NB = 1 two jobs split a full tile into
    // its two 128-row weight halves.
    const int xcd = blockIdx.x & 7;
    const int local = blockIdx.x >> 3;
    const int job = xcd * per_xcd + local;
    if (local >= per_xcd || job >= njobs) return;
    const int tile = tile0 + (NB == 2 ? job : job >> 1);
    const int group = tile / (kPGroupM * nblocks);
    const int within = tile - group * kPGroupM * nblocks;
    const int gm = min(kPGroupM, mblocks - group * kPGroupM);
    const int mb = group * kPGroupM + within % gm;
    const int nb = within / gm;
    const int m0 = mb * Shape::kRows;
    // first weight row of this workgroup and of this wave
    const int n0 = nb * kPN + (NB == 2 ? 0 : (job & 1) * (kPN / 2));

    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // 0 .. 4*KS-1
    const int wave = wave_id & 3;                   // weight column group
    const int kp = wave_id >> 2;                    // K half of each step (KS = 2)
    const int n32 = lane & 31;
    const int half = lane >> 5;
    const int steps = m.spr;

    const int nw0 = n0 + wave * 32 * NB;
    // B slots of this lane: [nb2][p] -> row tile 2*nb2 + n32/16 of the wave,
    // slot 16*(2p + half) + n32%16 (row tiles clamped; rows past the end are
    // never stored).  Slot indices fit 32 bits (planes below 4 GiB).
    uint32_t slot0[NB][kPL];
    float s[NB];
#pragma unroll
    for (int nb2 = 0; nb2 < NB; ++nb2) {
        s[nb2] = 0.0f;
        const int rt = min(nw0 / kTileRows + 2 * nb2 + (n32 >> 4), m.rtiles - 1);
#pragma unroll
        for (int pl = 0; pl < kPL; ++pl) {
            const int p = KS == 2 ? kp : pl;
            slot0[nb2][pl] = static_cast<uint32_t>(rt) * static_cast<uint32_t>(steps * kTileSlots) +
                             static_cast<uint32_t>(16 * (2 * p + half) + (n32 & 15));
        }
        if constexpr (MODE == kModeW) {
            const int row = rt * kTileRows + (n32 & 15);
            s[nb2] = row < m.rows ? m.scales[row] : 0.0f;
        }
    }

    // Activation loads of step st into stage `stage`: wave w fills rows
    // w*Shape::kRows/4 .. (w+1)*Shape::kRows/4 - 1, four rows (1 KB, one instruction) at a time; lane l
    // writes physical chunk l%16 of row l/16, i.e. logical chunk
    // (l%16) ^ (row & 15).  Per lane and instruction the source is a fixed
    // row (clamped to M-1) and a fixed chunk; only the column base moves.
    // The launcher guarantees cols % 8 == 0, a 16-byte aligned x and
    // M * cols * 2 below 4 GiB.
    // Instruction i covers rows w*Shape::kRows/4 + 4i + l/16; its chunk pattern
    // repeats every four instructions.
    constexpr int kAWaveRows = Shape::kRows / (4 * KS);   // rows each wave loads
    constexpr int kAWaveLoads = kAWaveRows / 4;          // 1 KB instructions per wave
    // swizzle of row wave_id * kAWaveRows + 4i + l/16 (not a multiple of 16
    // apart for every wave when kAWaveRows < 16)
    int achunk[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        achunk[i] = 8 * ((lane & 15) ^ ((wave_id * kAWaveRows + 4 * i + (lane >> 4)) & 15));
    const int arow0 = m0 + wave_id * kAWaveRows + (lane >> 4);
    const uint8_t* xb = reinterpret_cast<const uint8_t*>(x);
    auto load_a = [&](int st, int stage) {
        const int k0 = min(st, steps - 1) * kPK;
        const int kmax = m.cols - 8;
#pragma unroll
        for (int i = 0; i < kAWaveLoads; ++i) {
            const uint32_t row = static_cast<uint32_t>(min(arow0 + 4 * i, M - 1));
            const uint32_t off = 2u * (row * static_cast<uint32_t>(m.cols) +
                                       static_cast<uint32_t>(min(k0 + achunk[i & 3], kmax)));
            __builtin_amdgcn_global_load_lds(xb + off, (lds_void_ptr)(xs + stage * Shape::kStage +
                                                                      (wave_id * kAWaveRows + i * 4) * kPRow),
                                             16, 0, 0);
        }
    };
    auto load_b = [&](Bits (&bits)[NB][kPL], int st) {
        const uint32_t off = static_cast<uint32_t>(min(st, steps - 1) * kTileSlots);
#pragma unroll
        for (int nb2 = 0; nb2 < NB; ++nb2)
#pragma unroll
            for (int pl = 0; pl < kPL; ++pl) bits[nb2][pl].load32(m, slot0[nb2][pl] + off);
    };

    floatx16 acc[MI][NB];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // A operands of MFMA (p, t) for the MI 32-row blocks: row 32i + n32,
    // logical chunk 4*(2p + half) + t.
    auto read_a = [&](half8 (&a)[MI], int stage, int p, int t) {
        const int chunk = (4 * (2 * p + half) + t) ^ (n32 & 15);
        const uint8_t* base = xs + stage * Shape::kStage + n32 * kPRow + chunk * 16;
#pragma unroll
        for (int i = 0; i < MI; ++i) a[i] = *reinterpret_cast<const half8*>(base + 32 * i * kPRow);
    };
    // Slices pt = 0..7 of a step (group pair p = pt/4, codes t = pt%4).
    // Software pipeline per slice: read the A operands of slice pt+1 from
    // LDS and decode the B operands of slice pt+1 while the eight MFMAs of
    // slice pt run, then wait for the reads.  sched_barrier pins the slice
    // boundaries; inside a slice the compiler interleaves the decode VALU
    // with the MFMAs.
    auto decode_pt = [&](const Bits (&cur)[NB][kPL], half8 (&bop)[NB], int ps) {
#pragma unroll
        for (int nb2 = 0; nb2 < NB; ++nb2) bop[nb2] = cur[nb2][ps >> 2].operand(ps & 3, s[nb2]);
    };
    auto mfma_pt = [&](const half8 (&a)[MI], const half8 (&bop)[NB]) {
#pragma unroll
        for (int nb2 = 0; nb2 < NB; ++nb2) {
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                acc[i][nb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bop[nb2], acc[i][nb2], 0, 0, 0);
            }
        }
    };
    // Local slice ps covers group pair (KS == 2 ? kp : ps/4), codes t = ps%4.
    auto pair_of = [&](int ps) { return KS == 2 ? kp : (ps >> 2); };
    auto multiply = [&](const Bits (&cur)[NB][kPL], int stage) {
        constexpr int kSlices = 4 * kPL;
        half8 a0[MI], a1[MI];
        half8 b0[NB], b1[NB];
        read_a(a0, stage, pair_of(0), 0);
        decode_pt(cur, b0, 0);
        wait_lgkmcnt<0>();
#pragma unroll
        for (int ps = 0; ps < kSlices; ps += 2) {
            read_a(a1, stage, pair_of(ps + 1), (ps + 1) & 3);
            decode_pt(cur, b1, ps + 1);
            mfma_pt(a0, b0);
            __builtin_amdgcn_sched_barrier(0);
            wait_lgkmcnt<0>();
            if (ps + 2 < kSlices) {
                read_a(a0, stage, pair_of(ps + 2), (ps + 2) & 3);
                decode_pt(cur, b0, ps + 2);
            }
            mfma_pt(a1, b1);
            __builtin_amdgcn_sched_barrier(0);
            wait_lgkmcnt<0>();
        }
    };

    // Issue order matters (vector loads retire in order).  Per step: B of
    // step st+kBDist, then A of step st+kADist.  Before the barrier the wave
    // waits for everything except the batches just issued, i.e. for A(st+1)
    // and B(st+1).  sched_barrier keeps the compiler from sinking the loads
    // into the multiply.  With two waves per column group and codes of at
    // most 10 bits the register budget holds a third B buffer, so B is
    // prefetched two steps ahead; the buffers rotate by unrolling, so no
    // register copy is needed.
    constexpr int kBDist = (KS == 2 && MODE != kModeRaw && B <= 10) ? 2 : 1;
    constexpr int kBLoads = NB * kPL * GroupLoads<B, MODE>::value;   // B loads per step per wave
    auto step = [&](const Bits (&cur)[NB][kPL], Bits (&next)[NB][kPL], int st) {
        load_b(next, st + kBDist);
        __builtin_amdgcn_sched_barrier(0);
        load_a(st + Shape::kADist, (st + Shape::kADist) % Shape::kStages);
        __builtin_amdgcn_sched_barrier(0);
        multiply(cur, st % Shape::kStages);
        __builtin_amdgcn_sched_barrier(0);
        // A(st+1) and B(st+1) landed
        wait_vmcnt<kAWaveLoads * (Shape::kADist - 1) + kBLoads * (kBDist - 1)>();
        barrier_after_wait();
        __builtin_amdgcn_sched_barrier(0);
    };
    Bits b0[NB][kPL], b1[NB][kPL], b2[NB][kPL];
    load_b(b0, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_a(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kBDist == 2) load_b(b1, 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 1; d < Shape::kADist; ++d) load_a(d, d);
    __builtin_amdgcn_sched_barrier(0);
    // B(0) and A(0) landed; the later batches may be in flight
    wait_vmcnt<kAWaveLoads * (Shape::kADist - 1) + kBLoads * (kBDist - 1)>();
    barrier_after_wait();
    if constexpr (kBDist == 2) {
        for (int st = 0;; st += 3) {
            step(b0, b2, st);
            if (st + 1 >= steps) break;
            step(b1, b0, st + 1);
            if (st + 2 >= steps) break;
            step(b2, b1, st + 2);
            if (st + 3 >= steps) break;
        }
    } else {
        (void)b2;
        for (int st = 0;; st += 2) {
            step(b0, b1, st);
            if (st + 1 >= steps) break;
            step(b1, b0, st + 1);
            if (st + 2 >= steps) break;
        }
    }

    // ---- epilogue ----
    // 32x32 block element e of lane l is D[8*(e/4) + 4*(l/32) + e%4][l%32].
    // In passes of four row blocks (128 rows), each wave converts its part
    // of the tile to fp16 (scale, rounding, bias) into the workgroup's LDS
    // copy of the tile, then all waves write it back row by row with
    // 16-byte stores, each row one contiguous segment.  The activation
    // stages are free by now; the clamped re-reads of the last steps must
    // land before the LDS is reused.
    wait_vmcnt<0>();
    __syncthreads();
    if constexpr (KS == 2) {
        // The K-half-1 waves hand their partial sums to the K-half-0 waves
        // of the same column group through LDS, kRB row blocks at a time
        // (two when the four column groups' 4 * kRB * NB * 4 KB fit).
        constexpr int kRB = 4 * 2 * NB * 16 * 64 * 4 <= Shape::kLds ? 2 : 1;
        static_assert(4 * kRB * NB * 16 * 64 * 4 <= Shape::kLds, "K-split reduction exceeds the activation LDS");
        float* red = reinterpret_cast<float*>(xs) + wave * (kRB * NB * 16 * 64);
#pragma unroll
        for (int h = 0; h < MI / kRB; ++h) {
            if (kp == 1) {
#pragma unroll
                for (int i2 = 0; i2 < kRB; ++i2)
#pragma unroll
                    for (int nb2 = 0; nb2 < NB; ++nb2)
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            red[((i2 * NB + nb2) * 16 + e) * 64 + lane] = acc[kRB * h + i2][nb2][e];
            }
            __syncthreads();
            if (kp == 0) {
#pragma unroll
                for (int i2 = 0; i2 < kRB; ++i2)
#pragma unroll
                    for (int nb2 = 0; nb2 < NB; ++nb2)
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            acc[kRB * h + i2][nb2][e] += red[((i2 * NB + nb2) * 16 + e) * 64 + lane];
            }
            __syncthreads();
        }
    }
    constexpr int kCols = 32 * NB;               // output columns per wave
    constexpr int kTileCols = 4 * kCols;         // output columns per workgroup
    constexpr int kCPitch = 2 * kTileCols + 16;  // bytes per staged output row
    constexpr int kPassBlocks = MI < 4 ? MI : 4; // 32-row blocks per output pass
    constexpr int kCRows = 32 * kPassBlocks;     // rows per pass
    constexpr int kLanesPerRow = kTileCols / 8;  // 16-byte chunks per row
    constexpr int kThreads = 256 * KS;
    static_assert(kCRows * kCPitch <= Shape::kLds, "output staging exceeds the activation LDS");
    float sn[NB];
    uint16_t bn[NB];
#pragma unroll
    for (int nb2 = 0; nb2 < NB; ++nb2) {
        const int n = min(nw0 + 32 * nb2 + n32, m.rows - 1);
        sn[nb2] = 1.0f;
        bn[nb2] = 0;
        if constexpr (MODE == kModeQ) sn[nb2] = m.scales[n];
        if (bias) bn[nb2] = bias[n];
    }
    const bool yvec = (m.rows % 8 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0);
    const int chunk = threadIdx.x % kLanesPerRow;
#pragma unroll
    for (int pass = 0; pass < MI / kPassBlocks; ++pass) {
        if (pass > 0) __syncthreads();
        // the whole workgroup tile goes to LDS so that rows leave as
        // contiguous 2*kTileCols-byte segments
        if (kp == 0) {
            uint8_t* cw = xs + wave * kCols * 2;
#pragma unroll
            for (int nb2 = 0; nb2 < NB; ++nb2) {
#pragma unroll
                for (int i = 0; i < kPassBlocks; ++i) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int r = 32 * i + 8 * (e >> 2) + 4 * half + (e & 3);
                        *reinterpret_cast<uint16_t*>(cw + r * kCPitch + (32 * nb2 + n32) * 2) =
                            epilogue<MODE>(acc[kPassBlocks * pass + i][nb2][e], sn[nb2], bias != nullptr,
                                           bn[nb2]);
                    }
                }
            }
        }
        __syncthreads();
#pragma unroll 2
        for (int it = 0; it < kCRows * kLanesPerRow / kThreads; ++it) {
            const int r = it * (kThreads / kLanesPerRow) + static_cast<int>(threadIdx.x) / kLanesPerRow;
            const int gr = m0 + pass * kCRows + r;
            const int gn = n0 + chunk * 8;
            if (gr >= M || gn >= m.rows) continue;
            const uint4 v = *reinterpret_cast<const uint4*>(xs + r * kCPitch + chunk * 16);
            uint16_t* dst = y + static_cast<size_t>(gr) * m.rows + gn;
            if (yvec) {
                store_out16(dst, v);
            } else {
                const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    if (gn + k < m.rows) dst[k] = h[k];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// prefill, wide tiles (b <= 15): 256 activation rows x 256 weight rows per
// workgroup, four waves, one per SIMD.  Wave w owns weight rows
// 64w .. 64w + 63 of the tile for all 256 activation rows: 8 x 2 blocks of
// v_mfma_f32_32x32x16_f16 (256 accumulator registers per lane).
//
// Why this shape: per K step (128 columns) the CU moves 64 KB of activations
// (global -> LDS, shared by the four waves) and 40 KB of b = 10 weight bits
// (global -> registers, each wave its own 64 rows, nothing loaded twice)
// for 512 MFMAs; the 128 x 256 tile of linear_prefill_kernel moves 72 KB
// for 256, and the CU's vector memory pipe (64 B per clock) was what its
// waves stalled on.  Each decoded weight operand feeds eight MFMAs, each
// activation operand read from LDS two.
//
// Pipeline, per step st (8 slices of 16 columns; slice ps is group pair
// ps/4, codes 8*(ps%4)..+8):
//  * the operands of slice ps + 1 (A from LDS, B decoded in registers) are
//    prepared while the 16 MFMAs of slice ps run;
//  * activations go global -> LDS into two 64 KB stages; A(st+1) is issued
//    during slices 0..3 of step st, four 1 KB loads per slice;
//  * weight bits sit in a register ring of three half steps (a half step is
//    one group pair of one step: two groups per lane).  Those of half step
//    h + 2 are loaded in the first two slices of half step h, so every load
//    has at least five slices to land;
//  * the workgroup barrier sits before slice 7: by then every A read of the
//    step's stage has returned and A(st+1) has landed, and slice 7's MFMAs
//    overlap the first operand reads of step st + 1.
// Vector loads retire in issue order, so each wait is a count of the loads
// issued after the ones it needs.
// ---------------------------------------------------------------------------

// Widths the wide kernel takes: every packed width (b = 11..15 measured
// 16-23% faster than linear_prefill_kernel at 14336 x 4096 M = 2048, and
// spill-free with the ring of three half steps).
constexpr int kWideMaxBits = 15;
constexpr int kWRows = 256;                 // activation rows per workgroup
constexpr int kWN = 256;                    // weight rows per workgroup (4 waves x 64)
constexpr int kWHalfRow = kPRow / 2;        // bytes per staged row of a half step (64 columns)
constexpr int kWHalf = kWRows * kWHalfRow;  // bytes per half-stage (32 KB)
constexpr int kWGroupM = 4;                 // activation blocks per tile-order group

// AB: 32-row activation blocks of the tile (8: 256 x 256 tiles; 6: 192 x 256).
// The low operand half holds four blocks, the high half AB - 4.
template <int B, int MODE, int AB>
__global__ __launch_bounds__(256) void linear_prefill_wide_kernel(
    DevMatrix m, const uint16_t* __restrict__ x, int M, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ bias, const PrefillGrid g) {
    static_assert(B <= kWideMaxBits, "width beyond the wide kernel's ring");
    static_assert(AB == 8 || AB == 6, "six or eight activation blocks per tile");
    constexpr int kRows = 32 * AB;              // activation rows of a tile
    constexpr int AH = AB - 4;                  // blocks of the high operand half
    constexpr int AL = kRows / 32;              // A loads per wave per half step (eight rows each)
    using Bits = GroupBits<B, MODE>;
    constexpr int GL = GroupLoads<B, MODE>::value;  // vector loads per group
    __shared__ __attribute__((aligned(16))) uint8_t xs[4 * kWHalf];

    const int xcd = blockIdx.x & 7;
    const int local = blockIdx.x >> 3;
    int job = xcd * g.per_xcd + local;
    if (local >= g.per_xcd || job >= g.njobs) return;
    const bool second = job >= g.jobs0;
    const PrefillRect rc = second ? g.r[1] : g.r[0];
    if (second) job -= g.jobs0;
    const int group = job / (kWGroupM * rc.nblocks);
    const int within = job - group * kWGroupM * rc.nblocks;
    const int gm = min(kWGroupM, rc.mblocks - group * kWGroupM);
    const int mb = group * kWGroupM + within % gm;
    const int nb = rc.nb0 + within / gm;
    const int m0 = rc.m0 + mb * kRows;
    const int n0 = nb * kWN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n32 = lane & 31;
    const int half = lane >> 5;
    const int steps = m.spr;
    const int nw0 = n0 + wave * 64;

    // B slots [j][p]: 32-row block j (row tiles nw0/16 + 2j, +1), group pair p.
    uint32_t slot0[2][2];
    float s[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int rt = min(nw0 / kTileRows + 2 * j + (n32 >> 4), m.rtiles - 1);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            slot0[j][p] = static_cast<uint32_t>(rt) * static_cast<uint32_t>(steps * kTileSlots) +
                          static_cast<uint32_t>(16 * (2 * p + half) + (n32 & 15));
        }
        s[j] = 0.0f;
        if constexpr (MODE == kModeW) {
            const int row = rt * kTileRows + (n32 & 15);
            s[j] = row < m.rows ? m.scales[row] : 0.0f;
        }
    }

    // A: half step h (columns 64*(h%2) .. +63 of step h/2) of the tile's
    // rows goes global -> LDS into half-stage h % 4 (rows of 128 B).
    // Wave w fills rows 8 AL w .. 8 AL w + 8 AL - 1, eight rows (1 KB) per
    // instruction (8 AL w is a multiple of 16, so the swizzle below depends
    // on instruction i alone);
    // lane l writes physical chunk l%8 of row l/8, which holds logical chunk
    // (l%8) ^ ((row >> 1) & 7): with that swizzle the 16 rows read by lanes
    // 0..15 of an operand read land on distinct banks.  The launcher
    // guarantees cols % 8 == 0, a 16-byte aligned x and M * cols * 2 below
    // 4 GiB.
    int achunk[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) achunk[i] = 8 * ((lane & 7) ^ ((4 * i + (lane >> 4)) & 7));
    const int arow0 = m0 + wave * 8 * AL + (lane >> 3);
    const uint8_t* xb = reinterpret_cast<const uint8_t*>(x);
    auto load_a = [&](int h, int i) {
        const int k0 = min(h >> 1, steps - 1) * kPK + (h & 1) * (kPK / 2);
        const uint32_t row = static_cast<uint32_t>(min(arow0 + 8 * i, M - 1));
        const uint32_t off = 2u * (row * static_cast<uint32_t>(m.cols) +
                                   static_cast<uint32_t>(min(k0 + achunk[i & 1], m.cols - 8)));
        __builtin_amdgcn_global_load_lds(
            xb + off, (lds_void_ptr)(xs + (h & 3) * kWHalf + (wave * 8 * AL + 8 * i) * kWHalfRow), 16, 0, 0);
    };
    // weight bits of half step h, block j, into ring buffer r
    auto load_b = [&](Bits (&r)[2], int h, int j) {
        const uint32_t st = static_cast<uint32_t>(min(h >> 1, steps - 1));
        r[j].load32(m, slot0[j][h & 1] + st * kTileSlots);
    };

    floatx16 acc[AB][2];
#pragma unroll
    for (int i = 0; i < AB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // Operands.  The A operands of a slice are two halves of four and AB - 4
    // row blocks; each half is single-buffered: the high half of slice q is read
    // while the low-half MFMAs run, the low half of slice q + 1 while the
    // high-half MFMAs run.  The B operands (two decoded blocks) are
    // double-buffered by set.  set, hh and q are constants at every call, so
    // the arrays stay in registers.
    half8 pa[2][4], pb[2][2];
    const int aswz = (n32 >> 1) & 7;
    auto read_a = [&](int hh, int h, int q) {
        const int chunk = (4 * half + q) ^ aswz;
        const uint8_t* base = xs + (h & 3) * kWHalf + (128 * hh + n32) * kWHalfRow + chunk * 16;
#pragma unroll
        for (int i = 0; i < (hh == 0 ? 4 : AH); ++i) pa[hh][i] = *reinterpret_cast<const half8*>(base + 32 * i * kWHalfRow);
    };
    auto decode_b = [&](int set, int j, int q, const Bits (&r)[2]) { pb[set][j] = r[j].operand(q, s[j]); };
    auto mfma_half = [&](int hh, int set) {
#pragma unroll
        for (int i = 0; i < (hh == 0 ? 4 : AH); ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[4 * hh + i][j] =
                    __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[hh][i], pb[set][j], acc[4 * hh + i][j], 0, 0, 0);
    };

    // Half step h: four slices of 16 columns (codes 8q .. 8q + 7 of the
    // lane's group).  rc: its weight bits; rn: the bits of half step h + 1;
    // rf: the free ring buffer, filled with half step h + 2.  Every slice
    // issues two of the eight A loads of half step h + 2, slices 0 and 1 one
    // weight group each, so each CU's vector memory pipe sees an even load.
    //
    // Slice q, entered with A-low(q) read and B(q) decoded into set q % 2:
    //   loads; read A-high(q); wait A-low(q); low MFMAs + decode B(q+1)
    //   block 0; wait A-high(q); read A-low(q+1); high MFMAs + decode
    //   B(q+1) block 1.
    // Slice 3 instead waits for every load older than this half step's, so
    // that A and B of half step h + 1 have landed, and passes the workgroup
    // barrier before reading half-stage (h+1) % 4; its high-half MFMAs
    // overlap both decodes of slice 0 of half step h + 1.  The barrier also
    // retires every read of half-stage h % 4 before half step h + 1 refills
    // it... with the loads of half step h + 4, two half steps later.
    auto half_step = [&](const Bits (&rc)[2], const Bits (&rn)[2], Bits (&rf)[2], int h) {
        const bool more = h + 1 < 2 * steps;
        auto slice = [&](auto q_c) {
            constexpr int Q = decltype(q_c)::value;
            constexpr int SET = Q & 1;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                if (2 * Q + i < AL) load_a(h + 2, 2 * Q + i);
            }
            if constexpr (Q < 2) load_b(rf, h + 2, Q);
            __builtin_amdgcn_sched_barrier(0);
            read_a(1, h, Q);
            wait_lgkmcnt<AH>();                    // A-low(q) landed
            __builtin_amdgcn_sched_barrier(0);
            mfma_half(0, SET);
            if constexpr (Q < 3) decode_b(SET ^ 1, 0, Q + 1, rc);
            __builtin_amdgcn_sched_barrier(0);
            wait_lgkmcnt<0>();                     // A-high(q) landed
            if constexpr (Q == 3) {
                // A and B of half step h + 1 landed: the younger loads are
                // the AL A loads and two B groups of this half step
                wait_vmcnt<AL + 2 * GL>();
                barrier_after_wait();
                __builtin_amdgcn_sched_barrier(0);
                if (more) read_a(0, h + 1, 0);
            } else {
                read_a(0, h, Q + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            mfma_half(1, SET);
            if constexpr (Q < 3) {
                decode_b(SET ^ 1, 1, Q + 1, rc);
            } else {
                if (more) {
                    decode_b(0, 0, 0, rn);
                    decode_b(0, 1, 0, rn);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        slice(std::integral_constant<int, 0>{});
        slice(std::integral_constant<int, 1>{});
        slice(std::integral_constant<int, 2>{});
        slice(std::integral_constant<int, 3>{});
    };

    Bits ring0[2], ring1[2], ring2[2];
    // prologue: half steps 0 and 1 (A and B)
#pragma unroll
    for (int i = 0; i < AL; ++i) load_a(0, i);
#pragma unroll
    for (int j = 0; j < 2; ++j) load_b(ring0, 0, j);
#pragma unroll
    for (int i = 0; i < AL; ++i) load_a(1, i);
#pragma unroll
    for (int j = 0; j < 2; ++j) load_b(ring1, 1, j);
    wait_vmcnt<0>();
    barrier_after_wait();
    read_a(0, 0, 0);
    decode_b(0, 0, 0, ring0);
    decode_b(0, 1, 0, ring0);
    // One step (two half steps) per iteration.  The ring advances by two
    // buffers per step, (r0, r1, r2) <- (r2, r0, r1), by register copies
    // (at most 20 moves per step).  A loop body of three steps with an
    // exit after each needs no copies, but the accumulator merges at those
    // exits overflow the 256 accumulator registers and spill.
    for (int st = 0; st < steps; ++st) {
        half_step(ring0, ring1, ring2, 2 * st);
        half_step(ring1, ring2, ring0, 2 * st + 1);
        Bits t[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            t[j].copy_from(ring0[j]);
            ring0[j].copy_from(ring2[j]);
            ring2[j].copy_from(ring1[j]);
            ring1[j].copy_from(t[j]);
        }
    }

    // ---- epilogue: two passes of 128 activation rows through LDS ----
    // 32x32 block element e of lane l is D[8*(e/4) + 4*(l/32) + e%4][l%32].
    // The clamped re-loads of the last step must land before the LDS is
    // reused.
    wait_vmcnt<0>();
    __syncthreads();
    constexpr int kCPitch = 2 * kWN + 16;       // bytes per staged output row
    static_assert(128 * kCPitch <= 4 * kWHalf, "output staging exceeds the activation LDS");
    float sn[2];
    uint16_t bn[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = min(nw0 + 32 * j + n32, m.rows - 1);
        sn[j] = 1.0f;
        bn[j] = 0;
        if constexpr (MODE == kModeQ) sn[j] = m.scales[n];
        if (bias) bn[j] = bias[n];
    }
    const bool yvec = (m.rows % 8 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0);
    const int chunk = threadIdx.x & 31;         // 16-byte chunk of a 512-byte row
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const int pass_blocks = pass == 0 ? 4 : AH;   // 32-row blocks staged in this pass
        if (pass > 0) __syncthreads();
        uint8_t* cw = xs + wave * 128;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < pass_blocks; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int r = 32 * i + 8 * (e >> 2) + 4 * half + (e & 3);
                    *reinterpret_cast<uint16_t*>(cw + r * kCPitch + (32 * j + n32) * 2) =
                        epilogue<MODE>(acc[4 * pass + i][j][e], sn[j], bias != nullptr, bn[j]);
                }
        __syncthreads();
#pragma unroll 2
        for (int it = 0; it < 4 * pass_blocks; ++it) {
            const int r = it * 8 + (threadIdx.x >> 5);
            const int gr = m0 + pass * 128 + r;
            const int gn = n0 + chunk * 8;
            if (gr >= M || gn >= m.rows) continue;
            const uint4 v = *reinterpret_cast<const uint4*>(xs + r * kCPitch + chunk * 16);
            uint16_t* dst = y + static_cast<size_t>(gr) * m.rows + gn;
            if (yvec) {
                store_out16(dst, v);
            } else {
                const uint16_t* hh = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    if (gn + k < m.rows) dst[k] = hh[k];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// legacy flat-group op (bolt/ops_cuda.cu:2708-2750): one wave per output
// feature, four activation rows per wave, lanes stride over K.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float load_as_float(const void* p, int dtype, int64_t i) {
    if (dtype == 0) return static_cast<const float*>(p)[i];
    const uint16_t h = static_cast<const uint16_t*>(p)[i];
    if (dtype == 1) return h2f(h);
    return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ void store_from_float(void* p, int dtype, int64_t i, float v) {
    if (dtype == 0) {
        static_cast<float*>(p)[i] = v;
    } else if (dtype == 1) {
        static_cast<uint16_t*>(p)[i] = f2h(v);
    } else {
        // round to nearest even on the upper 16 bits; NaN stays a quiet NaN
        const uint32_t u = __builtin_bit_cast(uint32_t, v);
        uint16_t b;
        if ((u & 0x7FFFFFFFu) > 0x7F800000u) {
            b = static_cast<uint16_t>((u >> 16) | 0x40u);
        } else {
            b = static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
        }
        static_cast<uint16_t*>(p)[i] = b;
    }
}

__global__ void packed_linear_kernel(const void* __restrict__ x, int x_dtype, int64_t M,
                                     const uint8_t* __restrict__ packed, const void* __restrict__ scales,
                                     int s_dtype, const void* __restrict__ bias, int bits,
                                     int64_t group_size, int64_t N, int64_t K, void* __restrict__ y) {
    constexpr int kRows = 4;
    const int lane = threadIdx.x;
    const int64_t o = blockIdx.x;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kRows;
    const uint32_t mask = (1u << bits) - 1u;
    const int qmin = -(1 << (bits - 1));
    float acc[kRows] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t k = lane; k < K; k += 64) {
        const int64_t wi = o * K + k;
        const int64_t bit = wi * bits;
        const int64_t byte = bit >> 3;
        const int off = static_cast<int>(bit & 7);
        uint32_t word = packed[byte];
        if (off + bits > 8) word |= static_cast<uint32_t>(packed[byte + 1]) << 8;
        const int q = static_cast<int>((word >> off) & mask) + qmin;
        const float w = static_cast<float>(q) * load_as_float(scales, s_dtype, wi / group_size);
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            if (m0 + r < M) acc[r] += load_as_float(x, x_dtype, (m0 + r) * K + k) * w;
        }
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        float v = acc[r];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[r] = v;
    }
    if (lane == 0) {
        const float b = bias ? load_as_float(bias, x_dtype, o) : 0.0f;
        for (int r = 0; r < kRows; ++r) {
            if (m0 + r < M) store_from_float(y, x_dtype, (m0 + r) * N + o, acc[r] + b);
        }
    }
}

// ---------------------------------------------------------------------------
// dispatch helpers
// ---------------------------------------------------------------------------

// Compute units of the current device, cached per device (threads may race
// to fill an entry; they store the same value).
int device_cu_count() {
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

inline unsigned blocks_for(uint64_t n, unsigned threads) {
    return static_cast<unsigned>((n + threads - 1) / threads);
}

template <template <int> class F, typename... Args>
hipError_t dispatch_bits(int bits, Args&&... args) {
    switch (bits) {
        case 3: return F<3>::run(args...);
        case 4: return F<4>::run(args...);
        case 5: return F<5>::run(args...);
        case 6: return F<6>::run(args...);
        case 7: return F<7>::run(args...);
        case 8: return F<8>::run(args...);
        case 9: return F<9>::run(args...);
        case 10: return F<10>::run(args...);
        case 11: return F<11>::run(args...);
        case 12: return F<12>::run(args...);
        case 13: return F<13>::run(args...);
        case 14: return F<14>::run(args...);
        case 15: return F<15>::run(args...);
        default: return hipErrorInvalidValue;
    }
}

template <int B>
struct RepackOp {
    static hipError_t run(const uint8_t* canon, uint64_t canon_bytes, const DevMatrixOut& out, hipStream_t s) {
        const uint64_t slots = static_cast<uint64_t>(out.rtiles) * out.spr * kTileSlots;
        hipLaunchKernelGGL(repack_kernel<B>, dim3(blocks_for(slots, 256)), dim3(256), 0, s,
                           canon, canon_bytes, out, slots);
        return hipGetLastError();
    }
};

template <int B>
struct PackCodesOp {
    static hipError_t run(const int16_t* codes, uint64_t count, uint8_t* out, uint64_t out_bytes, int* bad,
                          hipStream_t s) {
        const uint64_t chunks = (count + 7) / 8;
        hipLaunchKernelGGL(pack_codes_kernel<B>, dim3(blocks_for(chunks, 256)), dim3(256), 0, s, codes, count, out,
                           out_bytes, bad);
        return hipGetLastError();
    }
};

template <int B>
struct UnpackOp {
    static hipError_t run(const DevMatrix& m, int16_t* out, hipStream_t s) {
        const uint64_t slots = static_cast<uint64_t>(m.rtiles) * m.spr * kTileSlots;
        hipLaunchKernelGGL(unpack_kernel<B>, dim3(blocks_for(slots, 256)), dim3(256), 0, s, m, out, slots);
        return hipGetLastError();
    }
};

template <int B>
struct MaterializeOp {
    static hipError_t run(const DevMatrix& m, uint16_t* out, hipStream_t s) {
        const uint64_t slots = static_cast<uint64_t>(m.rtiles) * m.spr * kTileSlots;
        hipLaunchKernelGGL(materialize_kernel<B>, dim3(blocks_for(slots, 256)), dim3(256), 0, s, m, out,
                           slots);
        return hipGetLastError();
    }
};

constexpr int kPrefillKS = 2;      // waves per column group of linear_prefill_kernel (K split)
constexpr int kDecodeWaves = 8;    // waves per workgroup of linear_decode_kernel
constexpr int kDecodeGpl = 1;      // weight tiles per wave batch of linear_decode_kernel
// Activation rows the decode kernel takes (in blocks of 16; above, the
// prefill kernels).
constexpr int kDecodeMaxM = 64;

// Whether linear_gemv_kernel takes an M = 1 launch (else
// linear_decode_kernel).  Not the decoded-fp16 mode (b >= 13, fullPrecision):
// it spends ~7 VALU instructions per code on the fp32 product and its
// rounding; at four waves per SIMD that work is exposed, and
// linear_decode_kernel is faster for it (8.7 vs 9.6 us at 4096 x 4096
// b = 15).  Measured on MI355X at M = 1 over rotated copies:
// with K at most 16 tiles (2048 columns) half or more of the 16 waves idle
// and the decode kernel is faster (4096 x 1024: 3.4-3.9 us against
// 3.7-5.3 us; 4096 x 2048 from b = 10); at b = 11 (the largest group
// loads) the GEMV kernel leads only with every wave holding two tiles,
// K = 4096 (4096 x 4096: 6.26 against 6.57 us; 11008 x 4096: 13.47
// against 13.60), and trails at 4096 x 3072 (5.84 against 5.74); at b <= 7
// with more than 256 row tiles (at most 28 bytes per lane and group) the
// decode kernel is 4-6% faster (14336 x 4096 b = 4: 8.3 against 8.7 us,
// b = 7: 12.3 against 13.0).  Elsewhere the GEMV kernel is ahead by up to
// 24% (1024 x 4096).
inline bool gemv_takes(const DevMatrix& m, int mode) {
    if (mode == kModeW) return false;
    if (m.spr <= kGemvMaxSteps / 2 || m.spr > kGemvMaxSteps) return false;
    if (mode != kModeRaw && ((m.bits == 11 && m.spr != kGemvMaxSteps) || (m.bits <= 7 && m.rtiles > 256)))
        return false;
    return true;
}

// Whether linear_gemv_kernel takes 2 <= M <= 16: the integer-code
// arithmetic where it takes M = 1, except b = 11; above eight rows only at
// K = 4096 (every wave holding two tiles).  Measured on MI355X (us, decode
// kernel -> GEMV kernel, b = 10): 4096 x 4096 M = 2 6.28 -> 5.79, M = 4
// 6.45 -> 5.96, M = 8 6.74 -> 6.24, M = 16 7.26 -> 6.99; 11008 x 4096 M = 4
// 12.57 -> 11.99, M = 7 13.92 -> 13.05; 14336 x 4096 M = 2 15.09 -> 14.41;
// 2048 x 4096 M = 16 6.20 -> 5.98; 4096 x 3072 M = 4 5.60 -> 5.44, M = 8
// 5.87 -> 5.76 but M = 16 6.12 -> 6.37.  At b = 11 the two are even (+-1%);
// raw fp16 (b = 16) is 1-2% slower at M = 2..4.
inline bool gemv_rows_takes(int64_t M, const DevMatrix& m, int mode) {
    if (mode != kModeQ || m.bits == 11 || !gemv_takes(m, mode)) return false;
    return M <= 8 || m.spr == kGemvMaxSteps;
}

// The kernel a forward of M <= 16 activation rows takes on matrix m in a
// launch of its own.  A multi-matrix launch fuses only matrices that all
// take the same route, so each output equals its matrix's own forward.
enum DecodeRoute { kRouteGemv1, kRouteGemv4, kRouteGemv16, kRouteRows, kRouteDecode };

inline DecodeRoute decode_route(int64_t M, const DevMatrix& m, int mode, int xvec, int cus) {
    if (M == 1 && xvec == 2 && gemv_takes(m, mode)) return kRouteGemv1;
    if (decode_rows_per_workgroup(M, m, mode, cus) > 0) return kRouteRows;
    if (M <= 16 && xvec == 2 && gemv_rows_takes(M, m, mode)) return M <= kGemvMaxM ? kRouteGemv4 : kRouteGemv16;
    return kRouteDecode;
}

inline int linear_mode(int bits, bool exact_w16) {
    return bits == 16 ? kModeRaw : (bits <= 12 && !exact_w16 ? kModeQ : kModeW);
}

std::atomic<int> g_prefill_tiles{0};   // eb_set_prefill_tiles

// Whether 256 x 256 tiles run with eight waves (eb_prefill.hip) rather than
// four.  Measured on MI355X, best of two interleaved runs after a 25 ms
// warm-up (us, four -> eight waves): integer-code widths 8..11 gain
// (14336 x 4096 M = 2048 b = 10 218.6 -> 215.2, b = 9 212.7 -> 211.0,
// b = 8 209.5 -> 203.3; 4096 x 4096 M = 8192 b = 10 238.3 -> 236.6;
// 14336 x 4096 M = 4096 b = 10 443.0 -> 427.4).  With two weight blocks
// per wave b = 7 lost (214.3 -> 219.0), and so did b = 12 (258.1 -> 262.8),
// the decoded-fp16 widths (b = 13: 296.0 -> 334.3) and raw fp16 (241.5 ->
// 254.1); with one block per wave (pp_weight_blocks) every packed width
// and arithmetic gains, so only raw fp16 keeps four waves.
template <int B, int MODE>
inline bool prefill_eight_waves() {
    const int mode = g_prefill_tiles.load(std::memory_order_relaxed);
    if (mode == kPrefillTilesWide8 || mode == kPrefillTilesWide8Plain || mode == kPrefillTilesWide8Short) return true;
    return mode == 0 && MODE != kModeRaw;
}

// Whether the 256 x 256 prefill tiles finish before the 128 x 256 ones.
// Cost in rounds of 128 x 256 tiles over the CUs: a full round of 256 x 256
// tiles takes about 1.7 of them (measured on MI355X, 14336 x 4096 b = 10:
// 116 us per wide round, 68 us per narrow round); the narrow kernel runs a
// last round that would leave half the CUs idle as half tiles, at about two
// thirds of a round.  The 256 x 256 launches, four or eight waves, are
// costed by prefill_pp_rounds: a sparse last round is cheaper than a full
// one, and may be balanced with 192-row tiles.
template <int B, int MODE>
inline bool prefer_wide_tiles(int64_t M, int rows, int cus) {
    const int mode = g_prefill_tiles.load(std::memory_order_relaxed);
    if (mode != 0) return mode >= 2;
    const int64_t narrow = ((M + 127) / 128) * ((rows + kPN - 1) / kPN);
    const double t_wide = 1.7 * prefill_pp_rounds(M, rows, cus, mode);
    const int64_t rem = narrow % cus;
    const double t_narrow = static_cast<double>(narrow / cus) + (rem == 0 ? 0.0 : (2 * rem <= cus ? 0.67 : 1.0));
    return t_wide < t_narrow;
}

// Tiles of linear_prefill_kernel with MI 32-row activation blocks: full
// tiles are 32 MI x 256; when the last round of full tiles would leave at
// least half the CUs idle, its tiles run as two 32 MI x 128 halves instead,
// so it takes half a round.  Returns the full tiles to launch of `tiles`.
inline int narrow_full_tiles(int tiles, int cus) {
    if (tiles <= cus / 2) return 0;
    if (tiles % cus != 0 && tiles % cus <= cus / 2) return tiles - tiles % cus;
    return tiles;
}

// Workgroups linear_prefill_kernel launches for M rows at MI.
inline int narrow_workgroups(int64_t M, int rows, int mi, int cus) {
    const int tiles = static_cast<int>((M + 32 * mi - 1) / (32 * mi)) * ((rows + kPN - 1) / kPN);
    const int full = narrow_full_tiles(tiles, cus);
    return full + 2 * (tiles - full);
}

// Whether linear_decode_kernel finishes 16 < M <= kDecodeMaxM rows before
// the prefill kernel.  The decode kernel reads the weights once, but every
// row tile re-reads all M x K activations from L2; the 64-row prefill tiles
// are few at these M, so their time is one tile's walk over K per round.
// Fitted on MI355X at b = 10 (us): decode ~ max(weight bytes at 5 TB/s,
// rtiles * M * K * 2 at R) + 2, with R the rate of the activation path the
// decode launch takes (6.5 TB/s staged whole up to 32 KB, 5.2 TB/s staged
// in LDS beyond that, 7.5 TB/s read per lane from L2); prefill ~
// (3 + 0.005 K) per round.  Measured (decode against prefill, us):
// 4096 x 4096 M = 64 19.8 / 24.6; 11008 x 4096 M = 17 20.5 / 23.3,
// M = 24 25.6 / 23.7; 14336 x 4096 M = 17 26.1 / 24.5; 4096 x 11008
// M = 64 46.8 / 61.1.
inline bool prefer_decode(int64_t M, const DevMatrix& m, int cus) {
    if (M <= 16) return true;
    if (M > kDecodeMaxM) return false;
    const double wbytes = static_cast<double>(m.rows) * m.cols * (m.bits == 16 ? 16 : m.bits) / 8.0;
    const double xbytes = static_cast<double>(m.rtiles) * static_cast<double>(M) * m.cols * 2.0;
    const double staged = static_cast<double>(M) * m.spr * kTileGroups * kGroup * 2.0;   // as launch_decode
    const double rate = staged <= kXLdsBytes ? 6.5e6
                        : (staged <= kXLdsDirectBytes || M <= 32) ? 5.2e6 : 7.5e6;
    const double t_decode = std::max(wbytes / 5.0e6, xbytes / rate) + 2.0;
    const int wgs = narrow_workgroups(M, m.rows, 2, cus);
    const double rounds = static_cast<double>((wgs + cus - 1) / cus);
    const double t_prefill = (3.0 + 0.005 * m.cols) * rounds;
    return t_decode < t_prefill;
}

// linear_prefill_kernel with MI = 4 (128-row tiles) or, where those would
// keep at most half the CUs busy, MI = 2 (64-row tiles).  Measured on MI355X
// at b = 10 (us, 128-row -> 64-row tiles): 4096 x 4096 M = 128..512
// 35 -> 24; 4096 x 11008 M = 128 88 -> 59; 1024 x 1024 M = 512 12.1 -> 8.1;
// with more tiles the 128-row tiles win (11008 x 4096 M = 512: 58.5
// against 65).
template <int B, int MODE, int MI>
void launch_narrow(const DevMatrix& m, const uint16_t* x, int64_t M, uint16_t* y, const uint16_t* bias,
                   hipStream_t s, int cus) {
    constexpr int kRows = 32 * MI;
    const int mblocks = static_cast<int>((M + kRows - 1) / kRows);
    const int nblocks = (m.rows + kPN - 1) / kPN;
    const int tiles = mblocks * nblocks;
    const int full = narrow_full_tiles(tiles, cus);
    if (full > 0) {
        const int per_xcd = (full + 7) / 8;
        hipLaunchKernelGGL((linear_prefill_kernel<B, MODE, MI, 2, kPrefillKS>), dim3(8 * per_xcd),
                           dim3(256 * kPrefillKS), 0, s, m, x, static_cast<int>(M), y, bias, mblocks, nblocks, 0,
                           full, per_xcd);
    }
    if (full < tiles) {
        const int jobs = 2 * (tiles - full);
        const int per_xcd = (jobs + 7) / 8;
        hipLaunchKernelGGL((linear_prefill_kernel<B, MODE, MI, 1, kPrefillKS>), dim3(8 * per_xcd),
                           dim3(256 * kPrefillKS), 0, s, m, x, static_cast<int>(M), y, bias, mblocks, nblocks,
                           full, jobs, per_xcd);
    }
}

// linear_decode_kernel for M <= 16 MB rows: activations staged in LDS when
// they fit (directly up to kXLdsDirectBytes when x's rows are whole tiles),
// in K chunks when they do not (whole tiles, M <= 32), read per lane from
// L2 otherwise.
template <int B, int MODE, int MB>
void launch_decode(const DevMatrix& m, const uint16_t* x, int64_t M, uint16_t* y, const uint16_t* bias, int xvec,
                   hipStream_t s, const MultiTail& mt, int tiles) {
    const size_t xbytes = static_cast<size_t>(M) * m.spr * kTileGroups * kGroup * 2;
    if (xbytes <= static_cast<size_t>(kXLdsBytes)) {
        hipLaunchKernelGGL((linear_decode_kernel<B, MODE, kDecodeWaves, kDecodeGpl, 1, MB>), dim3(tiles),
                           dim3(64 * kDecodeWaves), xbytes, s, m, x, static_cast<int>(M), y, bias, xvec, mt);
    } else if (xvec == 2 && xbytes <= static_cast<size_t>(kXLdsDirectBytes)) {
        hipLaunchKernelGGL((linear_decode_kernel<B, MODE, kDecodeWaves, kDecodeGpl, 2, MB>), dim3(tiles),
                           dim3(64 * kDecodeWaves), xbytes, s, m, x, static_cast<int>(M), y, bias, xvec, mt);
    } else if (MB <= 2 && xvec == 2) {
        if constexpr (MB <= 2) {
            constexpr int CT = MB == 1 ? 16 : 8;     // as in the kernel
            const int64_t Mp = (M + 32 / CT - 1) / (32 / CT) * (32 / CT);
            const size_t lds = static_cast<size_t>(2 * Mp * CT * kTileGroups * kGroup * 2);
            hipLaunchKernelGGL((linear_decode_kernel<B, MODE, kDecodeWaves, kDecodeGpl, 3, MB>), dim3(tiles),
                               dim3(64 * kDecodeWaves), lds, s, m, x, static_cast<int>(M), y, bias, xvec, mt);
        }
    } else {
        hipLaunchKernelGGL((linear_decode_kernel<B, MODE, kDecodeWaves, kDecodeGpl, 0, MB>), dim3(tiles),
                           dim3(64 * kDecodeWaves), 0, s, m, x, static_cast<int>(M), y, bias, xvec, mt);
    }
}

// mt: the other matrices of a multi-matrix decode launch (count 1 for a
// single matrix; only M <= kDecodeMaxM takes more than one).
template <int B, int MODE>
hipError_t run_linear_mode(const DevMatrix& m, const uint16_t* x, int64_t M, uint16_t* y,
                           const uint16_t* bias, int xvec, hipStream_t s, const MultiTail& mt) {
    const int tiles = mt.count > 1 ? mt.tile0[mt.count - 2] + mt.m[mt.count - 2].rtiles : m.rtiles;
    // The prefill kernels address x and the weight planes with 32-bit byte
    // offsets: x below 4 GiB, and the widest plane (32 bytes per group; the
    // raw fp16 weights load through 64-bit addresses) below 4 GiB.  Larger
    // operands take linear_gemm_kernel, whose addressing is 64-bit.
    const uint64_t groups = static_cast<uint64_t>(m.rtiles) * m.spr * kTileSlots;
    const bool offsets32 = static_cast<uint64_t>(M) * m.cols * 2 < (uint64_t(1) << 32) &&
                           (MODE == kModeRaw || groups * 32u < (uint64_t(1) << 32));
    const size_t gemv_lds = static_cast<size_t>(kGemvWaves) * M * 2 * kTileGroups * kGroup * 2;
    if (M <= 16) {
        // a multi-matrix launch reaches here only when every matrix takes this route
        switch (decode_route(M, m, MODE, xvec, device_cu_count())) {
            case kRouteGemv1:
                if constexpr (MODE != kModeW) {
                    hipLaunchKernelGGL((linear_gemv_kernel<B, MODE, 1>), dim3(tiles), dim3(64 * kGemvWaves), gemv_lds,
                                       s, m, x, 1, y, bias, mt);
                    return hipGetLastError();
                }
                return hipErrorInvalidValue;
            case kRouteGemv4:
            case kRouteGemv16:
                if constexpr (MODE == kModeQ && B != 11) {
                    if (M <= kGemvMaxM) {
                        hipLaunchKernelGGL((linear_gemv_kernel<B, MODE, kGemvMaxM>), dim3(tiles), dim3(64 * kGemvWaves),
                                           gemv_lds, s, m, x, static_cast<int>(M), y, bias, mt);
                    } else {
                        hipLaunchKernelGGL((linear_gemv_kernel<B, MODE, 16>), dim3(tiles), dim3(64 * kGemvWaves),
                                           gemv_lds, s, m, x, static_cast<int>(M), y, bias, mt);
                    }
                    return hipGetLastError();
                }
                return hipErrorInvalidValue;
            case kRouteRows:
                if (mt.count > 1) return hipErrorInvalidValue;
                return launch_decode_rows(m, MODE, decode_rows_per_workgroup(M, m, MODE, device_cu_count()), x, M, y,
                                          bias, xvec, s);
            case kRouteDecode:
                launch_decode<B, MODE, 1>(m, x, M, y, bias, xvec, s, mt, tiles);
                return hipGetLastError();
        }
    }
    if (M <= kDecodeMaxM && (mt.count > 1 || prefer_decode(M, m, device_cu_count()))) {
        if (M <= 32) {
            launch_decode<B, MODE, 2>(m, x, M, y, bias, xvec, s, mt, tiles);
        } else if constexpr (kDecodeMaxM > 32) {
            launch_decode<B, MODE, 4>(m, x, M, y, bias, xvec, s, mt, tiles);
        }
    } else if (mt.count > 1) {
        return hipErrorInvalidValue;      // the launcher splits prefill per matrix
    } else if (xvec && offsets32 && M >= kWRows && m.rows >= kWN &&
               prefer_wide_tiles<B, MODE>(M, m.rows, device_cu_count())) {
        if (prefill_eight_waves<B, MODE>()) {
            return launch_prefill_pp(m, MODE, x, M, y, bias, s, device_cu_count(),
                                     g_prefill_tiles.load(std::memory_order_relaxed));
        }
        if constexpr (B <= kWideMaxBits) {
            const PrefillPlan plan = prefill_plan(M, m.rows, device_cu_count(),
                                                  g_prefill_tiles.load(std::memory_order_relaxed));
            if (plan.full.njobs > 0) {
                hipLaunchKernelGGL((linear_prefill_wide_kernel<B, MODE, 8>), dim3(8 * plan.full.per_xcd), dim3(256),
                                   0, s, m, x, static_cast<int>(M), y, bias, plan.full);
            }
            if (plan.short_tiles.njobs > 0) {
                hipLaunchKernelGGL((linear_prefill_wide_kernel<B, MODE, 6>), dim3(8 * plan.short_tiles.per_xcd),
                                   dim3(256), 0, s, m, x, static_cast<int>(M), y, bias, plan.short_tiles);
            }
        }
    } else if (xvec && offsets32) {
        const int cus = device_cu_count();
        if (narrow_workgroups(M, m.rows, 4, cus) <= cus / 2) {
            launch_narrow<B, MODE, 2>(m, x, M, y, bias, s, cus);
        } else {
            launch_narrow<B, MODE, 4>(m, x, M, y, bias, s, cus);
        }
    } else {
        const dim3 grid((m.rows + kBN - 1) / kBN, static_cast<unsigned>((M + kBM - 1) / kBM));
        hipLaunchKernelGGL((linear_gemm_kernel<B, MODE>), grid, dim3(256), 0, s, m, x,
                           static_cast<int>(M), y, bias, xvec);
    }
    return hipGetLastError();
}

template <int B>
struct LinearOp {
    static hipError_t run(const DevMatrix& m, bool exact_w16, const uint16_t* x, int64_t M, uint16_t* y,
                          const uint16_t* bias, int xvec, hipStream_t s, const MultiTail& mt) {
        if constexpr (B <= 12) {
            if (!exact_w16) return run_linear_mode<B, kModeQ>(m, x, M, y, bias, xvec, s, mt);
        }
        return run_linear_mode<B, kModeW>(m, x, M, y, bias, xvec, s, mt);
    }
};

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

hipError_t launch_repack(const uint8_t* canon, uint64_t canon_bytes, const DevMatrixOut& out,
                         hipStream_t stream) {
    if (out.bits == 16) {
        const uint64_t slots = static_cast<uint64_t>(out.rtiles) * out.spr * kTileSlots;
        hipLaunchKernelGGL(repack16_kernel, dim3(blocks_for(slots, 256)), dim3(256), 0, stream,
                           reinterpret_cast<const uint16_t*>(canon), out, slots);
        return hipGetLastError();
    }
    return dispatch_bits<RepackOp>(out.bits, canon, canon_bytes, out, stream);
}

void set_prefill_tiles(int mode) { g_prefill_tiles.store(mode, std::memory_order_relaxed); }

int prefill_tiles_mode() { return g_prefill_tiles.load(std::memory_order_relaxed); }

hipError_t launch_pack_codes(const int16_t* codes, uint64_t count, int bits, uint8_t* out, uint64_t out_bytes,
                             int* bad, hipStream_t stream) {
    return dispatch_bits<PackCodesOp>(bits, codes, count, out, out_bytes, bad, stream);
}

hipError_t launch_unpack(const DevMatrix& m, int16_t* out, hipStream_t stream) {
    return dispatch_bits<UnpackOp>(m.bits, m, out, stream);
}

hipError_t launch_materialize(const DevMatrix& m, uint16_t* out, hipStream_t stream) {
    if (m.bits == 16) return MaterializeOp<16>::run(m, out, stream);
    return dispatch_bits<MaterializeOp>(m.bits, m, out, stream);
}

namespace {

// 1: rows of x can be read 16 bytes at a time; 2: and they span whole
// 128-column tiles, so x needs no zero padding
int x_vector_mode(const DevMatrix& m, const uint16_t* x) {
    int xvec = (m.cols % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    if (xvec && m.cols % (kTileGroups * kGroup) == 0) xvec = 2;
    return xvec;
}

hipError_t run_linear(const DevMatrix& m, bool exact_w16, const uint16_t* x, int64_t M, uint16_t* y,
                      const uint16_t* bias, hipStream_t stream, const MultiTail& mt) {
    const int xvec = x_vector_mode(m, x);
    if (m.bits == 16) return run_linear_mode<8, kModeRaw>(m, x, M, y, bias, xvec, stream, mt);
    return dispatch_bits<LinearOp>(m.bits, m, exact_w16, x, M, y, bias, xvec, stream, mt);
}

}  // namespace

hipError_t launch_linear(const DevMatrix& m, bool exact_w16, const uint16_t* x, int64_t M, uint16_t* y,
                         const uint16_t* bias, hipStream_t stream) {
    return run_linear(m, exact_w16, x, M, y, bias, stream, MultiTail{});
}

hipError_t launch_linear_multi(const DevMatrix* ms, int count, bool exact_w16, const uint16_t* x, int64_t M,
                               uint16_t* const* ys, const uint16_t* const* biases, hipStream_t stream) {
    if (count < 1 || count > kMultiMax) return hipErrorInvalidValue;
    for (int j = 1; j < count; ++j) {
        if (ms[j].cols != ms[0].cols || ms[j].bits != ms[0].bits) return hipErrorInvalidValue;
    }
    // The group shares one launch only when each matrix's own forward takes
    // the same kernel (and not linear_decode_rows_kernel, which fills the
    // device with one matrix), so that every output equals that forward's
    // bit for bit; otherwise it runs per matrix.
    bool fused = M <= kDecodeMaxM;
    const int cus = device_cu_count();
    const int xvec = x_vector_mode(ms[0], x);
    const int mode = linear_mode(ms[0].bits, exact_w16);
    const DecodeRoute route = decode_route(M, ms[0], mode, xvec, cus);
    for (int j = 0; j < count && fused; ++j) {
        fused = prefer_decode(M, ms[j], cus) &&
                (M > 16 || (decode_route(M, ms[j], mode, xvec, cus) == route && route != kRouteRows));
    }
    if (!fused) {
        for (int j = 0; j < count; ++j) {
            const hipError_t e = run_linear(ms[j], exact_w16, x, M, ys[j], biases ? biases[j] : nullptr, stream,
                                            MultiTail{});
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    MultiTail mt;
    mt.count = count;
    int tile = ms[0].rtiles;
    for (int j = 1; j < count; ++j) {
        mt.m[j - 1] = ms[j];
        mt.y[j - 1] = ys[j];
        mt.bias[j - 1] = biases ? biases[j] : nullptr;
        mt.tile0[j - 1] = tile;
        tile += ms[j].rtiles;
    }
    return run_linear(ms[0], exact_w16, x, M, ys[0], biases ? biases[0] : nullptr, stream, mt);
}

hipError_t launch_packed_linear(const void* x, int x_dtype, int64_t M, const uint8_t* packed,
                                const void* scales, int scale_dtype, const void* bias, int bits,
                                int64_t group_size, int64_t N, int64_t K, void* y, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(N), static_cast<unsigned>((M + 3) / 4));
    hipLaunchKernelGGL(packed_linear_kernel, grid, dim3(64), 0, stream, x, x_dtype, M, packed, scales,
                       scale_dtype, bias, bits, group_size, N, K, y);
    return hipGetLastError();
}

}  // namespace ebk
