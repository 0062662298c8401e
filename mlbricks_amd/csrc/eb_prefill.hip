// Prefill GEMM on 256 x 256 output tiles with eight waves, two per SIMD.
//
// y[M][rows] = x[M][cols] . W^T (+ bias) for M >= 256, W in the bit-plane
// layout of eb_internal.h, decoded in registers into the B operands of
// v_mfma_f32_32x32x16_f16; activations go global -> LDS directly.
//
// Why two waves per SIMD.  With one wave per SIMD (256 accumulators per
// lane), counters on configs[3] (14336 x 4096, M = 2048, b = 10) showed the
// matrix cores busy 47% of the cycles and the waves waiting on memory or
// LDS results 47% of theirs: nothing else could issue while the only wave
// of a SIMD waited.  Here every wave holds 128 accumulator registers per
// lane, so two waves fit a SIMD and one multiplies while the other waits.
// Two layouts (pp_weight_blocks):
//  * two weight blocks per wave: wave w owns weight rows 64 (w % 4) .. + 63
//    for activation rows 128 (w / 4) .. + 127, 4 x 2 blocks of 32 x 32.
//    The two waves of a column group load and decode the same weight bits
//    (the second load hits the CU's L1); each wave reads only its own 128
//    activation rows from LDS;
//  * one weight block per wave (every width but b = 8): wave w owns weight
//    rows 32 w .. 32 w + 31 for all 256 activation rows, 8 x 1 blocks.
//    Each weight bit is loaded and decoded once; each wave reads every
//    activation row from LDS.
//
// Per K step (128 columns = one plane tile) the CU moves 64 KB of
// activations global -> LDS and 40 KB (b = 10) of weight bits global ->
// registers, twice that with two weight blocks per wave, for 512 MFMAs.
//
// Pipeline, in half steps h (64 columns: group pair h % 2 of step h / 2):
//  * activations of half step h go to LDS half-stage h % 4 (32 KB; rows of
//    128 B whose 16-byte chunks are XOR-swizzled by (row >> 1) & 7, so the
//    rows read by one operand read land on distinct banks); half step h + 2
//    is loaded during half step h, one 1 KB load per wave and slice;
//  * weight bits sit in a register ring of D half steps: with D = 3 (b <= 12)
//    those of h + 2 are loaded in slices 0 (and 1, with two weight blocks)
//    of half step h; with D = 2
//    (b >= 13 and raw fp16, whose groups are larger) those of h + 1, in
//    slice 0, ahead of that slice's activation load;
//  * a slice (16 columns) is two halves of MFMAs (four each with two weight
//    blocks per wave; AB each with one); the A operands of one half are read
//    from LDS and the B operands of the next slice decoded while the other
//    half's MFMAs run;
//  * one workgroup barrier per half step, before the last slice's second
//    half: every read of the half-stage being retired has returned and the
//    next half step's activations and weight bits have landed.
// Vector loads retire in issue order, so each wait is a count of the loads
// issued after the ones it needs.  Loads past the last step re-read the
// last step (clamped addresses), which keeps every count uniform.
//
// Tried and slower: staging each 32-row block's weight bits once in LDS
// (global_load_lds into a ring of three stages, then LDS reads before the
// decode), which removes the duplicate loads of a column group and holds no
// registers while in flight: 4-5% slower at b = 8..10 (configs[3] b = 10:
// 225.5 against 215.2 us).  Without any weight-bit loads at all the kernel
// took 189 against 244 us on another box, so what costs is the traffic and
// latency of those bits, not the path they take.
//
// Launch: workgroup i runs on XCD i % 8, so each XCD walks a contiguous
// range of tiles, four activation blocks at a time, and the workgroups it
// runs at once share their activation and weight blocks in its L2.
#include "eb_device.h"

#include <algorithm>
#include <type_traits>

namespace ebk {
namespace {

constexpr int kQRows = 256;                  // activation rows per workgroup, at most
constexpr int kQN = 256;                     // weight rows per workgroup
constexpr int kQHalfRow = kPRow / 2;         // bytes per staged row of a half step
constexpr int kQHalf = kQRows * kQHalfRow;   // bytes per half-stage (32 KB)
constexpr int kQStages = 4;                  // half-stages in the ring
constexpr int kQCPitch = 2 * kQN + 16;       // bytes per staged output row
constexpr int kQLds = kQStages * kQHalf > kQRows * kQCPitch ? kQStages * kQHalf : kQRows * kQCPitch;
constexpr int kQGroupM = 4;                  // activation blocks per tile-order group
constexpr int kQWaves = 8;

using PPRect = PrefillRect;
using PPGrid = PrefillGrid;
using PPPlan = PrefillPlan;

// Depth of the weight-bit register ring (see the pipeline above).
template <int B, int MODE>
constexpr int ring_depth() {
    return (MODE == kModeRaw || B > 12) ? 2 : 3;
}

// Weight blocks per wave: 2 (wave w: weight rows 64 (w % 4) .. + 63 of
// activation rows 32 AB (w / 4) .. + 32 AB - 1) or 1 (wave w: weight rows
// 32 w .. 32 w + 31 of every activation row of the tile).  With one block a
// workgroup loads and decodes each weight bit once instead of twice and
// reads twice the activation operands from LDS.  Measured on MI355X
// (14336 x 4096 M = 2048 unless stated, us, two blocks -> one): b = 8
// 202.1 -> 205.5; b = 9 215.0 -> 212.4; b = 10 216.7 -> 215.8; b = 11
// 248.7 -> 231.5, 4096^2 M = 8192 272.6 -> 251.5; b = 12 250.6 -> 235.0
// (the four-wave kernel: 240.8).  Against the four-wave kernel, one block
// per wave also wins where two lost (us, four waves -> eight, one block):
// b = 3 216.5 -> 206.6, b = 5 220.2 -> 210.9, b = 7 228.2 -> 222.6,
// decoded fp16 at b = 10 278.2 -> 271.7, b = 13 292.4 -> 279.2, b = 15
// 307.0 -> 301.7.  Raw fp16 (b = 16) keeps the four-wave kernel.
template <int B, int MODE>
constexpr int pp_weight_blocks() {
    return (MODE == kModeRaw || (MODE == kModeQ && B == 8)) ? 2 : 1;
}

// AB: 32-row activation blocks per tile and weight-block column, so 64 AB
// activation rows per tile (AB = 4: 256 x 256 tiles; AB = 3: 192 x 256).
// A wave's activation blocks come in two operand halves: with two weight
// blocks per wave, two and AB - 2 blocks of its 32 AB rows; with one, AB
// and AB blocks of all 64 AB rows.
template <int B, int MODE, int AB>
__global__ __launch_bounds__(64 * kQWaves) void linear_prefill_pp_kernel(
    DevMatrix m, const uint16_t* __restrict__ x, int M, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ bias, const PPGrid g) {
    static_assert(AB == 3 || AB == 4, "three or four activation blocks per wave");
    constexpr int kRows = 64 * AB;              // activation rows of a tile
    constexpr int JB = pp_weight_blocks<B, MODE>();   // 32-row weight blocks per wave
    constexpr int AL = JB == 2 ? 2 : AB;        // activation blocks of the low operand half
    constexpr int AH = JB == 2 ? AB - 2 : AB;   // blocks of the high operand half
    using Bits = GroupBits<B, MODE>;
    constexpr int GL = GroupLoads<B, MODE>::value;  // vector loads per group
    constexpr int D = ring_depth<B, MODE>();
    constexpr bool kReadInGroup = MODE == kModeQ && B <= 10;   // see the slice order below
    __shared__ __attribute__((aligned(16))) uint8_t xs[kQLds];

    const int xcd = blockIdx.x & 7;
    const int local = blockIdx.x >> 3;
    int job = xcd * g.per_xcd + local;
    if (local >= g.per_xcd || job >= g.njobs) return;
    const bool second = job >= g.jobs0;
    const PPRect rc = second ? g.r[1] : g.r[0];
    if (second) job -= g.jobs0;
    const int group = job / (kQGroupM * rc.nblocks);
    const int within = job - group * kQGroupM * rc.nblocks;
    const int gm = min(kQGroupM, rc.mblocks - group * kQGroupM);
    const int mb = group * kQGroupM + within % gm;
    const int nb = rc.nb0 + within / gm;
    const int m0 = rc.m0 + mb * kRows;
    const int n0 = nb * kQN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // 0 .. 7
    const int colg = JB == 2 ? wave & 3 : wave;   // weight rows n0 + 32 JB colg ..
    const int mh = JB == 2 ? wave >> 2 : 0;       // activation rows m0 + 32 AB mh ..
    const int n32 = lane & 31;
    const int half = lane >> 5;
    const int steps = m.spr;
    const int nw0 = n0 + colg * 32 * JB;

    // B slots [j][p]: 32-row block j (row tiles nw0/16 + 2j, +1), group pair
    // p; lane (n32, half) holds group 2p + half of its row, whose codes
    // 8q .. 8q + 7 are the operand of slice q.
    uint32_t slot0[JB][2];
    float s[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
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

    // A of half step h: wave w fills rows 8 AB w .. 8 AB w + 8 AB - 1 of
    // half-stage h % 4, eight rows (1 KB) per instruction; lane l writes
    // physical chunk l % 8 of row l / 8, which holds logical chunk
    // (l % 8) ^ ((row >> 1) & 7).  Instruction i starts at row R = 8 (AB w +
    // i), so (row >> 1) & 7 = (4 ((R / 8) & 1) + l / 16) & 7.
    // The launcher guarantees cols % 8 == 0, a 16-byte aligned x and
    // M * cols * 2 below 4 GiB.
    int achunk[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) achunk[i] = 8 * ((lane & 7) ^ ((4 * i + (lane >> 4)) & 7));
    const int arow0 = m0 + wave * 8 * AB + (lane >> 3);
    const uint8_t* xb = reinterpret_cast<const uint8_t*>(x);
    auto load_a = [&](int h, int i) {
        const int k0 = min(h >> 1, steps - 1) * kPK + (h & 1) * (kPK / 2);
        const uint32_t row = static_cast<uint32_t>(min(arow0 + 8 * i, M - 1));
        const uint32_t off = 2u * (row * static_cast<uint32_t>(m.cols) +
                                   static_cast<uint32_t>(min(k0 + achunk[(wave * AB + i) & 1], m.cols - 8)));
        __builtin_amdgcn_global_load_lds(
            xb + off, (lds_void_ptr)(xs + (h & 3) * kQHalf + (wave * 8 * AB + 8 * i) * kQHalfRow), 16, 0, 0);
    };
    auto load_b = [&](Bits (&r)[JB], int h, int j) {
        const uint32_t st = static_cast<uint32_t>(min(h >> 1, steps - 1));
        r[j].load32(m, slot0[j][h & 1] + st * kTileSlots);
    };

    floatx16 acc[AL + AH][JB];
#pragma unroll
    for (int i = 0; i < AL + AH; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // Operands: A in two halves (hh) of AL and AH 32-row blocks, each half
    // single-buffered; B double-buffered by set.  hh, set and q are
    // constants at every call, so the arrays stay in registers.
    half8 pa[2][AL], pb[2][JB];
    const int aswz = (n32 >> 1) & 7;
    auto read_a = [&](int hh, int h, int q) {
        const int chunk = (4 * half + q) ^ aswz;
        const uint8_t* base = xs + (h & 3) * kQHalf + (32 * AB * mh + 32 * AL * hh + n32) * kQHalfRow + chunk * 16;
#pragma unroll
        for (int i = 0; i < (hh == 0 ? AL : AH); ++i) pa[hh][i] = *reinterpret_cast<const half8*>(base + 32 * i * kQHalfRow);
    };
    auto decode_b = [&](int set, int j, int q, const Bits (&r)[JB]) { pb[set][j] = r[j].operand(q, s[j]); };
    auto mfma_half = [&](int hh, int set) {
#pragma unroll
        for (int i = 0; i < (hh == 0 ? AL : AH); ++i)
#pragma unroll
            for (int j = 0; j < JB; ++j)
                acc[AL * hh + i][j] =
                    __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[hh][i], pb[set][j], acc[AL * hh + i][j], 0, 0, 0);
    };

    // Half step h.  rc: its weight bits; rn: those of h + 1 (decoded at the
    // end for slice 0 of h + 1); rf: the buffer this half step fills (h + 2
    // with D = 3; with D = 2 it is rn itself, filled with h + 1).
    //
    // Slice q, entered with A-low(q) read and B(q) decoded into set q % 2:
    //   loads; wait A-low(q); low MFMAs with the reads of A-high(q) after
    //   the first and the second of them + decode B(q+1) block 0; wait
    //   A-high(q); read A-low(q+1); high MFMAs + decode B(q+1) block 1.
    // The A-high reads issued from within the MFMA group keep their LDS
    // latency off the wave's critical path: read ahead of the low MFMAs, in
    // slices 1 and 3 the compiler joined their wait to that of A-low
    // (14336 x 4096, M = 2048, same box: b = 10 214.8 -> 213.0 us, b = 8
    // 203.3 -> 199.4, bit-identical).  At b = 11, whose decode is longer,
    // that order measured 1% slower; there A-high is read ahead as before.
    // Slice 3 instead waits for the loads of half step h + 1, passes the
    // barrier and reads A-low of slice 0 of h + 1; its high MFMAs overlap
    // both decodes of that slice.
    auto half_step = [&](const Bits (&rc)[JB], const Bits (&rn)[JB], Bits (&rf)[JB], int h) {
        const bool more = h + 1 < 2 * steps;
        auto slice = [&](auto q_c) {
            constexpr int Q = decltype(q_c)::value;
            constexpr int SET = Q & 1;
            if constexpr (D == 3) {
                if constexpr (Q < AB) load_a(h + 2, Q);
                if constexpr (Q < JB) load_b(rf, h + 2, Q);
            } else {
                if constexpr (Q == 0) {
#pragma unroll
                    for (int j = 0; j < JB; ++j) load_b(rf, h + 1, j);
                }
                if constexpr (Q < AB) load_a(h + 2, Q);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kReadInGroup) {
                wait_lgkmcnt<0>();                 // A-low(q) landed
                __builtin_amdgcn_sched_barrier(0);
                mfma_half(0, SET);
                read_a(1, h, Q);
                if constexpr (Q < 3) decode_b(SET ^ 1, 0, Q + 1, rc);
                if constexpr (JB == 2) {
                    // order: MFMA, read, MFMA, (read,) MFMA, eight VALU, MFMA, the rest
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if constexpr (AH == 2) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                } else {
                    // order: MFMA, read, ... (AB of each), eight VALU, the rest
#pragma unroll
                    for (int k = 0; k < AB; ++k) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    }
                    __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                }
            } else {
                read_a(1, h, Q);
                wait_lgkmcnt<AH>();                // A-low(q) landed
                __builtin_amdgcn_sched_barrier(0);
                mfma_half(0, SET);
                if constexpr (Q < 3) decode_b(SET ^ 1, 0, Q + 1, rc);
            }
            __builtin_amdgcn_sched_barrier(0);
            wait_lgkmcnt<0>();                     // A-high(q) landed
            if constexpr (Q == 3) {
                // A and B of half step h + 1 landed: younger are this half
                // step's AB activation loads and, with D = 3, its JB
                // weight groups (with D = 2 its weight groups are the ones
                // waited for, issued before its activation loads)
                wait_vmcnt<D == 3 ? AB + JB * GL : AB>();
                barrier_after_wait();
                __builtin_amdgcn_sched_barrier(0);
                if (more) read_a(0, h + 1, 0);
            } else {
                read_a(0, h, Q + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            mfma_half(1, SET);
            if constexpr (Q < 3) {
                if constexpr (JB == 2) decode_b(SET ^ 1, 1, Q + 1, rc);
            } else {
                if (more) {
#pragma unroll
                    for (int j = 0; j < JB; ++j) decode_b(0, j, 0, rn);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        slice(std::integral_constant<int, 0>{});
        slice(std::integral_constant<int, 1>{});
        slice(std::integral_constant<int, 2>{});
        slice(std::integral_constant<int, 3>{});
    };

    Bits ring0[JB], ring1[JB], ring2[JB];
    // prologue: A of half steps 0 and 1, weight bits of half step 0 (and 1
    // with D = 3)
#pragma unroll
    for (int i = 0; i < AB; ++i) load_a(0, i);
#pragma unroll
    for (int j = 0; j < JB; ++j) load_b(ring0, 0, j);
#pragma unroll
    for (int i = 0; i < AB; ++i) load_a(1, i);
    if constexpr (D == 3) {
#pragma unroll
        for (int j = 0; j < JB; ++j) load_b(ring1, 1, j);
    }
    wait_vmcnt<0>();
    barrier_after_wait();
    read_a(0, 0, 0);
#pragma unroll
    for (int j = 0; j < JB; ++j) decode_b(0, j, 0, ring0);
    if constexpr (D == 3) {
        // One step (two half steps) per iteration; the ring advances by two
        // buffers, (r0, r1, r2) <- (r2, r0, r1), by register copies.
        for (int st = 0; st < steps; ++st) {
            half_step(ring0, ring1, ring2, 2 * st);
            half_step(ring1, ring2, ring0, 2 * st + 1);
            Bits t[JB];
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                t[j].copy_from(ring0[j]);
                ring0[j].copy_from(ring2[j]);
                ring2[j].copy_from(ring1[j]);
                ring1[j].copy_from(t[j]);
            }
        }
    } else {
        (void)ring2;
        for (int st = 0; st < steps; ++st) {
            half_step(ring0, ring1, ring1, 2 * st);
            half_step(ring1, ring0, ring0, 2 * st + 1);
        }
    }

    // ---- epilogue: the whole 256 x 256 tile through LDS ----
    // 32x32 block element e of lane l is D[8*(e/4) + 4*(l/32) + e%4][l%32].
    // The clamped re-loads of the last step must land before the LDS is
    // reused.
    wait_vmcnt<0>();
    __syncthreads();
    static_assert(kQRows * kQCPitch <= kQLds, "output staging exceeds the LDS");
    float sn[JB];
    uint16_t bn[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int n = min(nw0 + 32 * j + n32, m.rows - 1);
        sn[j] = 1.0f;
        bn[j] = 0;
        if constexpr (MODE == kModeQ) sn[j] = m.scales[n];
        if (bias) bn[j] = bias[n];
    }
    {
        uint8_t* cw = xs + (32 * AB * mh) * kQCPitch + colg * 64 * JB;
#pragma unroll
        for (int j = 0; j < JB; ++j)
#pragma unroll
            for (int i = 0; i < AL + AH; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int r = 32 * i + 8 * (e >> 2) + 4 * half + (e & 3);
                    *reinterpret_cast<uint16_t*>(cw + r * kQCPitch + (32 * j + n32) * 2) =
                        epilogue<MODE>(acc[i][j][e], sn[j], bias != nullptr, bn[j]);
                }
    }
    __syncthreads();
    const bool yvec = (m.rows % 8 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0);
    const int chunk = threadIdx.x & 31;         // 16-byte chunk of a 512-byte row
#pragma unroll 4
    for (int it = 0; it < kRows / (64 * kQWaves / 32); ++it) {
        const int r = it * (64 * kQWaves / 32) + (threadIdx.x >> 5);
        const int gr = m0 + r;
        const int gn = n0 + chunk * 8;
        if (gr >= M || gn >= m.rows) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(xs + r * kQCPitch + chunk * 16);
        uint16_t* dst = y + static_cast<size_t>(gr) * m.rows + gn;
        if (yvec) {
            store_out16(dst, v);
        } else {
            const uint16_t* hv = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (gn + k < m.rows) dst[k] = hv[k];
            }
        }
    }
}

PPGrid pp_grid(const PPRect& a, const PPRect& b) {
    PPGrid g{};
    g.r[0] = a;
    g.r[1] = b;
    g.jobs0 = a.mblocks * a.nblocks;
    g.njobs = g.jobs0 + b.mblocks * b.nblocks;
    g.per_xcd = (g.njobs + 7) / 8;
    return g;
}

// The launches of one prefill: 256 x 256 tiles (full) and 192 x 256 tiles
// (short), either possibly empty, each one launch.
//
// Rounds.  Measured on MI355X (256 CUs), 14336 x 4096, b = 10, one launch of
// one tile height, us by tiles in the launch:
//   256-row tiles: 56: 78.9, 112: 80.0, 168: 93.0, 224: 110.8, 280: 192.0,
//   336: 196.8, 392: 203.4, 448: 214.2, 504: 230.0;
//   192-row tiles: 112: 70.3, 168: 79.6, 224: 90.3, 280: 160.9, 336: 163.4,
//   392: 168.8, 448: 176.3, 504: 193.0, 560: 257.9
// (b = 8 alike).  A round that keeps every CU busy is held by the chip as
// a whole, a sparse one by each CU's own tile: a round with a fraction f of
// the CUs busy costs about max(0.69, 0.45 + 0.55 f) of a full round of
// 256-row tiles, and of 192-row tiles max(0.60, 0.44 + 0.39 f) (0.83 when
// full).  So a 256 x 256 grid whose last round is sparse is better run as
// whole rounds of 256 x 256 tiles plus 192 x 256 tiles for the rest: every
// activation block of the first weight-row blocks and the first k of the
// last n stay 256 x 256, the rest of those n columns becomes 192 x 256.
// pp_plan picks k and n by that cost and takes the plan when it predicts at
// least 3% less time than the plain grid (same box, us, plain -> plan:
// 14336 x 4096 M = 1536 196.8 -> 175.5, 11008 x 4096 M = 2048 195.9 ->
// 183.1; the model rejects M = 2048 at 14336 x 4096, measured 214.0 ->
// 215.9).  Both tile shapes accumulate every output over K in the same
// order, so the output does not depend on the plan.
double pp_rounds_cost(int tiles, int cus, bool short_tiles) {
    if (tiles <= 0) return 0.0;
    const int whole = tiles / cus;
    const int rem = tiles % cus;
    const double f = static_cast<double>(rem) / cus;
    double cost = whole * (short_tiles ? 0.83 : 1.0);
    if (rem > 0) cost += short_tiles ? std::max(0.60, 0.44 + 0.39 * f) : std::max(0.69, 0.45 + 0.55 * f);
    return cost;
}

PPPlan pp_plan(int64_t M64, int rows, int cus, int tiles_mode) {
    const int M = static_cast<int>(M64);
    const int mb = (M + kQRows - 1) / kQRows;
    const int nb = (rows + kQN - 1) / kQN;
    const PPRect none{0, 0, 0, 0};
    PPPlan plan{pp_grid({0, mb, 0, nb}, none), pp_grid(none, none), pp_rounds_cost(mb * nb, cus, false)};
    if (tiles_mode == kPrefillTilesWide8Short || tiles_mode == kPrefillTilesWideShort) {
        const int sb = (M + 191) / 192;
        plan.full = pp_grid(none, none);
        plan.short_tiles = pp_grid({0, sb, 0, nb}, none);
        plan.cost = pp_rounds_cost(sb * nb, cus, true);
        return plan;
    }
    if (tiles_mode == kPrefillTilesWide8Plain || tiles_mode == kPrefillTilesWidePlain || (mb * nb) % cus == 0) {
        return plan;
    }
    double best = 0.97 * plan.cost;
    for (int k = 0; k < mb; ++k) {                     // 256-row blocks kept in the mixed columns
        const int s = (M - kQRows * k + 191) / 192;    // 192-row tiles below them
        for (int n = 1; n <= nb; ++n) {                // mixed columns: the last n weight-row blocks
            const int full = mb * (nb - n) + k * n;
            const double cost = pp_rounds_cost(full, cus, false) + pp_rounds_cost(s * n, cus, true);
            if (cost < best) {
                best = cost;
                plan.full = pp_grid({0, mb, 0, nb - n}, {0, k, nb - n, n});
                plan.short_tiles = pp_grid({kQRows * k, s, nb - n, n}, none);
                plan.cost = cost;
            }
        }
    }
    return plan;
}

// pp_plan searches k and n (tens of microseconds of host time for grids of
// thousands of tiles); a launch asks for the plan twice (route choice and
// launch), and a model asks for the same shapes again and again, so each host
// thread keeps its last plans.
PPPlan pp_plan_cached(int64_t M, int rows, int cus, int tiles_mode) {
    struct Entry {
        int64_t M;
        int rows, cus, mode;
        bool used;
        PPPlan plan;
    };
    constexpr int kEntries = 16;
    thread_local Entry cache[kEntries] = {};
    thread_local int next = 0;
    for (const Entry& e : cache) {
        if (e.used && e.M == M && e.rows == rows && e.cus == cus && e.mode == tiles_mode) return e.plan;
    }
    const PPPlan plan = pp_plan(M, rows, cus, tiles_mode);
    cache[next] = Entry{M, rows, cus, tiles_mode, true, plan};
    next = (next + 1) % kEntries;
    return plan;
}

template <int B, int MODE>
hipError_t launch_pp(const DevMatrix& m, const uint16_t* x, int64_t M, uint16_t* y, const uint16_t* bias,
                     hipStream_t s, int cus, int tiles_mode) {
    const PPPlan plan = pp_plan_cached(M, m.rows, cus, tiles_mode);
    if (plan.full.njobs > 0) {
        hipLaunchKernelGGL((linear_prefill_pp_kernel<B, MODE, 4>), dim3(8 * plan.full.per_xcd), dim3(64 * kQWaves),
                           0, s, m, x, static_cast<int>(M), y, bias, plan.full);
    }
    if (plan.short_tiles.njobs > 0) {
        hipLaunchKernelGGL((linear_prefill_pp_kernel<B, MODE, 3>), dim3(8 * plan.short_tiles.per_xcd),
                           dim3(64 * kQWaves), 0, s, m, x, static_cast<int>(M), y, bias, plan.short_tiles);
    }
    return hipGetLastError();
}

template <int B>
hipError_t launch_pp_bits(const DevMatrix& m, int mode, const uint16_t* x, int64_t M, uint16_t* y,
                          const uint16_t* bias, hipStream_t s, int cus, int tiles_mode) {
    if constexpr (B <= 12) {
        if (mode == kModeQ) return launch_pp<B, kModeQ>(m, x, M, y, bias, s, cus, tiles_mode);
    }
    if (mode == kModeW) return launch_pp<B, kModeW>(m, x, M, y, bias, s, cus, tiles_mode);
    return hipErrorInvalidValue;
}

}  // namespace

PrefillPlan prefill_plan(int64_t M, int rows, int cus, int tiles_mode) {
    return pp_plan_cached(M, rows, cus, tiles_mode);
}

double prefill_pp_rounds(int64_t M, int rows, int cus, int tiles_mode) {
    return pp_plan_cached(M, rows, cus, tiles_mode).cost;
}

double prefill_pp_plan_rects(int64_t M, int rows, int cus, int tiles_mode, int32_t* out) {
    const PPPlan plan = pp_plan_cached(M, rows, cus, tiles_mode);
    const PPRect* rects[3] = {&plan.full.r[0], &plan.full.r[1], &plan.short_tiles.r[0]};
    const int heights[3] = {kQRows, kQRows, 192};
    const bool used[3] = {plan.full.jobs0 > 0, plan.full.njobs > plan.full.jobs0, plan.short_tiles.njobs > 0};
    for (int i = 0; i < 3; ++i) {
        const PPRect& r = *rects[i];
        const int32_t v[5] = {r.m0, r.mblocks, heights[i], r.nb0, r.nblocks};
        for (int j = 0; j < 5; ++j) out[5 * i + j] = used[i] ? v[j] : 0;
    }
    return plan.cost;
}

hipError_t launch_prefill_pp(const DevMatrix& m, int mode, const uint16_t* x, int64_t M, uint16_t* y,
                             const uint16_t* bias, hipStream_t s, int cus, int tiles_mode) {
    if (mode == kModeRaw) return launch_pp<8, kModeRaw>(m, x, M, y, bias, s, cus, tiles_mode);
    switch (m.bits) {
        case 3: return launch_pp_bits<3>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 4: return launch_pp_bits<4>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 5: return launch_pp_bits<5>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 6: return launch_pp_bits<6>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 7: return launch_pp_bits<7>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 8: return launch_pp_bits<8>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 9: return launch_pp_bits<9>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 10: return launch_pp_bits<10>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 11: return launch_pp_bits<11>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 12: return launch_pp_bits<12>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 13: return launch_pp_bits<13>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 14: return launch_pp_bits<14>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        case 15: return launch_pp_bits<15>(m, mode, x, M, y, bias, s, cus, tiles_mode);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ebk
