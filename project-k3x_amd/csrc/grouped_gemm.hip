// grouped_gemm.hip -- the wide expert GEMM: experts with many rows (prefill
// chunks, verification windows) on bf16 MFMA, MXFP4 weights dequantised in
// registers.
//
// Workgroup = 8 waves, one 128-row chunk of one expert's rows (a work item
// listed by the grouping, so large experts spread over many workgroups) x
// NT 16-row output blocks per wave (gate/up: NT pairs of 16 gate + 16 up
// rows).  Per K tile (128 K):
//   * the chunk's activation rows (gathered through pair_token for the
//     routed gate/up) arrive in LDS by buffer loads that write LDS directly
//     (no registers), into a ring of kWideStages tiles.  A tile is stored as
//     32 KiB of row quads: rows 4q .. 4q + 3 fill 1 KiB, 16-byte chunk c of
//     row r at (r / 4) KiB + (c ^ (r / 4 % 4)) * 64 + (r % 4) * 16, a layout
//     measured at the ds_read_b128 rate of a linear read for the MFMA
//     operand pattern (16 lanes = 16 rows of one chunk), where row-major
//     XOR or padded layouts take about 1.4x as long;
//   * each wave dequantises its weight fragments once (v_cvt_scalef32_pk_
//     bf16_fp4 per code byte) and feeds each to the MFMAs of the chunk's
//     eight 16-row tiles (four when the chunk has at most 64 rows);
//   * software pipeline: step k multiplies tile k, then requests activation
//     and weight tile k + 3, then waits until only the requests of steps
//     k - 1 and k are outstanding (the vector-memory counter retires in issue
//     order) and meets the other waves at a barrier.  Tile k + 1 was
//     requested at step k - 2, so it is in LDS and registers; each request
//     has two steps of multiplies to arrive in.
// The weights of an expert are read once per 128-row chunk.  The N blocks of
// one item are numbered to land on one XCD, so its activation rows are
// fetched into that XCD's L2 once; the grouping deals the items to the XCDs'
// ranges by size, so the XCDs get equal work.
// Epilogues: GLU -> bf16 act (gate/up), fp32 rows scattered to the pair's
// (token, slot) row (routed down) or the token row (shared down).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "k3x_gemm.hpp"

using namespace k3x_dev;
using k3x_hip::kWideRows;
using k3x_hip::kWideStages;
using k3x_hip::WideGemmArgs;

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMTiles = kWideRows / 16;          // MFMA row tiles per chunk
constexpr int kTileChunks = kWideRows * 16;      // 16-byte chunks per activation tile
constexpr int kALoads = kTileChunks / kThreads;  // LDS-direct loads per wave per tile
static_assert(kALoads * kThreads == kTileChunks, "whole activation tile per step");

__device__ inline uint32_t prior_status(const uint32_t* status) { return *status; }
__device__ inline uint32_t wave_index() {
    return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Step (k % 4) of a block of four K tiles at which the MXFP4 weight scale
// dwords of the next block are requested: with the block's first step, or
// (q8 rows, which leave fewer registers) first thing at its third, so that
// they occupy registers for two steps instead of four.
template <bool Q>
constexpr int scale_step() {
    return Q ? 2 : 0;
}

// Vector-memory requests one wave issues at pipeline step k (activation tile,
// q8 scale dwords, weight tile; the MXFP4 scale dwords cover four K tiles and
// are requested at steps with k % 4 == scale_step).
template <bool FP4, int NT, int S, int U, bool Q>
constexpr int step_loads(int d) {
    return kALoads + (Q ? 1 : 0) + NT * S * U + ((FP4 && d == scale_step<Q>()) ? NT * S : 0);
}

// Waits until at most N of this wave's vector-memory requests are
// outstanding and all its LDS operations are done, then meets the workgroup.
// The memory clobber keeps the compiler from moving loads or LDS accesses
// across it.
template <int N>
__device__ inline void wait_and_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// End of pipeline step d (= k % 4): only the requests of steps k - 1 and k
// may stay outstanding.  d is a constant once the step loop is unrolled.
template <bool FP4, int NT, int S, int U, bool Q>
__device__ inline void end_step(int d) {
#define K3X_SL(i) step_loads<FP4, NT, S, U, Q>(i)
    switch (d) {
        case 0: wait_and_barrier<K3X_SL(3) + K3X_SL(0)>(); break;
        case 1: wait_and_barrier<K3X_SL(0) + K3X_SL(1)>(); break;
        case 2: wait_and_barrier<K3X_SL(1) + K3X_SL(2)>(); break;
        default: wait_and_barrier<K3X_SL(2) + K3X_SL(3)>(); break;
    }
#undef K3X_SL
}

// SPLIT: gate/up stores each activation as bf16 hi and lo halves (act_lo
// elements apart); down reads rows [hi | lo] of 2 kt tiles against the
// weights repeated along K.
// Q (MXFP4 only): the activation rows are q8 rows (hi and lo E4M3 codes of
// each K tile, 256 bytes like a bf16 tile row) with E8M0 scale dwords; each
// (row tile, weight block) pair takes two v_mfma_scale_f32_16x16x128_f8f6f4
// per K tile (hi, lo) on the weight codes as stored, in place of four bf16
// MFMAs on dequantised weights.
// MTC > 0 (routed kinds): a launch over one size class of the grouping's
// work items (each class's items in a list segment of its own, the class
// counts after the total in n_items), every chunk multiplied as MTC row
// tiles; MTC = 0 (shared kinds): every row chunk of the batch, the row tiles
// chosen per chunk below.
template <bool FP4, bool GATEUP, int NT, bool SPLIT, bool Q, int MTC = 0>
__global__ __launch_bounds__(kThreads, 1) void wide_gemm(WideGemmArgs a) {
    static_assert(!Q || (FP4 && !SPLIT), "q8 rows meet MXFP4 weights, one term pair per tile");
    // 128 KiB ring; the split gate/up's epilogue stages 128 rows of fp32
    // values in one pass, 16 bytes of pitch padding a row more than that.
    constexpr uint32_t kRingChunks = kWideStages * kTileChunks;
    constexpr uint32_t kStageChunks = GATEUP && SPLIT ? kWideRows * (kWaves * NT * 4 + 1) : 0;
    // Down's output row of each chunk row sits past the ring (or the split
    // epilogue's staging) in the same LDS array: as a second LDS variable it
    // made the compiler's wait counting fall back to a full drain of the
    // ring's LDS-DMA requests twice per four steps.  (Q's row scales stay a
    // variable of their own: folded in as well, the q8 kernels spilled.)
    constexpr uint32_t kA4 = kRingChunks > kStageChunks ? kRingChunks : kStageChunks;
    constexpr uint32_t kYrowChunks = GATEUP ? 0 : kWideRows * 4 / 16;
    __shared__ u32x4 s_a4[kA4 + kYrowChunks];
    uint32_t* const s_yrow = reinterpret_cast<uint32_t*>(s_a4 + kA4);
    // Q: scale dwords {hi, lo} of the chunk's rows per ring stage.
    __shared__ uint32_t s_qs[Q ? kWideStages * kWideRows * 2 : 1];
    constexpr int S = GATEUP ? 2 : 1;  // matrices per output row block (gate, up)
    constexpr int U = FP4 ? 1 : 4;     // 16-byte words per lane per tile
    static_assert(kWideStages == 4, "the step schedule below is written for four stages");
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const uint32_t g = lane >> 4, n = lane & 15;
    // One workgroup per (work item, output block set) on a 1-D grid sized
    // for the most items the grouping can list; the first nvalid workgroups
    // carry the listed items.  Consecutive workgroups go to the eight XCDs in
    // turn; renumber those nvalid so that each XCD takes an equal,
    // contiguous range of logical blocks (the blocks of one item share an
    // L2), and the unused tail of the grid is spread over all XCDs instead
    // of idling whole XCDs.
    if (prior_status(a.status)) return;
    const uint32_t nblk = a.nrb / (kWaves * NT);
    uint32_t ibase = 0, nlisted = a.items ? *a.n_items : 0;
    if constexpr (MTC > 0) {
        for (uint32_t c = 0; c < a.item_class; ++c) ibase += a.n_items[1 + c];
        nlisted = a.n_items[1 + a.item_class];
    }
    const uint32_t nvalid = a.items ? min(nlisted * nblk, gridDim.x) : gridDim.x;
    if (blockIdx.x >= nvalid) return;
    const uint32_t xcd = blockIdx.x % 8, per = nvalid / 8, rem = nvalid % 8;
    const uint32_t lb = xcd * per + min(xcd, rem) + blockIdx.x / 8;
    const uint32_t item = lb / nblk, jb = lb % nblk;
    uint32_t e = 0, cnt = a.tokens, off = 0, m0 = item * kWideRows;
    if (a.items) {
        const uint32_t it = a.items[ibase + item];
        e = it >> 16;
        m0 = (it & 0xffffu) * kWideRows;
        cnt = a.counts[e];
        off = a.offsets[e];
    }
    if (m0 >= cnt) return;
    const uint32_t kt = a.kt;  // multiple of kWideStages (checked on the host)
    // Activation tiles: kt, or 2 kt for split [hi | lo] rows, interleaved:
    // step k multiplies weight tile k / 2 with the hi (k even) or lo (k odd)
    // half's tile k / 2, so each weight tile is requested twice in a row and
    // its second request finds it in the L2 (a block of four steps covers two
    // weight tiles of one scale dword).
    constexpr bool kSplitIn = SPLIT && !GATEUP;
    const uint32_t kta = kSplitIn ? 2 * kt : kt;
    auto wtile = [&](uint32_t k) {
        if constexpr (kSplitIn) return k >> 1;
        else return k;
    };
    const uint32_t rows = min(cnt - m0, kWideRows);
    const uint32_t rb0 = (jb * kWaves + wave) * NT;
    // Weights of expert e through buffer resources: the per-lane offset is
    // the only vector register; block, tile and matrix offsets are scalar
    // (rb0 is wave-uniform), and reads past the expert's extent return 0.
    // Extent of one expert's tile array: nrb blocks x kt tiles x S x U KiB.
    const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(a.codes + e * a.codes_per_expert), (short)0,
        a.nrb * kt * (S * U * 1024u), 0x00020000);
    const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
        FP4 ? const_cast<uint32_t*>(a.scales + e * a.scales_per_expert) : nullptr, (short)0,
        FP4 ? (uint32_t)(a.scales_per_expert * 4) : 0u, 0x00020000);
    const uint32_t lane16 = lane * 16, lane4 = lane * 4;

    // Activation tile loads: wave w's load q fills the row quad 4 w + q
    // (rows 16 w + 4 q .. + 3, 1 KiB: lane l writes row 16 w + 4 q + l % 4 at
    // position l / 4, which holds the row's 16-byte chunk (l / 4) ^ q).  Rows
    // past the chunk's end repeat its last row (they are never stored).
    const __amdgpu_buffer_rsrc_t arsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.a), (short)0, a.a_bytes, 0x00020000);
    uint32_t aoff[kALoads];
#pragma unroll
    for (int q = 0; q < kALoads; ++q) {
        const uint32_t r = 16 * wave + 4 * q + (lane & 3);
        const uint32_t rr = off + m0 + min(r, rows - 1);
        const uint32_t src = a.gather ? a.pair_token[rr] : rr;
        aoff[q] = (src * a.a_stride + ((lane >> 2) ^ q) * 8) * 2;
    }
    // Q: scale loads also write LDS directly, one dword per lane: waves w
    // and w + 4 both fill quarter w % 4 of a stage (rows 32 (w % 4) ..
    // + 31, {hi, lo} each; the same values), so every wave issues the same
    // number of requests per step.
    const __amdgpu_buffer_rsrc_t qrsrc = __builtin_amdgcn_make_buffer_rsrc(
        Q ? const_cast<uint32_t*>(a.qs) : nullptr, (short)0, Q ? a.qs_bytes : 0u, 0x00020000);
    uint32_t qoff = 0;
    if constexpr (Q) {
        const uint32_t r = (wave & 3) * 32 + (lane >> 1);
        const uint32_t rr = off + m0 + min(r, rows - 1);
        const uint32_t src = a.gather ? a.pair_token[rr] : rr;
        qoff = (src * kt * 2 + (lane & 1)) * 4;
    }
    // Down: the output row of chunk row tid % 128 (the pair's token * top_k
    // + slot, or the row itself), requested first; it goes through LDS to
    // the lanes that store the row, stored there once the prologue's
    // requests are out (no register holds it through the step loop).
    uint32_t yv = 0;
    if constexpr (!GATEUP) {
        const uint32_t r = off + m0 + min(tid % kWideRows, rows - 1);
        yv = a.scatter ? a.pair_token[r] * a.top_k + a.pair_slot[r] : r;
    }
    // MFMA operand of lane (n, g), 8-column group j: row n (+ 16 per row
    // tile, 4 KiB), chunk 4 g + j; in 16-byte units.
    // Q: the E4M3 operand of lane (n, g) is K 16 g .. + 15 and 64 + 16 g ..
    // + 15 of row n (the scaled MFMA's 8-bit lane layout): chunks g and
    // g + 4 of the hi codes, 8 + g and 12 + g of the lo codes.  The swizzle
    // only touches c % 4, so they sit 0, 4, 8 and 12 chunk positions (16
    // units each) past chunk g: apos[0] serves all four.
    uint32_t apos[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = Q ? g : 4 * g + j;
        apos[j] = (n >> 2) * 64 + (c ^ (n >> 2)) * 4 + (n & 3);
    }

    // Weight stages: codes bc[d][nt][w][u] of K tile k in stage d = k % 4
    // (three are live at a time: tiles k .. k + 2 while tile k is
    // multiplied); scale dwords of the four tiles kb .. kb + 3 in sc (current
    // block) and scn (next block).  Plain arrays indexed only inside fully
    // unrolled loops, so they live in registers.
#define WIDE_LOAD_A(k, buf)                                                                  \
    _Pragma("unroll") for (int q = 0; q < kALoads; ++q)                                      \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(                                            \
            arsrc, (lds_ptr_t)&s_a4[(buf) * kTileChunks + (16 * wave + 4 * q) * 16], 16,      \
            aoff[q], (kSplitIn ? ((k) & 1) * kt + ((k) >> 1) : (k)) * 256, 0, 0);
#define WIDE_LOAD_B(d, k)                                                                    \
    _Pragma("unroll") for (int nt = 0; nt < NT; ++nt)                                        \
        _Pragma("unroll") for (int w = 0; w < S; ++w) {                                      \
            const uint32_t base_ = (((rb0 + nt) * kt + (k)) * S + w) * U * 1024;             \
            _Pragma("unroll") for (int u = 0; u < U; ++u) bc[d][nt][w][u] =                  \
                __builtin_amdgcn_raw_buffer_load_b128(wrsrc, lane16, base_ + u * 1024, 0);   \
        }
#define WIDE_LOAD_SCALES(dst, k)                                                             \
    if constexpr (FP4) {                                                                     \
        _Pragma("unroll") for (int nt = 0; nt < NT; ++nt)                                    \
            _Pragma("unroll") for (int w = 0; w < S; ++w) dst[nt][w] =                        \
                __builtin_amdgcn_raw_buffer_load_b32(                                        \
                    srsrc, lane4, (((rb0 + nt) * a.ks + (k) / 4) * S + w) * 256, 0);          \
    }
#define WIDE_LOAD_Q(k, buf)                                                                  \
    if constexpr (Q)                                                                         \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(                                            \
            qrsrc, (lds_ptr_t)&s_qs[(buf) * (kWideRows * 2) + (wave & 3) * 64], 4, qoff,     \
            (k) * 8, 0, 0);
#define WIDE_ORDER() asm volatile("" ::: "memory")

    // MT = row tiles multiplied: the chunk's rows rounded up to 32, 64, 96
    // or 128 rows, see the dispatch at the end (a workgroup-uniform choice
    // made once, so the step loop has no branches; tiles past the chunk's
    // rows hold copies of its last row and are not stored).
    auto run = [&](auto mt_count) {
        constexpr int MT = decltype(mt_count)::value;
        f32x4 acc[MT][NT][S];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int w = 0; w < S; ++w) acc[mt][nt][w] = f32x4{0.f, 0.f, 0.f, 0.f};
        u32x4 bc[kWideStages][NT][S][U];
        uint32_t sc[NT][S], scn[NT][S];

        // Prologue = steps -3 .. -1 of the schedule: step s requests
        // activation and weight tile s + 3 (the scales of tiles 0..3 with
        // step -3's).
        WIDE_LOAD_A(0u, 0)
        WIDE_LOAD_Q(0u, 0)
        WIDE_LOAD_B(0, wtile(0u))
        WIDE_LOAD_SCALES(sc, wtile(0u))
        WIDE_ORDER();
        WIDE_LOAD_A(1u, 1)
        WIDE_LOAD_Q(1u, 1)
        WIDE_LOAD_B(1, wtile(1u))
        WIDE_ORDER();
        WIDE_LOAD_A(2u, 2)
        WIDE_LOAD_Q(2u, 2)
        WIDE_LOAD_B(2, wtile(2u))
        if constexpr (!GATEUP) {
            if (tid < kWideRows) s_yrow[tid] = yv;
        }
        // Steps -2 and -1 may stay in flight; tile 0 (step -3) has arrived.
        wait_and_barrier<2 * (kALoads + (Q ? 1 : 0) + NT * S * U)>();

        for (uint32_t kb = 0; kb < kta; kb += kWideStages) {
#pragma unroll
            for (int d = 0; d < kWideStages; ++d) {
                const uint32_t k = kb + d;
                const u32x4* sa = s_a4 + d * kTileChunks;
                if constexpr (Q) {
                    // Scale bytes: the weights' byte d of each block dword
                    // (selected by the MFMA's op_sel), the rows' byte g of
                    // their {hi, lo} dwords (read as a byte from LDS).
                    const uint8_t* sq =
                        reinterpret_cast<const uint8_t*>(s_qs + d * (kWideRows * 2));
                    // All row tiles' hi terms, then their lo terms (an
                    // accumulator's two updates MT * NT * S MFMAs apart).
                    // The operand of the next row tile is read from LDS
                    // before the MFMAs of this one; the scheduling barrier
                    // keeps the compiler from hoisting more reads (their
                    // registers would spill).
                    auto operand = [&](int i) {
                        const int t = i / MT, mt = i % MT;
                        return q8_operand(sa[mt * 256 + t * 32 + apos[0]],
                                          sa[mt * 256 + t * 32 + 16 + apos[0]]);
                    };
                    auto exponent = [&](int i) {
                        const int t = i / MT, mt = i % MT;
                        return (uint32_t)sq[(mt * 16 + n) * 8 + t * 4 + g];
                    };
                    i32x8 av = operand(0);
                    uint32_t ea = exponent(0);
#pragma unroll
                    for (int i = 0; i < 2 * MT; ++i) {
                        i32x8 an = av;
                        uint32_t en = ea;
                        if (i + 1 < 2 * MT) {
                            an = operand(i + 1);
                            en = exponent(i + 1);
                        }
                        const int mt = i % MT;
#pragma unroll
                        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                            for (int w = 0; w < S; ++w)
                                acc[mt][nt][w] = mfma_q8_fp4_sel(d, av, bc[d][nt][w][0],
                                                                 acc[mt][nt][w], ea, sc[nt][w]);
                        __builtin_amdgcn_sched_barrier(0);
                        av = an;
                        ea = en;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        bf16x8 bw[NT][S];
#pragma unroll
                        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                            for (int w = 0; w < S; ++w) {
                                if constexpr (FP4) {
                                    const uint32_t word = bc[d][nt][w][0][j];
                                    // Scale byte of weight tile wtile(k)
                                    // in the block's dword.
                                    const uint32_t sb =
                                        kSplitIn ? 8 * (((kb >> 1) & 3) + (d >> 1)) : 8 * d;
                                    bw[nt][w] = dequant8(
                                        word, e8m0_to_f32((sc[nt][w] >> sb) & 0xffu));
                                } else {
                                    bw[nt][w] = as_bf16x8(bc[d][nt][w][j]);
                                }
                            }
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            const bf16x8 af = as_bf16x8(sa[mt * 256 + apos[j]]);
#pragma unroll
                            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                                for (int w = 0; w < S; ++w)
                                    acc[mt][nt][w] = mfma16x16x32(af, bw[nt][w], acc[mt][nt][w]);
                        }
                    }
                }
                // Step k's requests: tile k + 3 into the LDS buffer and
                // weight stage tile k - 1 used (all waves passed the barrier
                // after multiplying it); past the end they repeat the last
                // tile (the loads stay unconditional, the count exact).  The
                // next block's scales ride with step scale_step of the block
                // (with q8 rows requested first, so that waiting for them at
                // the next block does not wait for this step's tiles).
                constexpr bool kScalesFirst = Q;
                if (kScalesFirst && d == scale_step<Q>())
                    WIDE_LOAD_SCALES(scn, wtile(min(kb + 4, kta - 1)))
                WIDE_LOAD_A(min(k + 3, kta - 1), (d + 3) % kWideStages)
                WIDE_LOAD_Q(min(k + 3, kta - 1), (d + 3) % kWideStages)
                WIDE_LOAD_B((d + 3) % kWideStages, wtile(min(k + 3, kta - 1)))
                if (!kScalesFirst && d == scale_step<Q>())
                    WIDE_LOAD_SCALES(scn, wtile(min(kb + 4, kta - 1)))
                // Tile k + 1 (requested at step k - 2) is in LDS once only
                // steps k - 1 and k are outstanding.
                end_step<FP4, NT, S, U, Q>(d);
            }
            if constexpr (FP4) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int w = 0; w < S; ++w) sc[nt][w] = scn[nt][w];
            }
        }
        // The repeated last-tile requests of the final steps land before the
        // ring is reused for the output tile below.
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

        // Epilogue through LDS: the waves write their accumulators (GLU ->
        // bf16 for gate/up, fp32 for down) into the ring as row-major rows of
        // this workgroup's kCols output columns, then every lane stores 16
        // contiguous bytes of a row, so a wave writes whole 128-byte lines
        // where the accumulator layout (4 rows x 16 columns per store) wrote
        // 32- or 64-byte pieces of four rows.  Row pitch = row bytes + 16:
        // the four row groups of a write land 16 banks apart.  Down tiles
        // larger than the ring go in passes of RP rows.
        constexpr uint32_t kCols = kWaves * NT * 16;
        // Output element bytes: bf16 act, or fp32 (down's rows; split
        // gate/up's GLU values, rounded to the hi and lo halves as they are
        // copied out -- rounding them while the accumulators are live took
        // more registers than the step loop leaves).
        constexpr uint32_t kEs = GATEUP && !SPLIT ? 2 : 4;
        constexpr uint32_t kChunks = kCols * kEs / 16;              // 16-byte chunks per row
        constexpr uint32_t kPitch = kCols * kEs + 16;               // staged row bytes
        constexpr uint32_t kRing = kA4 * 16;  // the staging stays clear of s_yrow
        constexpr uint32_t RP0 = kRing / kPitch / 16 * 16;
        constexpr uint32_t RP = RP0 < MT * 16 ? RP0 : MT * 16;     // rows per pass
        static_assert(RP >= 16, "one row tile per pass at least");
        uint8_t* stage = reinterpret_cast<uint8_t*>(s_a4);
        const uint32_t col0 = jb * kCols;
#pragma unroll
        for (uint32_t p0 = 0; p0 < MT * 16; p0 += RP) {
            if (p0) __syncthreads();  // the previous pass has been copied out
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                if (mt * 16 < (int)p0 || mt * 16 >= (int)(p0 + RP)) continue;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t row = 16 * mt + 4 * g + i - p0;
                        const uint32_t col = (wave * NT + nt) * 16 + n;
                        if constexpr (GATEUP && SPLIT) {
                            *reinterpret_cast<float*>(stage + row * kPitch + col * 4) =
                                glu(acc[mt][nt][0][i], acc[mt][nt][1][i], a.glu);
                        } else if constexpr (GATEUP) {
                            uint16_t* sp = reinterpret_cast<uint16_t*>(stage + row * kPitch) + col;
                            *sp = f32_to_bf16(glu(acc[mt][nt][0][i], acc[mt][nt][1][i], a.glu));
                        } else {
                            *reinterpret_cast<float*>(stage + row * kPitch + col * 4) =
                                acc[mt][nt][0][i];
                        }
                    }
            }
            __syncthreads();
            const uint32_t prow = min(rows - min(rows, p0), RP);  // valid rows of this pass
            for (uint32_t c = tid; c < prow * kChunks; c += kThreads) {
                const uint32_t row = c / kChunks, ch = c % kChunks;
                const u32x4 v = *reinterpret_cast<const u32x4*>(stage + row * kPitch + ch * 16);
                if constexpr (GATEUP && SPLIT) {
                    // Four GLU values -> their hi and lo halves.
                    uint32_t h[2], l[2];
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const float v0 = __uint_as_float(v[2 * q]), v1 = __uint_as_float(v[2 * q + 1]);
                        const uint16_t h0 = f32_to_bf16(v0), h1 = f32_to_bf16(v1);
                        h[q] = (uint32_t)h0 | (uint32_t)h1 << 16;
                        l[q] = (uint32_t)act_lo_bf16(v0, h0) | (uint32_t)act_lo_bf16(v1, h1) << 16;
                    }
                    uint16_t* dst = a.act + (size_t)(off + m0 + p0 + row) * a.act_stride + col0 +
                                    ch * 4;
                    *reinterpret_cast<uint2*>(dst) = make_uint2(h[0], h[1]);
                    *reinterpret_cast<uint2*>(dst + a.act_lo) = make_uint2(l[0], l[1]);
                } else if constexpr (GATEUP) {
                    uint16_t* dst = a.act + (size_t)(off + m0 + p0 + row) * a.act_stride + col0;
                    *reinterpret_cast<u32x4*>(dst + ch * 8) = v;
                } else {
                    float* dst = a.y + (size_t)s_yrow[p0 + row] * a.y_stride + col0;
                    *reinterpret_cast<u32x4*>(dst + ch * 4) = v;
                }
            }
        }
    };
    // Routed kinds: the launch's class fixes the row tiles, one step loop a
    // kernel (with a choice of three or four row-tile counts inside one
    // kernel, the register allocator spilled in the routed gate/up's step
    // loop).  Shared kinds: four, six or eight row tiles, by the chunk's rows.
    if constexpr (MTC > 0) {
        // The grouping's class rule bounds the chunk's rows; a chunk past it
        // would lose rows, so it is an error, never a silent result.
        if (rows > 16u * MTC) {
            if (tid == 0)
                atomicCAS(const_cast<uint32_t*>(a.status), 0u, (uint32_t)K3X_ERR_INVALID_STATE);
            return;
        }
        run(std::integral_constant<int, MTC>{});
    } else {
        static_assert(!FP4, "routed kinds launch per size class");
        if (rows > kWideRows * 3 / 4)
            run(std::integral_constant<int, kMTiles>{});
        else if (rows > kWideRows / 2)
            run(std::integral_constant<int, kMTiles * 3 / 4>{});
        else
            run(std::integral_constant<int, kMTiles / 2>{});
    }
}

#undef WIDE_LOAD_A
#undef WIDE_LOAD_B
#undef WIDE_LOAD_SCALES
#undef WIDE_LOAD_Q
#undef WIDE_ORDER

// Output 16-row blocks per wave (kWaves * NT per workgroup): the more output
// rows a workgroup covers, the fewer times the chunk's activation rows are
// streamed from L2.
constexpr int kNtRoutedGateUp = 2, kNtRoutedDown = 4, kNtSharedGateUp = 1, kNtSharedDown = 2;

// bf16 rows -> q8 rows: one thread per 32-element block; the four threads of
// one K tile (consecutive lanes) merge their exponents into the tile's two
// scale dwords.
__global__ __launch_bounds__(256) void q8_rows_kernel(const uint16_t* __restrict__ src,
                                                      uint32_t rows, uint32_t cols,
                                                      uint32_t stride, uint16_t* __restrict__ q,
                                                      uint32_t* __restrict__ qs,
                                                      const uint32_t* status) {
    if (prior_status(status)) return;
    const uint32_t nb = cols / 32;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    // rows * nb is a multiple of 4: a tile's four threads are all in or out.
    if (i >= rows * nb) return;
    const uint32_t row = i / nb, b = i % nb, t = b / 4, bb = b % 4;
    const u32x4* in = reinterpret_cast<const u32x4*>(src + (size_t)row * stride + b * 32);
    float x[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u32x4 v = in[c];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[8 * c + 2 * j] = __uint_as_float(v[j] << 16);
            x[8 * c + 2 * j + 1] = __uint_as_float(v[j] & 0xffff0000u);
        }
    }
    uint32_t hi[8], lo[8], eh, el;
    q8_block(x, hi, lo, eh, el);
    u32x4* out = reinterpret_cast<u32x4*>(reinterpret_cast<uint8_t*>(q) + (size_t)row * cols * 2 +
                                          t * 256 + bb * 32);
    out[0] = u32x4{hi[0], hi[1], hi[2], hi[3]};
    out[1] = u32x4{hi[4], hi[5], hi[6], hi[7]};
    out[8] = u32x4{lo[0], lo[1], lo[2], lo[3]};
    out[9] = u32x4{lo[4], lo[5], lo[6], lo[7]};
    eh <<= 8 * bb;
    el <<= 8 * bb;
    eh |= __shfl_xor(eh, 1);
    el |= __shfl_xor(el, 1);
    eh |= __shfl_xor(eh, 2);
    el |= __shfl_xor(el, 2);
    if (bb == 0)
        *reinterpret_cast<uint2*>(qs + ((size_t)row * (cols / 128) + t) * 2) = make_uint2(eh, el);
}

}  // namespace

namespace k3x_hip {

uint32_t wide_rb_per_block(WideKind kind) {
    switch (kind) {
        case kWideRoutedGateUp: return kWaves * kNtRoutedGateUp;
        case kWideRoutedDown: return kWaves * kNtRoutedDown;
        case kWideSharedGateUp: return kWaves * kNtSharedGateUp;
        default: return kWaves * kNtSharedDown;
    }
}

int launch_wide_gemm(k3x_hip_ctx* ctx, WideKind kind, const WideGemmArgs& args,
                     uint32_t max_items, hipStream_t stream, int item_class) {
    if (!stream) stream = ctx->stream;
    const uint32_t per = wide_rb_per_block(kind);
    if (args.nrb % per || args.kt % kWideStages || !args.kt || !max_items)
        return K3X_ERR_INVALID_EXTENT;
    // Routed kinds: one size class of the grouping's items a launch; the
    // shared kinds take every row of the batch.
    const bool routed = kind == kWideRoutedGateUp || kind == kWideRoutedDown;
    if (routed ? (!args.items || item_class < 0 || item_class >= (int)kWideClasses)
               : item_class != -1)
        return K3X_ERR_INVALID_EXTENT;
    // The epilogue stores 16-byte row pieces.
    const bool gu = kind == kWideRoutedGateUp || kind == kWideSharedGateUp;
    if (gu ? ((uintptr_t)args.act % 16 || args.act_stride % 8 || args.act_lo % 8)
           : ((uintptr_t)args.y % 16 || args.y_stride % 4))
        return K3X_ERR_INVALID_EXTENT;
    if (args.kta && (args.kta != 2 * args.kt || gu)) return K3X_ERR_INVALID_EXTENT;
    const bool split = gu ? args.act_lo != 0 : args.kta != 0;
    // q8 rows: routed kinds only, no split halves, a scale dword pair per
    // row and K tile.
    const bool q8 = args.qs != nullptr;
    if (q8 && (split || !routed || (uintptr_t)args.qs % 8 || args.a_stride != args.kt * 128))
        return K3X_ERR_INVALID_EXTENT;
    WideGemmArgs a = args;
    a.item_class = routed ? (uint32_t)item_class : 0u;
    const dim3 grid(max_items * (a.nrb / per));
#define K3X_GO(...) hipLaunchKernelGGL((__VA_ARGS__), grid, dim3(kThreads), 0, stream, a)
    // Row tiles of the classes: 8, 6, 4, 2.
#define K3X_CLASS(GU_, NT_, SPLIT_, Q_)                                          \
    switch (item_class) {                                                       \
        case 0: K3X_GO(wide_gemm<true, GU_, NT_, SPLIT_, Q_, 8>); break;         \
        case 1: K3X_GO(wide_gemm<true, GU_, NT_, SPLIT_, Q_, 6>); break;         \
        case 2: K3X_GO(wide_gemm<true, GU_, NT_, SPLIT_, Q_, 4>); break;         \
        default: K3X_GO(wide_gemm<true, GU_, NT_, SPLIT_, Q_, 2>); break;        \
    }
    switch (kind) {
        case kWideRoutedGateUp:
            if (q8) K3X_CLASS(true, kNtRoutedGateUp, false, true)
            else if (split) K3X_CLASS(true, kNtRoutedGateUp, true, false)
            else K3X_CLASS(true, kNtRoutedGateUp, false, false)
            break;
        case kWideRoutedDown:
            if (q8) K3X_CLASS(false, kNtRoutedDown, false, true)
            else if (split) K3X_CLASS(false, kNtRoutedDown, true, false)
            else K3X_CLASS(false, kNtRoutedDown, false, false)
            break;
        case kWideSharedGateUp:
            if (split) K3X_GO(wide_gemm<false, true, kNtSharedGateUp, true, false>);
            else K3X_GO(wide_gemm<false, true, kNtSharedGateUp, false, false>);
            break;
        default:
            if (split) K3X_GO(wide_gemm<false, false, kNtSharedDown, true, false>);
            else K3X_GO(wide_gemm<false, false, kNtSharedDown, false, false>);
            break;
    }
#undef K3X_CLASS
#undef K3X_GO
    ctx->kernel_launches += 1;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

int launch_q8_rows(k3x_hip_ctx* ctx, const uint16_t* src, uint32_t rows, uint32_t cols,
                   uint32_t stride, uint16_t* q, uint32_t* qs, hipStream_t stream) {
    if (!stream) stream = ctx->stream;
    if (!rows) return K3X_OK;
    if (cols % 128 || stride < cols || stride % 8 || (uintptr_t)src % 16 || (uintptr_t)q % 16 ||
        (uintptr_t)qs % 8 || (uint64_t)rows * (cols / 32) >= (1ull << 32))
        return K3X_ERR_INVALID_EXTENT;
    const uint32_t n = rows * (cols / 32);
    hipLaunchKernelGGL(q8_rows_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, src, rows,
                       cols, stride, q, qs, ctx->status);
    ctx->kernel_launches += 1;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

}  // namespace k3x_hip
