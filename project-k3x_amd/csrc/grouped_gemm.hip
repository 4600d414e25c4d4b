// grouped_gemm.hip -- the wide expert GEMM: experts with many rows (prefill
// chunks, verification windows) on bf16 MFMA, MXFP4 weights dequantised in
// registers.
//
// Workgroup = 4 or 8 waves, one 128-row chunk of one expert's rows (a work item
// listed by the grouping, so large experts spread over many workgroups) x
// NT 16-row output blocks per wave (gate/up: NT pairs of 16 gate + 16 up
// rows).  Per K tile (128 K):
//   * the chunk's activation rows (gathered through pair_token for the
//     routed gate/up) are staged in LDS, double-buffered, rows padded to
//     272 B so the MFMA operand reads of 16 lanes hit 16 different banks;
//   * each wave dequantises its weight fragments once (v_cvt_scalef32_pk_
//     bf16_fp4 per code byte) and feeds each to the MFMAs of all eight
//     16-row tiles of the chunk (tiles past the chunk's rows are skipped);
//   * weights are prefetched DEPTH tiles ahead in registers, activations one
//     tile ahead; every load is unconditional (indices clamped) so the
//     compiler's in-order vector-memory waits never wait on later tiles.
// The weights of an expert are read once per 128-row chunk.  The N blocks of
// one expert are numbered to land on one XCD, so its activation rows are
// fetched into that XCD's L2 once.
// Epilogues: GLU -> bf16 act (gate/up), fp32 rows scattered to the pair's
// (token, slot) row (routed down) or the token row (shared down).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "k3x_gemm.hpp"

using namespace k3x_dev;
using k3x_hip::kWideRows;
using k3x_hip::WideGemmArgs;

namespace {

constexpr int kMTiles = kWideRows / 16;  // MFMA row tiles per chunk
constexpr int kPitch = 128 + 8;          // LDS row pitch, bf16 elements

__device__ inline uint32_t prior_status(const uint32_t* status) { return *status; }
__device__ inline uint32_t wave_index() {
    return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// OCC: minimum workgroups per CU the registers must allow (OCC * WAVES / 4
// waves per SIMD: two waves per SIMD keep one wave's loads in flight while
// the other multiplies); the 8 x NT x S accumulators are independent MFMA
// chains.
template <bool FP4, bool GATEUP, int WAVES, int NT, int DEPTH, int OCC>
__global__ __launch_bounds__(64 * WAVES, OCC) void wide_gemm(WideGemmArgs a) {
    constexpr int kThreads = 64 * WAVES;
    constexpr int kARowStep = kThreads / 16;            // 16 threads per 128-column row
    constexpr int kALoads = kWideRows / kARowStep;      // 16-byte activation loads per thread per tile
    __shared__ u32x4 s_a4[2][kWideRows * kPitch / 8];
    constexpr int S = GATEUP ? 2 : 1;  // matrices per output row block (gate, up)
    constexpr int U = FP4 ? 1 : 4;     // 16-byte words per lane per tile
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const uint32_t g = lane >> 4, n = lane & 15;
    // One workgroup per (work item, output block set) on a 1-D grid.
    // Consecutive workgroups go to the eight XCDs in turn; renumber so that
    // each XCD takes a contiguous range of logical blocks (the blocks of one
    // item share an L2).
    const uint32_t nb = gridDim.x, xcd = blockIdx.x % 8, per = nb / 8, rem = nb % 8;
    const uint32_t lb = xcd * per + min(xcd, rem) + blockIdx.x / 8;
    const uint32_t nblk = a.nrb / (WAVES * NT);
    const uint32_t item = lb / nblk, jb = lb % nblk;
    if (prior_status(a.status)) return;
    uint32_t e = 0, cnt = a.tokens, off = 0, m0 = item * kWideRows;
    if (a.items) {
        if (item >= *a.n_items) return;
        const uint32_t it = a.items[item];
        e = it >> 16;
        m0 = (it & 0xffffu) * kWideRows;
        cnt = a.counts[e];
        off = a.offsets[e];
    }
    if (m0 >= cnt) return;
    const uint32_t kt = a.kt;
    const uint32_t rb0 = (jb * WAVES + wave) * NT;
    const u32x4* codes = reinterpret_cast<const u32x4*>(a.codes + e * a.codes_per_expert) + lane;
    const uint32_t* scales = FP4 ? a.scales + e * a.scales_per_expert + lane : nullptr;

    // Weight stages: codes bc[d][nt][w][u] and scale dwords bs[d][nt][w] of
    // K tile k for stage d = k % DEPTH.  Plain arrays indexed only inside
    // fully unrolled loops, so they live in registers.
#define WIDE_LOAD_B(d, k)                                                                    \
    _Pragma("unroll") for (int nt = 0; nt < NT; ++nt)                                      \
        _Pragma("unroll") for (int w = 0; w < S; ++w) {                                    \
            const size_t base_ = (((size_t)(rb0 + nt) * kt + (k)) * S + w) * U * 64;       \
            _Pragma("unroll") for (int u = 0; u < U; ++u) bc[d][nt][w][u] =                \
                codes[base_ + u * 64];                                                       \
            if constexpr (FP4)                                                               \
                bs[d][nt][w] = scales[(((size_t)(rb0 + nt) * a.ks + (k) / 4) * S + w) * 64]; \
        }
#define WIDE_LOAD_A(k)                                                                       \
    _Pragma("unroll") for (int i = 0; i < kALoads; ++i) av[i] =                            \
        *reinterpret_cast<const u32x4*>(a.a + asrc[i] + (size_t)(k) * 128);
#define WIDE_STORE_A(buf)                                                                    \
    _Pragma("unroll") for (int i = 0; i < kALoads; ++i)                                    \
        s_a4[buf][((arow + kARowStep * i) * kPitch + acol) / 8] = av[i];

    // This thread's activation chunks: rows arow + kARowStep i, columns acol..+7.
    const uint32_t arow = tid / 16, acol = (tid % 16) * 8;
    {
        const uint32_t rows = min(cnt - m0, kWideRows);
        uint32_t asrc[kALoads];
#pragma unroll
        for (int i = 0; i < kALoads; ++i) {
            const uint32_t r = m0 + min(arow + kARowStep * i, rows - 1);  // clamped: valid row
            const uint32_t src = a.gather ? a.pair_token[off + r] : off + r;
            asrc[i] = src * a.a_stride + acol;
        }
        f32x4 acc[kMTiles][NT][S];
#pragma unroll
        for (int mt = 0; mt < kMTiles; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int w = 0; w < S; ++w) acc[mt][nt][w] = f32x4{0.f, 0.f, 0.f, 0.f};

        u32x4 bc[DEPTH][NT][S][U];
        uint32_t bs[DEPTH][NT][S];
        u32x4 av[kALoads];
        WIDE_LOAD_A(0)
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            WIDE_LOAD_B(d, min((uint32_t)d, kt - 1))
        }
        WIDE_STORE_A(0)
        WIDE_LOAD_A(min(1u, kt - 1))
        __syncthreads();

        // kt is a multiple of DEPTH (checked on the host): no branch in the
        // loop body.  Step k: stage tile k + 1 (loaded during step k - 1)
        // into the other LDS buffer, request tile k + 2, multiply tile k,
        // refill this weight stage with tile k + DEPTH.
        for (uint32_t kb = 0; kb < kt; kb += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                const uint32_t k = kb + d;
                WIDE_STORE_A((k + 1) & 1)  // at the last step: a copy of the last tile, unused
                WIDE_LOAD_A(min(k + 2, kt - 1))
                const uint16_t* sa =
                    reinterpret_cast<const uint16_t*>(s_a4[k & 1]) + n * kPitch + 32 * g;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bf16x8 bw[NT][S];
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                        for (int w = 0; w < S; ++w) {
                            if constexpr (FP4) {
                                const uint32_t word = bc[d][nt][w][0][j];
                                bw[nt][w] = dequant8(
                                    word, e8m0_to_f32((bs[d][nt][w] >> (8 * (k & 3))) & 0xffu));
                            } else {
                                bw[nt][w] = as_bf16x8(bc[d][nt][w][j]);
                            }
                        }
#pragma unroll
                    for (int mt = 0; mt < kMTiles; ++mt) {
                        if ((uint32_t)(16 * mt) < rows) {  // workgroup-uniform
                            const bf16x8 af =
                                *reinterpret_cast<const bf16x8*>(sa + 16 * mt * kPitch + 8 * j);
#pragma unroll
                            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                                for (int w = 0; w < S; ++w)
                                    acc[mt][nt][w] = mfma16x16x32(af, bw[nt][w], acc[mt][nt][w]);
                        }
                    }
                }
                WIDE_LOAD_B(d, min(k + DEPTH, kt - 1))
                __syncthreads();
            }
        }

#pragma unroll
        for (int mt = 0; mt < kMTiles; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t row = 16 * mt + 4 * g + i;
                    if (row >= rows) continue;
                    const uint32_t col = (rb0 + nt) * 16 + n;
                    const uint32_t r = off + m0 + row;
                    if constexpr (GATEUP) {
                        const float v = glu(acc[mt][nt][0][i], acc[mt][nt][1][i], a.glu);
                        a.act[(size_t)r * a.act_stride + col] = f32_to_bf16(v);
                    } else {
                        const size_t yrow = a.scatter ? (size_t)a.pair_token[r] * a.top_k + a.pair_slot[r]
                                                      : (size_t)r;
                        a.y[yrow * a.y_stride + col] = acc[mt][nt][0][i];
                    }
                }
    }
}

#undef WIDE_LOAD_B
#undef WIDE_LOAD_A
#undef WIDE_STORE_A

// Waves per workgroup and output 16-row blocks per wave (WAVES * NT per
// workgroup): the more output rows a workgroup covers, the fewer times the
// chunk's activation rows are streamed from L2.
constexpr int kWavesRouted = 8, kWavesShared = 4;
constexpr int kNtRoutedGateUp = 2, kNtRoutedDown = 4, kNtSharedGateUp = 1, kNtSharedDown = 2;
constexpr int kDepth = 2;

}  // namespace

namespace k3x_hip {

uint32_t wide_rb_per_block(WideKind kind) {
    switch (kind) {
        case kWideRoutedGateUp: return kWavesRouted * kNtRoutedGateUp;
        case kWideRoutedDown: return kWavesRouted * kNtRoutedDown;
        case kWideSharedGateUp: return kWavesShared * kNtSharedGateUp;
        default: return kWavesShared * kNtSharedDown;
    }
}

int launch_wide_gemm(k3x_hip_ctx* ctx, WideKind kind, const WideGemmArgs& a, uint32_t max_items) {
    const uint32_t per = wide_rb_per_block(kind);
    if (a.nrb % per || a.kt % kDepth || !max_items) return K3X_ERR_INVALID_EXTENT;
    const dim3 grid(max_items * (a.nrb / per));
    switch (kind) {
        case kWideRoutedGateUp:
            hipLaunchKernelGGL((wide_gemm<true, true, kWavesRouted, kNtRoutedGateUp, kDepth, 1>),
                               grid, dim3(64 * kWavesRouted), 0, ctx->stream, a);
            break;
        case kWideRoutedDown:
            hipLaunchKernelGGL((wide_gemm<true, false, kWavesRouted, kNtRoutedDown, kDepth, 1>),
                               grid, dim3(64 * kWavesRouted), 0, ctx->stream, a);
            break;
        case kWideSharedGateUp:
            hipLaunchKernelGGL((wide_gemm<false, true, kWavesShared, kNtSharedGateUp, kDepth, 2>),
                               grid, dim3(64 * kWavesShared), 0, ctx->stream, a);
            break;
        default:
            hipLaunchKernelGGL((wide_gemm<false, false, kWavesShared, kNtSharedDown, kDepth, 2>),
                               grid, dim3(64 * kWavesShared), 0, ctx->stream, a);
            break;
    }
    ctx->kernel_launches += 1;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

}  // namespace k3x_hip
