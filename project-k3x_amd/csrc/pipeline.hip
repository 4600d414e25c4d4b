// pipeline.hip -- the MoE-layer kernels and the forward entry points.
//
//   rmsnorm_kernel   x -> xn = bf16(x * inv_rms * gamma)      (canonical fp64 sum)
//   router_kernel    logits = W_r xn in fp64, canonical order  (bit-exact ids)
//   topk_kernel      sigmoid + bias, natural Top-K, renorm * routed_scale
//   group_kernel     expert-major CSR + first-use order         (bit-exact)
//   expert_gemm      MXFP4/bf16 weights x bf16 activations on MFMA; gate/up
//                    variant fuses the GLU, down variant scatters per pair
//                    (few rows per expert; many rows: grouped_gemm.hip)
//   combine_kernel   slot-ordered weighted sum + shared expert, bf16 cast
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "k3x_decode.hpp"
#include "k3x_device.hpp"
#include "k3x_gemm.hpp"
#include "k3x_internal.hpp"

using namespace k3x_dev;

namespace {

__device__ inline void latch(uint32_t* status, uint32_t code) { atomicCAS(status, 0u, code); }

// Canonical fp64 block reduction over 256 threads: xor butterfly inside each
// wave (pairwise tree of 64), then (w0 + w1) + (w2 + w3).  Every thread gets
// the result.
__device__ inline double block_tree_sum(double v, double* red) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    const double r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------------------
// RMSNorm: one block of 256 threads per token.  runtime/src/ops.cpp:10-18
// with the canonical order for the sum of squares and the bf16 rounding of
// the normalised activation.
// ---------------------------------------------------------------------------
constexpr uint32_t kNormRegHidden = 8192;  // rows up to this stay in registers

// Tile- and residue-major copy for router_mfma_kernel of token t's row held
// as b[j] = x[tid + 256 j] (bf16 bits, 0 past the row): j = 4m + q goes to
// slot 8q + m of the token's 32 terms of residue tid in its 16-token tile.
__device__ inline void store_xp(uint16_t* xp, uint32_t t, uint32_t tid, const uint32_t (&b)[32]) {
    u32x4* dst = reinterpret_cast<u32x4*>(xp + ((size_t)(t / 16) * 256 + tid) * (16 * 32) +
                                          (t % 16) * 32);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int s0 = 8 * c + 2 * h, s1 = s0 + 1;  // slots -> j = 4m + q
            w[h] = b[4 * (s0 % 8) + s0 / 8] | b[4 * (s1 % 8) + s1 / 8] << 16;
        }
        dst[c] = u32x4{w[0], w[1], w[2], w[3]};
    }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const float* __restrict__ gamma,
                                                      uint32_t H, float eps,
                                                      uint16_t* __restrict__ xn,
                                                      uint16_t* __restrict__ xp,
                                                      uint32_t* status) {
    __shared__ double red[4];
    if (*(volatile uint32_t*)status) return;
    const uint16_t* xr = x + (size_t)blockIdx.x * H;
    uint16_t* out = xn + (size_t)blockIdx.x * H;
    const uint32_t tid = threadIdx.x;
    if (H > kNormRegHidden) {
        double s = 0.0;
        int bad = 0;
        for (uint32_t k = tid; k < H; k += 256) {
            const float v = bf16_to_f32(xr[k]);
            bad |= !__builtin_isfinite(v);
            s = __builtin_fma((double)v, (double)v, s);  // exact product: fused == separate
        }
        if (__syncthreads_or(bad)) {
            if (tid == 0) latch(status, K3X_ERR_INVALID_MXFP4);
            return;
        }
        s = block_tree_sum(s, red);
        const float mean = (float)__ddiv_rn(s, (double)H);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
        for (uint32_t k = tid; k < H; k += 256)
            out[k] = f32_to_bf16(__fmul_rn(__fmul_rn(bf16_to_f32(xr[k]), inv), gamma[k]));
        return;
    }
    // The whole row in registers: this thread's k = tid + 256 j, j < 32.
    // Loads past the row read 0 (buffer range check), and the +0 terms they
    // add after the row's last term leave the sum of squares unchanged.  The
    // gamma loads go out with the row's, ahead of the reduction.
    const __amdgpu_buffer_rsrc_t xs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(xr), (short)0, H * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t gs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(gamma), (short)0, H * 4, 0x00020000);
    uint16_t xb[32];
    float gv[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) xb[j] = __builtin_amdgcn_raw_buffer_load_b16(xs, tid * 2, j * 512, 0);
#pragma unroll
    for (int j = 0; j < 32; ++j)
        gv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(gs, tid * 4, j * 1024, 0));
    double s = 0.0;
    int bad = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float v = bf16_to_f32(xb[j]);
        bad |= !__builtin_isfinite(v);
        s = __builtin_fma((double)v, (double)v, s);
    }
    if (__syncthreads_or(bad)) {
        if (tid == 0) latch(status, K3X_ERR_INVALID_MXFP4);
        return;
    }
    s = block_tree_sum(s, red);
    const float mean = (float)__ddiv_rn(s, (double)H);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    uint32_t b[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) b[j] = f32_to_bf16(__fmul_rn(__fmul_rn(bf16_to_f32(xb[j]), inv), gv[j]));
#pragma unroll
    for (int j = 0; j < 32; ++j)
        if (tid + 256u * j < H) out[tid + 256 * j] = (uint16_t)b[j];
    if (xp) store_xp(xp, blockIdx.x, tid, b);
}

// The residue-major copy of a bf16 row [H <= 8192] for router_mfma_kernel,
// one 256-thread block per token (inputs the router did not normalise).
__global__ __launch_bounds__(256) void xp_pack_kernel(const uint16_t* __restrict__ x, uint32_t H,
                                                      uint16_t* __restrict__ xp) {
    const __amdgpu_buffer_rsrc_t xs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(x + (size_t)blockIdx.x * H), (short)0, H * 2, 0x00020000);
    uint32_t b[32];
#pragma unroll
    for (int j = 0; j < 32; ++j)
        b[j] = __builtin_amdgcn_raw_buffer_load_b16(xs, threadIdx.x * 2, j * 512, 0);
    store_xp(xp, blockIdx.x, threadIdx.x, b);
}

// ---------------------------------------------------------------------------
// Router logits in fp64, canonical order: thread i accumulates k = i, i+256,
// ... sequentially, then block_tree_sum.  EPB experts x TPB tokens per block.
// Logit semantics: runtime/src/model.cpp:919-921 / backend_cpu.cpp:33-41.
// ---------------------------------------------------------------------------
template <int EPB, int TPB>
__global__ __launch_bounds__(256) void router_kernel(const float* __restrict__ W,
                                                     const uint16_t* __restrict__ xn,
                                                     uint32_t E, uint32_t H, uint32_t T,
                                                     float* __restrict__ logits,
                                                     const uint32_t* status) {
    __shared__ double red[4][EPB * TPB];
    if (*(volatile const uint32_t*)status) return;
    const uint32_t e0 = blockIdx.x * EPB, t0 = blockIdx.y * TPB;
    double acc[EPB][TPB];
#pragma unroll
    for (int a = 0; a < EPB; ++a)
#pragma unroll
        for (int b = 0; b < TPB; ++b) acc[a][b] = 0.0;
    for (uint32_t k = threadIdx.x; k < H; k += 256) {
        float w[EPB], xv[TPB];
#pragma unroll
        for (int a = 0; a < EPB; ++a) w[a] = e0 + a < E ? W[(size_t)(e0 + a) * H + k] : 0.0f;
#pragma unroll
        for (int b = 0; b < TPB; ++b)
            xv[b] = t0 + b < T ? bf16_to_f32(xn[(size_t)(t0 + b) * H + k]) : 0.0f;
#pragma unroll
        for (int a = 0; a < EPB; ++a)
#pragma unroll
            for (int b = 0; b < TPB; ++b)
                acc[a][b] = __builtin_fma((double)w[a], (double)xv[b], acc[a][b]);
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int a = 0; a < EPB; ++a)
#pragma unroll
        for (int b = 0; b < TPB; ++b) {
            double v = acc[a][b];
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
            if (lane == 0) red[wave][a * TPB + b] = v;
        }
    __syncthreads();
    if (threadIdx.x < EPB * TPB) {
        const int i = threadIdx.x, a = i / TPB, b = i % TPB;
        if (e0 + a < E && t0 + b < T)
            logits[(size_t)(t0 + b) * E + e0 + a] =
                (float)((red[0][i] + red[1][i]) + (red[2][i] + red[3][i]));
    }
}

// The same logits for H <= 8192 and T <= TPB with every load a thread needs
// -- its 32 residue terms of EPB expert rows and of the TPB token rows --
// issued before the first multiply-add (the loop above waits on each step's
// loads in turn).  Buffer loads: rows and terms past the ends read 0, and
// their +0 terms come after the last real one, leaving each partial
// unchanged (a partial started at +0 is never -0).
// Experts [blk * EPB, blk * EPB + EPB) by a workgroup of 256 threads.  The
// router rows are read once a call: non-temporal loads (the official layer at
// T=2: 198.8-199.3 -> 193.8-197.0 us).
constexpr int kLoadNonTemporal = 2;  // buffer load cache policy: nt
template <int EPB, int TPB>
__device__ __forceinline__ void router_reg_body(const float* __restrict__ W,
                                                const uint16_t* __restrict__ xn, uint32_t E,
                                                uint32_t H, uint32_t T,
                                                float* __restrict__ logits,
                                                const uint32_t* status, uint32_t blk) {
    __shared__ double red[4][EPB * TPB];
    if (*(volatile const uint32_t*)status) return;
    const uint32_t tid = threadIdx.x, e0 = blk * EPB;
    float w[EPB][32];
    uint32_t xb[TPB][32];
#pragma unroll
    for (int a = 0; a < EPB; ++a) {
        const uint32_t e = min(e0 + a, E - 1);
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(W + (size_t)e * H), (short)0, e0 + a < E ? H * 4 : 0, 0x00020000);
#pragma unroll
        for (int j = 0; j < 32; ++j)
            w[a][j] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(r, tid * 4, j * 1024, kLoadNonTemporal));
    }
#pragma unroll
    for (int b = 0; b < TPB; ++b) {
        const uint32_t t = min((uint32_t)b, T - 1);
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(xn + (size_t)t * H), (short)0, (uint32_t)b < T ? H * 2 : 0,
            0x00020000);
#pragma unroll
        for (int j = 0; j < 32; ++j)
            xb[b][j] = __builtin_amdgcn_raw_buffer_load_b16(r, tid * 2, j * 512, 0);
    }
    double acc[EPB][TPB];
#pragma unroll
    for (int a = 0; a < EPB; ++a)
#pragma unroll
        for (int b = 0; b < TPB; ++b) acc[a][b] = 0.0;
#pragma unroll
    for (int j = 0; j < 32; ++j)
#pragma unroll
        for (int a = 0; a < EPB; ++a)
#pragma unroll
            for (int b = 0; b < TPB; ++b)
                acc[a][b] = __builtin_fma((double)w[a][j], (double)bf16_to_f32((uint16_t)xb[b][j]),
                                          acc[a][b]);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int a = 0; a < EPB; ++a)
#pragma unroll
        for (int b = 0; b < TPB; ++b) {
            double v = acc[a][b];
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
            if (lane == 0) red[wave][a * TPB + b] = v;
        }
    __syncthreads();
    if (threadIdx.x < EPB * TPB) {
        const int i = threadIdx.x, a = i / TPB, b = i % TPB;
        if (e0 + a < E && (uint32_t)b < T)
            logits[(size_t)b * E + e0 + a] =
                (float)((red[0][i] + red[1][i]) + (red[2][i] + red[3][i]));
    }
}

template <int EPB, int TPB>
__global__ __launch_bounds__(256) void router_reg_kernel(const float* __restrict__ W,
                                                         const uint16_t* __restrict__ xn,
                                                         uint32_t E, uint32_t H, uint32_t T,
                                                         float* __restrict__ logits,
                                                         const uint32_t* status) {
    router_reg_body<EPB, TPB>(W, xn, E, H, T, logits, status, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Router logits for many tokens: the same fp64 canonical order as
// router_kernel (thread i sums k = i, i + 256, ... in sequence; then the
// balanced pairwise tree over the 256 thread partials in thread order), for
// an EPB x TPB (expert x token) tile per block of 256 threads.
//   * W and xn rows are clamped to valid rows, so every load is issued
//     unconditionally and the in-order vector-memory counter lets DEPTH
//     k-steps of loads stay in flight behind the multiply-adds.
//   * The 64 per-thread partials are reduced across the wave by halving
//     exchanges: at the step over lane bit m, each lane keeps half of its
//     outputs and adds the partner lane's copy of them.  Addition is
//     commutative, so each sum is bit-identical to the xor butterfly's and the
//     wave's lane L ends with output bitrev6(L).
// Products fp32 x bf16 are exact in fp64 (24 + 8 significand bits), so the
// fused multiply-add rounds exactly as the separate multiply and add do.
// ---------------------------------------------------------------------------
template <int EPB, int TPB, int DEPTH>
__global__ __launch_bounds__(256) void router_tile_kernel(const float* __restrict__ W,
                                                          const uint16_t* __restrict__ xn,
                                                          uint32_t E, uint32_t H, uint32_t T,
                                                          float* __restrict__ logits,
                                                          const uint32_t* status) {
    static_assert(EPB * TPB == 64, "one output per lane after the wave reduction");
    __shared__ double red[4][64];
    if (*(volatile const uint32_t*)status) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t e0 = blockIdx.x * EPB, t0 = blockIdx.y * TPB;
    const uint32_t nj = H / 256;  // k-steps every thread takes
    const float* wrow[EPB];
    const uint16_t* xrow[TPB];
#pragma unroll
    for (int a = 0; a < EPB; ++a) wrow[a] = W + (size_t)min(e0 + a, E - 1) * H + tid;
#pragma unroll
    for (int b = 0; b < TPB; ++b) xrow[b] = xn + (size_t)min(t0 + b, T - 1) * H + tid;
    double acc[EPB][TPB];
#pragma unroll
    for (int a = 0; a < EPB; ++a)
#pragma unroll
        for (int b = 0; b < TPB; ++b) acc[a][b] = 0.0;
    auto step = [&](const float* wv, const uint16_t* xv) {
        double wd[EPB], xd[TPB];
#pragma unroll
        for (int a = 0; a < EPB; ++a) wd[a] = (double)wv[a];
#pragma unroll
        for (int b = 0; b < TPB; ++b) xd[b] = (double)bf16_to_f32(xv[b]);
#pragma unroll
        for (int a = 0; a < EPB; ++a)
#pragma unroll
            for (int b = 0; b < TPB; ++b) acc[a][b] = __builtin_fma(wd[a], xd[b], acc[a][b]);
    };
    if (nj) {
        float wv[DEPTH][EPB];
        uint16_t xv[DEPTH][TPB];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const uint32_t j = min((uint32_t)d, nj - 1) * 256;
#pragma unroll
            for (int a = 0; a < EPB; ++a) wv[d][a] = wrow[a][j];
#pragma unroll
            for (int b = 0; b < TPB; ++b) xv[d][b] = xrow[b][j];
        }
        for (uint32_t jb = 0; jb < nj; jb += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                if (jb + d < nj) step(wv[d], xv[d]);  // block-uniform
                const uint32_t j = min(jb + d + DEPTH, nj - 1) * 256;
#pragma unroll
                for (int a = 0; a < EPB; ++a) wv[d][a] = wrow[a][j];
#pragma unroll
                for (int b = 0; b < TPB; ++b) xv[d][b] = xrow[b][j];
            }
        }
    }
    if (tid < H % 256) {  // the last, partial k-step
        float wv[EPB];
        uint16_t xv[TPB];
#pragma unroll
        for (int a = 0; a < EPB; ++a) wv[a] = wrow[a][nj * 256];
#pragma unroll
        for (int b = 0; b < TPB; ++b) xv[b] = xrow[b][nj * 256];
        step(wv, xv);
    }
    // Output o = b * EPB + a (consecutive experts of one token adjacent).
    double v[64];
#pragma unroll
    for (int a = 0; a < EPB; ++a)
#pragma unroll
        for (int b = 0; b < TPB; ++b) v[b * EPB + a] = acc[a][b];
#pragma unroll
    for (int m = 1, cnt = 64; m < 64; m <<= 1, cnt >>= 1) {
        const bool upper = lane & m;
#pragma unroll
        for (int i = 0; i < cnt / 2; ++i) {
            const double keep = upper ? v[cnt / 2 + i] : v[i];
            const double send = upper ? v[i] : v[cnt / 2 + i];
            v[i] = keep + __shfl_xor(send, m);
        }
    }
    const uint32_t o = __builtin_bitreverse32(lane) >> 26;
    red[wave][o] = v[0];
    __syncthreads();
    if (tid < 64) {
        const uint32_t a = tid % EPB, b = tid / EPB;
        if (e0 + a < E && t0 + b < T)
            logits[(size_t)(t0 + b) * E + e0 + a] =
                (float)((red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]));
    }
}

constexpr int kRouterEpb = 8, kRouterTpb = 8;  // router_tile_kernel tile for T > 4

// ---------------------------------------------------------------------------
// Router logits on the fp64 matrix cores.
//
// Tile- and residue-major operands: for residue i (k = i + 256 j), j = 4m + q
// and 16-row tiles (e = 16 et + n, t = 16 tt + n),
//   Wp[et][i][n][q][m] = W[e][k]   fp32, m < 8 (k >= H and e >= E padded with 0)
//   xp[tt][i][n][q][m] = xn[t][k]  bf16
// so lane l of a wave (row n = l % 16, q = l / 16) reads the 8 terms m of its
// (n, q) with one 32-byte (W) / 16-byte (x) load per residue, and one
// residue of a tile is a contiguous 2 KiB (W) / 1 KiB (x): consecutive
// residues, and the waves working on them, spread over the L2 channels.
//
// v_mfma_f64_16x16x4f64 computes D(e, t) = C(e, t) + sum_q A(e, q) B(q, t) as
// the sequential chain of fused multiply-adds q = 0, 1, 2, 3, so chaining the
// NM matrix ops m = 0 .. NM-1 from C = +0 visits j = 4m + q in order: exactly
// the sequential per-residue sum of router_tile_kernel.  A padded term adds
// 0 * 0 = +0 to a partial that is never -0 (it starts at +0 and a sum that
// cancels rounds to +0), so it changes nothing.  Products fp32 x bf16 are
// exact in fp64.  The 256 residue partials then meet in the same balanced
// pairwise tree over i: each wave folds its R = 256 / WPB consecutive residues
// with a binary carry stack (pairs (2a, 2a+1), then pairs of pairs, ...), and
// the block joins the WPB wave subtrees in tree order through LDS.
// One block per 16-expert x 16-token tile; D(e, t) lands in lane
// 16 (e % 4) + t, register e / 4.
// ---------------------------------------------------------------------------
constexpr int kRouterRes = 256;     // residues of k
constexpr int kRouterSlot = 32;     // padded terms per residue (4 q x 8 m)
constexpr uint32_t kRouterMaxHidden = kRouterRes * kRouterSlot;
constexpr uint32_t kRouterTileRes = 16 * kRouterSlot;  // elements of one tile residue
constexpr int kRouterWaves = 4;     // waves per block of router_mfma_kernel
constexpr int kRouterChains = 2;    // residues per wave in flight on the matrix core
constexpr uint32_t kRouterMfmaMinTokens = 256;

__global__ __launch_bounds__(256) void permute_router_kernel(const float* __restrict__ W,
                                                             uint32_t E, uint32_t H,
                                                             float* __restrict__ Wp) {
    const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t et = (uint32_t)(o / (kRouterRes * kRouterTileRes));
    if (et >= (E + 15) / 16) return;
    const uint32_t r = (uint32_t)(o % (kRouterRes * kRouterTileRes));
    const uint32_t i = r / kRouterTileRes, n = (r / kRouterSlot) % 16;
    const uint32_t q = (r / 8) % 4, m = r % 8;
    const uint32_t e = 16 * et + n, k = i + kRouterRes * (4 * m + q);
    Wp[o] = e < E && k < H ? W[(size_t)e * H + k] : 0.0f;
}

typedef __attribute__((ext_vector_type(4))) double f64x4;

template <int NM, int WPB>
__global__ __launch_bounds__(64 * WPB) void router_mfma_kernel(const float* __restrict__ Wp,
                                                               const uint16_t* __restrict__ xp,
                                                               uint32_t E, uint32_t T,
                                                               float* __restrict__ logits,
                                                               const uint32_t* status) {
    constexpr int R = kRouterRes / WPB;  // residues per wave
    constexpr int G = R / 16;            // groups of 16 residues per wave
    constexpr int LG = G == 1 ? 0 : G == 2 ? 1 : G == 4 ? 2 : G == 8 ? 3 : 4;
    constexpr int C = kRouterChains;     // residues whose chains run interleaved
    constexpr int LC = C == 1 ? 0 : C == 2 ? 1 : 2;
    constexpr int D = 2 * C > 4 ? 2 * C : 4;  // residues of loads in flight
    static_assert(NM >= 1 && NM <= 8 && (1 << LG) == G && R % 16 == 0, "tile shape");
    static_assert((1 << LC) == C && D % C == 0 && 16 % D == 0, "chains");
    __shared__ f64x4 red[WPB > 1 ? WPB - 1 : 1][64];
    if (*(volatile const uint32_t*)status) return;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar offsets
    const uint32_t e0 = blockIdx.x * 16, t0 = blockIdx.y * 16;
    const uint32_t row = lane % 16, q = lane / 16;
    // Per-block resources over this block's two tiles.  Rows past E read
    // the zero padding, rows past T whatever the padded scratch holds: either
    // only reaches outputs that are not stored.
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(Wp + (size_t)blockIdx.x * kRouterRes * kRouterTileRes), (short)0,
        kRouterRes * kRouterTileRes * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(xp + (size_t)blockIdx.y * kRouterRes * kRouterTileRes), (short)0,
        kRouterRes * kRouterTileRes * 2, 0x00020000);
    const uint32_t wv = row * (kRouterSlot * 4) + q * 32;
    const uint32_t xv = row * (kRouterSlot * 2) + q * 16;
    const uint32_t i0 = wave * R;
    u32x4 wa[D], wb[D], xa[D];
    auto load = [&](int slot, uint32_t i) {
        wa[slot] = __builtin_amdgcn_raw_buffer_load_b128(wr, wv, i * (kRouterTileRes * 4), 0);
        wb[slot] = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + 16, i * (kRouterTileRes * 4), 0);
        xa[slot] = __builtin_amdgcn_raw_buffer_load_b128(xr, xv, i * (kRouterTileRes * 2), 0);
    };
    auto wterm = [&](int slot, int m) {
        return (double)__uint_as_float(m < 4 ? wa[slot][m] : wb[slot][m - 4]);
    };
    auto xterm = [&](int slot, int m) {
        const uint32_t xw = xa[slot][m / 2];
        return (double)__uint_as_float(m % 2 ? xw & 0xffff0000u : xw << 16);
    };
    // Partials of C consecutive residues, their matrix-op chains interleaved.
    auto partials = [&](int r0, f64x4* p) {
#pragma unroll
        for (int c = 0; c < C; ++c) p[c] = f64x4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int c = 0; c < C; ++c)
                p[c] = __builtin_amdgcn_mfma_f64_16x16x4f64(wterm((r0 + c) % D, m),
                                                            xterm((r0 + c) % D, m), p[c], 0, 0, 0);
    };
#pragma unroll
    for (int d = 0; d < D; ++d) load(d, i0 + d);
    f64x4 so[LG > 0 ? LG : 1];
    f64x4 v;
    for (int g = 0; g < G; ++g) {
        f64x4 st[4];
#pragma unroll
        for (int r = 0; r < 16; r += C) {
            f64x4 p[C];
            partials(r, p);
            // Scheduling fences keep the refill of these slots D residues
            // ahead of its use (the scheduler would otherwise sink it).
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < C; ++c) load((r + c) % D, min(i0 + 16 * g + r + c + D, i0 + R - 1));
            __builtin_amdgcn_sched_barrier(0);
            // Residues r .. r+C-1 (r a multiple of C) form a subtree; fold it,
            // then carry it into the levels above.
#pragma unroll
            for (int w = 1; w < C; w *= 2)
#pragma unroll
                for (int c = 0; c < C; c += 2 * w) p[c] = p[c] + p[c + w];
            v = p[0];
#pragma unroll
            for (int L = LC; L < 4; ++L) {
                if (!((r >> L) & 1)) {
                    st[L] = v;
                    break;
                }
                v = st[L] + v;
            }
        }
        // v: the subtree of group g; carry it into the levels above.
#pragma unroll
        for (int L = 0; L < LG; ++L) {
            if (!((g >> L) & 1)) {
                so[L] = v;
                break;
            }
            v = so[L] + v;
        }
    }
    // v: this wave's subtree of R residues.
    if (wave) red[wave - 1][lane] = v;
    __syncthreads();
    if (wave) return;
    if constexpr (WPB == 2) {
        v = v + red[0][lane];
    } else if constexpr (WPB == 4) {
        v = (v + red[0][lane]) + (red[1][lane] + red[2][lane]);
    } else if constexpr (WPB == 8) {
        v = ((v + red[0][lane]) + (red[1][lane] + red[2][lane])) +
            ((red[3][lane] + red[4][lane]) + (red[5][lane] + red[6][lane]));
    }
    const uint32_t t = t0 + row;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t e = e0 + 4 * r + q;
        if (e < E && t < T) logits[(size_t)t * E + e] = (float)v[r];
    }
}

// ---------------------------------------------------------------------------
// Top-K: one wave per token.  Scores, validation and renormalisation follow
// runtime/src/routing_policy.cpp:40-95,146-157 (FLOAT) or
// runtime/src/official_moe.cpp:214-242 (DOUBLE); contributions are then
// multiplied by routed_scale (runtime/src/model.cpp:1004-1009).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void topk_kernel(const float* __restrict__ logits,
                                                  const float* __restrict__ bias, uint32_t E,
                                                  uint32_t K, float routed_scale,
                                                  uint32_t renorm, uint32_t* __restrict__ ids,
                                                  float* __restrict__ weights,
                                                  uint32_t* status) {
    extern __shared__ uint64_t keys[];  // [E] keys then [E] scores
    float* sc = reinterpret_cast<float*>(keys + E);
    __shared__ uint32_t sel[64];
    __shared__ float selsc[64];
    if (*(volatile uint32_t*)status) return;
    const uint32_t t = blockIdx.x, lane = threadIdx.x;
    uint32_t bad = 0;
    for (uint32_t e = lane; e < E; e += 64) {
        const float lg = logits[(size_t)t * E + e];
        const float b = bias[e];
        if (renorm == K3X_RENORM_DOUBLE && (!__builtin_isfinite(lg) || !__builtin_isfinite(b)))
            bad = K3X_ERR_INVALID_EXTENT;
        const float s = sigmoid_cr(lg);
        const float adj = __fadd_rn(s, b);
        if (renorm == K3X_RENORM_FLOAT &&
            (!__builtin_isfinite(s) || s < 0.0f || s > 1.0f || !__builtin_isfinite(b) ||
             !__builtin_isfinite(adj)))
            bad = K3X_ERR_INVALID_STATE;
        sc[e] = s;
        keys[e] = topk_key(adj, e);
    }
    for (int d = 1; d < 64; d <<= 1) bad = max(bad, (uint32_t)__shfl_xor((int)bad, d));
    if (bad) {
        if (lane == 0) latch(status, bad);
        return;
    }
    __syncthreads();
    for (uint32_t slot = 0; slot < K; ++slot) {
        uint64_t best = 0;
        for (uint32_t e = lane; e < E; e += 64) best = max(best, keys[e]);
        for (int d = 1; d < 64; d <<= 1) {
            const uint64_t o = __shfl_xor(best, d);
            best = max(best, o);
        }
        const uint32_t win = 0xffffffffu - (uint32_t)best;
        __syncthreads();
        if (lane == 0) {
            sel[slot] = win;
            selsc[slot] = sc[win];
            keys[win] = 0;
        }
        __syncthreads();
    }
    if (lane != 0) return;
    if (renorm == K3X_RENORM_DOUBLE) {
        double total = 0.0;
        for (uint32_t s = 0; s < K; ++s) total = __dadd_rn(total, (double)selsc[s]);
        if (!__builtin_isfinite(total) || !(total > 0.0)) {
            latch(status, K3X_ERR_INVALID_EXTENT);
            return;
        }
        for (uint32_t s = 0; s < K; ++s) {
            ids[(size_t)t * K + s] = sel[s];
            weights[(size_t)t * K + s] =
                __fmul_rn((float)__ddiv_rn((double)selsc[s], total), routed_scale);
        }
    } else {
        float den = 0.0f;
        for (uint32_t s = 0; s < K; ++s) den = __fadd_rn(den, selsc[s]);
        if (!__builtin_isfinite(den) || !(den > 0.0f)) {
            latch(status, K3X_ERR_INVALID_STATE);
            return;
        }
        for (uint32_t s = 0; s < K; ++s) {
            ids[(size_t)t * K + s] = sel[s];
            weights[(size_t)t * K + s] = __fmul_rn(__fdiv_rn(selsc[s], den), routed_scale);
        }
    }
}

// The same Top-K with each lane's keys in registers (E <= 64 KPL): one wave
// per token, topk_wave's sorted lane lists and DPP wave maxima; every logit
// and bias load is issued before the status check.
template <int KPL>
__global__ __launch_bounds__(64) void topk_reg_kernel(const float* __restrict__ logits,
                                                      const float* __restrict__ bias, uint32_t E,
                                                      uint32_t K, float routed_scale,
                                                      uint32_t renorm, uint32_t* __restrict__ ids,
                                                      float* __restrict__ weights,
                                                      uint32_t* status) {
    const uint32_t t = blockIdx.x, lane = threadIdx.x;
    float lv[KPL], bv[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
        const uint32_t e = min(lane + 64u * i, E - 1);
        lv[i] = logits[(size_t)t * E + e];
        bv[i] = bias[e];
    }
    if (*(volatile uint32_t*)status) return;
    uint32_t selid;
    float w;
    const uint32_t err =
        topk_wave<KPL>(lv, bv, E, K, renorm == K3X_RENORM_DOUBLE, routed_scale, &selid, &w);
    if (err) {
        if (lane == 0) latch(status, err);
        return;
    }
    if (lane < K) {
        ids[(size_t)t * K + lane] = selid;
        weights[(size_t)t * K + lane] = w;
    }
}

// The same Top-K by one 256-thread workgroup per token, for few tokens (one
// wave per token leaves the device idle while it works through K rounds of
// wave maxima).  Thread tid owns experts tid + 256 i, i < EPT (E <= 256 EPT):
//   keys       sigmoid + bias, the validation and the sort key of topk_wave;
//   threshold  the maximum score half of each 16-expert group (DPP row
//              rotates); with G groups and K <= G, the K-th largest group
//              maximum tau has at least K keys at or above it, so no key with
//              score half below tau is selected;
//   survivors  the keys at or above tau (every key when K > G), compacted,
//              ranked exactly by the full 64-bit key (keys are distinct: the
//              low half holds the expert); rank r < K is router slot r;
//   renorm     one wave, sequential sums in slot order, as topk_wave.
// Same results as topk_reg_kernel, bit for bit.
constexpr uint32_t kTopkThrThreads = 256;
constexpr uint32_t kTopkThrMaxTokens = 256;  // tokens up to which launch_topk_any uses it

// PUBLISH: ids and weights are stored at device scope (coherent across the
// XCDs' L2s), for a workgroup of the same launch to read them.
// Token t by a workgroup of kTopkThrThreads.
template <int EPT, bool PUBLISH>
__device__ __forceinline__ void topk_thr_body(
    const float* __restrict__ logits, const float* __restrict__ bias, uint32_t E, uint32_t K,
    float routed_scale, uint32_t renorm, uint32_t* __restrict__ ids,
    float* __restrict__ weights, uint32_t* status, uint32_t t) {
    constexpr uint32_t kN = kTopkThrThreads * EPT;
    __shared__ __align__(16) uint64_t ckey[kN];  // survivors' keys, compacted, 0 past them
    __shared__ uint32_t cid[kN];
    __shared__ float csc[kN];
    __shared__ __align__(16) uint32_t gmax[kN / 16];  // every group written (0 past E)
    __shared__ uint32_t sel[64];
    __shared__ float selsc[64];
    __shared__ uint32_t ncand, thr, bad, prior;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool dbl = renorm == K3X_RENORM_DOUBLE;
    constexpr uint32_t kErrExtent = K3X_ERR_INVALID_EXTENT, kErrState = K3X_ERR_INVALID_STATE;
    float lv[EPT], bv[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const uint32_t e = min(tid + kTopkThrThreads * i, E - 1);
        lv[i] = logits[(size_t)t * E + e];
        bv[i] = bias[e];
    }
    if (tid == 0) {
        ncand = 0;
        bad = 0;
        prior = *(volatile uint32_t*)status;  // one read: the block decides as one
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) ckey[tid + kTopkThrThreads * i] = 0;
    __syncthreads();
    if (prior) return;
    uint64_t key[EPT];
    float sc[EPT];
    uint32_t err = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const uint32_t e = tid + kTopkThrThreads * i;
        key[i] = 0;
        sc[i] = 0.0f;
        if (e < E) {
            if (dbl && (!__builtin_isfinite(lv[i]) || !__builtin_isfinite(bv[i]))) err = kErrExtent;
            const float sg = sigmoid_cr(lv[i]);
            const float adj = __fadd_rn(sg, bv[i]);
            if (!dbl && (!__builtin_isfinite(sg) || sg < 0.0f || sg > 1.0f ||
                         !__builtin_isfinite(bv[i]) || !__builtin_isfinite(adj)))
                err = kErrState;
            sc[i] = sg;
            key[i] = topk_key(adj, e);
        }
        uint32_t m = (uint32_t)(key[i] >> 32);
        m = dpp_max_step<0x128, 0xf>(m);  // row_ror:8
        m = dpp_max_step<0x124, 0xf>(m);  // row_ror:4
        m = dpp_max_step<0x122, 0xf>(m);  // row_ror:2
        m = dpp_max_step<0x121, 0xf>(m);  // row_ror:1
        if ((lane & 15) == 0) gmax[(tid + kTopkThrThreads * i) >> 4] = m;
    }
    if (err) atomicMax(&bad, err);
    __syncthreads();
    if (bad) {
        if (tid == 0) latch(status, bad);
        return;
    }
    // tau by wave 0: the group maximum m with fewer than K larger maxima and
    // at least K at or above it (groups past G hold 0).
    const uint32_t G = (E + 15) / 16;
    if (wave == 0) {
        uint32_t th = 0;
        if (K <= G) {
            const uint32_t m = lane < G ? gmax[lane] : 0u;
            uint32_t gt = 0, ge = 0;
            const uint4* gm = reinterpret_cast<const uint4*>(gmax);
            for (uint32_t g4 = 0; g4 < (G + 3) / 4; ++g4) {  // groups past G hold 0
                const uint4 v = gm[g4];
                gt += (v.x > m) + (v.y > m) + (v.z > m) + (v.w > m);
                ge += (v.x >= m) + (v.y >= m) + (v.z >= m) + (v.w >= m);
            }
            const uint64_t q = __ballot(lane < G && gt < K && K <= ge);
            if (q) th = (uint32_t)__builtin_amdgcn_readlane((int)m, (int)__builtin_ctzll(q));
        }
        if (lane == 0) thr = th;
    }
    __syncthreads();
    const uint32_t tau = thr;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const uint32_t e = tid + kTopkThrThreads * i;
        const bool surv = e < E && (uint32_t)(key[i] >> 32) >= tau;
        const uint64_t m = __ballot(surv);
        if (!m) continue;
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&ncand, (uint32_t)__popcll(m));
        base = __builtin_amdgcn_readfirstlane(base);
        if (surv) {
            const uint32_t c = base + (uint32_t)__popcll(m & ((1ull << lane) - 1));
            ckey[c] = key[i];
            cid[c] = e;
            csc[c] = sc[i];
        }
    }
    __syncthreads();
    const uint32_t n = ncand;
    const ulonglong2* ck = reinterpret_cast<const ulonglong2*>(ckey);
    for (uint32_t c = tid; c < n; c += kTopkThrThreads) {
        const uint64_t k = ckey[c];
        uint32_t r = 0;
        for (uint32_t c2 = 0; c2 < n; c2 += 8) {  // zero-padded past n (kN is a multiple of 8)
            ulonglong2 kk[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) kk[q] = ck[c2 / 2 + q];
#pragma unroll
            for (int q = 0; q < 4; ++q) r += (kk[q].x > k) + (kk[q].y > k);
        }
        if (r < K) {
            sel[r] = cid[c];
            selsc[r] = csc[c];
        }
    }
    __syncthreads();
    if (wave != 0) return;
    // Renormalise in slot order (sequential sums as the reference).
    const float v = lane < K ? selsc[lane] : 0.0f;
    float den_f = 0.0f;
    double den_d = 0.0;
    for (uint32_t s2 = 0; s2 < K; ++s2) {
        const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), s2));
        den_f = __fadd_rn(den_f, x);
        den_d = __dadd_rn(den_d, (double)x);
    }
    if (dbl ? !(__builtin_isfinite(den_d) && den_d > 0.0)
            : !(__builtin_isfinite(den_f) && den_f > 0.0f)) {
        if (lane == 0) latch(status, dbl ? kErrExtent : kErrState);
        return;
    }
    if (lane < K) {
        const float w = dbl ? __fmul_rn((float)__ddiv_rn((double)v, den_d), routed_scale)
                            : __fmul_rn(__fdiv_rn(v, den_f), routed_scale);
        if constexpr (PUBLISH) {
            __hip_atomic_store(ids + (size_t)t * K + lane, sel[lane], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(weights + (size_t)t * K + lane, w, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        } else {
            ids[(size_t)t * K + lane] = sel[lane];
            weights[(size_t)t * K + lane] = w;
        }
    }
}

template <int EPT>
__global__ __launch_bounds__(kTopkThrThreads) void topk_thr_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, uint32_t E, uint32_t K,
    float routed_scale, uint32_t renorm, uint32_t* __restrict__ ids,
    float* __restrict__ weights, uint32_t* status) {
    topk_thr_body<EPT, false>(logits, bias, E, K, routed_scale, renorm, ids, weights, status,
                              blockIdx.x);
}

// ---------------------------------------------------------------------------
// Expert-major grouping in three launches.  Produces the ascending-expert CSR
// (counts, offsets, pair_token, pair_slot; rows of one expert in (token,
// slot) order) plus first_use = min(token*K + slot) and the active experts
// sorted by it, which is the group order of build_expert_major_plan
// (runtime/src/expert_major.cpp:10-54).  Tokens are taken in chunks of
// tps = min(64, 1024 / K):
//   group_count_kernel    one workgroup per chunk: checks the ids (< E, no
//                         expert twice in one token: invalid_state, as
//                         expert_major.cpp:30-35), ranks each pair among the
//                         chunk's pairs of its expert (popcount of earlier
//                         tokens in a per-expert token bitmap), and writes
//                         the chunk's per-expert count and first use;
//   group_scan_kernel     one workgroup: per expert, the running row base of
//                         every chunk, its count and first use; CSR offsets,
//                         the active lists, and (witems non-null) the wide
//                         GEMM's (expert << 16 | row chunk) work items,
//                         dealt by size class over the XCDs' list segments;
//   group_scatter_kernel  one workgroup per chunk: row offsets[e] +
//                         base[chunk][e] + rank gets (token, slot).
// ---------------------------------------------------------------------------
__device__ inline uint32_t group_tps(uint32_t K) { return min(64u, 1024u / K); }

// ready (may be null): [E] words, 0 for a slot that holds no admitted expert.
__device__ inline bool group_count_body(uint32_t c, const uint32_t* __restrict__ ids,
                                        uint32_t T, uint32_t K, uint32_t E,
                                        const uint32_t* __restrict__ ready,
                                        uint32_t* __restrict__ chunk_cnt,
                                        uint32_t* __restrict__ chunk_fu,
                                        uint8_t* __restrict__ rank, uint32_t* status) {
    extern __shared__ uint32_t smem[];
    uint32_t* s_ids = smem;          // [1024] the chunk's ids
    uint32_t* mask = s_ids + 1024;   // [E][2] token bitmap per expert
    uint32_t* fu = mask + 2 * E;     // [E]
    if (*(volatile uint32_t*)status) return false;
    const uint32_t tid = threadIdx.x, tps = group_tps(K);
    const uint32_t tl = tid / K, s = tid % K, t = c * tps + tl;
    const bool valid = tl < tps && t < T;
    const uint32_t p = t * K + s;
    for (uint32_t e = tid; e < E; e += 1024) {
        mask[2 * e] = 0;
        mask[2 * e + 1] = 0;
        fu[e] = 0xffffffffu;
    }
    const uint32_t e = valid ? ids[p] : 0u;
    s_ids[tid] = e;
    __syncthreads();
    int bad = valid && (e >= E || (ready && !ready[e]));
    if (valid)
        for (uint32_t q = 0; q < s; ++q) bad |= s_ids[tl * K + q] == e;
    if (__syncthreads_or(bad)) {
        if (tid == 0) latch(status, K3X_ERR_INVALID_STATE);
        return false;
    }
    if (valid) {
        atomicOr(&mask[2 * e + (tl >> 5)], 1u << (tl & 31));
        atomicMin(&fu[e], p);
    }
    __syncthreads();
    if (valid) {
        const uint32_t lo = mask[2 * e], hi = mask[2 * e + 1];
        rank[p] = (uint8_t)(tl < 32 ? __popc(lo & ((1u << tl) - 1u))
                                    : __popc(lo) + __popc(hi & ((1u << (tl - 32)) - 1u)));
    }
    for (uint32_t q = tid; q < E; q += 1024) {
        chunk_cnt[(size_t)c * E + q] = __popc(mask[2 * q]) + __popc(mask[2 * q + 1]);
        chunk_fu[(size_t)c * E + q] = fu[q];
    }
    return true;
}

__global__ __launch_bounds__(1024) void group_count_kernel(
    const uint32_t* __restrict__ ids, uint32_t T, uint32_t K, uint32_t E,
    const uint32_t* __restrict__ ready, uint32_t* __restrict__ chunk_cnt,
    uint32_t* __restrict__ chunk_fu, uint8_t* __restrict__ rank, uint32_t* status) {
    (void)group_count_body(blockIdx.x, ids, T, K, E, ready, chunk_cnt, chunk_fu, rank, status);
}

// Exclusive scan of one 64-bit value per thread over a 1024-thread block;
// returns this thread's prefix, *total gets the block total.
__device__ inline uint64_t block_exclusive_scan(uint64_t v, uint64_t* red, uint64_t* total) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint64_t y = __shfl_up(x, d);
        if (lane >= (uint32_t)d) x += y;
    }
    if (lane == 63) red[wave] = x;
    __syncthreads();
    if (wave == 0) {
        uint64_t w = lane < 16 ? red[lane] : 0;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            const uint64_t y = __shfl_up(w, d);
            if (lane >= (uint32_t)d) w += y;
        }
        if (lane < 16) red[16 + lane] = w;
    }
    __syncthreads();
    const uint64_t before = (wave ? red[16 + wave - 1] : 0) + x - v;
    *total = red[31];
    __syncthreads();
    return before;
}

// Per-expert fields packed for one scan: rows (bits 0..26), wide GEMM items
// (27..47), active flag (48..60).
constexpr uint32_t kScanItemShift = 27, kScanActiveShift = 48;

__device__ inline bool group_scan_body(
    uint32_t T, uint32_t K, uint32_t E, uint32_t* __restrict__ chunk_cnt,
    const uint32_t* __restrict__ chunk_fu, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ offsets, uint32_t* __restrict__ first_use,
    uint32_t* __restrict__ n_active, uint32_t* __restrict__ active_asc,
    uint32_t* __restrict__ active_fu, uint32_t* __restrict__ witems,
    uint32_t* __restrict__ n_witems, uint32_t chunk_rows, uint4* __restrict__ arec,
    uint32_t* status) {
    extern __shared__ uint32_t smem[];
    uint32_t* s_cnt = smem;          // [E]
    uint32_t* s_fu = s_cnt + E;      // [E]
    uint32_t* s_alist = s_fu + E;    // [E] active experts, ascending
    __shared__ uint64_t red[32];
    if (*(volatile uint32_t*)status) return false;
    const uint32_t tid = threadIdx.x, nch = (T + group_tps(K) - 1) / group_tps(K);
    // Running base of every chunk, per expert (chunks loaded 16 at a time).
    for (uint32_t e = tid; e < E; e += 1024) {
        uint32_t acc = 0, f = 0xffffffffu;
        for (uint32_t c0 = 0; c0 < nch; c0 += 16) {
            uint32_t v[16], g[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t c = min(c0 + i, nch - 1);
                v[i] = chunk_cnt[(size_t)c * E + e];
                g[i] = chunk_fu[(size_t)c * E + e];
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (c0 + i >= nch) break;
                chunk_cnt[(size_t)(c0 + i) * E + e] = acc;
                acc += v[i];
                f = min(f, g[i]);
            }
        }
        s_cnt[e] = acc;
        s_fu[e] = f;
    }
    __syncthreads();
    // Thread tid owns experts [tid * per, tid * per + per).
    const uint32_t per = (E + 1023) / 1024, e0 = tid * per;
    uint64_t mine = 0;
    for (uint32_t i = 0; i < per; ++i) {
        const uint32_t e = e0 + i;
        if (e >= E) break;
        const uint64_t c = s_cnt[e];
        mine += c | ((c + chunk_rows - 1) / chunk_rows) << kScanItemShift |
                (uint64_t)(c != 0) << kScanActiveShift;
    }
    uint64_t total;
    uint64_t pre = block_exclusive_scan(mine, red, &total);
    for (uint32_t i = 0; i < per; ++i) {
        const uint32_t e = e0 + i;
        if (e >= E) break;
        const uint32_t c = s_cnt[e];
        const uint32_t row = (uint32_t)(pre & ((1ull << kScanItemShift) - 1));
        const uint32_t item = (uint32_t)((pre >> kScanItemShift) & ((1ull << 21) - 1));
        const uint32_t act = (uint32_t)(pre >> kScanActiveShift);
        (void)item;
        offsets[e] = row;
        counts[e] = c;
        first_use[e] = s_fu[e];
        if (c) {
            active_asc[act] = e;
            s_alist[act] = e;
            if (arec) arec[act] = make_uint4(e, c, row, 0u);
        }
        pre += c | (uint64_t)((c + chunk_rows - 1) / chunk_rows) << kScanItemShift |
               (uint64_t)(c != 0) << kScanActiveShift;
    }
    const uint32_t na = (uint32_t)(total >> kScanActiveShift);
    const uint32_t n_items = (uint32_t)((total >> kScanItemShift) & ((1ull << 21) - 1));
    if (tid == 0) {
        offsets[E] = (uint32_t)(total & ((1ull << kScanItemShift) - 1));
        *n_active = na;
        if (witems) *n_witems = n_items;
    }
    if (witems) {
        // Wide GEMM work items in kWideClasses segments, one launch each:
        // class 0 holds every full chunk and the last chunks of more than
        // 3/4 of chunk_rows, classes 1, 2 and 3 the last chunks of more than
        // 1/2, more than 1/4 and at most 1/4 of it (a launch multiplies its
        // class's chunks as 8, 6, 4 or 2 row tiles).  Rank k of a class (by
        // expert) goes to segment position k % 8 * q + min(k % 8, r) + k / 8
        // (q, r = the class's count / 8, % 8): the GEMM hands each XCD one
        // contiguous eighth of the segment, so each XCD gets every eighth
        // item.
        auto cls = [&](uint32_t c) -> uint32_t {  // class of an expert's last chunk
            const uint32_t last = c - (c - 1) / chunk_rows * chunk_rows;
            return last * 4 > chunk_rows * 3 ? 0u
                   : last * 2 > chunk_rows   ? 1u
                   : last * 4 > chunk_rows   ? 2u
                                             : 3u;
        };
        auto counts01 = [&](uint32_t c) -> uint64_t {  // items of classes 0 | 1
            if (!c) return 0;
            const uint32_t nq = (c + chunk_rows - 1) / chunk_rows, k = cls(c);
            return (uint64_t)(nq - 1 + (k == 0)) | (uint64_t)(k == 1) << 32;
        };
        auto counts23 = [&](uint32_t c) -> uint64_t {  // items of classes 2 | 3
            if (!c) return 0;
            const uint32_t k = cls(c);
            return (uint64_t)(k == 2) | (uint64_t)(k == 3) << 32;
        };
        uint64_t mine01 = 0, mine23 = 0;
        for (uint32_t i = 0; i < per; ++i)
            if (e0 + i < E) {
                mine01 += counts01(s_cnt[e0 + i]);
                mine23 += counts23(s_cnt[e0 + i]);
            }
        uint64_t total01, total23;
        uint64_t pre01 = block_exclusive_scan(mine01, red, &total01);
        uint64_t pre23 = block_exclusive_scan(mine23, red, &total23);
        const uint32_t ncls[4] = {(uint32_t)total01, (uint32_t)(total01 >> 32), (uint32_t)total23,
                                  (uint32_t)(total23 >> 32)};
        const uint32_t base[4] = {0u, ncls[0], ncls[0] + ncls[1], ncls[0] + ncls[1] + ncls[2]};
        if (tid == 0)
            for (int c = 0; c < 4; ++c) n_witems[1 + c] = ncls[c];
        auto place = [&](uint32_t c, uint32_t k) {  // list position of rank k of class c
            const uint32_t x = k % 8;
            return base[c] + x * (ncls[c] / 8) + min(x, ncls[c] % 8) + k / 8;
        };
        for (uint32_t i = 0; i < per; ++i) {
            const uint32_t e = e0 + i;
            if (e >= E) break;
            const uint32_t c = s_cnt[e];
            if (c) {
                const uint32_t nq = (c + chunk_rows - 1) / chunk_rows, k = cls(c);
                const uint32_t p0 = (uint32_t)pre01;
                for (uint32_t q = 0; q + 1 < nq; ++q) witems[place(0, p0 + q)] = (e << 16) | q;
                const uint32_t kl = k == 0   ? p0 + nq - 1
                                    : k == 1 ? (uint32_t)(pre01 >> 32)
                                    : k == 2 ? (uint32_t)pre23
                                             : (uint32_t)(pre23 >> 32);
                witems[place(k, kl)] = (e << 16) | (nq - 1);
            }
            pre01 += counts01(c);
            pre23 += counts23(c);
        }
    }
    __syncthreads();
    // First uses are distinct pair indices: ranks are a permutation.
    for (uint32_t a = tid; a < na; a += 1024) {
        const uint32_t e = s_alist[a], key = s_fu[e];
        uint32_t r = 0;
        for (uint32_t b = 0; b < na; ++b) r += s_fu[s_alist[b]] < key;
        active_fu[r] = e;
    }
    return true;
}

__global__ __launch_bounds__(1024) void group_scan_kernel(
    uint32_t T, uint32_t K, uint32_t E, uint32_t* __restrict__ chunk_cnt,
    const uint32_t* __restrict__ chunk_fu, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ offsets, uint32_t* __restrict__ first_use,
    uint32_t* __restrict__ n_active, uint32_t* __restrict__ active_asc,
    uint32_t* __restrict__ active_fu, uint32_t* __restrict__ witems,
    uint32_t* __restrict__ n_witems, uint32_t chunk_rows, uint4* __restrict__ arec,
    uint32_t* status) {
    (void)group_scan_body(T, K, E, chunk_cnt, chunk_fu, counts, offsets, first_use, n_active,
                          active_asc, active_fu, witems, n_witems, chunk_rows, arec, status);
}

__device__ inline void group_scatter_body(uint32_t c, 
    const uint32_t* __restrict__ ids, uint32_t T, uint32_t K, uint32_t E,
    const uint32_t* __restrict__ chunk_base, const uint8_t* __restrict__ rank,
    const uint32_t* __restrict__ offsets, uint32_t* __restrict__ pair_token,
    uint32_t* __restrict__ pair_slot, uint32_t* status) {
    if (*(volatile uint32_t*)status) return;
    const uint32_t tid = threadIdx.x, tps = group_tps(K);
    const uint32_t tl = tid / K, s = tid % K, t = c * tps + tl;
    if (tl >= tps || t >= T) return;
    const uint32_t p = t * K + s, e = ids[p];
    const uint32_t r = offsets[e] + chunk_base[(size_t)c * E + e] + rank[p];
    pair_token[r] = t;
    pair_slot[r] = s;
}

__global__ __launch_bounds__(1024) void group_scatter_kernel(
    const uint32_t* __restrict__ ids, uint32_t T, uint32_t K, uint32_t E,
    const uint32_t* __restrict__ chunk_base, const uint8_t* __restrict__ rank,
    const uint32_t* __restrict__ offsets, uint32_t* __restrict__ pair_token,
    uint32_t* __restrict__ pair_slot, uint32_t* status) {
    group_scatter_body(blockIdx.x, ids, T, K, E, chunk_base, rank, offsets, pair_token, pair_slot,
                       status);
}

// All T tokens in one chunk (T <= group_tps(K)): the three steps in one
// workgroup, separated by barriers (the chunk values pass through global
// memory written and read by this workgroup only).
__global__ __launch_bounds__(1024) void group_single_kernel(
    const uint32_t* __restrict__ ids, uint32_t T, uint32_t K, uint32_t E,
    const uint32_t* __restrict__ ready, uint32_t* __restrict__ chunk_cnt, uint32_t* __restrict__ chunk_fu, uint8_t* __restrict__ rank,
    uint32_t* __restrict__ counts, uint32_t* __restrict__ offsets,
    uint32_t* __restrict__ first_use, uint32_t* __restrict__ n_active,
    uint32_t* __restrict__ active_asc, uint32_t* __restrict__ active_fu,
    uint32_t* __restrict__ witems, uint32_t* __restrict__ n_witems, uint32_t chunk_rows,
    uint4* __restrict__ arec, uint32_t* __restrict__ pair_token, uint32_t* __restrict__ pair_slot,
    uint32_t* status) {
    if (!group_count_body(0, ids, T, K, E, ready, chunk_cnt, chunk_fu, rank, status)) return;
    __syncthreads();
    if (!group_scan_body(T, K, E, chunk_cnt, chunk_fu, counts, offsets, first_use, n_active,
                         active_asc, active_fu, witems, n_witems, chunk_rows, arec, status))
        return;
    __syncthreads();
    group_scatter_body(0, ids, T, K, E, chunk_cnt, rank, offsets, pair_token, pair_slot, status);
}

// ---------------------------------------------------------------------------
// Grouped expert GEMM on v_mfma_f32_16x16x32_bf16.
//
// Work item of one wave: NT row blocks of 16 output rows (GATEUP: NT pairs of
// 16 gate + 16 up rows) of one expert, for all of the expert's pair rows in
// chunks of 16*MT, over the full K.  B (weights) is read straight from the
// tile layout into registers -- MXFP4 codes dequantised by dequant8, bf16
// used as is -- so every weight byte is fetched once per chunk.  A
// (activations) is read per lane from the bf16 rows the lane's MFMA row maps
// to (gathered through pair_token for gate/up).
//
// Accumulator layout (16x16 MFMA): lane l, element i holds row 4(l/16)+i of
// the M (pair) dimension and column l%16 of the output rows.
// ---------------------------------------------------------------------------
struct GemmArgs {
    const uint8_t* codes;       // expert 0 base of the tile array
    const uint32_t* scales;     // MXFP4 only
    size_t codes_per_expert;    // bytes
    size_t scales_per_expert;   // dwords
    uint32_t kt, ks;            // K tiles, scale dword groups
    uint32_t blocks_per_expert; // workgroups per expert
    const uint16_t* a;          // activation rows (bf16)
    uint32_t a_stride;          // elements per activation row
    uint32_t a_lo;              // split rows [hi | lo]: element offset of the lo half (0: none)
    uint32_t gather;            // A row = pair_token[off+m] (1) or off+m (0)
    const uint32_t* n_active;   // grouping (nullptr = single block of `tokens` rows)
    const uint32_t* active;
    const uint32_t* counts;
    const uint32_t* offsets;
    const uint32_t* pair_token;
    const uint32_t* pair_slot;
    uint32_t tokens;
    uint32_t top_k;
    uint16_t* act;              // GATEUP output [row][act_stride] bf16
    uint32_t act_stride;
    uint32_t act_lo;            // GATEUP: element offset of the lo half in a row (0: none)
    float* y;                   // down output [row][y_stride] fp32
    uint32_t y_stride;
    uint32_t scatter;           // y row = token*top_k + slot (1) or off+m (0)
    GluParams glu;
    const uint32_t* status;
};

constexpr int kGemmDepth = 4;  // K steps in flight per wave of a one-row-tile GEMM

// SPLIT: activation rows [hi | lo] (a_lo elements apart), an fp32 value in
// two bf16 halves; each weight fragment meets both (two MFMAs, the weights
// read once).
template <bool FP4, bool GATEUP, int MT, int NT, bool SPLIT>
__global__ __launch_bounds__(256) void expert_gemm(GemmArgs a) {
    if (*(volatile const uint32_t*)a.status) return;
    const uint32_t eb = blockIdx.x / a.blocks_per_expert;
    const uint32_t jb = blockIdx.x % a.blocks_per_expert;
    uint32_t e = 0, cnt = a.tokens, off = 0;
    if (a.active) {
        if (eb >= *a.n_active) return;
        e = a.active[eb];
        cnt = a.counts[e];
        off = a.offsets[e];
    }
    constexpr int S = GATEUP ? 2 : 1;  // tiles per row block and K step
    constexpr int U = FP4 ? 1 : 4;     // 16-byte words per lane per tile
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, n = lane & 15;
    const uint32_t rb0 = (jb * 4 + wave) * NT;
    const uint4* codes = reinterpret_cast<const uint4*>(a.codes + e * a.codes_per_expert);
    const uint32_t* scales = FP4 ? a.scales + e * a.scales_per_expert : nullptr;
    constexpr int H2 = SPLIT ? 2 : 1;  // activation halves

    for (uint32_t m0 = 0; m0 < cnt; m0 += 16 * MT) {
        // Rows past the block's end read its last row (their products are
        // zeroed): every activation load is unconditional, so none waits
        // behind a branch for all older loads.
        const uint16_t* arow[MT];
        bool live[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const uint32_t row = m0 + 16 * mt + n;
            live[mt] = row < cnt;
            const uint32_t r = min(row, cnt - 1);
            const uint32_t src = a.gather ? a.pair_token[off + r] : off + r;
            arow[mt] = a.a + (size_t)src * a.a_stride + 32 * g;
        }
        f32x4 acc[MT][NT][S];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int w = 0; w < S; ++w) acc[mt][nt][w] = f32x4{0.f, 0.f, 0.f, 0.f};

        // One row tile: D K steps of loads issued together (steps past the
        // last tile clamped, their activations zeroed), since a lone step's
        // round trip would bound the wave.
        constexpr int D = MT == 1 ? kGemmDepth : 1;
        for (uint32_t k0 = 0; k0 < a.kt; k0 += D) {
            uint4 bt[D][NT][S][U];
            float sc[D][NT][S];
            bf16x8 af[D][MT][H2][4];
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const uint32_t k = min(k0 + d, a.kt - 1);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int w = 0; w < S; ++w) {
                        const size_t base = (((size_t)(rb0 + nt) * a.kt + k) * S + w) * U * 64 + lane;
#pragma unroll
                        for (int u = 0; u < U; ++u) bt[d][nt][w][u] = codes[base + u * 64];
                        if constexpr (FP4) {
                            const uint32_t sw =
                                scales[(((size_t)(rb0 + nt) * a.ks + k / 4) * S + w) * 64 + lane];
                            sc[d][nt][w] = e8m0_to_f32((sw >> (8 * (k & 3))) & 0xffu);
                        }
                    }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int h = 0; h < H2; ++h) {
                        const uint4* p = reinterpret_cast<const uint4*>(
                            arow[mt] + (h ? a.a_lo : 0u) + (size_t)k * 128);
                        const bool use = live[mt] && k0 + d < a.kt;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const uint4 v = p[j];
                            af[d][mt][h][j] = as_bf16x8(use ? v : make_uint4(0, 0, 0, 0));
                        }
                    }
            }
#pragma unroll
            for (int d = 0; d < D; ++d)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                        for (int w = 0; w < S; ++w) {
                            bf16x8 b;
                            if constexpr (FP4) {
                                const uint4 c = bt[d][nt][w][0];
                                const uint32_t word = j == 0 ? c.x : j == 1 ? c.y : j == 2 ? c.z : c.w;
                                b = dequant8(word, sc[d][nt][w]);
                            } else {
                                b = as_bf16x8(bt[d][nt][w][j]);
                            }
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                                for (int h = 0; h < H2; ++h)
                                    acc[mt][nt][w] = mfma16x16x32(af[d][mt][h][j], b, acc[mt][nt][w]);
                        }
                }
        }

#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t row = m0 + 16 * mt + 4 * g + i;
                    if (row >= cnt) continue;
                    const uint32_t col = (rb0 + nt) * 16 + n;
                    if constexpr (GATEUP) {
                        const float v = glu(acc[mt][nt][0][i], acc[mt][nt][1][i], a.glu);
                        uint16_t* dst = a.act + (size_t)(off + row) * a.act_stride + col;
                        const uint16_t hi = f32_to_bf16(v);
                        *dst = hi;
                        if (a.act_lo) dst[a.act_lo] = act_lo_bf16(v, hi);
                    } else {
                        const uint32_t r = off + row;
                        const size_t yrow = a.scatter
                                                ? (size_t)a.pair_token[r] * a.top_k + a.pair_slot[r]
                                                : (size_t)r;
                        a.y[yrow * a.y_stride + col] = acc[mt][nt][0][i];
                    }
                }
    }
}

// ---------------------------------------------------------------------------
// Dense bf16 projection of a few rows (T <= 16) in the bank's tile layout:
// one workgroup of kGemvWaves waves per 16 output rows (S = 2: 16 gate + 16
// up rows); wave w takes the K tiles w, w + kGemvWaves, ..., with D tiles of
// weight loads issued per step (indices clamped, activations of steps past
// the last tile zeroed, so no load sits behind a branch).  The waves'
// accumulators are summed in wave order through LDS.  Activations: lane l
// reads token l % 16 (clamped to the last token and zeroed past it).
// OUT: 0 fp32 y, 1 bf16 y, 2 bf16 GLU(gate, up) (S == 2), 3 the official
// layer's output bf16(bf16(prefix) + bf16(bf16(y) + bf16(shared))), y also
// stored in fp32 (runtime/src/official_moe.cpp:336-340).
// ---------------------------------------------------------------------------
constexpr int kGemvWaves = 16;
constexpr uint32_t kGemvMaxTokens = k3x_hip::kDenseDirectTokens;

// Weight tiles are read once a call: non-temporal loads (the lines are not
// kept in L2 / MALL), which stream faster than cached ones (the official
// layer at T=2: 202.6-202.9 -> 192.7-197.1 us).
__device__ inline uint4 ntl_tile(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

struct GemvArgs {
    const uint4* tiles;   // [N/16][kt][S][4][64]
    uint32_t kt;          // K tiles
    const uint16_t* x;    // [T][x_stride] bf16
    uint32_t x_stride;
    uint32_t tokens;
    void* out;            // [T][out_stride]
    uint32_t out_stride;
    GluParams glu;
    const uint32_t* status;
    // OUT 3 (the official layer's output): prefix, shared (may be null) and
    // the fp32 projection (routed) at the output's [T][out_stride] layout.
    const float* prefix;
    const float* shared;
    float* routed;
    // Split activations: x rows [hi | lo], the lo half x_lo elements after
    // hi (SPLIT kernels; each weight tile meets both halves); OUT 2 also
    // stores lo = bf16(v - hi) out_lo elements after hi (0: none).
    uint32_t x_lo;
    uint32_t out_lo;
    // NORM kernels: x is the T raw rows; each workgroup applies RMSNorm with
    // these weights to them in LDS first.
    const float* gamma;
    float eps;
};

// NORM: tokens a workgroup normalises (256 threads each) and 16-byte chunks
// of the raw rows and of gamma its threads load (two and one a thread).
constexpr uint32_t kNormOutTokens = 4;
constexpr uint32_t kNormOutRowChunks = 2 * 64 * kGemvWaves;
constexpr uint32_t kNormOutGammaChunks = 64 * kGemvWaves;

// Output rows [16 rb, 16 rb + 16) by a workgroup of W waves.
// LDSX: the T activation rows (x 16-byte aligned, x_stride == K, at most
// 64 W 16-byte chunks, K tiles <= W D: one step) are copied into LDS once by
// the workgroup, their loads issued before the weights', so a wave holds only
// its weight tiles in registers (the kernel then fits two workgroups a
// compute unit).  The products and sums are those of the register path.
// NORM (LDSX, W = kGemvWaves, T <= kNormOutTokens): the rows are first
// normalised in LDS by rmsnorm_kernel's arithmetic in its order -- 256
// threads a token, thread r summing the squares of elements r + 256 j in
// fp64 (j ascending), the wave butterfly, then (w0 + w1) + (w2 + w3) --
// so the GEMV meets the same bf16 rows as after a separate RMSNorm launch;
// a non-finite element latches K3X_ERR_INVALID_MXFP4, as there.  The
// workgroup's barriers wait for LDS only: its weight tiles stay in flight
// through the norm.
template <int S, int D, int OUT, int W, bool SPLIT, bool LDSX = false, bool NORM = false>
__device__ __forceinline__ void dense_gemv_body(const GemvArgs& a, uint32_t rb) {
    __shared__ f32x4 part[W][S][64];
    if (*(volatile const uint32_t*)a.status) return;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;
    const uint32_t row = min((uint32_t)n, a.tokens - 1);
    const bool live_row = (uint32_t)n < a.tokens;
    if constexpr (LDSX) {
        static_assert(!SPLIT, "one activation half");
        static_assert(!NORM || W == kGemvWaves, "256 threads a token");
        extern __shared__ uint4 s_gx[];                // [T][K] bf16 (NORM: then [K] fp32)
        const uint32_t tid = threadIdx.x;
        const uint32_t chunks = a.tokens * a.kt * 16;  // 16-byte chunks of the T rows
        const uint4* x4 = reinterpret_cast<const uint4*>(a.x);
        const uint4 xv = x4[min(tid, chunks - 1)];
        uint4 xv2, gv;
        if constexpr (NORM) {
            xv2 = x4[min(tid + 64 * W, chunks - 1)];
            gv = reinterpret_cast<const uint4*>(a.gamma)[min(tid, a.kt * 32 - 1)];
        }
        const uint4* wt = a.tiles + (size_t)rb * a.kt * S * 256 + lane;
        uint4 b[D][S][4];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const uint32_t k = min(wave + d * W, a.kt - 1);
#pragma unroll
            for (int w = 0; w < S; ++w)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    b[d][w][u] = ntl_tile(&wt[((size_t)k * S + w) * 256 + u * 64]);
        }
        if (tid < chunks) s_gx[tid] = xv;
        if constexpr (NORM) {
            __shared__ double nred[W];
            __shared__ uint32_t nbad[W];
            const uint32_t K = a.kt * 128;
            uint16_t* xs = reinterpret_cast<uint16_t*>(s_gx);
            const float* gs = reinterpret_cast<const float*>(s_gx + chunks);
            if (tid + 64 * W < chunks) s_gx[tid + 64 * W] = xv2;
            if (tid < a.kt * 32) s_gx[chunks + tid] = gv;
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            const uint32_t t = tid / 256, r = tid % 256;  // token, its thread
            const bool mine = t < a.tokens;               // wave-uniform
            double sq = 0.0;
            bool bad = false;
            if (mine) {
                for (uint32_t k = r; k < K; k += 256) {
                    const float v = bf16_to_f32(xs[(size_t)t * K + k]);
                    bad |= !__builtin_isfinite(v);
                    sq = __builtin_fma((double)v, (double)v, sq);
                }
#pragma unroll
                for (int d = 1; d < 64; d <<= 1) sq += __shfl_xor(sq, d);
            }
            const bool wbad = __any(bad);
            if (lane == 0) {
                nred[wave] = sq;
                nbad[wave] = wbad;
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            uint32_t any_bad = 0;
            for (uint32_t q = 0; q < 4 * a.tokens; ++q) any_bad |= nbad[q];
            if (any_bad) {
                if (tid == 0) latch(const_cast<uint32_t*>(a.status), K3X_ERR_INVALID_MXFP4);
                return;
            }
            if (mine) {
                const double* nr = nred + 4 * t;
                const double tot = (nr[0] + nr[1]) + (nr[2] + nr[3]);
                const float mean = (float)__ddiv_rn(tot, (double)K);
                const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, a.eps)));
                for (uint32_t k = r; k < K; k += 256) {
                    uint16_t* e = xs + (size_t)t * K + k;
                    *e = f32_to_bf16(__fmul_rn(__fmul_rn(bf16_to_f32(*e), inv), gs[k]));
                }
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const uint16_t* xrow =
            reinterpret_cast<const uint16_t*>(s_gx) + (size_t)row * a.kt * 128 + 32 * g;
        f32x4 acc[S];
#pragma unroll
        for (int w = 0; w < S; ++w) acc[w] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const uint32_t k = wave + d * W;
            const bool live = live_row && k < a.kt;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint4 xv4 =
                    live ? *reinterpret_cast<const uint4*>(xrow + (size_t)k * 128 + 8 * j)
                         : make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int w = 0; w < S; ++w)
                    acc[w] = mfma16x16x32(as_bf16x8(xv4), as_bf16x8(b[d][w][j]), acc[w]);
            }
        }
#pragma unroll
        for (int w = 0; w < S; ++w) part[wave][w][lane] = acc[w];
    } else {
        const uint4* xr = reinterpret_cast<const uint4*>(a.x + (size_t)row * a.x_stride + 32 * g);
        const uint4* wt = a.tiles + (size_t)rb * a.kt * S * 256 + lane;
        f32x4 acc[S];
#pragma unroll
        for (int w = 0; w < S; ++w) acc[w] = f32x4{0.f, 0.f, 0.f, 0.f};
        constexpr int H2 = SPLIT ? 2 : 1;  // activation halves
        const uint4* xl = reinterpret_cast<const uint4*>(a.x + (size_t)row * a.x_stride + a.x_lo +
                                                         32 * g);
        for (uint32_t k0 = wave; k0 < a.kt; k0 += W * D) {
            uint4 b[D][S][4], xa[D][H2][4];
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const uint32_t k = min(k0 + d * W, a.kt - 1);
#pragma unroll
                for (int w = 0; w < S; ++w)
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        b[d][w][u] = ntl_tile(&wt[((size_t)k * S + w) * 256 + u * 64]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    xa[d][0][j] = xr[(size_t)k * 16 + j];
                    if constexpr (SPLIT) xa[d][H2 - 1][j] = xl[(size_t)k * 16 + j];
                }
            }
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const bool live = live_row && k0 + d * W < a.kt;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int h = 0; h < H2; ++h) {
                        const uint4 xv = live ? xa[d][h][j] : make_uint4(0, 0, 0, 0);
#pragma unroll
                        for (int w = 0; w < S; ++w)
                            acc[w] = mfma16x16x32(as_bf16x8(xv), as_bf16x8(b[d][w][j]), acc[w]);
                    }
            }
        }
#pragma unroll
        for (int w = 0; w < S; ++w) part[wave][w][lane] = acc[w];
    }
    __syncthreads();
    // Thread 16 t + c finishes output (t, c): lane 16 (t / 4) + c, element
    // t % 4 of every wave's accumulator, summed in wave order.
    const uint32_t t = threadIdx.x / 16, c = threadIdx.x % 16;
    if (t >= a.tokens) return;
    const uint32_t pl = 16 * (t / 4) + c, pi = t % 4;
    float v[S];
#pragma unroll
    for (int w = 0; w < S; ++w) {
        v[w] = part[0][w][pl][pi];
#pragma unroll
        for (int q = 1; q < W; ++q) v[w] = __fadd_rn(v[w], part[q][w][pl][pi]);
    }
    const size_t at = (size_t)t * a.out_stride + (size_t)rb * 16 + c;
    if constexpr (OUT == 0) static_cast<float*>(a.out)[at] = v[0];
    else if constexpr (OUT == 1) static_cast<uint16_t*>(a.out)[at] = f32_to_bf16(v[0]);
    else if constexpr (OUT == 2) {
        const float g = glu(v[0], v[S - 1], a.glu);
        const uint16_t hi = f32_to_bf16(g);
        static_cast<uint16_t*>(a.out)[at] = hi;
        if (a.out_lo) static_cast<uint16_t*>(a.out)[at + a.out_lo] = act_lo_bf16(g, hi);
    }
    else {
        auto r16 = [](float x) { return __uint_as_float((uint32_t)f32_to_bf16(x) << 16); };
        a.routed[at] = v[0];
        const float sh = a.shared ? r16(a.shared[at]) : 0.0f;
        const float combined = r16(__fadd_rn(r16(v[0]), sh));
        static_cast<uint16_t*>(a.out)[at] = f32_to_bf16(__fadd_rn(r16(a.prefix[at]), combined));
    }
}

template <int S, int D, int OUT, int W = kGemvWaves, bool SPLIT = false, bool LDSX = false,
          bool NORM = false>
__global__ __launch_bounds__(64 * W) void dense_gemv_kernel(GemvArgs a) {
    dense_gemv_body<S, D, OUT, W, SPLIT, LDSX, NORM>(a, blockIdx.x);
}

// ---------------------------------------------------------------------------
// out[t][h] = bf16(sum_{slot in router order} w[t][slot] * y[t][slot][h]
//                  + shared[t][h]), float mul then float add per term
// (runtime/src/backend_cpu.cpp:295-301, runtime/src/model.cpp:1145).
// ---------------------------------------------------------------------------
// VEC adjacent h per thread; the slots' loads are issued in batches of 16
// ahead of the slot-ordered multiply-adds.  H % VEC == 0.
// The per-pair rows are read once, with non-temporal loads (they pass
// through the L2 without being kept).
template <int VEC>
struct CombineVec { typedef float T __attribute__((ext_vector_type(VEC))); };
template <>
struct CombineVec<1> { typedef float T; };

template <int VEC>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ shared,
                                                      uint32_t K, uint32_t H,
                                                      uint16_t* __restrict__ out,
                                                      float* __restrict__ out_f32,
                                                      uint32_t round_y,
                                                      const uint32_t* status) {
    typedef typename CombineVec<VEC>::T vec_t;
    constexpr uint32_t kBatch = 16;
    if (*(volatile const uint32_t*)status) return;
    const uint32_t h = (blockIdx.x * 256 + threadIdx.x) * VEC;
    const uint32_t t = blockIdx.y;
    if (h >= H) return;
    const float* yt = y + (size_t)t * K * H + h;
    const float* wt = w + (size_t)t * K;
    float mix[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) mix[c] = 0.0f;
    for (uint32_t s0 = 0; s0 < K; s0 += kBatch) {
        vec_t v[kBatch];
        float ws[kBatch];
#pragma unroll
        for (uint32_t i = 0; i < kBatch; ++i) {
            const uint32_t s = min(s0 + i, K - 1);  // clamped: loads stay unconditional
            v[i] = __builtin_nontemporal_load(reinterpret_cast<const vec_t*>(yt + (size_t)s * H));
            ws[i] = wt[s];
        }
#pragma unroll
        for (uint32_t i = 0; i < kBatch; ++i) {
            if (s0 + i >= K) break;
            const float* vi = reinterpret_cast<const float*>(&v[i]);
#pragma unroll
            for (int c = 0; c < VEC; ++c) {
                // The official layer rounds each expert output to bf16 first
                // (runtime/src/official_moe.cpp:99-101).
                const float yv = round_y ? __uint_as_float((uint32_t)f32_to_bf16(vi[c]) << 16)
                                         : vi[c];
                mix[c] = __fadd_rn(mix[c], __fmul_rn(ws[i], yv));
            }
        }
    }
    if (shared) {
        const vec_t sh = *reinterpret_cast<const vec_t*>(shared + (size_t)t * H + h);
        const float* sv = reinterpret_cast<const float*>(&sh);
#pragma unroll
        for (int c = 0; c < VEC; ++c) mix[c] = __fadd_rn(mix[c], sv[c]);
    }
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
        out[(size_t)t * H + h + c] = f32_to_bf16(mix[c]);
        if (out_f32) out_f32[(size_t)t * H + h + c] = mix[c];
    }
}

constexpr int kCombineVec = 1;  // h per thread of combine_kernel

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

using Scratch = k3x_hip::LayerBuffers;
using k3x_hip::begin_stage;
using k3x_hip::end_stage;

// Tokens from which the general path runs the wide grouped GEMM.
constexpr uint32_t kWideMinTokens = 128;

// Lays the per-call buffers out in the context scratch; returns bytes needed
// (base == nullptr only measures).
// Upper bound of the wide GEMM's (expert, chunk) items: every pair row in a
// full chunk plus at most one partial chunk per active expert.
uint32_t wide_max_items(const k3x_hip_layer_desc& d, uint32_t T, uint32_t K) {
    const uint64_t P = (uint64_t)T * K;
    return (uint32_t)(P / k3x_hip::kWideRows + std::min<uint64_t>(d.experts, P));
}

// Scratch bytes of the grouping: per-chunk counts and first uses, pair ranks.
size_t group_scratch_bytes(uint32_t T, uint32_t K, uint32_t E) {
    const size_t tps = std::min(64u, 1024u / K), nch = (T + tps - 1) / tps;
    return 2 * nch * E * 4 + (((size_t)T * K + 255) & ~(size_t)255);
}

// K3X_FLAG_SCALED_FP4 in effect: not with split activations or inputs.
bool scaled_fp4(const k3x_hip_moe_params* p) {
    return (p->flags & K3X_FLAG_SCALED_FP4) &&
           !(p->flags & (K3X_FLAG_SPLIT_ACT | K3X_FLAG_SPLIT_INPUT));
}

// split: the routed activation rows hold [hi | lo] halves (K3X_FLAG_SPLIT_ACT);
// q8: room for the q8 rows of the scaled FP4 wide GEMM.
size_t carve(uint8_t* base, const k3x_hip_layer_desc& d, uint32_t T, uint32_t K, bool split,
             bool q8, Scratch* s) {
    size_t at = 0;
    auto take = [&](size_t bytes) {
        uint8_t* p = base ? base + at : nullptr;
        at += (bytes + 255) & ~(size_t)255;
        return p;
    };
    const size_t P = (size_t)T * K;
    s->xn = (uint16_t*)take((size_t)T * d.hidden * 2);
    s->logits = (float*)take((size_t)T * d.experts * 4);
    s->ids = (uint32_t*)take(P * 4);
    s->weights = (float*)take(P * 4);
    s->counts = (uint32_t*)take((size_t)d.experts * 4);
    s->offsets = (uint32_t*)take(((size_t)d.experts + 1) * 4);
    s->pair_token = (uint32_t*)take(P * 4);
    s->pair_slot = (uint32_t*)take(P * 4);
    s->first_use = (uint32_t*)take((size_t)d.experts * 4);
    s->n_active = (uint32_t*)take(4);
    s->active_asc = (uint32_t*)take((size_t)d.experts * 4);
    s->active_fu = (uint32_t*)take((size_t)d.experts * 4);
    s->act = (uint16_t*)take(P * d.inter * (split ? 4 : 2));
    // y is first written by the down projection, after the router: the
    // residue-major xn copy of router_mfma_kernel lives in the same bytes.
    const size_t xp_bytes = (size_t)(T + 15) / 16 * kRouterRes * kRouterTileRes * 2;
    s->y = (float*)take(std::max(P * d.hidden * 4, xp_bytes));
    s->xp = reinterpret_cast<uint16_t*>(s->y);
    s->sact = (uint16_t*)take((size_t)T * d.shared_inter * 2);
    s->sy = (float*)take((size_t)T * d.hidden * 4);
    s->arec = (uint4*)take((size_t)d.experts * 16);
    s->witems = (uint32_t*)take((size_t)wide_max_items(d, T, K) * 4);
    s->n_witems = (uint32_t*)take(4 * (1 + k3x_hip::kWideClasses));
    s->gscratch = take(group_scratch_bytes(T, K, d.experts));
    s->qx = q8 ? (uint16_t*)take((size_t)T * d.hidden * 2) : nullptr;
    s->qxs = q8 ? (uint32_t*)take((size_t)T * (d.hidden / 128) * 8) : nullptr;
    s->qact = q8 ? (uint16_t*)take(P * d.inter * 2) : nullptr;
    s->qacts = q8 ? (uint32_t*)take(P * (d.inter / 128) * 8) : nullptr;
    return at;
}

bool finite_pos(float v) { return std::isfinite(v) && v > 0.0f; }

// all_experts: every bank slot must be admitted (routes decided on the
// device may pick any); routes given by the caller check their own slots
// instead (on the host copy when there is one, else in the grouping).
int validate_params(const k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                    bool all_experts = true) {
    const auto& d = bank->desc;
    if (!p->tokens || p->tokens > (1u << 20) || !p->top_k || p->top_k > 64 ||
        p->top_k > d.experts)
        return K3X_ERR_INVALID_EXTENT;
    if (!finite_pos(p->rms_epsilon) || !std::isfinite(p->routed_scale) || p->glu > 1 ||
        p->renorm > 1 ||
        (p->flags & ~(uint32_t)(K3X_FLAG_GENERAL_PATH | K3X_FLAG_ROUND_EXPERT_OUT |
                                K3X_FLAG_SPLIT_ACT | K3X_FLAG_SPLIT_INPUT |
                                K3X_FLAG_SCALED_FP4)))
        return K3X_ERR_INVALID_MXFP4;
    if (p->glu == K3X_GLU_SITU &&
        (!finite_pos(p->situ_beta) || (p->has_situ_linear && !finite_pos(p->situ_linear_beta))))
        return K3X_ERR_INVALID_MXFP4;
    if (all_experts)
        for (uint8_t r : bank->expert_ready)
            if (!r) return K3X_ERR_INVALID_STATE;
    if (d.shared_inter && !bank->shared_ready) return K3X_ERR_INVALID_STATE;
    return K3X_OK;
}

int launched(k3x_hip_ctx* ctx, unsigned n) {
    ctx->kernel_launches += n;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}


// ready (may be null): the bank's admitted-slot words; a route to another
// slot is latched as K3X_ERR_INVALID_STATE.
// The grouping of a small route (P = T * K <= kGroupSmallPairs pairs, no
// wide-GEMM work items) by one workgroup with the route in LDS: every output
// is a count over the P pairs, no pass goes through global memory.  For pair
// p = token * K + slot of expert e: rin = earlier pairs of e, below = pairs
// of smaller experts; its CSR row is below + rin (rows of one expert in pair
// order, as the count/scan/scatter kernels order them).  Per expert: counts,
// offsets (pairs of smaller experts; offsets[E] = P), first_use (its first
// pair, 0xffffffff unused).  The pair with rin = 0 places its expert in
// active_asc (rank among the first uses of smaller experts) and active_fu
// (rank among earlier first uses).  Validation as group_count_body: an id
// past E, a slot that holds no admitted expert, or an expert twice in one
// token latches K3X_ERR_INVALID_STATE.  arec: the active slot records of
// the decode kernels, {expert, rows, CSR offset, tokens of the first four
// rows (8 bits each)}, in active_asc order.
constexpr uint32_t kGroupSmallPairs = 256;
static_assert(kGroupSmallPairs == kTopkThrThreads, "the fused Top-K launch groups with its threads");

// ATOMIC: the ids are read at device scope (written in the same launch by
// other workgroups).
template <bool ATOMIC>
__device__ __forceinline__ void group_small_body(
    const uint32_t* __restrict__ ids, uint32_t T, uint32_t K, uint32_t E,
    const uint32_t* __restrict__ ready, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ offsets, uint32_t* __restrict__ first_use,
    uint32_t* __restrict__ n_active, uint32_t* __restrict__ active_asc,
    uint32_t* __restrict__ active_fu, uint32_t* __restrict__ pair_token,
    uint32_t* __restrict__ pair_slot, uint4* __restrict__ arec, uint32_t* status) {
    __shared__ __align__(16) uint32_t s_id[kGroupSmallPairs];   // 0xffffffff past P
    __shared__ __align__(16) uint32_t s_first[kGroupSmallPairs];  // 1: pair is its expert's first use
    __shared__ uint32_t prior;
    const uint32_t tid = threadIdx.x, P = T * K;
    if (tid == 0)
        prior = ATOMIC ? __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : *(volatile uint32_t*)status;
    uint32_t e = 0xffffffffu;
    if (tid < P)
        e = ATOMIC ? __hip_atomic_load(ids + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : ids[tid];
    s_id[tid] = e;
    __syncthreads();
    if (prior) return;
    const uint32_t tok = tid / K, slot = tid % K;
    int bad = tid < P && (e >= E || (ready && !ready[e]));
    if (tid < P)
        for (uint32_t q = 0; q < slot; ++q) bad |= s_id[tok * K + q] == e;
    if (__syncthreads_or(bad)) {
        if (tid == 0) latch(status, K3X_ERR_INVALID_STATE);
        return;
    }
    const uint4* id4 = reinterpret_cast<const uint4*>(s_id);
    uint32_t rin = 0, below = 0;
    if (tid < P) {
        for (uint32_t q0 = 0; q0 < P; q0 += 4) {  // entries past P hold 0xffffffff
            const uint4 v = id4[q0 / 4];
            const uint32_t f[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                rin += q0 + i < tid && f[i] == e;
                below += f[i] < e;
            }
        }
        pair_token[below + rin] = tok;
        pair_slot[below + rin] = slot;
    }
    s_first[tid] = tid < P && rin == 0;
    __syncthreads();
    if (tid < P && rin == 0) {
        uint32_t asc = 0, fu = 0, rows = 0, toks = 0;
        for (uint32_t q = 0; q < P; ++q) {
            if (s_id[q] == e) {  // the expert's rows in pair order (at most one per token)
                if (rows < 4) toks |= (q / K) << (8 * rows);
                ++rows;
            }
            if (!s_first[q]) continue;
            asc += s_id[q] < e;
            fu += q < tid;
        }
        active_asc[asc] = e;
        active_fu[fu] = e;
        if (arec) arec[asc] = make_uint4(e, rows, below, toks);
    }
    // Per expert: counts over the pairs (E * P / 256 comparisons a thread).
    for (uint32_t x = tid; x < E; x += kGroupSmallPairs) {
        uint32_t c = 0, b = 0, f = 0xffffffffu;
        for (uint32_t q0 = 0; q0 < P; q0 += 4) {
            const uint4 v = id4[q0 / 4];
            const uint32_t g[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                c += g[i] == x;
                b += g[i] < x;
                if (g[i] == x) f = min(f, q0 + i);
            }
        }
        counts[x] = c;
        offsets[x] = b;
        first_use[x] = f;
    }
    if (tid == 0) {
        offsets[E] = P;
        uint32_t na = 0;
        for (uint32_t q = 0; q < P; ++q) na += s_first[q];
        *n_active = na;
    }
}

__global__ __launch_bounds__(kGroupSmallPairs) void group_small_kernel(
    const uint32_t* __restrict__ ids, uint32_t T, uint32_t K, uint32_t E,
    const uint32_t* __restrict__ ready, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ offsets, uint32_t* __restrict__ first_use,
    uint32_t* __restrict__ n_active, uint32_t* __restrict__ active_asc,
    uint32_t* __restrict__ active_fu, uint32_t* __restrict__ pair_token,
    uint32_t* __restrict__ pair_slot, uint4* __restrict__ arec, uint32_t* status) {
    group_small_body<false>(ids, T, K, E, ready, counts, offsets, first_use, n_active, active_asc,
                            active_fu, pair_token, pair_slot, arec, status);
}

// The Top-K of T tokens (topk_thr_body, one workgroup a token) and the
// small-route grouping (group_small_body) in one launch: every workgroup
// publishes its token's ids at device scope, waits for the stores, and
// counts itself in; the workgroup whose count completes T groups all T * K
// pairs, reading the ids at device scope, then resets the counter to zero
// for the next launch.  Every workgroup counts itself, whatever its Top-K
// found (a latched error makes the grouping return at once), so the
// counter always completes and is left at zero.  No workgroup waits for
// another.
struct TopkGroupArgs {
    const float* logits;
    const float* bias;
    uint32_t E, K, T;
    float routed_scale;
    uint32_t renorm;
    uint32_t* ids;
    float* weights;
    const uint32_t* ready;
    uint32_t *counts, *offsets, *first_use, *n_active, *active_asc, *active_fu, *pair_token,
        *pair_slot;
    uint4* arec;
    uint32_t* counter;
    uint32_t* status;
};

// Token t's workgroup (t < T).
template <int EPT>
__device__ __forceinline__ void topk_group_body(const TopkGroupArgs& a, uint32_t t) {
    __shared__ uint32_t last;
    topk_thr_body<EPT, true>(a.logits, a.bias, a.E, a.K, a.routed_scale, a.renorm, a.ids,
                             a.weights, a.status, t);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               a.T - 1;
    __syncthreads();
    if (!last) return;  // block-uniform
    group_small_body<true>(a.ids, a.T, a.K, a.E, a.ready, a.counts, a.offsets, a.first_use,
                           a.n_active, a.active_asc, a.active_fu, a.pair_token, a.pair_slot,
                           a.arec, a.status);
    if (threadIdx.x == 0)
        __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int EPT>
__global__ __launch_bounds__(kTopkThrThreads) void topk_group_kernel(TopkGroupArgs a) {
    topk_group_body<EPT>(a, blockIdx.x);
}

// ---------------------------------------------------------------------------
// The official layer's few-token launches: each a set of roles by workgroup
// index, 256 threads a workgroup, every role reading only what an earlier
// launch wrote (so no workgroup waits for another role).
//   front   router logits (router_reg_body, 2 experts a workgroup); the
//           latent projection, bf16 out; the shared gate/up + GLU, split
//           [hi | lo] activation rows (a GEMV row block of 16 outputs a
//           workgroup, 4 waves over the K tiles);
//   select  the Top-K and grouping of topk_group_kernel (one workgroup a
//           token, the last to arrive groups); the shared down projection
//           over the split rows, fp32 out.
// The router's workgroups come first, then the Top-K's: the latency-bound
// route starts at once and the projections' weight streams fill the rest of
// the device meanwhile.
// ---------------------------------------------------------------------------
constexpr int kOfficialWaves = 4;
// One expert a router workgroup: router_reg_body<2, 2> alone takes 205
// VGPRs (two waves a SIMD), <1, 2> 110 (four), which the GEMV roles beside
// it need.
constexpr int kOfficialRouterEpb = 1;
static_assert(64 * kOfficialWaves == kTopkThrThreads, "one workgroup size for every role");

struct OfficialFrontArgs {
    const float* router;  // [E][H] fp32
    const uint16_t* hidden;
    uint32_t E, H, T;
    float* logits;
    GemvArgs latent;  // 1 matrix, bf16 out
    GemvArgs shared;  // gate + up, GLU out (tiles null: no shared FFN)
    uint32_t n_router, n_latent;
    const uint32_t* status;
};

template <int TPB>
__global__ __launch_bounds__(64 * kOfficialWaves) void official_front_kernel(OfficialFrontArgs a) {
    const uint32_t b = blockIdx.x;
    if (b < a.n_router)
        router_reg_body<kOfficialRouterEpb, TPB>(a.router, a.hidden, a.E, a.H, a.T, a.logits,
                                                 a.status, b);
    else if (b < a.n_router + a.n_latent)
        dense_gemv_body<1, 3, 1, kOfficialWaves, false>(a.latent, b - a.n_router);
    else
        dense_gemv_body<2, 2, 2, kOfficialWaves, false>(a.shared, b - a.n_router - a.n_latent);
}

struct OfficialSelectArgs {
    TopkGroupArgs route;
    GemvArgs shared_down;  // split rows, fp32 out (tiles null: none)
};

template <int EPT>
__global__ __launch_bounds__(64 * kOfficialWaves) void official_select_kernel(
    OfficialSelectArgs a) {
    if (blockIdx.x < a.route.T)
        topk_group_body<EPT>(a.route, blockIdx.x);
    else
        dense_gemv_body<1, 2, 0, kOfficialWaves, true>(a.shared_down, blockIdx.x - a.route.T);
}

int launch_group(k3x_hip_ctx* ctx, const uint32_t* ids, uint32_t T, uint32_t K, uint32_t E,
                 const uint32_t* ready, uint32_t* counts, uint32_t* offsets,
                 uint32_t* pair_token, uint32_t* pair_slot, uint32_t* first_use,
                 uint32_t* n_active, uint32_t* active_asc, uint32_t* active_fu,
                 uint8_t* gscratch, uint32_t* witems = nullptr, uint32_t* n_witems = nullptr,
                 uint4* arec = nullptr) {
    const uint32_t tps = std::min(64u, 1024u / K), nch = (T + tps - 1) / tps;
    uint32_t* chunk_cnt = reinterpret_cast<uint32_t*>(gscratch);
    uint32_t* chunk_fu = chunk_cnt + (size_t)nch * E;
    uint8_t* rank = reinterpret_cast<uint8_t*>(chunk_fu + (size_t)nch * E);
    if (!witems && T * K <= kGroupSmallPairs) {
        hipLaunchKernelGGL(group_small_kernel, dim3(1), dim3(kGroupSmallPairs), 0, ctx->stream,
                           ids, T, K, E, ready, counts, offsets, first_use, n_active, active_asc,
                           active_fu, pair_token, pair_slot, arec, ctx->status);
        return launched(ctx, 1);
    }
    if (nch == 1) {
        hipLaunchKernelGGL(group_single_kernel, dim3(1), dim3(1024), (size_t)(1024 + 3 * E) * 4,
                           ctx->stream, ids, T, K, E, ready, chunk_cnt, chunk_fu, rank, counts,
                           offsets,
                           first_use, n_active, active_asc, active_fu, witems, n_witems,
                           k3x_hip::kWideRows, arec, pair_token, pair_slot, ctx->status);
        return launched(ctx, 1);
    }
    hipLaunchKernelGGL(group_count_kernel, dim3(nch), dim3(1024), (size_t)(1024 + 3 * E) * 4,
                       ctx->stream, ids, T, K, E, ready, chunk_cnt, chunk_fu, rank, ctx->status);
    hipLaunchKernelGGL(group_scan_kernel, dim3(1), dim3(1024), (size_t)3 * E * 4, ctx->stream, T,
                       K, E, chunk_cnt, chunk_fu, counts, offsets, first_use, n_active, active_asc,
                       active_fu, witems, n_witems, k3x_hip::kWideRows, arec, ctx->status);
    hipLaunchKernelGGL(group_scatter_kernel, dim3(nch), dim3(1024), 0, ctx->stream, ids, T, K, E,
                       chunk_cnt, rank, offsets, pair_token, pair_slot, ctx->status);
    return launched(ctx, 3);
}

template <bool FP4, bool GATEUP, int MT, int NT>
void launch_gemm(k3x_hip_ctx* ctx, GemmArgs& g, uint32_t experts_in_grid, uint32_t rows,
                 hipStream_t stream = nullptr) {
    g.blocks_per_expert = rows / 16 / (4 * NT);
    const dim3 grid(experts_in_grid * g.blocks_per_expert);
    if (!stream) stream = ctx->stream;
    if (g.a_lo)
        hipLaunchKernelGGL((expert_gemm<FP4, GATEUP, MT, NT, true>), grid, dim3(256), 0, stream,
                           g);
    else
        hipLaunchKernelGGL((expert_gemm<FP4, GATEUP, MT, NT, false>), grid, dim3(256), 0, stream,
                           g);
}

// The shared expert below the wide GEMM's row counts: gate/up + GLU -> sact,
// down -> sy, each as one block of T rows on the narrow GEMM, on `stream`
// (stage marks only on the context stream).
int run_shared_narrow(k3x_hip_ctx* ctx, const k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                      const Scratch& s, const uint16_t* xn, const GluParams& glu, bool split_in,
                      hipStream_t stream) {
    const auto& d = bank->desc;
    const uint32_t T = p->tokens;
    const bool wide = T > 16;  // more than one 16-row MFMA tile
    const bool marks = stream == ctx->stream;
    GemmArgs sg{};
    sg.status = ctx->status;
    sg.glu = glu;
    sg.top_k = p->top_k;
    sg.codes = bank->sh_gu;
    sg.kt = bank->sgate.kt;
    sg.a = xn;
    sg.a_stride = split_in ? 2 * d.hidden : d.hidden;
    sg.a_lo = split_in ? d.hidden : 0;
    sg.tokens = T;
    sg.act = s.sact;
    sg.act_stride = d.shared_inter;
    sg.act_lo = 0;  // the bank's shared expert keeps bf16 activations
    int mark = marks ? begin_stage(ctx, K3X_STAGE_SHARED_GATE_UP) : -1;
    if (wide) launch_gemm<false, true, 4, 1>(ctx, sg, 1, d.shared_inter, stream);
    else launch_gemm<false, true, 1, 1>(ctx, sg, 1, d.shared_inter, stream);
    if (marks) end_stage(ctx, mark);
    GemmArgs sd = sg;
    sd.codes = bank->sh_dn;
    sd.kt = bank->sdown.kt;
    sd.a = s.sact;
    sd.a_stride = d.shared_inter;
    sd.a_lo = 0;
    sd.y = s.sy;
    sd.y_stride = d.hidden;
    sd.scatter = 0;
    mark = marks ? begin_stage(ctx, K3X_STAGE_SHARED_DOWN) : -1;
    if (wide) launch_gemm<false, false, 4, 2>(ctx, sd, 1, d.hidden, stream);
    else launch_gemm<false, false, 1, 2>(ctx, sd, 1, d.hidden, stream);
    if (marks) end_stage(ctx, mark);
    return launched(ctx, 2);
}

// Many rows per expert: the wide grouped GEMM (128-row chunks, activations
// staged in LDS) for the routed and the shared expert.  Shapes it needs: K
// tile counts even, output rows a multiple of the workgroup's row blocks,
// element offsets of the activation rows below 2^32.
bool use_wide_gemm(const k3x_hip_layer_desc& d, uint32_t T, uint32_t K, bool split) {
    using k3x_hip::wide_rb_per_block;
    constexpr uint32_t kq = 128 * k3x_hip::kWideStages;  // K extents: whole pipeline blocks
    const uint64_t rows = (uint64_t)T * K;
    // Activation and weight byte offsets are 32-bit (buffer loads).
    return T >= kWideMinTokens && d.hidden % kq == 0 && d.inter % kq == 0 &&
           (d.inter / 16) % wide_rb_per_block(k3x_hip::kWideRoutedGateUp) == 0 &&
           (d.hidden / 16) % wide_rb_per_block(k3x_hip::kWideRoutedDown) == 0 &&
           (!d.shared_inter ||
            (d.shared_inter % kq == 0 &&
             (d.shared_inter / 16) % wide_rb_per_block(k3x_hip::kWideSharedGateUp) == 0 &&
             (d.hidden / 16) % wide_rb_per_block(k3x_hip::kWideSharedDown) == 0)) &&
           rows * std::max(d.hidden, std::max(d.inter * (split ? 2 : 1), d.shared_inter)) * 2 <
               (1ull << 32) &&
           // weight byte offsets within one matrix pair are 32-bit as well
           (uint64_t)std::max(d.inter, d.shared_inter) * d.hidden * 4 < (1ull << 32);
}

// Arguments of the routed gate/up launch; the other three derive from them.
k3x_hip::WideGemmArgs wide_gate_up_args(k3x_hip_ctx* ctx, const k3x_hip_bank* bank,
                                        const k3x_hip_moe_params* p, const Scratch& s,
                                        const uint16_t* xn, const GluParams& glu) {
    const auto& d = bank->desc;
    const uint32_t T = p->tokens, K = p->top_k;
    k3x_hip::WideGemmArgs g{};
    g.items = s.witems;
    g.n_items = s.n_witems;
    g.status = ctx->status;
    g.glu = glu;
    g.top_k = K;
    g.counts = s.counts;
    g.offsets = s.offsets;
    g.pair_token = s.pair_token;
    g.pair_slot = s.pair_slot;
    g.codes = bank->gu_codes;
    g.scales = bank->gu_scales;
    g.codes_per_expert = bank->gu_codes_per_expert;
    g.scales_per_expert = bank->gu_scales_per_expert;
    g.kt = bank->gate.kt;
    g.ks = bank->gate.ks;
    g.nrb = d.inter / 16;
    g.a = xn;
    g.a_stride = d.hidden;
    g.a_bytes = T * d.hidden * 2;
    g.gather = 1;
    g.act = s.act;
    const bool split = (p->flags & K3X_FLAG_SPLIT_ACT) != 0;
    g.act_stride = split ? 2 * d.inter : d.inter;
    g.act_lo = split ? d.inter : 0;
    return g;
}

// The shared expert on the wide GEMM: gate/up + GLU -> sact, down -> sy, on
// `stream` (stage marks only on the context stream).
int run_shared_wide(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                    const Scratch& s, const uint16_t* xn, const GluParams& glu,
                    hipStream_t stream) {
    using namespace k3x_hip;
    const auto& d = bank->desc;
    const uint32_t T = p->tokens;
    const uint32_t all_chunks = (T + kWideRows - 1) / kWideRows;
    const bool marks = stream == ctx->stream;
    WideGemmArgs sg = wide_gate_up_args(ctx, bank, p, s, xn, glu);
    sg.codes = bank->sh_gu;
    sg.scales = nullptr;
    sg.codes_per_expert = 0;
    sg.kt = bank->sgate.kt;
    sg.nrb = d.shared_inter / 16;
    sg.gather = 0;
    sg.items = nullptr;
    sg.tokens = T;
    sg.act = s.sact;
    sg.act_stride = d.shared_inter;
    sg.act_lo = 0;  // the bank's shared expert keeps bf16 activations
    int mark = marks ? begin_stage(ctx, K3X_STAGE_SHARED_GATE_UP) : -1;
    int st = launch_wide_gemm(ctx, kWideSharedGateUp, sg, all_chunks, stream);
    end_stage(ctx, mark);
    if (st) return st;
    WideGemmArgs sd = sg;
    sd.codes = bank->sh_dn;
    sd.kt = bank->sdown.kt;
    sd.nrb = d.hidden / 16;
    sd.a = s.sact;
    sd.a_stride = d.shared_inter;
    sd.a_bytes = T * d.shared_inter * 2;
    sd.act = nullptr;
    sd.y = s.sy;
    sd.y_stride = d.hidden;
    sd.scatter = 0;
    mark = marks ? begin_stage(ctx, K3X_STAGE_SHARED_DOWN) : -1;
    st = launch_wide_gemm(ctx, kWideSharedDown, sd, all_chunks, stream);
    end_stage(ctx, mark);
    return st;
}

// Routed gate/up + GLU, then down; with shared_inline the shared expert's
// GEMMs run on the context stream after each routed one.  The routed GEMMs
// run per size class of the grouping's items (kWideClasses): classes 0 (full
// chunks) and 1 (last chunks of 65-96 rows) on the context stream; classes 2
// and 3 (last chunks at 4 and 2 row tiles) on the side stream beside them
// (behind the shared expert's GEMMs when they run there), forked after the
// grouping and joined before the return -- a class's down GEMM needs only its
// own gate/up rows.  In line with stage profiling and with q8 rows (quantised
// for every class at once on the context stream).
int run_wide(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
             const Scratch& s, const uint16_t* xn, const GluParams& glu, bool shared_inline) {
    using namespace k3x_hip;
    const auto& d = bank->desc;
    const uint32_t T = p->tokens, K = p->top_k;
    // Routed: one workgroup column per (expert, 128-row chunk) item the
    // grouping listed, up to wide_max_items in class 0 and one an active
    // expert (its last chunk) in each of the others.
    const uint32_t routed_chunks = wide_max_items(d, T, K);
    const uint32_t last_chunks = std::min(routed_chunks, std::min(d.experts, T * K));
    // q8 rows are quantised for all classes at once on the context stream.
    const bool q8 = s.qx != nullptr;
    const bool beside = !ctx->profiling && ctx->side_stream && !q8;
    hipStream_t cstream = beside ? ctx->side_stream : ctx->stream;
    struct ClassJoin {
        k3x_hip_ctx* ctx;
        bool armed = false;
        int join() {
            if (!armed) return K3X_OK;
            armed = false;
            if (hipEventRecord(ctx->class_join_ev, ctx->side_stream) != hipSuccess) {
                (void)hipStreamSynchronize(ctx->side_stream);
                return K3X_ERR_BACKEND_UNAVAILABLE;
            }
            return hipStreamWaitEvent(ctx->stream, ctx->class_join_ev, 0) == hipSuccess
                       ? K3X_OK
                       : K3X_ERR_BACKEND_UNAVAILABLE;
        }
        ~ClassJoin() { (void)join(); }
    } cjoin{ctx};
    if (beside) {
        if (hipEventRecord(ctx->class_fork_ev, ctx->stream) != hipSuccess ||
            hipStreamWaitEvent(ctx->side_stream, ctx->class_fork_ev, 0) != hipSuccess)
            return K3X_ERR_BACKEND_UNAVAILABLE;
        cjoin.armed = true;
    }
    // Classes 0 and 1 on the context stream, 2 and 3 beside them (class 1
    // beside as well left the side stream finishing last: prefill c5
    // 3594-3624 against 3571-3610 us, the official layer at T=2048 5512-5530
    // against 5415-5428; class 2 moved too, c5 3679-3704).
    auto beside_class = [](int c) { return c >= 2; };
    auto routed = [&](WideKind kind, const WideGemmArgs& a, bool main) {
        int r = K3X_OK;
        for (int c = 0; !r && c < (int)kWideClasses; ++c)
            if (beside_class(c) != main)
                r = launch_wide_gemm(ctx, kind, a, c ? last_chunks : routed_chunks,
                                     main ? ctx->stream : cstream, c);
        return r;
    };
    WideGemmArgs g = wide_gate_up_args(ctx, bank, p, s, xn, glu);
    // Scaled FP4: the experts read q8 rows of xn, then of act (quantised
    // in the stage that consumes them).
    int mark = begin_stage(ctx, K3X_STAGE_GATE_UP);
    int st = K3X_OK;
    if (q8) {
        st = launch_q8_rows(ctx, xn, T, d.hidden, d.hidden, s.qx, s.qxs);
        g.a = s.qx;
        g.qs = s.qxs;
        g.qs_bytes = T * (d.hidden / 128) * 8;
    }
    if (!st) st = routed(kWideRoutedGateUp, g, false);
    if (!st) st = routed(kWideRoutedGateUp, g, true);
    end_stage(ctx, mark);
    if (st) return st;
    if (shared_inline && d.shared_inter &&
        (st = run_shared_wide(ctx, bank, p, s, xn, glu, ctx->stream)))
        return st;
    WideGemmArgs dn = g;
    dn.codes = bank->dn_codes;
    dn.scales = bank->dn_scales;
    dn.codes_per_expert = bank->dn_codes_per_expert;
    dn.scales_per_expert = bank->dn_scales_per_expert;
    dn.kt = bank->down.kt;
    dn.ks = bank->down.ks;
    dn.nrb = d.hidden / 16;
    dn.a = s.act;
    dn.a_stride = g.act_stride;
    dn.a_bytes = T * K * g.act_stride * 2;
    dn.kta = g.act_lo ? 2 * dn.kt : 0;
    dn.gather = 0;
    dn.act = nullptr;
    dn.y = s.y;
    dn.y_stride = d.hidden;
    dn.scatter = 1;
    dn.qs = nullptr;
    mark = begin_stage(ctx, K3X_STAGE_DOWN);
    if (q8) {
        st = launch_q8_rows(ctx, s.act, T * K, d.inter, d.inter, s.qact, s.qacts);
        dn.a = s.qact;
        dn.qs = s.qacts;
        dn.qs_bytes = T * K * (d.inter / 128) * 8;
    }
    if (!st) st = routed(kWideRoutedDown, dn, false);
    if (!st) st = routed(kWideRoutedDown, dn, true);
    end_stage(ctx, mark);
    const int jst = cjoin.join();
    return st ? st : jst;
}

// Grouping, expert GEMMs, shared expert, combine.  xn is the bf16 input of
// the experts; ids/weights [T][K] device.
// Whether a call's shared expert runs on the context's second stream: the
// wide path (the routed GEMMs run for milliseconds) and the verification
// windows on the decode kernels (hundreds of microseconds of routed
// streaming beside a few dozen shared workgroups).  With stage profiling on,
// everything stays on the context stream.
bool shared_on_side(const k3x_hip_ctx* ctx, const k3x_hip_bank* bank, const k3x_hip_moe_params* p) {
    const auto& d = bank->desc;
    const uint32_t T = p->tokens, K = p->top_k;
    const bool split = (p->flags & K3X_FLAG_SPLIT_ACT) != 0;
    const bool split_in = (p->flags & K3X_FLAG_SPLIT_INPUT) != 0;
    const bool wide_path = !split_in && use_wide_gemm(d, T, K, split);
    const bool chunked_rows = !wide_path && !split_in && T > k3x_hip::kMaxDecodeTokens &&
                              T <= k3x_hip::kChunkedMaxTokens &&
                              k3x_hip::few_row_experts_eligible(ctx, bank,
                                                                k3x_hip::kMaxDecodeTokens, split);
    return (wide_path || chunked_rows) && d.shared_inter && !ctx->profiling && ctx->side_stream;
}

// Launches the shared expert on the second stream after the context
// stream's work so far (it needs xn only) and records the event the context
// stream joins on.
int fork_shared(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                const Scratch& s, const uint16_t* xn, const GluParams& glu) {
    const auto& d = bank->desc;
    const bool split = (p->flags & K3X_FLAG_SPLIT_ACT) != 0;
    const bool split_in = (p->flags & K3X_FLAG_SPLIT_INPUT) != 0;
    const bool wide_path = !split_in && use_wide_gemm(d, p->tokens, p->top_k, split);
    if (hipEventRecord(ctx->fork_ev, ctx->stream) != hipSuccess ||
        hipStreamWaitEvent(ctx->side_stream, ctx->fork_ev, 0) != hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    const int sst = wide_path ? run_shared_wide(ctx, bank, p, s, xn, glu, ctx->side_stream)
                              : run_shared_narrow(ctx, bank, p, s, xn, glu, split_in,
                                                  ctx->side_stream);
    if (hipEventRecord(ctx->join_ev, ctx->side_stream) != hipSuccess) {
        // Without the event, order the streams the blunt way.
        (void)hipStreamSynchronize(ctx->side_stream);
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    return sst;
}

// forked: the caller has already launched the shared expert on the second
// stream (fork_shared); the context stream still joins it before the
// combine and on every return.
int run_tail(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
             const Scratch& s, const uint16_t* xn, const uint32_t* ids, const float* weights,
             uint16_t* out, float* out_f32, bool forked = false) {
    const auto& d = bank->desc;
    const uint32_t T = p->tokens, K = p->top_k;
    GluParams glu{(int)p->glu, p->situ_beta, (int)p->has_situ_linear, p->situ_linear_beta};
    // Wide path with a shared expert: its GEMMs depend only on xn, so they
    // go to the side stream now and run beside the grouping and the routed
    // GEMMs (filling the small grouping launches and the routed GEMMs'
    // tails); the context stream waits for them before the combine, and on
    // every early return (they read and write this call's scratch).  With
    // stage profiling on, everything stays on the context stream.
    const bool split = (p->flags & K3X_FLAG_SPLIT_ACT) != 0;
    // Split input rows [hi | lo] (2 H): the narrow GEMMs, gate/up over both
    // halves.
    const bool split_in = (p->flags & K3X_FLAG_SPLIT_INPUT) != 0;
    const bool wide_path = !split_in && use_wide_gemm(d, T, K, split);
    // Verification windows on the decode kernels (below): the routed experts
    // stream for hundreds of microseconds, the shared expert's narrow GEMMs
    // run a few dozen workgroups; on the side stream they overlap.
    const bool chunked_rows = !wide_path && !split_in && T > k3x_hip::kMaxDecodeTokens &&
                              T <= k3x_hip::kChunkedMaxTokens &&
                              k3x_hip::few_row_experts_eligible(ctx, bank,
                                                                k3x_hip::kMaxDecodeTokens, split);
    const bool side = shared_on_side(ctx, bank, p);
    struct Join {
        k3x_hip_ctx* ctx;
        bool armed = false;
        int join() {
            if (!armed) return K3X_OK;
            armed = false;
            return hipStreamWaitEvent(ctx->stream, ctx->join_ev, 0) == hipSuccess
                       ? K3X_OK
                       : K3X_ERR_BACKEND_UNAVAILABLE;
        }
        ~Join() { (void)join(); }
    } joiner{ctx};
    if (side) {
        joiner.armed = true;
        if (!forked) {
            const int sst = fork_shared(ctx, bank, p, s, xn, glu);
            if (sst) return sst;
        }
    }
    int mark = begin_stage(ctx, K3X_STAGE_GROUP);
    // Work items of the wide GEMM only where it runs (without them a small
    // route is grouped by one workgroup).
    // Few tokens: the routed experts on the decode path's kernels, fed by
    // the active-slot records of the small-route grouping.
    // Up to kChunkedMaxTokens tokens (verification windows): the same
    // kernels over slots of any size, rows through LDS a few at a time.
    const bool few = !wide_path && !split_in && T * K <= kGroupSmallPairs &&
                     k3x_hip::few_row_experts_eligible(ctx, bank, T, split);
    const bool chunked = !few && chunked_rows;
    // A route grouped with its Top-K (topk_group_kernel) holds what the
    // small-route grouping below would write: no wide path there.
    if (s.grouped && (wide_path || T * K > kGroupSmallPairs)) return K3X_ERR_INVALID_EXTENT;
    int st = s.grouped ? K3X_OK
                       : launch_group(ctx, ids, T, K, d.experts, bank->ready_dev, s.counts,
                                      s.offsets, s.pair_token, s.pair_slot, s.first_use,
                                      s.n_active, s.active_asc, s.active_fu, s.gscratch,
                                      wide_path ? s.witems : nullptr,
                                      wide_path ? s.n_witems : nullptr,
                                      few || chunked ? s.arec : nullptr);
    end_stage(ctx, mark);
    if (st) return st;
    const uint32_t max_active = std::min<uint32_t>(d.experts, T * K);
    const bool wide = T > 16;  // more than one 16-row MFMA tile per expert possible
    if (wide_path) {
        if ((st = run_wide(ctx, bank, p, s, xn, glu, !side))) return st;
        if ((st = joiner.join())) return st;
        return k3x_hip::launch_combine(ctx, s.y, weights, d.shared_inter ? s.sy : nullptr, K,
                                       d.hidden, T, out, out_f32,
                                       (p->flags & K3X_FLAG_ROUND_EXPERT_OUT) != 0);
    }

    GemmArgs g{};
    g.status = ctx->status;
    g.glu = glu;
    g.top_k = K;
    // Routed gate/up + GLU.
    g.codes = bank->gu_codes;
    g.scales = bank->gu_scales;
    g.codes_per_expert = bank->gu_codes_per_expert;
    g.scales_per_expert = bank->gu_scales_per_expert;
    g.kt = bank->gate.kt;
    g.ks = bank->gate.ks;
    g.a = xn;
    g.a_stride = split_in ? 2 * d.hidden : d.hidden;
    g.a_lo = split_in ? d.hidden : 0;
    g.gather = 1;
    g.n_active = s.n_active;
    g.active = s.active_asc;
    g.counts = s.counts;
    g.offsets = s.offsets;
    g.pair_token = s.pair_token;
    g.pair_slot = s.pair_slot;
    g.act = s.act;
    g.act_stride = split ? 2 * d.inter : d.inter;
    g.act_lo = split ? d.inter : 0;
    mark = begin_stage(ctx, K3X_STAGE_GATE_UP);
    if (few || chunked) {
        if ((st = k3x_hip::launch_few_row_gate_up(ctx, bank, T, K, s, xn, glu, split, chunked)))
            return st;
    } else if (wide) {
        launch_gemm<true, true, 4, 1>(ctx, g, max_active, d.inter);
    } else {
        launch_gemm<true, true, 1, 1>(ctx, g, max_active, d.inter);
    }
    end_stage(ctx, mark);
    // Routed down, scattered to [token][slot].
    GemmArgs dn = g;
    dn.codes = bank->dn_codes;
    dn.scales = bank->dn_scales;
    dn.codes_per_expert = bank->dn_codes_per_expert;
    dn.scales_per_expert = bank->dn_scales_per_expert;
    dn.kt = bank->down.kt;
    dn.ks = bank->down.ks;
    dn.a = s.act;
    dn.a_stride = g.act_stride;
    dn.a_lo = split ? d.inter : 0;
    dn.gather = 0;
    dn.y = s.y;
    dn.y_stride = d.hidden;
    dn.scatter = 1;
    // Few tokens: the combine rides in the down launch (the decode path's
    // fused mix), after the shared expert, whose output it adds.
    if (few && k3x_hip::few_row_mix_eligible(bank, T)) {
        if (d.shared_inter && !side &&
            (st = run_shared_narrow(ctx, bank, p, s, xn, glu, split_in, ctx->stream)))
            return st;
        if ((st = joiner.join())) return st;
        const k3x_hip::FewRowMix mix{weights, d.shared_inter ? s.sy : nullptr, out, out_f32,
                                     (p->flags & K3X_FLAG_ROUND_EXPERT_OUT) != 0};
        mark = begin_stage(ctx, K3X_STAGE_DOWN);
        st = k3x_hip::launch_few_row_down(ctx, bank, T, K, s, split, false, &mix);
        end_stage(ctx, mark);
        return st;
    }
    mark = begin_stage(ctx, K3X_STAGE_DOWN);
    if (few || chunked) {
        if ((st = k3x_hip::launch_few_row_down(ctx, bank, T, K, s, split, chunked))) return st;
    } else if (wide) {
        launch_gemm<true, false, 4, 2>(ctx, dn, max_active, d.hidden);
    } else {
        launch_gemm<true, false, 1, 2>(ctx, dn, max_active, d.hidden);
    }
    end_stage(ctx, mark);
    if ((st = launched(ctx, few || chunked ? 0 : 2))) return st;
    if (d.shared_inter && !side &&
        (st = run_shared_narrow(ctx, bank, p, s, xn, glu, split_in, ctx->stream)))
        return st;
    if ((st = joiner.join())) return st;
    return k3x_hip::launch_combine(ctx, s.y, weights, d.shared_inter ? s.sy : nullptr, K,
                                   d.hidden, T, out, out_f32,
                                       (p->flags & K3X_FLAG_ROUND_EXPERT_OUT) != 0);
}

int copy_taps(k3x_hip_ctx* ctx, const k3x_hip_bank* bank, const k3x_hip_moe_params* p,
              const Scratch& s, const uint16_t* xn, const uint32_t* ids, const float* weights,
              const k3x_hip_moe_taps* taps) {
    if (!taps) return K3X_OK;
    const auto& d = bank->desc;
    const size_t T = p->tokens, K = p->top_k, P = T * K, E = d.experts;
    const bool split = (p->flags & K3X_FLAG_SPLIT_ACT) != 0;
    // Split rows [hi | lo]: the taps receive the hi halves.
    if ((p->flags & K3X_FLAG_SPLIT_INPUT) && taps->normed_x && taps->normed_x != xn &&
        hipMemcpy2DAsync(taps->normed_x, d.hidden * 2, xn, d.hidden * 4, d.hidden * 2, T,
                         hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    if (split && taps->act &&
        hipMemcpy2DAsync(taps->act, d.inter * 2, s.act, d.inter * 4, d.inter * 2, P,
                         hipMemcpyDeviceToDevice, ctx->stream) != hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    struct Item { void* dst; const void* src; size_t bytes; };
    const Item items[] = {
        {taps->normed_x, (p->flags & K3X_FLAG_SPLIT_INPUT) ? nullptr : xn, T * d.hidden * 2},
        {taps->logits, s.logits, T * E * 4},
        {taps->ids, ids, P * 4},
        {taps->weights, weights, P * 4},
        {taps->counts, s.counts, E * 4},
        {taps->offsets, s.offsets, (E + 1) * 4},
        {taps->pair_token, s.pair_token, P * 4},
        {taps->pair_slot, s.pair_slot, P * 4},
        {taps->first_use, s.first_use, E * 4},
        {taps->n_active, s.n_active, 4},
        {taps->active_first_use, s.active_fu, E * 4},
        {taps->act, split ? nullptr : s.act, P * d.inter * 2},
        {taps->expert_out, s.y, P * d.hidden * 4},
        {taps->shared_out, d.shared_inter ? s.sy : nullptr, T * d.hidden * 4},
        {taps->shared_act, d.shared_inter ? s.sact : nullptr, T * d.shared_inter * 2},
    };
    for (const auto& it : items) {
        if (!it.dst || !it.src || it.dst == it.src) continue;
        if (hipMemcpyAsync(it.dst, it.src, it.bytes, hipMemcpyDeviceToDevice, ctx->stream) !=
            hipSuccess)
            return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    return K3X_OK;
}

// Router logits of T rows of xn: router_mfma_kernel when the residue-major
// router copy Wp is given (xp then already holds, or -- pack -- is made to
// hold, the residue-major copy of xn), the register kernel for up to four
// rows of at most kRouterMaxHidden, else the loop or tile kernel.  All of
// them produce the same canonical fp64 logits.
int launch_router(k3x_hip_ctx* ctx, const float* W, const float* Wp, const uint16_t* xn,
                  uint16_t* xp, uint32_t E, uint32_t H, uint32_t T, float* logits,
                  bool pack = false) {
    if (Wp) {
        if (H > kRouterMaxHidden) return K3X_ERR_INVALID_EXTENT;
        if (pack)
            hipLaunchKernelGGL(xp_pack_kernel, dim3(T), dim3(256), 0, ctx->stream, xn, H, xp);
        const dim3 grid((E + 15) / 16, (T + 15) / 16);
        const uint32_t nm = (H + 4 * kRouterRes - 1) / (4 * kRouterRes);
        switch (nm) {
#define K3X_ROUTER_NM(n)                                                                        \
    case n:                                                                                     \
        hipLaunchKernelGGL((router_mfma_kernel<n, kRouterWaves>), grid, dim3(64 * kRouterWaves), \
                           0, ctx->stream, Wp, xp, E, T, logits, ctx->status);                  \
        break;
            K3X_ROUTER_NM(1) K3X_ROUTER_NM(2) K3X_ROUTER_NM(3) K3X_ROUTER_NM(4)
            K3X_ROUTER_NM(5) K3X_ROUTER_NM(6) K3X_ROUTER_NM(7) K3X_ROUTER_NM(8)
#undef K3X_ROUTER_NM
            default: return K3X_ERR_INVALID_EXTENT;
        }
        return launched(ctx, pack ? 2 : 1);
    }
    if (T <= 4 && H <= kRouterMaxHidden) {
        const dim3 grid((E + 1) / 2);
        if (T == 1)
            hipLaunchKernelGGL((router_reg_kernel<2, 1>), grid, dim3(256), 0, ctx->stream, W, xn,
                               E, H, T, logits, ctx->status);
        else if (T == 2)
            hipLaunchKernelGGL((router_reg_kernel<2, 2>), grid, dim3(256), 0, ctx->stream, W, xn,
                               E, H, T, logits, ctx->status);
        else
            hipLaunchKernelGGL((router_reg_kernel<2, 4>), grid, dim3(256), 0, ctx->stream, W, xn,
                               E, H, T, logits, ctx->status);
    } else if (T <= 4) {
        hipLaunchKernelGGL((router_kernel<1, 4>), dim3(E, 1), dim3(256), 0, ctx->stream, W, xn, E,
                           H, T, logits, ctx->status);
    } else {
        hipLaunchKernelGGL((router_tile_kernel<kRouterEpb, kRouterTpb, 4>),
                           dim3((E + kRouterEpb - 1) / kRouterEpb, (T + kRouterTpb - 1) / kRouterTpb),
                           dim3(256), 0, ctx->stream, W, xn, E, H, T, logits, ctx->status);
    }
    return launched(ctx, 1);
}

// Top-K of T rows of logits: for few tokens the threshold kernel (257 to
// 1024 experts), else the register kernel up to 1024 experts.
int launch_topk_any(k3x_hip_ctx* ctx, const float* logits, const float* bias, uint32_t E,
                    uint32_t K, uint32_t T, float routed_scale, uint32_t renorm, uint32_t* ids,
                    float* weights) {
#define K3X_TOPK(kpl)                                                                          \
    hipLaunchKernelGGL(topk_reg_kernel<kpl>, dim3(T), dim3(64), 0, ctx->stream, logits, bias, E, \
                       K, routed_scale, renorm, ids, weights, ctx->status)
#define K3X_TOPK_THR(ept)                                                                      \
    hipLaunchKernelGGL(topk_thr_kernel<ept>, dim3(T), dim3(kTopkThrThreads), 0, ctx->stream,    \
                       logits, bias, E, K, routed_scale, renorm, ids, weights, ctx->status)
    if (T <= kTopkThrMaxTokens && E > 256 && E <= 512) K3X_TOPK_THR(2);
    else if (T <= kTopkThrMaxTokens && E > 512 && E <= 1024) K3X_TOPK_THR(4);
#undef K3X_TOPK_THR
    else if (E <= 256) K3X_TOPK(4);
    else if (E <= 512) K3X_TOPK(8);
    else if (E <= 1024) K3X_TOPK(16);
#undef K3X_TOPK
    else
        hipLaunchKernelGGL(topk_kernel, dim3(T), dim3(64), (size_t)E * 12, ctx->stream, logits,
                           bias, E, K, routed_scale, renorm, ids, weights, ctx->status);
    return launched(ctx, 1);
}

// The fused Top-K and grouping launch (topk_group_kernel) over the routed
// call's grouping buffers and the context's arrival counter.
int launch_topk_group_impl(k3x_hip_ctx* ctx, const float* logits, const float* bias, uint32_t E,
                           uint32_t K, uint32_t T, float routed_scale, uint32_t renorm,
                           uint32_t* ids, float* weights, const uint32_t* ready,
                           const Scratch& s) {
    TopkGroupArgs a{logits,        bias,        E,         K,           T,
                    routed_scale,  renorm,      ids,       weights,     ready,
                    s.counts,      s.offsets,   s.first_use, s.n_active, s.active_asc,
                    s.active_fu,   s.pair_token, s.pair_slot, s.arec,    ctx->route_counter,
                    ctx->status};
    if (E <= 512)
        hipLaunchKernelGGL(topk_group_kernel<2>, dim3(T), dim3(kTopkThrThreads), 0, ctx->stream,
                           a);
    else
        hipLaunchKernelGGL(topk_group_kernel<4>, dim3(T), dim3(kTopkThrThreads), 0, ctx->stream,
                           a);
    return launched(ctx, 1);
}

int prepare(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p, Scratch* s) {
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    const bool split = (p->flags & K3X_FLAG_SPLIT_ACT) != 0;
    const bool q8 = scaled_fp4(p);
    const size_t need = carve(nullptr, bank->desc, p->tokens, p->top_k, split, q8, s);
    int st = k3x_hip::ensure_scratch(ctx, need);
    if (st) return st;
    carve(static_cast<uint8_t*>(ctx->scratch), bank->desc, p->tokens, p->top_k, split, q8, s);
    s->mix = ctx->mix_counts;
    return K3X_OK;
}

}  // namespace

namespace k3x_hip {

int permute_router_matrix(k3x_hip_ctx* ctx, const float* W, uint32_t E, uint32_t H, float* Wp) {
    const size_t n = router_wp_floats(E);
    hipLaunchKernelGGL(permute_router_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       ctx->stream, W, E, H, Wp);
    return launched(ctx, 1);
}

int permute_router(k3x_hip_bank* bank) {
    const auto& d = bank->desc;
    if (!bank->router_wp) return K3X_OK;
    return permute_router_matrix(bank->ctx, bank->router_w, d.experts, d.hidden, bank->router_wp);
}

bool router_mfma_eligible(uint32_t hidden) { return hidden <= kRouterMaxHidden; }

bool official_decode_eligible(uint32_t E, uint32_t H, uint32_t L, uint32_t I_s, uint32_t K,
                              uint32_t T) {
    return T >= 1 && T <= 4 && topk_group_eligible(E, K, T) && H <= kRouterMaxHidden &&
           !router_uses_mfma(H, T) && H % 128 == 0 && L % 128 == 0 && I_s % 128 == 0;
}

int launch_official_front(k3x_hip_ctx* ctx, const OfficialDecode& d) {
    if (!official_decode_eligible(d.E, d.H, d.L, d.I_s, d.K, d.T)) return K3X_ERR_INVALID_EXTENT;
    OfficialFrontArgs a{};
    a.router = d.router;
    a.hidden = d.hidden;
    a.E = d.E;
    a.H = d.H;
    a.T = d.T;
    a.logits = d.logits;
    a.latent = GemvArgs{d.latent_tiles, d.H / 128, d.hidden, d.H, d.T, d.latent, d.L, {},
                        ctx->status};
    a.shared = GemvArgs{d.shared_gu, d.H / 128, d.hidden, d.H, d.T, d.sact, 2 * d.I_s, d.glu,
                        ctx->status};
    a.shared.out_lo = d.I_s;
    a.n_router = (d.E + kOfficialRouterEpb - 1) / kOfficialRouterEpb;
    a.n_latent = d.L / 16;
    a.status = ctx->status;
    const dim3 grid(a.n_router + a.n_latent + d.I_s / 16), block(64 * kOfficialWaves);
    if (d.T == 1)
        hipLaunchKernelGGL(official_front_kernel<1>, grid, block, 0, ctx->stream, a);
    else if (d.T == 2)
        hipLaunchKernelGGL(official_front_kernel<2>, grid, block, 0, ctx->stream, a);
    else
        hipLaunchKernelGGL(official_front_kernel<4>, grid, block, 0, ctx->stream, a);
    return launched(ctx, 1);
}

int launch_official_select(k3x_hip_ctx* ctx, const OfficialDecode& d, const LayerBuffers& s) {
    if (!official_decode_eligible(d.E, d.H, d.L, d.I_s, d.K, d.T) || !ctx->route_counter)
        return K3X_ERR_INVALID_EXTENT;
    OfficialSelectArgs a{};
    a.route = TopkGroupArgs{d.logits,   d.correction, d.E,          d.K,          d.T,
                            1.0f,       K3X_RENORM_DOUBLE, d.ids,   d.weights,    d.ready,
                            s.counts,   s.offsets,    s.first_use,  s.n_active,   s.active_asc,
                            s.active_fu, s.pair_token, s.pair_slot, s.arec,       ctx->route_counter,
                            ctx->status};
    a.shared_down = GemvArgs{d.shared_dn, d.I_s / 128, d.sact, 2 * d.I_s, d.T, d.shared, d.H, {},
                             ctx->status};
    a.shared_down.x_lo = d.I_s;
    const dim3 grid(d.T + (d.I_s ? d.H / 16 : 0)), block(64 * kOfficialWaves);
    if (d.E <= 512)
        hipLaunchKernelGGL(official_select_kernel<2>, grid, block, 0, ctx->stream, a);
    else
        hipLaunchKernelGGL(official_select_kernel<4>, grid, block, 0, ctx->stream, a);
    return launched(ctx, 1);
}

bool topk_group_eligible(uint32_t E, uint32_t K, uint32_t T) {
    return E > 256 && E <= 1024 && T >= 1 && T <= kTopkThrMaxTokens && K >= 1 && K <= 64 &&
           (size_t)T * K <= kGroupSmallPairs && T < kWideMinTokens;
}

int launch_topk_group(k3x_hip_ctx* ctx, const float* logits, const float* bias, uint32_t E,
                      uint32_t K, uint32_t T, float routed_scale, uint32_t renorm, uint32_t* ids,
                      float* weights, const uint32_t* ready, const LayerBuffers& s) {
    if (!topk_group_eligible(E, K, T) || !ctx->route_counter) return K3X_ERR_INVALID_EXTENT;
    return launch_topk_group_impl(ctx, logits, bias, E, K, T, routed_scale, renorm, ids, weights,
                                  ready, s);
}

int launch_rmsnorm(k3x_hip_ctx* ctx, const uint16_t* x, const float* gamma, uint32_t T,
                   uint32_t H, float eps, uint16_t* xn) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, ctx->stream, x, gamma, H, eps, xn,
                       (uint16_t*)nullptr, ctx->status);
    return launched(ctx, 1);
}

int launch_router_logits(k3x_hip_ctx* ctx, const float* W, const float* Wp, const uint16_t* xn,
                         uint16_t* xp, uint32_t E, uint32_t H, uint32_t T, float* logits) {
    return launch_router(ctx, W, Wp, xn, xp, E, H, T, logits, true);
}

bool router_uses_mfma(uint32_t H, uint32_t T) {
    return H <= kRouterMaxHidden && T >= kRouterMfmaMinTokens;
}

size_t router_xp_bytes(uint32_t T) {
    return (size_t)(T + 15) / 16 * kRouterRes * kRouterTileRes * 2;
}

int launch_topk(k3x_hip_ctx* ctx, const float* logits, const float* bias, uint32_t E, uint32_t K,
                uint32_t T, float routed_scale, uint32_t renorm, uint32_t* ids, float* weights) {
    return launch_topk_any(ctx, logits, bias, E, K, T, routed_scale, renorm, ids, weights);
}

// Dense bf16 projections in the bank's tile layout: the wide grouped GEMM
// (one item per 128-row chunk of the T rows) from kWideMinTokens rows when
// the shapes fit it, else expert_gemm over the T rows as one block.
int dense_down_output(k3x_hip_ctx* ctx, const uint4* tiles, uint32_t N, uint32_t K,
                      const uint16_t* a, uint32_t T, const float* prefix, const float* shared,
                      float* routed, uint16_t* out) {
    if (!T || T > kGemvMaxTokens || N % 128 || K % 128) return K3X_ERR_INVALID_EXTENT;
    GemvArgs g{tiles, K / 128, a, K, T, out, N, {}, ctx->status, prefix, shared, routed};
    if (K / 128 <= 2 * kGemvWaves && (size_t)T * K / 8 <= 64 * kGemvWaves &&
        (uintptr_t)a % 16 == 0)
        hipLaunchKernelGGL((dense_gemv_kernel<1, 2, 3, kGemvWaves, false, true>), dim3(N / 16),
                           dim3(64 * kGemvWaves), (size_t)T * K * 2, ctx->stream, g);
    else
        hipLaunchKernelGGL((dense_gemv_kernel<1, 3, 3>), dim3(N / 16), dim3(64 * kGemvWaves), 0,
                           ctx->stream, g);
    return launched(ctx, 1);
}

bool dense_norm_output_ok(uint32_t N, uint32_t K, uint32_t T) {
    return T && T <= kNormOutTokens && N % 128 == 0 && K % 128 == 0 &&
           K / 128 <= 2 * kGemvWaves && (size_t)T * K / 8 <= kNormOutRowChunks &&
           K / 4 <= kNormOutGammaChunks;
}

int dense_norm_output(k3x_hip_ctx* ctx, const uint4* tiles, uint32_t N, uint32_t K,
                      const uint16_t* x, const float* gamma, float eps, uint32_t T,
                      const float* prefix, const float* shared, float* routed, uint16_t* out) {
    if (!dense_norm_output_ok(N, K, T) || (uintptr_t)x % 16 || (uintptr_t)gamma % 16)
        return K3X_ERR_INVALID_EXTENT;
    GemvArgs g{tiles, K / 128, x, K, T, out, N, {}, ctx->status, prefix, shared, routed};
    g.gamma = gamma;
    g.eps = eps;
    hipLaunchKernelGGL((dense_gemv_kernel<1, 2, 3, kGemvWaves, false, true, true>), dim3(N / 16),
                       dim3(64 * kGemvWaves), (size_t)T * K * 2 + (size_t)K * 4, ctx->stream, g);
    return launched(ctx, 1);
}

bool dense_wide_ok(WideKind kind, uint32_t N, uint32_t K, uint32_t T) {
    return T >= kWideMinTokens && K % (128 * kWideStages) == 0 &&
           (N / 16) % wide_rb_per_block(kind) == 0 && N % 16 == 0 &&
           (uint64_t)T * std::max(N, K) * 4 < (1ull << 32) && (uint64_t)N * K * 4 < (1ull << 32);
}

bool dense_mlp_any_stream(uint32_t I, uint32_t H, uint32_t T) {
    return T <= kDenseDirectTokens ||
           (dense_wide_ok(kWideSharedGateUp, I, H, T) && dense_wide_ok(kWideSharedDown, H, I, T));
}

bool dense_down_any_stream(uint32_t N, uint32_t K, uint32_t T) {
    return T <= kDenseDirectTokens || dense_wide_ok(kWideSharedDown, N, K, T);
}

int dense_gate_up(k3x_hip_ctx* ctx, const uint4* tiles, uint32_t I, uint32_t H, const uint16_t* x,
                  uint32_t T, const GluParams& glu, uint16_t* act, hipStream_t stream,
                  bool split) {
    if (!T || I % 64 || H % 128) return K3X_ERR_INVALID_EXTENT;
    const uint32_t act_stride = split ? 2 * I : I, act_lo = split ? I : 0;
    if (dense_wide_ok(kWideSharedGateUp, I, H, T)) {
        WideGemmArgs g{};
        g.codes = reinterpret_cast<const uint8_t*>(tiles);
        g.kt = H / 128;
        g.nrb = I / 16;
        g.a = x;
        g.a_stride = H;
        g.a_bytes = T * H * 2;
        g.tokens = T;
        g.act = act;
        g.act_stride = act_stride;
        g.act_lo = act_lo;
        g.glu = glu;
        g.status = ctx->status;
        return launch_wide_gemm(ctx, kWideSharedGateUp, g, (T + kWideRows - 1) / kWideRows, stream);
    }
    if (T <= kGemvMaxTokens) {
        GemvArgs g{tiles, H / 128, x, H, T, act, act_stride, glu, ctx->status};
        g.out_lo = act_lo;
        // Beside the context stream: half-size workgroups, so that the
        // other stream's launches find room on every compute unit.
        if (stream == ctx->stream)
            hipLaunchKernelGGL((dense_gemv_kernel<2, 2, 2>), dim3(I / 16), dim3(64 * kGemvWaves), 0,
                               stream, g);
        else
            hipLaunchKernelGGL((dense_gemv_kernel<2, 2, 2, kGemvWaves / 2>), dim3(I / 16),
                               dim3(32 * kGemvWaves), 0, stream, g);
        return launched(ctx, 1);
    }
    if (stream != ctx->stream) return K3X_ERR_INVALID_EXTENT;
    GemmArgs g{};
    g.codes = reinterpret_cast<const uint8_t*>(tiles);
    g.kt = H / 128;
    g.a = x;
    g.a_stride = H;
    g.tokens = T;
    g.act = act;
    g.act_stride = act_stride;
    g.act_lo = act_lo;
    g.glu = glu;
    g.status = ctx->status;
    if (T > 16) launch_gemm<false, true, 4, 1>(ctx, g, 1, I);
    else launch_gemm<false, true, 1, 1>(ctx, g, 1, I);
    return launched(ctx, 1);
}

int dense_down(k3x_hip_ctx* ctx, const uint4* tiles, uint32_t N, uint32_t K, const uint16_t* a,
               uint32_t T, float* y, hipStream_t stream, uint16_t* y_bf16, bool split) {
    if (!T || N % 128 || K % 128) return K3X_ERR_INVALID_EXTENT;
    // Split rows [hi | lo] of 2 K: each weight tile meets both halves.
    const uint32_t a_stride = split ? 2 * K : K;
    if (T <= kGemvMaxTokens) {
        GemvArgs g{tiles, K / 128, a, a_stride, T, y_bf16 ? (void*)y_bf16 : (void*)y, N, {},
                   ctx->status};
        g.x_lo = split ? K : 0;
        const dim3 grid(N / 16);
        if (y_bf16 && split) return K3X_ERR_INVALID_EXTENT;
        if (y_bf16)
            hipLaunchKernelGGL((dense_gemv_kernel<1, 3, 1>), grid, dim3(64 * kGemvWaves), 0, stream,
                               g);
        else if (stream == ctx->stream && split)
            hipLaunchKernelGGL((dense_gemv_kernel<1, 2, 0, kGemvWaves, true>), grid,
                               dim3(64 * kGemvWaves), 0, stream, g);
        else if (stream == ctx->stream)
            hipLaunchKernelGGL((dense_gemv_kernel<1, 3, 0>), grid, dim3(64 * kGemvWaves), 0, stream,
                               g);
        else if (split)
            hipLaunchKernelGGL((dense_gemv_kernel<1, 3, 0, kGemvWaves / 2, true>), grid,
                               dim3(32 * kGemvWaves), 0, stream, g);
        else
            hipLaunchKernelGGL((dense_gemv_kernel<1, 3, 0, kGemvWaves / 2>), grid,
                               dim3(32 * kGemvWaves), 0, stream, g);
        return launched(ctx, 1);
    }
    if (y_bf16) return K3X_ERR_INVALID_EXTENT;
    if (dense_wide_ok(kWideSharedDown, N, K, T)) {
        WideGemmArgs g{};
        g.codes = reinterpret_cast<const uint8_t*>(tiles);
        g.kt = K / 128;
        g.kta = split ? 2 * g.kt : 0;  // the weights repeated along K
        g.nrb = N / 16;
        g.a = a;
        g.a_stride = a_stride;
        g.a_bytes = T * a_stride * 2;
        g.tokens = T;
        g.y = y;
        g.y_stride = N;
        g.status = ctx->status;
        return launch_wide_gemm(ctx, kWideSharedDown, g, (T + kWideRows - 1) / kWideRows, stream);
    }
    if (stream != ctx->stream) return K3X_ERR_INVALID_EXTENT;
    GemmArgs g{};
    g.codes = reinterpret_cast<const uint8_t*>(tiles);
    g.kt = K / 128;
    g.a_lo = split ? K : 0;
    g.a = a;
    g.a_stride = a_stride;
    g.tokens = T;
    g.y = y;
    g.y_stride = N;
    g.status = ctx->status;
    if (T > 16) launch_gemm<false, false, 4, 2>(ctx, g, 1, N);
    else launch_gemm<false, false, 1, 2>(ctx, g, 1, N);
    return launched(ctx, 1);
}

size_t router_wp_floats(uint32_t experts) {
    return (size_t)(experts + 15) / 16 * kRouterRes * kRouterTileRes;
}

int launch_combine(k3x_hip_ctx* ctx, const float* y, const float* weights, const float* shared,
                   uint32_t K, uint32_t H, uint32_t T, uint16_t* out, float* out_f32,
                   bool round_y) {
    const int mark = begin_stage(ctx, K3X_STAGE_COMBINE);
    hipLaunchKernelGGL(combine_kernel<kCombineVec>, dim3((H / kCombineVec + 255) / 256, T),
                       dim3(256), 0, ctx->stream, y, weights, shared, K, H, out, out_f32,
                       (uint32_t)round_y, ctx->status);
    end_stage(ctx, mark);
    return launched(ctx, 1);
}

}  // namespace k3x_hip

extern "C" {

}  // extern "C"

namespace {

// The layer with device routing over the per-call buffers `s` (already laid
// out): the decode path when it applies, else the general path.
int forward_device_routed(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                          const Scratch& s, const uint16_t* x, uint16_t* out,
                          const k3x_hip_moe_taps* taps) {
    int st = K3X_OK;
    if (!(p->flags &
          (K3X_FLAG_GENERAL_PATH | K3X_FLAG_ROUND_EXPERT_OUT | K3X_FLAG_SPLIT_ACT)) &&
        k3x_hip::decode_eligible(ctx, bank, p, x)) {
        const bool group_taps = taps && (taps->counts || taps->offsets || taps->first_use ||
                                         taps->active_first_use);
        if ((st = k3x_hip::decode_forward(ctx, bank, p, s, x, out,
                                           taps ? taps->out_f32 : nullptr, group_taps)))
            return st;
        ++ctx->forward_calls;
        return copy_taps(ctx, bank, p, s, s.xn, s.ids, s.weights, taps);
    }
    const auto& d = bank->desc;
    const uint32_t T = p->tokens, K = p->top_k;
    const int mark = k3x_hip::begin_stage(ctx, K3X_STAGE_ROUTE);
    const bool mfma_router = bank->router_wp && T >= kRouterMfmaMinTokens;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, ctx->stream, x, bank->gamma,
                       d.hidden, p->rms_epsilon, s.xn, mfma_router ? s.xp : nullptr,
                       ctx->status);
    // The shared expert needs xn only: on the second stream it runs beside
    // the router, the Top-K and the grouping, not only the routed GEMMs.
    const bool forked = shared_on_side(ctx, bank, p);
    if (forked) {
        const GluParams glu{(int)p->glu, p->situ_beta, (int)p->has_situ_linear,
                            p->situ_linear_beta};
        if ((st = fork_shared(ctx, bank, p, s, s.xn, glu))) {
            (void)hipStreamWaitEvent(ctx->stream, ctx->join_ev, 0);
            return st;
        }
    }
    st = launch_router(ctx, bank->router_w, mfma_router ? bank->router_wp : nullptr, s.xn, s.xp,
                       d.experts, d.hidden, T, s.logits);
    // Few pairs: the Top-K groups its own route (one launch fewer); the
    // routed tail then skips its grouping.
    Scratch g = s;
    g.grouped = k3x_hip::topk_group_eligible(d.experts, K, T) && ctx->route_counter &&
                !(p->flags & K3X_FLAG_SPLIT_INPUT);
    if (g.grouped)
        st = st ? st : launch_topk_group_impl(ctx, s.logits, bank->router_bias, d.experts, K, T,
                                              p->routed_scale, p->renorm, s.ids, s.weights,
                                              bank->ready_dev, s);
    else
        st = st ? st : launch_topk_any(ctx, s.logits, bank->router_bias, d.experts, K, T,
                                       p->routed_scale, p->renorm, s.ids, s.weights);
    if (!st) k3x_hip::end_stage(ctx, mark);
    if (!st) st = launched(ctx, 1);
    if (st) {
        if (forked) (void)hipStreamWaitEvent(ctx->stream, ctx->join_ev, 0);
        return st;
    }
    if ((st = run_tail(ctx, bank, p, g, s.xn, s.ids, s.weights, out, taps ? taps->out_f32 : nullptr,
                       forked)))
        return st;
    ++ctx->forward_calls;
    return copy_taps(ctx, bank, p, s, s.xn, s.ids, s.weights, taps);
}

}  // namespace

// Scratch of k3x_hip_moe_forward_noalloc: the per-call buffers live in this
// fixed array instead of the context's grow-only allocation.  In host code
// `scratch` names a host-side stand-in, never the device memory: the device
// address comes from hipGetSymbolAddress, taken once per device
// (k3x_hip::noalloc_scratch) and kept in the context; only that address is
// passed to kernels.  Each device holds its own copy for the life of the
// process, shared by every no-allocation call on that device.
static __device__ __align__(256) uint8_t scratch[K3X_HIP_NOALLOC_SCRATCH_BYTES];

namespace k3x_hip {

int routed_begin(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                 LayerBuffers* s) {
    if (!ctx || !bank || !p || !s || bank->ctx != ctx) return K3X_ERR_INVALID_EXTENT;
    const int st = validate_params(bank, p, false);
    return st ? st : prepare(ctx, bank, p, s);
}

int routed_finish(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                  const LayerBuffers& s, const uint16_t* xn, const uint32_t* ids,
                  const float* weights, uint16_t* out, const k3x_hip_moe_taps* taps) {
    if (!xn || !ids || !weights || !out) return K3X_ERR_INVALID_EXTENT;
    int st = run_tail(ctx, bank, p, s, xn, ids, weights, out, taps ? taps->out_f32 : nullptr);
    if (st) return st;
    ++ctx->forward_calls;
    return copy_taps(ctx, bank, p, s, xn, ids, weights, taps);
}

int noalloc_scratch(int device, void** out) {
    static std::mutex mu;
    static std::vector<void*> by_device;
    std::lock_guard<std::mutex> lock(mu);
    if (device < 0) return K3X_ERR_INVALID_EXTENT;
    if ((size_t)device >= by_device.size()) by_device.resize((size_t)device + 1, nullptr);
    if (!by_device[device]) {
        void* ptr = nullptr;  // with `device` current (the caller's hipSetDevice)
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return K3X_ERR_BACKEND_UNAVAILABLE;
        }
        by_device[device] = ptr;
    }
    *out = by_device[device];
    return K3X_OK;
}

}  // namespace k3x_hip

extern "C" {

int k3x_hip_moe_forward(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                        const uint16_t* x, uint16_t* out, const k3x_hip_moe_taps* taps) {
    if (!ctx || !bank || !p || !x || !out || bank->ctx != ctx) return K3X_ERR_INVALID_EXTENT;
    int st = validate_params(bank, p);
    if (st) return st;
    if (p->flags & K3X_FLAG_SPLIT_INPUT) return K3X_ERR_INVALID_MXFP4;  // x is raw bf16 here
    if (!bank->router_ready) return K3X_ERR_INVALID_STATE;
    Scratch s;
    if ((st = prepare(ctx, bank, p, &s))) return st;
    return forward_device_routed(ctx, bank, p, s, x, out, taps);
}

int k3x_hip_moe_forward_noalloc(k3x_hip_ctx* ctx, k3x_hip_bank* bank,
                                const k3x_hip_moe_params* p, const uint16_t* x, uint16_t* out,
                                const k3x_hip_moe_taps* taps) {
    if (!ctx || !bank || !p || !x || !out || bank->ctx != ctx) return K3X_ERR_INVALID_EXTENT;
    int st = validate_params(bank, p);
    if (st) return st;
    if (p->flags & K3X_FLAG_SPLIT_INPUT) return K3X_ERR_INVALID_MXFP4;  // x is raw bf16 here
    if (!bank->router_ready) return K3X_ERR_INVALID_STATE;
    if (!ctx->noalloc_scratch) return K3X_ERR_BACKEND_UNAVAILABLE;
    Scratch s;
    const bool split = (p->flags & K3X_FLAG_SPLIT_ACT) != 0, q8 = scaled_fp4(p);
    // The fixed scratch's last kDecodeMixBytes hold the decode combine's
    // counters (zero from load time, left zero by every call); the carve
    // stays below them.
    constexpr size_t kCarveMax = K3X_HIP_NOALLOC_SCRATCH_BYTES - k3x_hip::kDecodeMixBytes;
    if (carve(nullptr, bank->desc, p->tokens, p->top_k, split, q8, &s) > kCarveMax)
        return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    carve(static_cast<uint8_t*>(ctx->noalloc_scratch), bank->desc, p->tokens, p->top_k, split,
          q8, &s);
    s.mix = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ctx->noalloc_scratch) + kCarveMax);
    // Stage timing takes events from a pool that may have to create them:
    // not on this path.
    const bool profiling = ctx->profiling;
    ctx->profiling = false;
    st = forward_device_routed(ctx, bank, p, s, x, out, taps);
    ctx->profiling = profiling;
    return st;
}

int k3x_hip_moe_forward_routed(k3x_hip_ctx* ctx, k3x_hip_bank* bank,
                               const k3x_hip_moe_params* p, const uint16_t* xn,
                               const uint32_t* ids, const float* weights,
                               const uint32_t* host_ids, const float* host_weights,
                               uint16_t* out, const k3x_hip_moe_taps* taps) {
    if (!ctx || !bank || !p || !xn || !ids || !weights || !out || bank->ctx != ctx)
        return K3X_ERR_INVALID_EXTENT;
    int st = validate_params(bank, p, false);
    if (st) return st;
    const uint32_t T = p->tokens, K = p->top_k, E = bank->desc.experts;
    // Route contract of build_expert_major_plan (expert_major.cpp:21-36);
    // a routed slot must hold an admitted expert.
    if (host_ids) {
        for (uint32_t t = 0; t < T; ++t)
            for (uint32_t s = 0; s < K; ++s) {
                const uint32_t e = host_ids[(size_t)t * K + s];
                if (e >= E || !bank->expert_ready[e]) return K3X_ERR_INVALID_STATE;
                for (uint32_t q = 0; q < s; ++q)
                    if (host_ids[(size_t)t * K + q] == e) return K3X_ERR_INVALID_STATE;
            }
    }
    if (host_weights)
        for (size_t i = 0; i < (size_t)T * K; ++i)
            if (!std::isfinite(host_weights[i])) return K3X_ERR_INVALID_STATE;
    Scratch s;
    if ((st = prepare(ctx, bank, p, &s))) return st;
    return k3x_hip::routed_finish(ctx, bank, p, s, xn, ids, weights, out, taps);
}

int k3x_hip_expert_major_plan(k3x_hip_ctx* ctx, const uint32_t* ids, uint32_t tokens,
                              uint32_t top_k, uint32_t experts, const k3x_hip_moe_taps* t) {
    if (!ctx || !ids || !t || !tokens || tokens > (1u << 20) || !top_k || top_k > 64 ||
        !experts || experts > 4096 ||
        !t->counts || !t->offsets || !t->pair_token || !t->pair_slot || !t->first_use ||
        !t->n_active || !t->active_first_use)
        return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    // Scratch: the ascending active list, then the grouping's own buffers.
    const size_t asc = ((size_t)experts * 4 + 255) & ~(size_t)255;
    int st = k3x_hip::ensure_scratch(ctx, asc + group_scratch_bytes(tokens, top_k, experts));
    if (st) return st;
    uint8_t* base = static_cast<uint8_t*>(ctx->scratch);
    return launch_group(ctx, ids, tokens, top_k, experts, nullptr, t->counts, t->offsets,
                        t->pair_token,
                        t->pair_slot, t->first_use, t->n_active, reinterpret_cast<uint32_t*>(base),
                        t->active_first_use, base + asc);
}

}  // extern "C"
