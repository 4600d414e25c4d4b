// decode.hip -- the decode path of the MoE layer (T <= 4 tokens): six
// launches on two streams, no cross-workgroup synchronisation inside any of
// them.
//
// Context stream (the routing chain):
//   decode_router_kernel  every block rebuilds xn = bf16(RMSNorm(x) * gamma)
//                         in LDS and streams the fp32 router, one wave per
//                         expert row (fp64, canonical order), into logits.
//   decode_select_kernel  sigmoid + bias Top-K of every token and the
//                         expert-major grouping (one block).
//   decode_gateup_kernel  routed MXFP4 gate/up + GLU per active expert, four
//                         16-row blocks per workgroup (K split over two waves
//                         when the extra waves still fit on the device at
//                         once), weights dequantised in registers.
//   decode_down_kernel    one workgroup per 16 output rows: its waves take
//                         the active experts in turn (MXFP4 down projection
//                         of each expert's pairs into LDS), then the block
//                         forms out = bf16(sum over slots in router order of
//                         w * y + shared) for its rows.
// Side stream (the shared expert, which needs only xn):
//   decode_shared_gateup_kernel  bf16 shared gate/up + GLU, one 16-row block
//                         of S per workgroup, K split over 16 waves.
//   decode_shared_down_kernel    bf16 shared down, one 16-row block of H per
//                         workgroup, K split over four waves.
// The side stream forks from the context stream at entry and joins it before
// decode_down_kernel, so its ~90 MB stream overlaps the router and Top-K
// steps, which leave most of the device idle.
//
// The streaming loops keep one weight tile in flight per wave and few
// registers, so that eight waves fit on each SIMD: for these HBM streams
// the number of resident waves matters more than per-wave prefetch depth.
// Numerics: the same canonical fp64 order for the RMS sum and the router
// logits as the general path, the same Top-K keys and renormalisation, the
// same slot-ordered combine; fp32 MFMA accumulation for the projections.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "k3x_decode.hpp"
#include "k3x_device.hpp"
#include "k3x_internal.hpp"

using namespace k3x_dev;
using k3x_hip::kMaxDecodeTokens;
using k3x_hip::begin_stage;
using k3x_hip::end_stage;

namespace {

constexpr int kFrontThreads = 512;  // 8 waves
constexpr int kFrontWaves = kFrontThreads / 64;
constexpr int kKeysPerLane = 8;     // Top-K candidates per lane: E <= 512

__device__ inline void latch(uint32_t* status, uint32_t code) { atomicCAS(status, 0u, code); }

__device__ inline float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Sort key: larger adjusted score first, then lower expert index
// (runtime/src/official_moe.cpp:226-232).  -0 folds into +0; 0 = no entry.
__device__ inline uint64_t topk_key(float adj, uint32_t e) {
    const float a = adj == 0.0f ? 0.0f : adj;
    const uint32_t u = __float_as_uint(a);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - e);
}

// Maximum of v over the 64 lanes with DPP moves (quad permutes, row
// rotates, row broadcasts): VALU latency instead of LDS-crossbar shuffles.
// Rows not selected by a row_bcast keep their own value (max(v, v) = v).
template <int Ctrl, int RowMask>
__device__ inline uint32_t dpp_max_step(uint32_t x) {
    const uint32_t y =
        (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, Ctrl, RowMask, 0xf, false);
    return x > y ? x : y;
}

__device__ inline uint32_t wave_max_u32(uint32_t v) {
    v = dpp_max_step<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_max_step<0x124, 0xf>(v);  // row_ror:4
    v = dpp_max_step<0x128, 0xf>(v);  // row_ror:8
    v = dpp_max_step<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    v = dpp_max_step<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Canonical combination of one lane's four partial sums (partials 4l..4l+3
// of the 256-way strided order) and the 64-lane butterfly: the pairwise tree
// over all 256 partials.
__device__ inline double canon_reduce(const double p[4]) {
    double v = (p[0] + p[1]) + (p[2] + p[3]);
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
    return v;
}

// Block-wide exclusive scan of one value per thread (512 threads).  Returns
// the exclusive prefix; *total receives the sum.
__device__ inline uint32_t block_scan_excl(uint32_t v, uint32_t* wave_sums, uint32_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
    }
    if (lane == 63) wave_sums[wave] = incl;
    __syncthreads();
    uint32_t base = 0, all = 0;
    for (int w = 0; w < kFrontWaves; ++w) {
        const uint32_t s = wave_sums[w];
        if (w < wave) base += s;
        all += s;
    }
    __syncthreads();
    *total = all;
    return base + incl - v;
}

// ---------------------------------------------------------------------------
// MXFP4 step helpers: one 128-K tile of S 16-row blocks (codes [S][64] x
// 16 B, one E8M0 byte per lane per block), dequantised in registers and
// multiplied by the activation slice av[4] (K = 32g + 8j .. +7 of the tile).
// ---------------------------------------------------------------------------
__device__ inline f32x4 mxfp4_tile(const uint4& c, float scale, const uint4 av[4], f32x4 acc) {
    const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = mfma16x16x32(as_bf16x8(av[j]), dequant8(cw[j], scale), acc);
    return acc;
}

__device__ inline void load_act(const uint16_t* ap, bool arow, uint32_t k, uint4 av[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
        av[j] = arow ? *reinterpret_cast<const uint4*>(ap + k * 128 + 8 * j) : make_uint4(0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// xn prologue of the router and shared gate/up kernels
// ---------------------------------------------------------------------------
struct NormShared {
    float inv[kMaxDecodeTokens];
    int bad;
};

// x -> LDS (16-byte chunks), inverse RMS per token from the sum of squares in
// the canonical fp64 order, then xn = bf16(x * inv * gamma) in place; the
// block then holds xn as [T][H] bf16 at s_x4.  Returns false when x holds a
// non-finite value (latched into *status when status is non-null).  Needs
// at least T waves; xn_out, when non-null, receives a global copy.
template <int kThreads>
__device__ __forceinline__ bool build_xn(const uint16_t* x, const float* gamma, uint32_t T, uint32_t H, float eps,
                         uint4* s_x4, NormShared& ns, uint16_t* xn_out, uint32_t* status) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint16_t* s_x = reinterpret_cast<const uint16_t*>(s_x4);
    if (tid == 0) ns.bad = 0;
    const uint32_t chunks = T * H / 8;
    for (uint32_t c0 = 0; c0 < chunks; c0 += 4 * kThreads) {
        uint4 v[4];
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const uint32_t c = c0 + tid + kThreads * it;
            v[it] = c < chunks ? reinterpret_cast<const uint4*>(x)[c] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const uint32_t c = c0 + tid + kThreads * it;
            if (c < chunks) s_x4[c] = v[it];
        }
    }
    __syncthreads();
    if (wave < T) {
        const uint16_t* xr = s_x + (size_t)wave * H;
        double p[4] = {0.0, 0.0, 0.0, 0.0};
        int bad = 0;
        for (uint32_t j = 0; j < H / 256; ++j) {
            const uint2 w = *reinterpret_cast<const uint2*>(xr + 256 * j + 4 * lane);
            const float f[4] = {lo_bf16(w.x), hi_bf16(w.x), lo_bf16(w.y), hi_bf16(w.y)};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                bad |= !__builtin_isfinite(f[c]);
                p[c] += (double)f[c] * (double)f[c];
            }
        }
        const double s = canon_reduce(p);
        bad = __any(bad);
        if (lane == 0) {
            if (bad) ns.bad = 1;
            const float mean = (float)__ddiv_rn(s, (double)H);
            ns.inv[wave] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
        }
    }
    __syncthreads();
    if (ns.bad) {
        if (status && tid == 0) latch(status, K3X_ERR_INVALID_MXFP4);
        return false;
    }
    for (uint32_t c = tid; c < chunks; c += kThreads) {
        const uint32_t t = (c * 8) / H, k = (c * 8) % H;
        const uint4 w = s_x4[c];
        const float4 g0 = *reinterpret_cast<const float4*>(gamma + k);
        const float4 g1 = *reinterpret_cast<const float4*>(gamma + k + 4);
        const float inv = ns.inv[t];
        const uint32_t in[4] = {w.x, w.y, w.z, w.w};
        const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t lo = f32_to_bf16(__fmul_rn(__fmul_rn(lo_bf16(in[q]), inv), g[2 * q]));
            const uint32_t hi =
                f32_to_bf16(__fmul_rn(__fmul_rn(hi_bf16(in[q]), inv), g[2 * q + 1]));
            o[q] = lo | (hi << 16);
        }
        const uint4 ov = make_uint4(o[0], o[1], o[2], o[3]);
        s_x4[c] = ov;
        if (xn_out) reinterpret_cast<uint4*>(xn_out)[c] = ov;
    }
    __syncthreads();
    return true;
}

// ---------------------------------------------------------------------------
// Router kernel: xn and router logits
// ---------------------------------------------------------------------------
struct RouterArgs {
    const uint16_t* x;
    const float* gamma;
    const float* router_w;  // [E][H] fp32
    uint32_t T, H, E;
    float eps;
    uint16_t* xn;           // [T][H] global copy (block 0 writes it)
    float* logits;          // [T][E]
    uint32_t* status;
};

constexpr int kRouterBatch = 14;  // float4 row loads per lane per buffer (two buffers)

// One wave per expert row.  The wave's first two batches of row loads are
// issued before the xn prologue, so the row fetch overlaps it; each partial
// 4l + c still accumulates j = 0, 1, ... in order (canonical order).
// TT bounds the token count (register arrays sized by it).
template <int TT>
__global__ __launch_bounds__(kFrontThreads) void decode_router_kernel(RouterArgs a) {
    extern __shared__ uint4 dyn_lds[];
    __shared__ NormShared ns;
    if (*(volatile uint32_t*)a.status) return;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t T = a.T, H = a.H, J = H / 256;
    const uint32_t e = blockIdx.x * kFrontWaves + wave;
    const bool row = e < a.E;
    const float* wr = a.router_w + (size_t)(row ? e : 0) * H + 4 * lane;
    float4 wb[2][kRouterBatch];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int u = 0; u < kRouterBatch; ++u) {
            const uint32_t j = b * kRouterBatch + u;
            if (row && j < J) wb[b][u] = *reinterpret_cast<const float4*>(wr + 256 * j);
        }
    if (!build_xn<kFrontThreads>(a.x, a.gamma, T, H, a.eps, dyn_lds, ns,
                                 blockIdx.x == 0 ? a.xn : nullptr, a.status))
        return;
    if (!row) return;
    const uint16_t* s_x = reinterpret_cast<const uint16_t*>(dyn_lds);
    double p[TT][4];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) p[t][c] = 0.0;
    for (uint32_t j0 = 0; j0 < J; j0 += 2 * kRouterBatch) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int u = 0; u < kRouterBatch; ++u) {
                const uint32_t j = j0 + b * kRouterBatch + u;
                if (j >= J) continue;
                const float wv[4] = {wb[b][u].x, wb[b][u].y, wb[b][u].z, wb[b][u].w};
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    if ((uint32_t)t >= T) continue;
                    const uint2 xv =
                        *reinterpret_cast<const uint2*>(s_x + (size_t)t * H + 256 * j + 4 * lane);
                    const float f[4] = {lo_bf16(xv.x), hi_bf16(xv.x), lo_bf16(xv.y),
                                        hi_bf16(xv.y)};
#pragma unroll
                    for (int c = 0; c < 4; ++c) p[t][c] += (double)wv[c] * (double)f[c];
                }
            }
            // Refill this buffer with the batch two ahead.
#pragma unroll
            for (int u = 0; u < kRouterBatch; ++u) {
                const uint32_t j = j0 + (b + 2) * kRouterBatch + u;
                if (j < J) wb[b][u] = *reinterpret_cast<const float4*>(wr + 256 * j);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        if ((uint32_t)t >= T) continue;
        const double v = canon_reduce(p[t]);
        if (lane == 0) a.logits[(size_t)t * a.E + e] = (float)v;
    }
}

// ---------------------------------------------------------------------------
// Shared expert (side stream): gate/up + GLU, then down
// ---------------------------------------------------------------------------
constexpr int kSharedGuWaves = 16;  // K split of one 16-row block of the shared gate/up
constexpr int kSharedDnWaves = 4;   // K split of one 16-row block of the shared down

struct SharedGateUpArgs {
    const uint16_t* x;
    const float* gamma;
    uint32_t T, H, S;
    float eps;
    const uint4* sh_gu;  // shared gate/up tiles [S/16][H/128][2][4][64] x 16 B
    GluParams glu;
    uint16_t* sact;      // [T][S] bf16 shared activation
    const uint32_t* status;
};

struct SharedGateUpLds {
    NormShared ns;
    f32x4 red[kSharedGuWaves][2][64];
};

// Workgroup = one 16-row block of S and the whole K = H range, split over
// 16 waves (first weight tile requested before the xn prologue); the wave
// partials are added in a fixed tree in LDS (wave w += wave w + h for
// h = 8, 4, 2, 1) and the block writes sact = bf16(GLU(gate, up)) for its 16
// columns.
__global__ __launch_bounds__(64 * kSharedGuWaves) void decode_shared_gateup_kernel(
    SharedGateUpArgs a) {
    extern __shared__ uint4 dyn_lds[];
    __shared__ SharedGateUpLds sh;
    if (*(volatile const uint32_t*)a.status) return;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t T = a.T, H = a.H, rb = blockIdx.x, kt = H / 128;
    const uint32_t k0 = wave * kt / kSharedGuWaves, k1 = (wave + 1) * kt / kSharedGuWaves;
    const uint4* tiles = a.sh_gu + (size_t)rb * kt * 2 * 4 * 64 + lane;
    uint4 bn[2][4];
    if (k0 < k1)
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int j = 0; j < 4; ++j) bn[w][j] = tiles[(((size_t)k0 * 2 + w) * 4 + j) * 64];
    // A non-finite x is reported by the router kernel.
    if (!build_xn<64 * kSharedGuWaves>(a.x, a.gamma, T, H, a.eps, dyn_lds, sh.ns, nullptr, nullptr))
        return;
    const uint16_t* s_x = reinterpret_cast<const uint16_t*>(dyn_lds);
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const bool arow = n < T;
    for (uint32_t k = k0; k < k1; ++k) {
        bf16x8 af[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (arow)
                v = *reinterpret_cast<const uint4*>(s_x + (size_t)n * H + k * 128 + 32 * g + 8 * j);
            af[j] = as_bf16x8(v);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int w = 0; w < 2; ++w) acc[w] = mfma16x16x32(af[j], as_bf16x8(bn[w][j]), acc[w]);
        if (k + 1 < k1)  // refill after use: one tile of registers
#pragma unroll
            for (int w = 0; w < 2; ++w)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    bn[w][j] = tiles[(((size_t)(k + 1) * 2 + w) * 4 + j) * 64];
    }
    sh.red[wave][0][lane] = acc[0];
    sh.red[wave][1][lane] = acc[1];
#pragma unroll
    for (uint32_t h = kSharedGuWaves / 2; h >= 1; h /= 2) {
        __syncthreads();
        if (wave < h) {
            sh.red[wave][0][lane] = sh.red[wave][0][lane] + sh.red[wave + h][0][lane];
            sh.red[wave][1][lane] = sh.red[wave][1][lane] + sh.red[wave + h][1][lane];
        }
    }
    if (wave != 0) return;
    const f32x4 gs = sh.red[0][0][lane], us = sh.red[0][1][lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = 4 * g + i;
        if (t < T) a.sact[(size_t)t * a.S + rb * 16 + n] = f32_to_bf16(glu(gs[i], us[i], a.glu));
    }
}

struct SharedDownArgs {
    const uint4* sh_dn;    // shared down tiles [H/16][S/128][4][64] x 16 B
    const uint16_t* sact;  // [T][S]
    uint32_t T, H, S;
    float* sy;             // [T][H] shared expert output, fp32
    const uint32_t* status;
};

// Workgroup = one 16-row block of H, K = S split over four waves (one tile
// ahead in flight), partials added pairwise: (w0 + w1) + (w2 + w3).
__global__ __launch_bounds__(64 * kSharedDnWaves) void decode_shared_down_kernel(SharedDownArgs a) {
    __shared__ f32x4 red[kSharedDnWaves][64];
    if (*(volatile const uint32_t*)a.status) return;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t rb = blockIdx.x, skt = a.S / 128;
    const uint32_t k0 = wave * skt / kSharedDnWaves, k1 = (wave + 1) * skt / kSharedDnWaves;
    const uint4* tiles = a.sh_dn + (size_t)rb * skt * 4 * 64 + lane;
    const bool arow = n < a.T;
    const uint16_t* ap = a.sact + (size_t)(arow ? n : 0) * a.S + 32 * g;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 bn[4];
    if (k0 < k1)
#pragma unroll
        for (int j = 0; j < 4; ++j) bn[j] = tiles[((size_t)k0 * 4 + j) * 64];
    for (uint32_t k = k0; k < k1; ++k) {
        uint4 b[4], av[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = bn[j];
        if (k + 1 < k1)
#pragma unroll
            for (int j = 0; j < 4; ++j) bn[j] = tiles[((size_t)(k + 1) * 4 + j) * 64];
        load_act(ap, arow, k, av);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = mfma16x16x32(as_bf16x8(av[j]), as_bf16x8(b[j]), acc);
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    const f32x4 tot = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t t = 4 * g + q;
        if (t < a.T) a.sy[(size_t)t * a.H + rb * 16 + n] = tot[q];
    }
}
// ---------------------------------------------------------------------------
// Select kernel: Top-K + expert-major grouping (one block)
// ---------------------------------------------------------------------------
struct SelectArgs {
    const float* logits;
    const float* bias;
    uint32_t T, E, K;
    float routed_scale;
    uint32_t renorm;
    uint32_t* ids;       // [T][K]
    float* weights;      // [T][K]
    uint32_t* counts;
    uint32_t* offsets;
    uint32_t* pair_token;
    uint32_t* pair_slot;
    uint32_t* first_use;
    uint32_t* n_active;
    uint32_t* active_asc;
    uint32_t* active_fu;
    uint4* arec;         // [E] per active slot: {expert, rows, offset, row tokens}
    uint32_t* status;
};

struct SelectShared {
    int bad;
    uint32_t wave_sums[kFrontWaves];
    uint32_t ids[kMaxDecodeTokens * 64];
    uint32_t cnt[kKeysPerLane * 64];
    uint32_t fu[kKeysPerLane * 64];
    uint32_t off[kKeysPerLane * 64];
    uint32_t active[kMaxDecodeTokens * 64];
    uint32_t ptok[kMaxDecodeTokens * 64];
};

// Top-K of one token by one wave: keys held 8 per lane, popped K times.
// Scores, validation and renormalisation as runtime/src/routing_policy.cpp
// :40-95,146-157 (FLOAT) or runtime/src/official_moe.cpp:214-242 (DOUBLE),
// then * routed_scale (runtime/src/model.cpp:1004-1009).
__device__ void topk_token(const SelectArgs& a, uint32_t t, SelectShared& sh) {
    const int lane = threadIdx.x & 63;
    const uint32_t E = a.E, K = a.K;
    uint64_t key[kKeysPerLane];
    float score[kKeysPerLane];
    uint32_t bad = 0;
#pragma unroll
    for (int i = 0; i < kKeysPerLane; ++i) {
        const uint32_t e = lane + 64u * i;
        key[i] = 0;
        score[i] = 0.0f;
        if (e < E) {
            const float lg = a.logits[(size_t)t * E + e];
            const float b = a.bias[e];
            if (a.renorm == K3X_RENORM_DOUBLE &&
                (!__builtin_isfinite(lg) || !__builtin_isfinite(b)))
                bad = K3X_ERR_INVALID_EXTENT;
            const float s = sigmoid_cr(lg);
            const float adj = __fadd_rn(s, b);
            if (a.renorm == K3X_RENORM_FLOAT &&
                (!__builtin_isfinite(s) || s < 0.0f || s > 1.0f || !__builtin_isfinite(b) ||
                 !__builtin_isfinite(adj)))
                bad = K3X_ERR_INVALID_STATE;
            score[i] = s;
            key[i] = topk_key(adj, e);
        }
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) bad = max(bad, (uint32_t)__shfl_xor((int)bad, d));
    if (bad) {
        if (lane == 0) {
            latch(a.status, bad);
            sh.bad = 1;
        }
        return;
    }
    // Local selection sort, descending: the lane's head is key[0].
#pragma unroll
    for (int i = 0; i < kKeysPerLane; ++i)
#pragma unroll
        for (int j = i + 1; j < kKeysPerLane; ++j)
            if (key[j] > key[i]) {
                const uint64_t tk = key[i];
                key[i] = key[j];
                key[j] = tk;
                const float ts = score[i];
                score[i] = score[j];
                score[j] = ts;
            }
    float selsc = 0.0f;  // lane s < K keeps the score of slot s
    uint32_t selid = 0;
    for (uint32_t s = 0; s < K; ++s) {
        // Largest head: first the score half of the key, then, among lanes
        // whose heads tie on it, the expert half (a larger value there is a
        // lower expert index).
        const uint32_t hi = (uint32_t)(key[0] >> 32);
        const uint32_t mhi = wave_max_u32(hi);
        uint64_t tie = __ballot(hi == mhi);
        if (__popcll(tie) > 1) {
            const uint32_t lo = hi == mhi ? (uint32_t)key[0] : 0u;
            const uint32_t mlo = wave_max_u32(lo);
            tie = __ballot(hi == mhi && lo == mlo);
        }
        const int wlane = __ffsll((unsigned long long)tie) - 1;
        const uint32_t win = 0xffffffffu - (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key[0], wlane);
        const float wsc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(score[0]), wlane));
        const bool mine = lane == wlane;
        if ((uint32_t)lane == s) {
            selsc = wsc;
            selid = win;
        }
        if (mine) {
#pragma unroll
            for (int i = 0; i < kKeysPerLane - 1; ++i) {
                key[i] = key[i + 1];
                score[i] = score[i + 1];
            }
            key[kKeysPerLane - 1] = 0;
        }
    }
    // Renormalise in slot order (sequential sums as the reference).
    float den_f = 0.0f;
    double den_d = 0.0;
    for (uint32_t s = 0; s < K; ++s) {
        const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(selsc), s));
        den_f = __fadd_rn(den_f, v);
        den_d = __dadd_rn(den_d, (double)v);
    }
    uint32_t err = 0;
    if (a.renorm == K3X_RENORM_DOUBLE) {
        if (!__builtin_isfinite(den_d) || !(den_d > 0.0)) err = K3X_ERR_INVALID_EXTENT;
    } else if (!__builtin_isfinite(den_f) || !(den_f > 0.0f)) {
        err = K3X_ERR_INVALID_STATE;
    }
    if (err) {
        if (lane == 0) {
            latch(a.status, err);
            sh.bad = 1;
        }
        return;
    }
    if ((uint32_t)lane < K) {
        const float w = a.renorm == K3X_RENORM_DOUBLE
                            ? __fmul_rn((float)__ddiv_rn((double)selsc, den_d), a.routed_scale)
                            : __fmul_rn(__fdiv_rn(selsc, den_f), a.routed_scale);
        a.ids[(size_t)t * K + lane] = selid;
        a.weights[(size_t)t * K + lane] = w;
        sh.ids[t * K + lane] = selid;
    }
}

// Expert-major grouping of the T*K selected pairs by the whole block:
// ascending-expert CSR, rows of one expert in (token, slot) order, plus
// first-use keys and the first-use order of the active experts
// (runtime/src/expert_major.cpp:10-54).
__device__ void group_pairs(const SelectArgs& a, SelectShared& sh) {
    const uint32_t tid = threadIdx.x;
    const uint32_t P = a.T * a.K, E = a.E;
    for (uint32_t e = tid; e < E; e += kFrontThreads) {
        sh.cnt[e] = 0;
        sh.fu[e] = 0xffffffffu;
    }
    __syncthreads();
    if (tid < P) {
        const uint32_t e = sh.ids[tid];
        atomicAdd(&sh.cnt[e], 1u);
        atomicMin(&sh.fu[e], tid);
    }
    __syncthreads();
    // E <= 512: one expert per thread.
    const uint32_t c = tid < E ? sh.cnt[tid] : 0u;
    uint32_t total = 0, na = 0;
    const uint32_t excl = block_scan_excl(c, sh.wave_sums, &total);
    const uint32_t aidx = block_scan_excl(c ? 1u : 0u, sh.wave_sums, &na);
    if (tid < E) {
        sh.off[tid] = excl;
        a.offsets[tid] = excl;
        a.counts[tid] = c;
        a.first_use[tid] = sh.fu[tid];
        if (c) {
            a.active_asc[aidx] = tid;
            sh.active[aidx] = tid;
        }
    }
    if (tid == 0) {
        a.offsets[E] = total;
        *a.n_active = na;
    }
    __syncthreads();
    if (tid < P) {
        const uint32_t e = sh.ids[tid];
        uint32_t rank = 0;
        for (uint32_t q = 0; q < tid; ++q) rank += sh.ids[q] == e;
        const uint32_t r = sh.off[e] + rank;
        a.pair_token[r] = tid / a.K;
        a.pair_slot[r] = tid % a.K;
        sh.ptok[r] = tid / a.K;
    }
    __syncthreads();
    if (tid < na) {  // record of active slot tid: rows' tokens packed 8 bits each
        const uint32_t e = sh.active[tid], c = sh.cnt[e], o = sh.off[e];
        uint32_t toks = 0;
        for (uint32_t q = 0; q < c && q < 4; ++q) toks |= sh.ptok[o + q] << (8 * q);
        a.arec[tid] = make_uint4(e, c, o, toks);
    }
    if (tid < na) {
        const uint32_t e = sh.active[tid];
        const uint32_t key = sh.fu[e];
        uint32_t rank = 0;
        for (uint32_t b = 0; b < na; ++b) rank += sh.fu[sh.active[b]] < key;
        a.active_fu[rank] = e;
    }
}

__global__ __launch_bounds__(kFrontThreads) void decode_select_kernel(SelectArgs a) {
    __shared__ SelectShared sh;
    if (*(volatile uint32_t*)a.status) return;
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    if (tid == 0) sh.bad = 0;
    __syncthreads();
    if (wave < a.T) topk_token(a, wave, sh);
    __syncthreads();
    if (sh.bad) return;
    group_pairs(a, sh);
}

// ---------------------------------------------------------------------------
// Routed gate/up + GLU
// ---------------------------------------------------------------------------
struct GateUpArgs {
    const uint4* gu_codes;     // expert 0 base, tiles [I/16][H/128][2][64] x 16 B
    const uint32_t* gu_scales; // [I/16][ks][2][64]
    size_t codes_per_expert;   // uint4 units
    size_t scales_per_expert;  // dwords
    uint32_t kt, ks;           // H/128 tiles, scale groups
    uint32_t I, H;
    const uint16_t* xn;        // [T][H]
    const uint32_t* n_active;
    const uint4* arec;         // per active slot {expert, rows, offset, row tokens}
    uint16_t* act;             // [pairs][I] bf16, CSR row order
    GluParams glu;
    const uint32_t* status;
};

// Workgroup = 4 * KS waves: four 16-row blocks; with KS = 2 each block's K
// range is split over waves w and w + 4 (first half, second half), added in
// that order before the GLU.
template <int KS>
__global__ __launch_bounds__(256 * KS) void decode_gateup_kernel(GateUpArgs a) {
    __shared__ f32x4 red[KS == 2 ? 4 : 1][2][64];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t per_expert = a.I / 64;
    const uint32_t ai = blockIdx.x / per_expert;
    // Status, active count and this slot's record in one round trip (the
    // record of an inactive slot is not used).
    const uint32_t st = *(volatile const uint32_t*)a.status;
    const uint32_t na = *a.n_active;
    const uint4 rec = a.arec[ai];  // ai < min(E, T*K): in bounds
    if (st || ai >= na) return;
    const uint32_t e = rec.x;
    const uint32_t rb = (blockIdx.x % per_expert) * 4 + (wave & 3);
    const uint32_t half = wave >> 2;
    const uint32_t kt = a.kt;
    // Split on a scale-group boundary, never past the last tile.
    const uint32_t kmid = KS == 1 ? kt : min(kt, (kt / 2 + 3) & ~3u);
    const uint32_t k0 = half ? kmid : 0, k1 = half ? kt : kmid;
    const uint4* codes = a.gu_codes + e * a.codes_per_expert + (size_t)rb * kt * 2 * 64 + lane;
    const uint32_t* scales = a.gu_scales + e * a.scales_per_expert + (size_t)rb * a.ks * 2 * 64 + lane;
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const uint32_t cnt = rec.y, off = rec.z;
    if (k0 < k1) {
        uint4 cn0 = codes[(size_t)k0 * 128], cn1 = codes[(size_t)k0 * 128 + 64];
        const bool arow = n < cnt;
        const uint16_t* ap = a.xn + (size_t)(arow ? (rec.w >> (8 * n)) & 0xffu : 0u) * a.H + 32 * g;
        uint32_t sw0 = 0, sw1 = 0;
        for (uint32_t k = k0; k < k1; ++k) {
            const uint4 c0 = cn0, c1 = cn1;
            if (k + 1 < k1) {
                cn0 = codes[(size_t)(k + 1) * 128];
                cn1 = codes[(size_t)(k + 1) * 128 + 64];
            }
            if ((k & 3) == 0 || k == k0) {
                sw0 = scales[(size_t)(k >> 2) * 128];
                sw1 = scales[(size_t)(k >> 2) * 128 + 64];
            }
            uint4 av[4];
            load_act(ap, arow, k, av);
            acc[0] = mxfp4_tile(c0, e8m0_to_f32((sw0 >> (8 * (k & 3))) & 0xffu), av, acc[0]);
            acc[1] = mxfp4_tile(c1, e8m0_to_f32((sw1 >> (8 * (k & 3))) & 0xffu), av, acc[1]);
        }
    }
    if (KS == 2) {
        if (half) {
            red[wave & 3][0][lane] = acc[0];
            red[wave & 3][1][lane] = acc[1];
        }
        __syncthreads();
        if (half) return;
        acc[0] = acc[0] + red[wave & 3][0][lane];
        acc[1] = acc[1] + red[wave & 3][1][lane];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = 4 * g + i;
        if (row >= cnt) continue;
        const float v = glu(acc[0][i], acc[1][i], a.glu);
        a.act[(size_t)(off + row) * a.I + rb * 16 + n] = f32_to_bf16(v);
    }
}

// ---------------------------------------------------------------------------
// Routed down projection and slot-ordered combine
// ---------------------------------------------------------------------------
constexpr int kMaxDecodePairs = 256;

struct DownArgs {
    const uint4* dn_codes;     // expert 0 base, tiles [H/16][I/128][64] x 16 B
    const uint32_t* dn_scales; // [H/16][ks][64]
    size_t codes_per_expert;
    size_t scales_per_expert;
    uint32_t kt, ks;           // I/128, scale groups
    uint32_t I, H, T, K;
    const uint16_t* act;       // [pairs][I] CSR order
    const uint32_t* n_active;
    const uint4* arec;         // per active slot {expert, rows, offset, row tokens}
    const uint32_t* pair_token;
    const uint32_t* pair_slot;
    const float* weights;      // [T][K]
    const float* shared_y;     // [T][H] shared expert output (null: no shared expert)
    float* y;                  // [T][K][H] per-pair outputs (kept for inspection)
    uint16_t* out;             // [T][H] bf16
    float* out_f32;            // optional
    const uint32_t* status;
};

// Workgroup = 16 waves and one 16-row block of the output.  Wave w projects
// active experts w, w + 16, ... as one stream of (expert, tile) steps (every
// pair of an expert in one pass over its tiles, the next step's codes in
// flight).  The block then sums over slots in router order:
// out[t][h] = bf16(sum_s w[t][s] * y[t][s][h] + shared[t][h]), float mul then
// float add per term (runtime/src/backend_cpu.cpp:295-301,
// runtime/src/model.cpp:1145).
constexpr int kDownWaves = 16;

__global__ __launch_bounds__(64 * kDownWaves) void decode_down_kernel(DownArgs a) {
    __shared__ float ys[kMaxDecodePairs][16];
    __shared__ uint32_t rowof[kMaxDecodePairs];
    __shared__ uint32_t s_e[kMaxDecodePairs], s_cnt[kMaxDecodePairs], s_off[kMaxDecodePairs];
    if (*(volatile const uint32_t*)a.status) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t rb = blockIdx.x;
    const uint32_t P = a.T * a.K;
    const uint32_t na = *a.n_active;
    // Stage the active experts and the (token, slot) -> CSR row map.
    for (uint32_t i = tid; i < na; i += 64 * kDownWaves) {
        const uint4 rec = a.arec[i];
        s_e[i] = rec.x;
        s_cnt[i] = rec.y;
        s_off[i] = rec.z;
    }
    for (uint32_t r = tid; r < P; r += 64 * kDownWaves)
        rowof[a.pair_token[r] * a.K + a.pair_slot[r]] = r;
    __syncthreads();

    // Routed experts: wave w streams experts w, w + 16, ...
    const uint32_t kt = a.kt;
    const uint32_t nexp = na > wave ? (na - wave + kDownWaves - 1) / kDownWaves : 0;
    const uint32_t steps = nexp * kt;
    auto code_at = [&](uint32_t s) {
        const uint32_t e = s_e[wave + kDownWaves * (s / kt)];
        return a.dn_codes[e * a.codes_per_expert + ((size_t)rb * kt + s % kt) * 64 + lane];
    };
    uint4 cn = steps ? code_at(0) : make_uint4(0, 0, 0, 0);
    uint32_t sw = 0;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t s = 0; s < steps; ++s) {
        const uint32_t i = wave + kDownWaves * (s / kt), k = s % kt;
        const uint4 c = cn;
        if (s + 1 < steps) cn = code_at(s + 1);
        const uint32_t e = s_e[i], cnt = s_cnt[i], off = s_off[i];
        if ((k & 3) == 0)
            sw = a.dn_scales[e * a.scales_per_expert + ((size_t)rb * a.ks + k / 4) * 64 + lane];
        const bool arow = n < cnt;
        uint4 av[4];
        load_act(a.act + (size_t)(off + (arow ? n : 0)) * a.I + 32 * g, arow, k, av);
        acc = mxfp4_tile(c, e8m0_to_f32((sw >> (8 * (k & 3))) & 0xffu), av, acc);
        if (k == kt - 1) {  // expert done: its pair rows -> LDS (and y)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t row = 4 * g + q;
                if (row < cnt) {
                    const uint32_t r = off + row;
                    ys[r][n] = acc[q];
                    a.y[((size_t)a.pair_token[r] * a.K + a.pair_slot[r]) * a.H + rb * 16 + n] =
                        acc[q];
                }
            }
            acc = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < a.T * 16; i += 64 * kDownWaves) {
        const uint32_t t = i / 16, c = i % 16, h = rb * 16 + c;
        float mix = 0.0f;
        for (uint32_t s = 0; s < a.K; ++s)
            mix = __fadd_rn(mix, __fmul_rn(a.weights[(size_t)t * a.K + s], ys[rowof[t * a.K + s]][c]));
        const float v = a.shared_y ? __fadd_rn(mix, a.shared_y[(size_t)t * a.H + h]) : mix;
        a.out[(size_t)t * a.H + h] = f32_to_bf16(v);
        if (a.out_f32) a.out_f32[(size_t)t * a.H + h] = v;
    }
}

}  // namespace

namespace k3x_hip {

namespace {

size_t router_lds(uint32_t T, uint32_t H) { return (size_t)T * H * 2 + sizeof(NormShared); }
size_t shared_gateup_lds(uint32_t T, uint32_t H) {
    return (size_t)T * H * 2 + sizeof(SharedGateUpLds);
}

}  // namespace

bool decode_eligible(const k3x_hip_ctx* ctx, const k3x_hip_bank* bank,
                     const k3x_hip_moe_params* p, const void* x) {
    const auto& d = bank->desc;
    if (reinterpret_cast<uintptr_t>(x) % 16) return false;  // 16-byte input loads
    const size_t lds = std::max(router_lds(p->tokens, d.hidden),
                                shared_gateup_lds(p->tokens, d.hidden));
    return p->tokens <= (uint32_t)kMaxDecodeTokens && lds <= ctx->max_lds_per_block &&
           d.hidden % 256 == 0 && d.experts <= (uint32_t)(kKeysPerLane * 64) &&
           p->top_k <= 64 && p->tokens * p->top_k <= (uint32_t)kMaxDecodePairs &&
           d.inter % 64 == 0 && d.shared_inter % 256 == 0;
}

// Launch order: the router, Top-K/grouping and routed gate/up run on the
// context stream; the shared expert, which needs only xn, runs on the
// context's side stream from a fork event recorded at entry, so it overlaps
// the latency-bound router and Top-K steps.  The routed down/combine kernel
// waits for the side stream's join event.  The next call's side work is
// ordered after this call's combine by its own fork event, so the per-call
// buffers are never written while still being read.
int decode_forward(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                   const LayerBuffers& b, const uint16_t* x, uint16_t* out, float* out_f32) {
    const auto& d = bank->desc;
    const uint32_t T = p->tokens, K = p->top_k, S = d.shared_inter;
    const GluParams glu{(int)p->glu, p->situ_beta, (int)p->has_situ_linear, p->situ_linear_beta};
    hipStream_t main = ctx->stream, side = ctx->side_stream;
    if (S && (hipEventRecord(ctx->fork_event, main) != hipSuccess ||
              hipStreamWaitEvent(side, ctx->fork_event, 0) != hipSuccess))
        return K3X_ERR_BACKEND_UNAVAILABLE;

    RouterArgs r{};
    r.x = x;
    r.gamma = bank->gamma;
    r.router_w = bank->router_w;
    r.T = T;
    r.H = d.hidden;
    r.E = d.experts;
    r.eps = p->rms_epsilon;
    r.xn = b.xn;
    r.logits = b.logits;
    r.status = ctx->status;
    const dim3 router_grid((d.experts + kFrontWaves - 1) / kFrontWaves);
    int mark = begin_stage(ctx, K3X_STAGE_DECODE_FRONT, main);
    if (T <= 2)
        hipLaunchKernelGGL((decode_router_kernel<2>), router_grid, dim3(kFrontThreads),
                           (size_t)T * d.hidden * 2, main, r);
    else
        hipLaunchKernelGGL((decode_router_kernel<kMaxDecodeTokens>), router_grid,
                           dim3(kFrontThreads), (size_t)T * d.hidden * 2, main, r);
    end_stage(ctx, mark, main);

    if (S) {
        SharedGateUpArgs sg{};
        sg.x = x;
        sg.gamma = bank->gamma;
        sg.T = T;
        sg.H = d.hidden;
        sg.S = S;
        sg.eps = p->rms_epsilon;
        sg.sh_gu = reinterpret_cast<const uint4*>(bank->sh_gu);
        sg.glu = glu;
        sg.sact = b.sact;
        sg.status = ctx->status;
        mark = begin_stage(ctx, K3X_STAGE_SHARED_GATE_UP, side);
        hipLaunchKernelGGL(decode_shared_gateup_kernel, dim3(S / 16), dim3(64 * kSharedGuWaves),
                           (size_t)T * d.hidden * 2, side, sg);
        end_stage(ctx, mark, side);
        SharedDownArgs sd{};
        sd.sh_dn = reinterpret_cast<const uint4*>(bank->sh_dn);
        sd.sact = b.sact;
        sd.T = T;
        sd.H = d.hidden;
        sd.S = S;
        sd.sy = b.sy;
        sd.status = ctx->status;
        mark = begin_stage(ctx, K3X_STAGE_SHARED_DOWN, side);
        hipLaunchKernelGGL(decode_shared_down_kernel, dim3(d.hidden / 16),
                           dim3(64 * kSharedDnWaves), 0, side, sd);
        end_stage(ctx, mark, side);
        if (hipEventRecord(ctx->join_event, side) != hipSuccess)
            return K3X_ERR_BACKEND_UNAVAILABLE;
    }

    SelectArgs sa{};
    sa.logits = b.logits;
    sa.bias = bank->router_bias;
    sa.T = T;
    sa.E = d.experts;
    sa.K = K;
    sa.routed_scale = p->routed_scale;
    sa.renorm = p->renorm;
    sa.ids = b.ids;
    sa.weights = b.weights;
    sa.counts = b.counts;
    sa.offsets = b.offsets;
    sa.pair_token = b.pair_token;
    sa.pair_slot = b.pair_slot;
    sa.first_use = b.first_use;
    sa.n_active = b.n_active;
    sa.active_asc = b.active_asc;
    sa.active_fu = b.active_fu;
    sa.arec = b.arec;
    sa.status = ctx->status;
    mark = begin_stage(ctx, K3X_STAGE_DECODE_SELECT, main);
    hipLaunchKernelGGL(decode_select_kernel, dim3(1), dim3(kFrontThreads), 0, main, sa);
    end_stage(ctx, mark, main);

    const uint32_t max_active = std::min<uint32_t>(d.experts, T * K);
    GateUpArgs gu{};
    gu.gu_codes = reinterpret_cast<const uint4*>(bank->gu_codes);
    gu.gu_scales = bank->gu_scales;
    gu.codes_per_expert = bank->gu_codes_per_expert / 16;
    gu.scales_per_expert = bank->gu_scales_per_expert;
    gu.kt = bank->gate.kt;
    gu.ks = bank->gate.ks;
    gu.I = d.inter;
    gu.H = d.hidden;
    gu.xn = b.xn;
    gu.n_active = b.n_active;
    gu.arec = b.arec;
    gu.act = b.act;
    gu.glu = glu;
    gu.status = ctx->status;
    // Split K over two waves only while every workgroup of the launch fits
    // on the device at once; otherwise the extra waves run as a second,
    // partly empty round.
    if (!ctx->gateup_split_blocks) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_gateup_kernel<2>, 512,
                                                         0) != hipSuccess)
            (void)hipGetLastError();
        ctx->gateup_split_blocks = (uint32_t)std::max(per_cu, 0) * ctx->cu_count + 1;
    }
    const uint32_t gu_blocks = max_active * (d.inter / 64);
    mark = begin_stage(ctx, K3X_STAGE_DECODE_GATE_UP, main);
    if (gu_blocks < ctx->gateup_split_blocks)
        hipLaunchKernelGGL((decode_gateup_kernel<2>), dim3(gu_blocks), dim3(512), 0, main, gu);
    else
        hipLaunchKernelGGL((decode_gateup_kernel<1>), dim3(gu_blocks), dim3(256), 0, main, gu);
    end_stage(ctx, mark, main);

    if (S && hipStreamWaitEvent(main, ctx->join_event, 0) != hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    DownArgs dn{};
    dn.dn_codes = reinterpret_cast<const uint4*>(bank->dn_codes);
    dn.dn_scales = bank->dn_scales;
    dn.codes_per_expert = bank->dn_codes_per_expert / 16;
    dn.scales_per_expert = bank->dn_scales_per_expert;
    dn.kt = bank->down.kt;
    dn.ks = bank->down.ks;
    dn.I = d.inter;
    dn.H = d.hidden;
    dn.T = T;
    dn.K = K;
    dn.act = b.act;
    dn.n_active = b.n_active;
    dn.arec = b.arec;
    dn.pair_token = b.pair_token;
    dn.pair_slot = b.pair_slot;
    dn.weights = b.weights;
    dn.shared_y = S ? b.sy : nullptr;
    dn.y = b.y;
    dn.out = out;
    dn.out_f32 = out_f32;
    dn.status = ctx->status;
    mark = begin_stage(ctx, K3X_STAGE_DECODE_DOWN, main);
    hipLaunchKernelGGL(decode_down_kernel, dim3(d.hidden / 16), dim3(64 * kDownWaves), 0, main,
                       dn);
    end_stage(ctx, mark, main);
    ctx->kernel_launches += S ? 6 : 4;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

}  // namespace k3x_hip
