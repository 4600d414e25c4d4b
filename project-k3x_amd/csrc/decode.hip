// decode.hip -- the decode path of the MoE layer (T <= 4 tokens), five
// launches with no cross-workgroup synchronisation inside any of them:
//
//   decode_front_kernel   every block rebuilds xn = bf16(RMSNorm(x) * gamma)
//                         in LDS.  Router blocks stream the fp32 router (one
//                         wave per expert row, fp64, canonical order) into
//                         logits; shared blocks run the bf16 shared-expert
//                         gate/up + GLU with the K range split over 8 waves.
//   decode_select_kernel  block 0: sigmoid + bias Top-K of every token and the
//                         expert-major grouping; the other blocks run the
//                         shared down projection (K split over 8 waves), so
//                         the selection's latency hides behind that stream.
//   decode_gateup_kernel  routed MXFP4 gate/up + GLU per active expert: four
//                         16-row blocks per workgroup, K split over two waves
//                         each, weights dequantised in registers.
//   decode_down_kernel    routed MXFP4 down projection to per-pair fp32 rows.
//   combine (pipeline.hip) out = bf16(sum over slots in router order of
//                         w * y + shared).
//
// Numerics are identical to the general path in pipeline.hip: the same
// canonical fp64 order for the RMS sum and the router logits, the same
// Top-K keys and renormalisation, the same per-accumulator MFMA order for
// the routed experts, the same slot-ordered combine.
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

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint64_t o = __shfl_xor(v, d);
        v = o > v ? o : v;
    }
    return v;
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
// Front kernel: xn, router logits, shared gate/up
// ---------------------------------------------------------------------------
struct FrontArgs {
    const uint16_t* x;
    const float* gamma;
    const float* router_w;
    uint32_t T, H, E, S;
    float eps;
    uint32_t router_blocks;
    const uint4* sh_gu;  // shared gate/up tiles [S/16][H/128][2][4][64] x 16 B
    GluParams glu;
    uint16_t* xn;        // [T][H] global copy (block 0 writes it)
    float* logits;       // [T][E]
    uint16_t* sact;      // [T][S] shared-expert activation
    uint32_t* status;
};

struct FrontShared {
    float inv[kMaxDecodeTokens];
    int bad;
    f32x4 red[kFrontWaves][2][64];  // shared blocks: split-K partials
};

__global__ __launch_bounds__(kFrontThreads) void decode_front_kernel(FrontArgs a) {
    extern __shared__ uint4 dyn_lds[];
    uint16_t* s_x = reinterpret_cast<uint16_t*>(dyn_lds);  // [T][H]
    __shared__ FrontShared sh;
    if (*(volatile uint32_t*)a.status) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t T = a.T, H = a.H;

    // -- 1. x -> LDS in 16-byte chunks; T*H/8 <= 3584 chunks. --------------
    if (tid == 0) sh.bad = 0;
    const uint32_t chunks = T * H / 8;
    {
        constexpr int kMaxIt = (kMaxDecodeTokens * 7168 / 8 + kFrontThreads - 1) / kFrontThreads;
        uint4 v[kMaxIt];
#pragma unroll
        for (int it = 0; it < kMaxIt; ++it) {
            const uint32_t c = tid + kFrontThreads * it;
            if (c < chunks) v[it] = reinterpret_cast<const uint4*>(a.x)[c];
        }
#pragma unroll
        for (int it = 0; it < kMaxIt; ++it) {
            const uint32_t c = tid + kFrontThreads * it;
            if (c < chunks) dyn_lds[c] = v[it];
        }
    }
    __syncthreads();
    // -- 2. sum of squares in the canonical order; inverse RMS per token. ---
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
            if (bad) sh.bad = 1;
            const float mean = (float)__ddiv_rn(s, (double)H);
            sh.inv[wave] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, a.eps)));
        }
    }
    __syncthreads();
    if (sh.bad) {
        if (tid == 0) latch(a.status, K3X_ERR_INVALID_MXFP4);
        return;
    }
    // -- 3. xn = bf16(x * inv * gamma) in place. ---------------------------
    for (uint32_t c = tid; c < chunks; c += kFrontThreads) {
        const uint32_t t = (c * 8) / H, k = (c * 8) % H;
        const uint4 w = dyn_lds[c];
        const float4 g0 = *reinterpret_cast<const float4*>(a.gamma + k);
        const float4 g1 = *reinterpret_cast<const float4*>(a.gamma + k + 4);
        const float inv = sh.inv[t];
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
        dyn_lds[c] = ov;
        if (blockIdx.x == 0) reinterpret_cast<uint4*>(a.xn)[c] = ov;
    }
    __syncthreads();

    if (blockIdx.x < a.router_blocks) {
        // -- 4. router logits: wave -> expert row, fp64 canonical order. ---
        const uint32_t e = blockIdx.x * kFrontWaves + wave;
        if (e >= a.E) return;
        const float* wr = a.router_w + (size_t)e * H;
        double p[kMaxDecodeTokens][4];
#pragma unroll
        for (int t = 0; t < kMaxDecodeTokens; ++t)
#pragma unroll
            for (int c = 0; c < 4; ++c) p[t][c] = 0.0;
        const uint32_t J = H / 256;
        constexpr int kBatch = 14;
        for (uint32_t j0 = 0; j0 < J; j0 += kBatch) {
            float4 w[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (j0 + u < J)
                    w[u] = *reinterpret_cast<const float4*>(wr + 256 * (j0 + u) + 4 * lane);
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                if (j0 + u >= J) continue;
                const float wv[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
                for (int t = 0; t < kMaxDecodeTokens; ++t) {
                    if ((uint32_t)t >= T) continue;
                    const uint2 xv = *reinterpret_cast<const uint2*>(
                        s_x + (size_t)t * H + 256 * (j0 + u) + 4 * lane);
                    const float f[4] = {lo_bf16(xv.x), hi_bf16(xv.x), lo_bf16(xv.y),
                                        hi_bf16(xv.y)};
#pragma unroll
                    for (int c = 0; c < 4; ++c) p[t][c] += (double)wv[c] * (double)f[c];
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kMaxDecodeTokens; ++t) {
            if ((uint32_t)t >= T) continue;
            const double v = canon_reduce(p[t]);
            if (lane == 0) a.logits[(size_t)t * a.E + e] = (float)v;
        }
        return;
    }

    // -- 5. shared expert gate/up + GLU: 16 rows, K split over 8 waves. ---
    const uint32_t rb = blockIdx.x - a.router_blocks;
    const uint32_t kt = H / 128;
    const uint32_t k0 = wave * kt / kFrontWaves, k1 = (wave + 1) * kt / kFrontWaves;
    const uint32_t g = lane >> 4, n = lane & 15;
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const uint4* tiles = a.sh_gu + (size_t)rb * kt * 2 * 4 * 64 + lane;
    const bool arow = n < T;
    for (uint32_t k = k0; k < k1; ++k) {
        uint4 b[2][4];
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int j = 0; j < 4; ++j) b[w][j] = tiles[(((size_t)k * 2 + w) * 4 + j) * 64];
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
            for (int w = 0; w < 2; ++w) acc[w] = mfma16x16x32(af[j], as_bf16x8(b[w][j]), acc[w]);
    }
    sh.red[wave][0][lane] = acc[0];
    sh.red[wave][1][lane] = acc[1];
    __syncthreads();
    if (wave == 0) {
        f32x4 r[2];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const f32x4 s01 = sh.red[0][w][lane] + sh.red[1][w][lane];
            const f32x4 s23 = sh.red[2][w][lane] + sh.red[3][w][lane];
            const f32x4 s45 = sh.red[4][w][lane] + sh.red[5][w][lane];
            const f32x4 s67 = sh.red[6][w][lane] + sh.red[7][w][lane];
            r[w] = (s01 + s23) + (s45 + s67);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t row = 4 * g + i;  // token
            if (row >= T) continue;
            const float v = glu(r[0][i], r[1][i], a.glu);
            a.sact[(size_t)row * a.S + rb * 16 + n] = f32_to_bf16(v);
        }
    }
}

// ---------------------------------------------------------------------------
// Select kernel: Top-K + grouping (block 0), shared down (other blocks)
// ---------------------------------------------------------------------------
struct SelectArgs {
    const float* logits;
    const float* bias;
    uint32_t T, H, E, K, S;
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
    const uint4* sh_dn;  // shared down tiles [H/16][S/128][4][64] x 16 B
    const uint16_t* sact;
    float* shared_y;     // [T][H]
    uint32_t* status;
};

struct SelectShared {
    int bad;
    uint32_t wave_sums[kFrontWaves];
    union {
        struct {
            uint32_t ids[kMaxDecodeTokens * 64];
            uint32_t cnt[kKeysPerLane * 64];
            uint32_t fu[kKeysPerLane * 64];
            uint32_t off[kKeysPerLane * 64];
            uint32_t active[kMaxDecodeTokens * 64];
        } g;
        f32x4 red[kFrontWaves][64];
    } u;
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
        const uint64_t best = wave_max_u64(key[0]);
        const uint32_t win = 0xffffffffu - (uint32_t)best;
        const bool mine = key[0] == best;
        const int wlane = __ffsll((unsigned long long)__ballot(mine)) - 1;
        const float wsc = __shfl(score[0], wlane);
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
        const float v = __shfl(selsc, s);
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
        sh.u.g.ids[t * K + lane] = selid;
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
        sh.u.g.cnt[e] = 0;
        sh.u.g.fu[e] = 0xffffffffu;
    }
    __syncthreads();
    if (tid < P) {
        const uint32_t e = sh.u.g.ids[tid];
        atomicAdd(&sh.u.g.cnt[e], 1u);
        atomicMin(&sh.u.g.fu[e], tid);
    }
    __syncthreads();
    // E <= 512: one expert per thread.
    const uint32_t c = tid < E ? sh.u.g.cnt[tid] : 0u;
    uint32_t total = 0, na = 0;
    const uint32_t excl = block_scan_excl(c, sh.wave_sums, &total);
    const uint32_t aidx = block_scan_excl(c ? 1u : 0u, sh.wave_sums, &na);
    if (tid < E) {
        sh.u.g.off[tid] = excl;
        a.offsets[tid] = excl;
        a.counts[tid] = c;
        a.first_use[tid] = sh.u.g.fu[tid];
        if (c) {
            a.active_asc[aidx] = tid;
            sh.u.g.active[aidx] = tid;
        }
    }
    if (tid == 0) {
        a.offsets[E] = total;
        *a.n_active = na;
    }
    __syncthreads();
    if (tid < P) {
        const uint32_t e = sh.u.g.ids[tid];
        uint32_t rank = 0;
        for (uint32_t q = 0; q < tid; ++q) rank += sh.u.g.ids[q] == e;
        const uint32_t r = sh.u.g.off[e] + rank;
        a.pair_token[r] = tid / a.K;
        a.pair_slot[r] = tid % a.K;
    }
    if (tid < na) {
        const uint32_t e = sh.u.g.active[tid];
        const uint32_t key = sh.u.g.fu[e];
        uint32_t rank = 0;
        for (uint32_t b = 0; b < na; ++b) rank += sh.u.g.fu[sh.u.g.active[b]] < key;
        a.active_fu[rank] = e;
    }
}

__global__ __launch_bounds__(kFrontThreads) void decode_select_kernel(SelectArgs a) {
    __shared__ SelectShared sh;
    if (*(volatile uint32_t*)a.status) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (blockIdx.x == 0) {
        if (tid == 0) sh.bad = 0;
        __syncthreads();
        if (wave < a.T) topk_token(a, wave, sh);
        __syncthreads();
        if (sh.bad) return;
        group_pairs(a, sh);
        return;
    }
    // Shared down: one 16-row block per workgroup, K split over 8 waves.
    const uint32_t rb = blockIdx.x - 1;
    const uint32_t kt = a.S / 128;
    const uint32_t k0 = wave * kt / kFrontWaves, k1 = (wave + 1) * kt / kFrontWaves;
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint4* tiles = a.sh_dn + (size_t)rb * kt * 4 * 64 + lane;
    const bool arow = n < a.T;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t k = k0; k < k1; ++k) {
        uint4 b[4], av[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            b[j] = tiles[((size_t)k * 4 + j) * 64];
            av[j] = arow ? *reinterpret_cast<const uint4*>(a.sact + (size_t)n * a.S + k * 128 +
                                                           32 * g + 8 * j)
                         : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = mfma16x16x32(as_bf16x8(av[j]), as_bf16x8(b[j]), acc);
    }
    sh.u.red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        const f32x4 s01 = sh.u.red[0][lane] + sh.u.red[1][lane];
        const f32x4 s23 = sh.u.red[2][lane] + sh.u.red[3][lane];
        const f32x4 s45 = sh.u.red[4][lane] + sh.u.red[5][lane];
        const f32x4 s67 = sh.u.red[6][lane] + sh.u.red[7][lane];
        const f32x4 r = (s01 + s23) + (s45 + s67);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t row = 4 * g + i;
            if (row < a.T) a.shared_y[(size_t)row * a.H + rb * 16 + n] = r[i];
        }
    }
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
    const uint32_t* active;
    const uint32_t* counts;
    const uint32_t* offsets;
    const uint32_t* pair_token;
    uint16_t* act;             // [pairs][I] bf16, CSR row order
    GluParams glu;
    const uint32_t* status;
};

// One MXFP4 K-range of a 16-row block: codes/scales from the tile layout,
// activations from rows `ap` (lanes with arow), MFMAs into acc.  Tiles are
// loaded one ahead of the MFMAs that consume them.
template <int S>
__device__ inline void mxfp4_krange(const uint4* codes, const uint32_t* scales, uint32_t k0,
                                    uint32_t k1, const uint16_t* ap, bool arow, f32x4* acc) {
    if (k0 >= k1) return;
    uint4 cn[S], an[4];
#pragma unroll
    for (int w = 0; w < S; ++w) cn[w] = codes[(size_t)k0 * 64 * S + 64 * w];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        an[j] = arow ? *reinterpret_cast<const uint4*>(ap + k0 * 128 + 8 * j) : make_uint4(0, 0, 0, 0);
    for (uint32_t k = k0; k < k1; ++k) {
        uint4 c[S], av[4];
#pragma unroll
        for (int w = 0; w < S; ++w) c[w] = cn[w];
#pragma unroll
        for (int j = 0; j < 4; ++j) av[j] = an[j];
        uint32_t sw[S];
#pragma unroll
        for (int w = 0; w < S; ++w) sw[w] = scales[(size_t)(k >> 2) * 64 * S + 64 * w];
        if (k + 1 < k1) {
#pragma unroll
            for (int w = 0; w < S; ++w) cn[w] = codes[(size_t)(k + 1) * 64 * S + 64 * w];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                an[j] = arow ? *reinterpret_cast<const uint4*>(ap + (k + 1) * 128 + 8 * j)
                             : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int w = 0; w < S; ++w) {
            const float sc = e8m0_to_f32((sw[w] >> (8 * (k & 3))) & 0xffu);
            const uint32_t cw[4] = {c[w].x, c[w].y, c[w].z, c[w].w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[w] = mfma16x16x32(as_bf16x8(av[j]), dequant8(cw[j], sc), acc[w]);
        }
    }
}

// Workgroup = 8 waves: four 16-row blocks, each block's K range split over
// waves w and w + 4 (first half, second half); the halves are added in that
// order before the GLU.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(6, 6))) void
decode_gateup_kernel(GateUpArgs a) {
    __shared__ f32x4 red[4][2][64];
    if (*(volatile const uint32_t*)a.status) return;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t per_expert = a.I / 64;
    const uint32_t ai = blockIdx.x / per_expert;
    if (ai >= *a.n_active) return;
    const uint32_t e = a.active[ai];
    const uint32_t cnt = a.counts[e], off = a.offsets[e];
    const uint32_t rb = (blockIdx.x % per_expert) * 4 + (wave & 3);
    const uint32_t half = wave >> 2;
    const uint32_t kt = a.kt;
    // Split on a scale-group boundary, never past the last tile.
    const uint32_t kmid = min(kt, (kt / 2 + 3) & ~3u);
    const uint32_t k0 = half ? kmid : 0, k1 = half ? kt : kmid;
    const uint4* codes = a.gu_codes + e * a.codes_per_expert + (size_t)rb * kt * 2 * 64 + lane;
    const uint32_t* scales = a.gu_scales + e * a.scales_per_expert + (size_t)rb * a.ks * 2 * 64 + lane;
    const bool arow = n < cnt;
    const uint16_t* ap = arow ? a.xn + (size_t)a.pair_token[off + n] * a.H + 32 * g : a.xn;
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    mxfp4_krange<2>(codes, scales, k0, k1, ap, arow, acc);
    if (half) {
        red[wave & 3][0][lane] = acc[0];
        red[wave & 3][1][lane] = acc[1];
    }
    __syncthreads();
    if (half) return;
    const f32x4 gsum = acc[0] + red[wave][0][lane];
    const f32x4 usum = acc[1] + red[wave][1][lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = 4 * g + i;
        if (row >= cnt) continue;
        const float v = glu(gsum[i], usum[i], a.glu);
        a.act[(size_t)(off + row) * a.I + rb * 16 + n] = f32_to_bf16(v);
    }
}

// ---------------------------------------------------------------------------
// Routed down projection -> per-pair fp32 rows
// ---------------------------------------------------------------------------
struct DownArgs {
    const uint4* dn_codes;     // expert 0 base, tiles [H/16][I/128][64] x 16 B
    const uint32_t* dn_scales; // [H/16][ks][64]
    size_t codes_per_expert;
    size_t scales_per_expert;
    uint32_t kt, ks;           // I/128, scale groups
    uint32_t I, H, K;
    const uint16_t* act;       // [pairs][I] CSR order
    const uint32_t* n_active;
    const uint32_t* active;
    const uint32_t* counts;
    const uint32_t* offsets;
    const uint32_t* pair_token;
    const uint32_t* pair_slot;
    float* y;                  // [T][K][H]
    const uint32_t* status;
};

// Workgroup = 4 waves, one 16-row block each, the whole K range.
__global__ __launch_bounds__(256) void decode_down_kernel(DownArgs a) {
    if (*(volatile const uint32_t*)a.status) return;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t per_expert = a.H / 64;
    const uint32_t ai = blockIdx.x / per_expert;
    if (ai >= *a.n_active) return;
    const uint32_t e = a.active[ai];
    const uint32_t cnt = a.counts[e], off = a.offsets[e];
    const uint32_t rb = (blockIdx.x % per_expert) * 4 + wave;
    const uint32_t kt = a.kt;
    const uint4* codes = a.dn_codes + e * a.codes_per_expert + (size_t)rb * kt * 64 + lane;
    const uint32_t* scales = a.dn_scales + e * a.scales_per_expert + (size_t)rb * a.ks * 64 + lane;
    const bool arow = n < cnt;
    const uint16_t* ap = a.act + (size_t)(off + (arow ? n : 0)) * a.I + 32 * g;
    f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
    mxfp4_krange<1>(codes, scales, 0, kt, ap, arow, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = 4 * g + i;
        if (row >= cnt) continue;
        const uint32_t r = off + row;
        const size_t yrow = (size_t)a.pair_token[r] * a.K + a.pair_slot[r];
        a.y[yrow * a.H + rb * 16 + n] = acc[0][i];
    }
}

}  // namespace

namespace k3x_hip {

bool decode_eligible(const k3x_hip_ctx* ctx, const k3x_hip_bank* bank,
                     const k3x_hip_moe_params* p, const void* x) {
    const auto& d = bank->desc;
    if (reinterpret_cast<uintptr_t>(x) % 16) return false;  // 16-byte input loads
    const size_t lds = (size_t)p->tokens * d.hidden * 2 + sizeof(FrontShared);
    return p->tokens <= (uint32_t)kMaxDecodeTokens && lds <= ctx->max_lds_per_block &&
           d.hidden % 256 == 0 && d.hidden <= 7168 && d.experts <= (uint32_t)(kKeysPerLane * 64) &&
           p->top_k <= 64 && p->tokens * p->top_k <= 256 && d.inter % 64 == 0 &&
           d.hidden % 64 == 0;
}

int decode_forward(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                   const LayerBuffers& b, const uint16_t* x, uint16_t* out, float* out_f32) {
    const auto& d = bank->desc;
    const uint32_t T = p->tokens, K = p->top_k;
    const GluParams glu{(int)p->glu, p->situ_beta, (int)p->has_situ_linear, p->situ_linear_beta};

    FrontArgs f{};
    f.x = x;
    f.gamma = bank->gamma;
    f.router_w = bank->router_w;
    f.T = T;
    f.H = d.hidden;
    f.E = d.experts;
    f.S = d.shared_inter;
    f.eps = p->rms_epsilon;
    f.router_blocks = (d.experts + kFrontWaves - 1) / kFrontWaves;
    f.sh_gu = reinterpret_cast<const uint4*>(bank->sh_gu);
    f.glu = glu;
    f.xn = b.xn;
    f.logits = b.logits;
    f.sact = b.sact;
    f.status = ctx->status;
    const size_t lds = (size_t)T * d.hidden * 2;
    int mark = begin_stage(ctx, K3X_STAGE_DECODE_FRONT);
    hipLaunchKernelGGL(decode_front_kernel, dim3(f.router_blocks + d.shared_inter / 16),
                       dim3(kFrontThreads), lds, ctx->stream, f);
    end_stage(ctx, mark);

    SelectArgs sa{};
    sa.logits = b.logits;
    sa.bias = bank->router_bias;
    sa.T = T;
    sa.H = d.hidden;
    sa.E = d.experts;
    sa.K = K;
    sa.S = d.shared_inter;
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
    sa.sh_dn = reinterpret_cast<const uint4*>(bank->sh_dn);
    sa.sact = b.sact;
    sa.shared_y = b.sy;
    sa.status = ctx->status;
    mark = begin_stage(ctx, K3X_STAGE_DECODE_SELECT);
    hipLaunchKernelGGL(decode_select_kernel, dim3(1 + (d.shared_inter ? d.hidden / 16 : 0)),
                       dim3(kFrontThreads), 0, ctx->stream, sa);
    end_stage(ctx, mark);

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
    gu.active = b.active_asc;
    gu.counts = b.counts;
    gu.offsets = b.offsets;
    gu.pair_token = b.pair_token;
    gu.act = b.act;
    gu.glu = glu;
    gu.status = ctx->status;
    mark = begin_stage(ctx, K3X_STAGE_DECODE_GATE_UP);
    hipLaunchKernelGGL(decode_gateup_kernel, dim3(max_active * (d.inter / 64)), dim3(512), 0,
                       ctx->stream, gu);
    end_stage(ctx, mark);

    DownArgs dn{};
    dn.dn_codes = reinterpret_cast<const uint4*>(bank->dn_codes);
    dn.dn_scales = bank->dn_scales;
    dn.codes_per_expert = bank->dn_codes_per_expert / 16;
    dn.scales_per_expert = bank->dn_scales_per_expert;
    dn.kt = bank->down.kt;
    dn.ks = bank->down.ks;
    dn.I = d.inter;
    dn.H = d.hidden;
    dn.K = K;
    dn.act = b.act;
    dn.n_active = b.n_active;
    dn.active = b.active_asc;
    dn.counts = b.counts;
    dn.offsets = b.offsets;
    dn.pair_token = b.pair_token;
    dn.pair_slot = b.pair_slot;
    dn.y = b.y;
    dn.status = ctx->status;
    mark = begin_stage(ctx, K3X_STAGE_DECODE_DOWN);
    hipLaunchKernelGGL(decode_down_kernel, dim3(max_active * (d.hidden / 64)), dim3(256), 0,
                       ctx->stream, dn);
    end_stage(ctx, mark);
    ctx->kernel_launches += 4;
    if (hipGetLastError() != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    return launch_combine(ctx, b.y, b.weights, d.shared_inter ? b.sy : nullptr, K, d.hidden, T,
                          out, out_f32);
}

}  // namespace k3x_hip
