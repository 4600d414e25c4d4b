// decode.hip -- the decode path of the MoE layer (T <= 4 tokens): four
// launches; no workgroup ever waits for another (the fused combine is done
// by whichever workgroup completes a counter).
//
//   decode_front_kernel   router blocks rebuild xn = bf16(RMSNorm(x) * gamma)
//                         in LDS and stream the fp32 router, one wave per
//                         expert row (fp64, canonical order), into logits;
//                         shared blocks (same xn prologue) stream the bf16
//                         shared-expert gate/up, K split over the waves, and
//                         write the shared activation bf16(GLU(gate, up)).
//   decode_select_kernel  block 0: sigmoid + bias Top-K of every token and
//                         the expert-major grouping; the other blocks stream
//                         the bf16 shared down projection.
//   decode_gateup_kernel  routed MXFP4 gate/up + GLU: one wave per (active
//                         expert, 16-row block), weights dequantised in
//                         registers.
//   decode_down_kernel    routed MXFP4 down projection: one wave per (active
//                         expert, 16-row block) -> per-pair rows y; the
//                         workgroup that stores the last of a token's K rows
//                         of a 64-column group writes that group of
//                         out = bf16(sum over slots in router order of w * y
//                         + shared).
// The shared expert needs only xn, so it rides along as extra workgroups of
// the two latency-bound launches (router, Top-K), whose own blocks leave
// most of the device idle.
//
// Streaming loops keep several steps of loads in flight per wave with no
// branch around a weight load (indices clamped instead), so the compiler's
// in-order wait on the vector-memory counter never waits for a later step.
// Work units of one wave spread evenly over the CUs.
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

// Canonical combination of one lane's four partial sums (partials 4l..4l+3
// of the 256-way strided order) and the 64-lane butterfly: the pairwise tree
// over all 256 partials.
__device__ inline double canon_reduce(const double p[4]) {
    double v = (p[0] + p[1]) + (p[2] + p[3]);
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
    return v;
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

// The same tile against split activations hi + lo (each weight fragment
// dequantised once, two MFMAs).
__device__ inline f32x4 mxfp4_tile2(const uint4& c, float scale, const uint4 ah[4],
                                    const uint4 al[4], f32x4 acc) {
    const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bf16x8 b = dequant8(cw[j], scale);
        acc = mfma16x16x32(as_bf16x8(ah[j]), b, acc);
        acc = mfma16x16x32(as_bf16x8(al[j]), b, acc);
    }
    return acc;
}

// Activation slice for K tile k, loaded only by the lanes whose MFMA row is
// used: row m of an MFMA result depends only on row m of A, and unused rows
// are never stored, so the other lanes' registers may hold anything.  Issued
// before a step's weight loads, so that the weight loads of later steps,
// which every path issues, stay counted behind a step's own loads and the
// compiler can wait for one step while later steps remain in flight.
__device__ inline void load_act(const uint16_t* ap, bool arow, uint32_t k, uint4 av[4]) {
    if (arow)
#pragma unroll
        for (int j = 0; j < 4; ++j) av[j] = *reinterpret_cast<const uint4*>(ap + k * 128 + 8 * j);
}


// Routed expert weights are read once per call (each expert's tiles by one
// workgroup set) and not again before other layers' weights have passed
// through the caches: non-temporal loads, which do not keep the lines in
// the L2 / MALL, leave those caches to the activations, per-pair rows and
// counters that are re-read (C3 decode: gate/up 76.3 -> 74.8 us, down
// 47.0 -> 44.1 us).
__device__ inline uint4 ntl(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ inline uint32_t ntl(const uint32_t* p) { return __builtin_nontemporal_load(p); }

// Wave index as a wave-uniform (scalar) value.
__device__ inline uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Latched error word as left by earlier launches: a plain load from a
// uniform address (a scalar load, counted apart from the vector loads, so
// that checking it does not wait for weight prefetches already issued).
__device__ inline uint32_t prior_status(const uint32_t* status) { return *status; }

// ---------------------------------------------------------------------------
// xn prologue of the router and shared gate/up kernels
// ---------------------------------------------------------------------------
struct NormShared {
    float inv[kMaxDecodeTokens];
    double part[kFrontWaves];  // per-wave sums of squares
    int bad;
};

// x and gamma -> LDS in one batch of 16-byte loads, inverse RMS per token
// from the sum of squares in the canonical fp64 order, then xn = bf16(x *
// inv * gamma) in place; the block then holds xn as [T][H] bf16 at s_x4
// (gamma follows as [H] fp32).  Returns false when x holds a non-finite
// value (latched into *status when status is non-null).  Needs at least T
// waves; xn_out, when non-null, receives a global copy.  mid() runs once
// the first batch of x / gamma loads is issued (the caller's weight
// prefetch goes there: vector loads complete in order, so loads issued
// before x / gamma would delay the prologue); then the latched error word of
// earlier launches is checked (false, for the whole block, when it is set).
// late() runs once this wave's x / gamma loads have arrived, before the sum
// of squares and the xn pass (loads issued there overlap them without
// queueing ahead of any block's x / gamma).
template <int kThreads, typename Mid, typename Late>
__device__ __forceinline__ bool build_xn(const uint16_t* x, const float* gamma, uint32_t T,
                                         uint32_t H, float eps, uint4* s_x4, NormShared& ns,
                                         uint16_t* xn_out, uint32_t* status,
                                         const uint32_t* prior, Mid&& mid, Late&& late) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint16_t* s_x = reinterpret_cast<const uint16_t*>(s_x4);
    const uint32_t chunks = T * H / 8;          // x chunks; gamma chunks follow
    const uint32_t all = chunks + H / 4;
    const float* s_g = reinterpret_cast<const float*>(s_x4 + chunks);
    if (tid == 0) ns.bad = 0;
    constexpr int kLoads = 8;
    // Every block of the launch reads the same x and gamma: each starts at
    // its own offset so that they do not all request the same lines at once.
    const uint32_t rot = (blockIdx.x * 613u) % all;
    // Slot c of the rotated order (c < all, rot < all): one compare and
    // subtract, not a division.
    auto rotated = [&](uint32_t c) {
        c += rot;
        return c >= all ? c - all : c;
    };
    for (uint32_t c0 = 0; c0 < all; c0 += kLoads * kThreads) {
        // One unconditional load and store per slot (slots past the end
        // copy the last chunk again, the same value to the same place): no
        // branch, so the loads are all in flight together.
        uint4 v[kLoads];
#pragma unroll
        for (int it = 0; it < kLoads; ++it) {
            const uint32_t c = rotated(min(c0 + tid + kThreads * it, all - 1));
            const uint4* src = c < chunks ? reinterpret_cast<const uint4*>(x) + c
                                          : reinterpret_cast<const uint4*>(gamma) + (c - chunks);
            v[it] = *src;
        }
        if (c0 == 0) {
            mid();
            if (prior_status(prior)) return false;
        }
#pragma unroll
        for (int it = 0; it < kLoads; ++it)
            s_x4[rotated(min(c0 + tid + kThreads * it, all - 1))] = v[it];
    }
    // x and gamma have arrived (this wave's, and the block's after the
    // barrier): late() may now request what the block needs after xn.
    late();
    __syncthreads();
    // Sum of squares per token in the canonical order -- partial q (of 256)
    // sums the elements 256 j + q over j in sequence, then the balanced
    // pairwise tree over q -- spread over nw = 4 (T <= 2) or 2 waves per
    // token: wave u of token t owns partials [256 u / nw, 256 (u + 1) / nw),
    // reduces them across lanes (the tree's lower levels) and the top levels
    // add the wave sums.  Every tree node adds the same two children as a
    // one-wave reduction (canon_reduce), so the sum is bit-identical.
    static_assert(kThreads / 64 >= 2 * kMaxDecodeTokens, "two waves per token");
    const uint32_t nw = T <= 2 ? 4 : 2, t = wave / nw, u = wave % nw;
    if (t < T) {
        const uint16_t* xr = s_x + (size_t)t * H;
        double v;
        int bad = 0;
        // The values of eight steps j are read from LDS before their eight
        // dependent FMAs (one LDS round trip per eight steps, not per step);
        // reads past the row end repeat its last group and are not added.
        constexpr uint32_t kB = 8;
        const uint32_t J = H / 256;
        if (nw == 4) {
            double p = 0.0;
            for (uint32_t j0 = 0; j0 < J; j0 += kB) {
                float f[kB];
#pragma unroll
                for (uint32_t i = 0; i < kB; ++i)
                    f[i] = bf16_to_f32(xr[256 * min(j0 + i, J - 1) + 64 * u + lane]);
#pragma unroll
                for (uint32_t i = 0; i < kB; ++i) {
                    if (j0 + i >= J) break;
                    bad |= !__builtin_isfinite(f[i]);
                    p = __builtin_fma((double)f[i], (double)f[i], p);  // exact product
                }
            }
            v = p;
        } else {
            double p0 = 0.0, p1 = 0.0;
            for (uint32_t j0 = 0; j0 < J; j0 += kB) {
                uint32_t w[kB];
#pragma unroll
                for (uint32_t i = 0; i < kB; ++i)
                    w[i] = *reinterpret_cast<const uint32_t*>(xr + 256 * min(j0 + i, J - 1) +
                                                              128 * u + 2 * lane);
#pragma unroll
                for (uint32_t i = 0; i < kB; ++i) {
                    if (j0 + i >= J) break;
                    const float f0 = lo_bf16(w[i]), f1 = hi_bf16(w[i]);
                    bad |= !__builtin_isfinite(f0) | !__builtin_isfinite(f1);
                    p0 = __builtin_fma((double)f0, (double)f0, p0);
                    p1 = __builtin_fma((double)f1, (double)f1, p1);
                }
            }
            v = p0 + p1;
        }
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
        if (__any(bad) && lane == 0) ns.bad = 1;
        if (lane == 0) ns.part[wave] = v;
    }
    __syncthreads();
    if (tid < T) {
        const double* q = ns.part + tid * nw;
        const double s = nw == 4 ? (q[0] + q[1]) + (q[2] + q[3]) : q[0] + q[1];
        const float mean = (float)__ddiv_rn(s, (double)H);
        ns.inv[tid] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    }
    __syncthreads();
    if (ns.bad) {
        if (status && tid == 0) latch(status, K3X_ERR_INVALID_MXFP4);
        return false;
    }
    // xn = bf16(x * inv * gamma) in place: thread per 8-element column chunk,
    // its gamma read once for all tokens, all tokens' chunks read before any
    // is written.
    float inv[kMaxDecodeTokens];
#pragma unroll
    for (uint32_t t2 = 0; t2 < (uint32_t)kMaxDecodeTokens; ++t2) inv[t2] = t2 < T ? ns.inv[t2] : 0.f;
    const uint32_t rc = H / 8;  // chunks per row
    for (uint32_t k8 = tid; k8 < rc; k8 += kThreads) {
        const float4 g0 = *reinterpret_cast<const float4*>(s_g + 8 * k8);
        const float4 g1 = *reinterpret_cast<const float4*>(s_g + 8 * k8 + 4);
        const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        uint4 w[kMaxDecodeTokens];
#pragma unroll
        for (uint32_t t2 = 0; t2 < (uint32_t)kMaxDecodeTokens; ++t2)
            if (t2 < T) w[t2] = s_x4[t2 * rc + k8];
#pragma unroll
        for (uint32_t t2 = 0; t2 < (uint32_t)kMaxDecodeTokens; ++t2) {
            if (t2 >= T) break;
            const uint32_t in[4] = {w[t2].x, w[t2].y, w[t2].z, w[t2].w};
            uint32_t o[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                o[q] = pack_bf16x2(__fmul_rn(__fmul_rn(lo_bf16(in[q]), inv[t2]), g[2 * q]),
                                   __fmul_rn(__fmul_rn(hi_bf16(in[q]), inv[t2]), g[2 * q + 1]));
            const uint4 ov = make_uint4(o[0], o[1], o[2], o[3]);
            s_x4[t2 * rc + k8] = ov;
            if (xn_out) reinterpret_cast<uint4*>(xn_out)[t2 * rc + k8] = ov;
        }
    }
    __syncthreads();
    return true;
}

// Dynamic LDS of a block that runs build_xn: x [T][H] bf16 + gamma [H] fp32.
inline size_t xn_lds_bytes(uint32_t T, uint32_t H) { return (size_t)T * H * 2 + (size_t)H * 4; }

// ---------------------------------------------------------------------------
// Front kernel: xn, router logits (router blocks) and the shared expert's
// gate/up + GLU (shared blocks)
// ---------------------------------------------------------------------------
struct FrontArgs {
    const uint16_t* x;
    const float* gamma;
    const float* router_w;  // [E][H] fp32
    uint32_t T, H, E, S;
    float eps;
    uint32_t router_blocks;
    const uint4* sh_gu;     // shared gate/up tiles [S/16][H/128][2][4][64] x 16 B
    GluParams glu;
    uint16_t* xn;           // [T][H] global copy (block 0 writes it)
    float* logits;          // [T][E]
    uint16_t* sact;         // [T][S] bf16 shared activation
    uint32_t* status;
};

constexpr int kRouterBatch = 14;  // float4 row loads per lane per buffer (two buffers)
constexpr int kRouterRows = 4;    // router rows per router block (all 8 waves build xn)
constexpr int kSharedGuDepth = 2; // shared gate/up tiles in flight per wave

struct FrontLds {
    NormShared ns;
    f32x4 red[kFrontWaves][2][64];  // shared blocks: K-split partials
};

// Router block: kRouterRows expert rows; wave w takes row w % kRouterRows
// for the tokens t = w / kRouterRows, w / kRouterRows + 2, ... (so with two
// or more tokens all eight waves form dot products, each over half the
// tokens; both waves of a row fetch it), and all eight build xn.  A row
// wave's two batches of row loads are issued right after the xn prologue's
// loads, so the row fetch overlaps the prologue; each partial 4l + c still
// accumulates j = 0, 1, ... in order (the canonical order).  TT bounds the
// token count (register arrays sized by it).
template <int TT>
__device__ __forceinline__ void router_block(const FrontArgs& a, uint32_t blk, uint4* dyn_lds,
                                             NormShared& ns) {
    constexpr uint32_t kPhases = kFrontWaves / kRouterRows;  // waves per row
    constexpr int NT = (TT + kPhases - 1) / kPhases;         // tokens per wave
    const uint32_t lane = threadIdx.x & 63, wave = wave_id();
    const uint32_t T = a.T, H = a.H, J = H / 256;
    const uint32_t ph = wave / kRouterRows, e = blk * kRouterRows + wave % kRouterRows;
    const bool dots = ph < T;  // wave-uniform: this wave has tokens
    const bool row = dots && e < a.E;
    // Loads are unconditional (a row past E reads row 0, a batch index past
    // the row end reads its last chunk; neither is used), so that they are
    // all in flight together.
    const float* wr = a.router_w + (size_t)(row ? e : 0) * H + 4 * lane;
    float4 wb[2][kRouterBatch];
    auto prefetch = [&]() {
        if (dots)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int u = 0; u < kRouterBatch; ++u) {
                    const uint32_t j = min((uint32_t)(b * kRouterBatch + u), J - 1);
                    wb[b][u] = *reinterpret_cast<const float4*>(wr + 256 * j);
                }
    };
    if (!build_xn<kFrontThreads>(a.x, a.gamma, T, H, a.eps, dyn_lds, ns,
                                 blk == 0 ? a.xn : nullptr, a.status, a.status, prefetch, [] {}))
        return;
    if (!row) return;
    const uint16_t* s_x = reinterpret_cast<const uint16_t*>(dyn_lds);
    double p[NT][4];
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) p[i][c] = 0.0;
    for (uint32_t j0 = 0; j0 < J; j0 += 2 * kRouterBatch) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int u = 0; u < kRouterBatch; ++u) {
                const uint32_t j = j0 + b * kRouterBatch + u;
                if (j >= J) continue;
                const double wv[4] = {(double)wb[b][u].x, (double)wb[b][u].y, (double)wb[b][u].z,
                                      (double)wb[b][u].w};
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    const uint32_t t = ph + kPhases * i;
                    if (t >= T) continue;
                    const uint2 xv =
                        *reinterpret_cast<const uint2*>(s_x + (size_t)t * H + 256 * j + 4 * lane);
                    const float f[4] = {lo_bf16(xv.x), hi_bf16(xv.x), lo_bf16(xv.y),
                                        hi_bf16(xv.y)};
#pragma unroll
                    for (int c = 0; c < 4; ++c) p[i][c] = __builtin_fma(wv[c], (double)f[c], p[i][c]);
                }
            }
            // Refill this buffer with the batch two ahead (clamped).
            if (j0 + (b + 2) * kRouterBatch < J)
#pragma unroll
                for (int u = 0; u < kRouterBatch; ++u) {
                    const uint32_t j = min(j0 + (b + 2) * kRouterBatch + u, J - 1);
                    wb[b][u] = *reinterpret_cast<const float4*>(wr + 256 * j);
                }
        }
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const uint32_t t = ph + kPhases * i;
        if (t >= T) continue;
        const double v = canon_reduce(p[i]);
        if (lane == 0) a.logits[(size_t)t * a.E + e] = (float)v;
    }
}

// Shared gate/up block: one 16-row block rb of S and the whole K = H range,
// split over the eight waves (kSharedGuDepth tiles of registers in flight
// per wave, the first ones requested during the xn prologue, refills
// clamped to the last tile); the wave partials are added in a fixed tree in LDS (wave w += wave
// w + h for h = 4, 2, 1) and the block writes sact = bf16(GLU(gate, up)) for
// its 16 columns.
__device__ __forceinline__ void shared_gateup_block(const FrontArgs& a, uint32_t rb,
                                                    uint4* dyn_lds, FrontLds& sh) {
    const uint32_t lane = threadIdx.x & 63, wave = wave_id();
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t T = a.T, H = a.H, kt = H / 128;
    const uint32_t k0 = wave * kt / kFrontWaves, k1 = (wave + 1) * kt / kFrontWaves;
    const uint32_t N = k1 - k0;
    const uint4* tiles = a.sh_gu + (size_t)rb * kt * 2 * 4 * 64 + lane;
    constexpr int PD = kSharedGuDepth;
    uint4 bn[PD][2][4];
    auto load = [&](uint4 (&b)[2][4], uint32_t k) {
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int j = 0; j < 4; ++j) b[w][j] = tiles[(((size_t)k * 2 + w) * 4 + j) * 64];
    };
    // The weights are requested once this block's x / gamma have arrived
    // (and so, nearly, every block's): requested with the x / gamma loads,
    // the 59 MB of shared gate/up tiles would queue ahead of the router
    // blocks' x / gamma and router rows, which are on the layer's critical
    // path.  A non-finite x is reported by the router blocks.
    auto prefetch = [&]() {
#pragma unroll
        for (int d = 0; d < PD; ++d) load(bn[d], min(k0 + d, kt - 1));
    };
    if (!build_xn<kFrontThreads>(a.x, a.gamma, T, H, a.eps, dyn_lds, sh.ns, nullptr, nullptr,
                                 a.status, [] {}, prefetch))
        return;
    const uint16_t* s_x = reinterpret_cast<const uint16_t*>(dyn_lds);
    const uint16_t* xrow = s_x + (size_t)(n < T ? n : 0) * H + 32 * g;  // unused rows: row 0
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    auto step = [&](const uint4 (&b)[2][4], uint32_t k) {
        bf16x8 af[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            af[j] = as_bf16x8(*reinterpret_cast<const uint4*>(xrow + k * 128 + 8 * j));
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int w = 0; w < 2; ++w) acc[w] = mfma16x16x32(af[j], as_bf16x8(b[w][j]), acc[w]);
    };
    if (N) {
        uint32_t kb = 0;
        for (; kb + PD <= N; kb += PD) {
#pragma unroll
            for (int d = 0; d < PD; ++d) {
                step(bn[d], k0 + kb + d);
                load(bn[d], k0 + min(kb + d + PD, N - 1));
            }
        }
#pragma unroll
        for (int d = 0; d < PD; ++d)
            if (kb + d < N) step(bn[d], k0 + kb + d);
    }
    sh.red[wave][0][lane] = acc[0];
    sh.red[wave][1][lane] = acc[1];
#pragma unroll
    for (uint32_t h = kFrontWaves / 2; h >= 1; h /= 2) {
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

// Blocks [0, router_blocks) are router blocks, the rest shared gate/up
// blocks (16-row block rb = block - router_blocks).
template <int TT>
__global__ __launch_bounds__(kFrontThreads) void decode_front_kernel(FrontArgs a) {
    extern __shared__ uint4 dyn_lds[];
    __shared__ FrontLds sh;
    if (blockIdx.x < a.router_blocks)
        router_block<TT>(a, blockIdx.x, dyn_lds, sh.ns);
    else
        shared_gateup_block(a, blockIdx.x - a.router_blocks, dyn_lds, sh);
}

// ---------------------------------------------------------------------------
// Select kernel: Top-K + expert-major grouping (block 0) and the shared
// expert's down projection (the other blocks)
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
    uint32_t group_taps; // nonzero: also counts, offsets, first_use, active_asc, active_fu
    uint32_t local_only; // nonzero: the results stay in LDS (rec, na, selw), no global store
    uint32_t* status;
};

// The shared expert's down projection: the select launch's other workgroups.
struct SharedDownArgs {
    const uint4* sh_dn;    // shared down tiles [H/16][S/128][4][64] x 16 B
    const uint16_t* sact;  // [T][S] bf16 shared activation
    uint32_t T, H, S;
    float* sy;             // [T][H] shared expert output, fp32
    const uint32_t* status;
};

// Block 0 of the select kernel: natural Top-K of every token and the
// expert-major grouping, by all eight waves.  Thread e owns expert e of every
// token (E <= kSelExperts).
//   keys       sigmoid + bias, the validation and the sort key of topk_wave
//              (score order, then the lower expert index);
//   threshold  the maximum score half of each 16-expert group (DPP row
//              rotates); with G groups and K <= G, the K-th largest group
//              maximum tau has at least K keys at or above it (one per group
//              at or above tau), so no key with score half below tau can be
//              selected;
//   survivors  the keys at or above tau (every key when K > G) are compacted
//              per token and ranked exactly among themselves by the full
//              64-bit key (keys are distinct: the low half holds the
//              expert); rank r < K is router slot r;
//   renorm     one wave per token, sequential sums in slot order, as
//              topk_wave;
//   grouping   per pair p = token * K + slot, counts of equal and smaller
//              expert ids among the P = T * K pairs give the CSR row, the
//              active index and the first-use rank directly
//              (runtime/src/expert_major.cpp:10-54), with no atomics.
constexpr uint32_t kSelExperts = kKeysPerLane * 64;  // experts per token: E <= 512
constexpr uint32_t kSelGroups = kSelExperts / 16;    // 16-expert groups
constexpr uint32_t kSelMaxPairs = kMaxDecodeTokens * 64;
constexpr uint32_t kRankThreads = kFrontThreads / kMaxDecodeTokens;  // per token
static_assert(kSelGroups <= 32, "one lane per group in half a wave");
static_assert(kFrontWaves >= 2 * kMaxDecodeTokens, "renormalisation waves apart from the pairs'");

struct SelectShared {
    uint64_t ckey[kMaxDecodeTokens][kSelExperts];  // survivors' keys, compacted, 0 past them
    uint32_t cid[kMaxDecodeTokens][kSelExperts];   // survivors' experts
    float csc[kMaxDecodeTokens][kSelExperts];      // survivors' sigmoid scores
    uint32_t gmax[kMaxDecodeTokens][kSelGroups];   // group maxima of the score half
    uint32_t thr[kMaxDecodeTokens];                // survivor threshold tau
    uint32_t ncand[kMaxDecodeTokens];
    uint32_t sel[kSelMaxPairs];      // expert of pair t * K + s
    float selsc[kSelMaxPairs];       // its sigmoid score
    float selw[kSelMaxPairs];        // its contribution
    uint32_t first[kSelMaxPairs];    // 1: the pair is its expert's first use
    uint32_t rowtok[kSelMaxPairs];   // token of CSR row r
    uint4 rec[kSelMaxPairs];         // active slot records {expert, rows, offset, row tokens}
    uint32_t na;                     // active slots
    uint32_t bad;
};

// Top-K of the T tokens into sh.sel / sh.selsc (router order); false (error
// latched) when a score fails its check.  lg[t]: logit of expert tid for
// token t; b: bias of expert tid.
__device__ bool select_topk(const SelectArgs& a, SelectShared& sh,
                            const float (&lg)[kMaxDecodeTokens], float b) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t T = a.T, K = a.K, e = tid;
    const bool dbl = a.renorm == K3X_RENORM_DOUBLE;
    const bool valid = e < a.E;
    constexpr uint32_t kErrExtent = K3X_ERR_INVALID_EXTENT, kErrState = K3X_ERR_INVALID_STATE;
    if (tid < kMaxDecodeTokens) sh.ncand[tid] = 0;
    if (tid == 0) sh.bad = 0;
    // Candidate keys past the survivors stay 0, below every real key, and
    // pairs past T * K hold expert 0xffffffff, above every real one (the
    // loops read whole batches of eight).
#pragma unroll
    for (int t = 0; t < kMaxDecodeTokens; ++t) sh.ckey[t][tid] = 0;
    if (tid < kSelMaxPairs) {
        sh.sel[tid] = 0xffffffffu;
        sh.first[tid] = 0;
    }
    // Keys and validation (runtime/src/routing_policy.cpp:40-95,
    // runtime/src/official_moe.cpp:214-232), as topk_wave; experts past E
    // hold key 0, below every real key.  Group maxima over rows of 16 lanes
    // (all lanes active for the DPP moves).
    uint64_t key[kMaxDecodeTokens];
    float sc[kMaxDecodeTokens];
    uint32_t err = 0;
#pragma unroll
    for (int t = 0; t < kMaxDecodeTokens; ++t) {
        key[t] = 0;
        sc[t] = 0.0f;
        if ((uint32_t)t >= T) continue;
        if (valid) {
            if (dbl && (!__builtin_isfinite(lg[t]) || !__builtin_isfinite(b))) err = kErrExtent;
            const float s = sigmoid_cr(lg[t]);
            const float adj = __fadd_rn(s, b);
            if (!dbl && (!__builtin_isfinite(s) || s < 0.0f || s > 1.0f || !__builtin_isfinite(b) ||
                         !__builtin_isfinite(adj)))
                err = kErrState;
            sc[t] = s;
            key[t] = topk_key(adj, e);
        }
        uint32_t m = (uint32_t)(key[t] >> 32);
        m = dpp_max_step<0x128, 0xf>(m);  // row_ror:8
        m = dpp_max_step<0x124, 0xf>(m);  // row_ror:4
        m = dpp_max_step<0x122, 0xf>(m);  // row_ror:2
        m = dpp_max_step<0x121, 0xf>(m);  // row_ror:1
        if ((lane & 15) == 0) sh.gmax[t][tid >> 4] = m;
    }
    __syncthreads();
    if (err) atomicMax(&sh.bad, err);
    // tau of token t by wave t: the group maximum m with fewer than K larger
    // maxima and at least K at or above it (lanes 32..63 repeat 0..31).
    const uint32_t G = (a.E + 15) / 16;
    if (wave < T) {
        const uint32_t t = wave, g = lane & 31;
        uint32_t th = 0;
        if (K <= G) {
            const uint32_t m = sh.gmax[t][g];
            uint32_t gt = 0, ge = 0;
            const uint4* gm = reinterpret_cast<const uint4*>(sh.gmax[t]);
            for (uint32_t g4 = 0; g4 < (G + 3) / 4; ++g4) {  // groups past G hold 0
                const uint4 v = gm[g4];
                gt += (v.x > m) + (v.y > m) + (v.z > m) + (v.w > m);
                ge += (v.x >= m) + (v.y >= m) + (v.z >= m) + (v.w >= m);
            }
            const uint64_t q = __ballot(g < G && gt < K && K <= ge);
            if (q) th = (uint32_t)__builtin_amdgcn_readlane((int)m, (int)__builtin_ctzll(q));
        }
        if (lane == 0) sh.thr[t] = th;
    }
    __syncthreads();
    if (sh.bad) {
        if (tid == 0) latch(a.status, sh.bad);
        return false;
    }
    // Compact the survivors (their order in the list does not matter: the
    // ranking is exact).
#pragma unroll
    for (int t = 0; t < kMaxDecodeTokens; ++t) {
        if ((uint32_t)t >= T) continue;
        const bool surv = valid && (uint32_t)(key[t] >> 32) >= sh.thr[t];
        const uint64_t m = __ballot(surv);
        if (!m) continue;
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&sh.ncand[t], (uint32_t)__popcll(m));
        base = __builtin_amdgcn_readfirstlane(base);
        if (surv) {
            const uint32_t c = base + (uint32_t)__popcll(m & ((1ull << lane) - 1));
            sh.ckey[t][c] = key[t];
            sh.cid[t][c] = e;
            sh.csc[t][c] = sc[t];
        }
    }
    __syncthreads();
    // Exact rank among the survivors, kRankThreads threads per token; rank
    // r < K is slot r.
    const uint32_t rt = tid / kRankThreads;
    if (rt < T) {
        const uint32_t n = sh.ncand[rt];
        const ulonglong2* ck = reinterpret_cast<const ulonglong2*>(&sh.ckey[rt][0]);
        for (uint32_t c = tid % kRankThreads; c < n; c += kRankThreads) {
            const uint64_t k = sh.ckey[rt][c];
            uint32_t r = 0;
            for (uint32_t c2 = 0; c2 < n; c2 += 8) {  // zero-padded past n
                ulonglong2 kk[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) kk[q] = ck[c2 / 2 + q];
#pragma unroll
                for (int q = 0; q < 4; ++q) r += (kk[q].x > k) + (kk[q].y > k);
            }
            if (r < K) {
                sh.sel[rt * K + r] = sh.cid[rt][c];
                sh.selsc[rt * K + r] = sh.csc[rt][c];
            }
        }
    }
    __syncthreads();
    return true;
}

// Renormalisation of the Top-K and the expert-major grouping of the P = T *
// K selected pairs (pair p = token * K + slot): ascending-expert CSR with the
// rows of one expert in pair order and the active-slot records of the
// decode kernels; with group_taps also the per-expert counts, offsets and
// first-use keys and both orders of the active experts
// (runtime/src/expert_major.cpp:10-54).  Every quantity is a count over the
// P pairs.
__device__ void select_group(const SelectArgs& a, SelectShared& sh) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t K = a.K, P = a.T * K, E = a.E;
    const bool dbl = a.renorm == K3X_RENORM_DOUBLE;
    // Pairs are read eight at a time (two 16-byte LDS reads per wait); the
    // padding past P matches no expert and is below no expert.
    const uint4* sel4 = reinterpret_cast<const uint4*>(sh.sel);
    const uint4* first4 = reinterpret_cast<const uint4*>(sh.first);
#define SEL_BATCH(q0, body)                                                                     \
    {                                                                                           \
        const uint4 u0_ = sel4[(q0) / 4], u1_ = sel4[(q0) / 4 + 1];                             \
        const uint32_t fv_[8] = {u0_.x, u0_.y, u0_.z, u0_.w, u1_.x, u1_.y, u1_.z, u1_.w};      \
        _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_) {                                      \
            const uint32_t q = (q0) + i_, f = fv_[i_];                                          \
            body                                                                                \
        }                                                                                       \
    }
    uint32_t e = 0, rin = 0, below = 0, cnt = 0;
    if (tid < P) {
        e = sh.sel[tid];
        for (uint32_t q0 = 0; q0 < P; q0 += 8)
            SEL_BATCH(q0, rin += q < tid && f == e; cnt += f == e; below += f < e;)
        sh.first[tid] = rin == 0;
        sh.rowtok[below + rin] = tid / K;
    }
    // Renormalise in slot order (sequential sums as the reference), then
    // * routed_scale (runtime/src/routing_policy.cpp:146-157,
    // runtime/src/official_moe.cpp:235-242, runtime/src/model.cpp:1004-1009),
    // on waves kMaxDecodeTokens.. (the pairs' own waves are 0..).
    if (wave >= kMaxDecodeTokens && wave - kMaxDecodeTokens < a.T) {
        const uint32_t t = wave - kMaxDecodeTokens;
        const float v = lane < K ? sh.selsc[t * K + lane] : 0.0f;
        float den_f = 0.0f;
        double den_d = 0.0;
        for (uint32_t s = 0; s < K; ++s) {
            const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), s));
            den_f = __fadd_rn(den_f, x);
            den_d = __dadd_rn(den_d, (double)x);
        }
        const bool ok = dbl ? (__builtin_isfinite(den_d) && den_d > 0.0)
                            : (__builtin_isfinite(den_f) && den_f > 0.0f);
        if (!ok) {
            if (lane == 0) {
                latch(a.status, dbl ? K3X_ERR_INVALID_EXTENT : K3X_ERR_INVALID_STATE);
                atomicMax(&sh.bad, 1u);
            }
        } else if (lane < K) {
            sh.selw[t * K + lane] = dbl ? __fmul_rn((float)__ddiv_rn((double)v, den_d),
                                                    a.routed_scale)
                                        : __fmul_rn(__fdiv_rn(v, den_f), a.routed_scale);
        }
    }
    // The last barrier: every global store of the block comes after it, so
    // no barrier waits for stores to drain.
    __syncthreads();
    if (sh.bad) return;
    if (tid < P && !a.local_only) {
        const uint32_t r = below + rin;  // CSR row
        a.pair_token[r] = tid / K;
        a.pair_slot[r] = tid % K;
        a.ids[tid] = e;
        a.weights[tid] = sh.selw[tid];
    }
    if (tid < P && sh.first[tid]) {
        uint32_t ai = 0, fr = 0, na = 0;
        for (uint32_t q0 = 0; q0 < P; q0 += 8) {
            const uint4 g0 = first4[q0 / 4], g1 = first4[q0 / 4 + 1];
            const uint32_t fq_[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            SEL_BATCH(q0, const bool fq = fq_[i_] != 0;
                      ai += fq && f < e;    /* active experts below e: ascending index */
                      fr += fq && q < tid;  /* first uses before e's: first-use rank */
                      na += fq;)
        }
        uint32_t toks = 0;  // tokens of e's first four rows, 8 bits each
        for (uint32_t j = 0; j < min(cnt, 4u); ++j) toks |= sh.rowtok[below + j] << (8 * j);
        sh.rec[ai] = make_uint4(e, cnt, below, toks);
        if (ai == 0) sh.na = na;
        if (a.local_only) return;
        a.arec[ai] = make_uint4(e, cnt, below, toks);
        if (ai == 0) *a.n_active = na;
        if (a.group_taps) {
            a.active_asc[ai] = e;
            a.active_fu[fr] = e;
        }
    }
    if (!a.group_taps || a.local_only) return;
    // Per expert: count, CSR offset, first use (0xffffffff when unused).
    for (uint32_t x = tid; x < E; x += kFrontThreads) {
        uint32_t c = 0, o = 0, fu = 0xffffffffu;
        for (uint32_t q0 = 0; q0 < P; q0 += 8)
            SEL_BATCH(q0, c += f == x; o += f < x; if (f == x && fu == 0xffffffffu) fu = q;)
        a.counts[x] = c;
        a.offsets[x] = o;
        a.first_use[x] = fu;
    }
    if (tid == 0) a.offsets[E] = P;
#undef SEL_BATCH
}

// Shared down block: one 16-row block rb of H, K = S split over the eight
// waves (up to two tiles in flight per wave, refills clamped to the last
// tile), partials added in a fixed tree in LDS (wave w += wave w + h for
// h = 4, 2, 1).
__device__ __forceinline__ void shared_down_block(const SharedDownArgs& a, uint32_t rb,
                                                  f32x4 (&red)[kFrontWaves][64]) {
    const uint32_t lane = threadIdx.x & 63, wave = wave_id();
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t skt = a.S / 128;
    const uint32_t k0 = wave * skt / kFrontWaves, k1 = (wave + 1) * skt / kFrontWaves;
    const uint32_t N = k1 - k0;
    const uint4* tiles = a.sh_dn + (size_t)rb * skt * 4 * 64 + lane;
    const bool arow = n < a.T;
    const uint16_t* ap = a.sact + (size_t)(arow ? n : 0) * a.S + 32 * g;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int PD = 2;
    struct Step {
        uint4 b[4], av[4];
    };
    auto load = [&](Step& r, uint32_t k) {
        load_act(ap, arow, k, r.av);
#pragma unroll
        for (int j = 0; j < 4; ++j) r.b[j] = tiles[((size_t)k * 4 + j) * 64];
    };
    auto step = [&](const Step& r) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = mfma16x16x32(as_bf16x8(r.av[j]), as_bf16x8(r.b[j]), acc);
    };
    Step r[PD];
#pragma unroll
    for (int d = 0; d < PD; ++d) {
        r[d].av[0] = r[d].av[1] = r[d].av[2] = r[d].av[3] = make_uint4(0, 0, 0, 0);
        load(r[d], min(k0 + d, skt - 1));
    }
    if (prior_status(a.status)) return;  // the same value for the whole block
    uint32_t kb = 0;
    for (; kb + PD <= N; kb += PD) {
#pragma unroll
        for (int d = 0; d < PD; ++d) {
            step(r[d]);
            load(r[d], min(k0 + kb + d + PD, skt - 1));
        }
    }
#pragma unroll
    for (int d = 0; d < PD; ++d)
        if (kb + d < N) step(r[d]);
    red[wave][lane] = acc;
#pragma unroll
    for (uint32_t h = kFrontWaves / 2; h >= 1; h /= 2) {
        __syncthreads();
        if (wave < h) red[wave][lane] = red[wave][lane] + red[wave + h][lane];
    }
    if (wave != 0) return;
    const f32x4 tot = red[0][lane];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t t = 4 * g + q;
        if (t < a.T) a.sy[(size_t)t * a.H + rb * 16 + n] = tot[q];
    }
}

union SelectLds {
    SelectShared sel;
    f32x4 red[kFrontWaves][64];
};

// Block 0: the Top-K of every token and the grouping; blocks 1.. the shared
// expert's down projection, which streams while block 0 works.
__global__ __launch_bounds__(kFrontThreads) void decode_select_kernel(SelectArgs a,
                                                                     SharedDownArgs sd) {
    __shared__ SelectLds lds;
    if (blockIdx.x) {
        shared_down_block(sd, blockIdx.x - 1, lds.red);
        return;
    }
    SelectShared& sh = lds.sel;
    // Logits of expert tid for every token and its bias, loaded
    // unconditionally (indices clamped) before the status check.
    const uint32_t e = min(threadIdx.x, a.E - 1);
    float lg[kMaxDecodeTokens];
#pragma unroll
    for (int t = 0; t < kMaxDecodeTokens; ++t)
        lg[t] = a.logits[(size_t)min((uint32_t)t, a.T - 1) * a.E + e];
    const float b = a.bias[e];
    if (prior_status(a.status)) return;
    if (select_topk(a, sh, lg, b)) select_group(a, sh);
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
    const uint32_t* pair_token;  // ROWS kernels: token of each CSR row
    uint16_t* act;             // [pairs][act_stride] bf16, CSR row order
    uint32_t act_stride;       // elements per act row
    uint32_t act_lo;           // element offset of the lo halves (split activations), 0: none
    GluParams glu;
    const uint32_t* status;
};

// Workgroup = one unit (active slot ai = block / (I / 16), 16-row block rb =
// block % (I / 16)) with the K range split over kGuWaves waves of at most
// kGuTiles tiles each.  The xn rows of the slot's tokens are copied into LDS
// by the whole block; their loads are issued first, then each wave's gate
// and up code tiles and scale dwords, all in flight together (unconditional
// loads, clamped indices), so a unit costs about one memory round trip.
// Wave partials are added in a fixed tree in LDS (wave w += wave w + h for
// h = 4, 2, 1) before the GLU.
constexpr int kGuWaves = 8;
constexpr int kGuTiles = 8;       // K tiles per wave: H <= 128 * 8 * 8
constexpr int kGuActLoads = 7;    // 16-byte xn loads per thread: T * H / 8 <= 7 * 512
// Rows of a slot in LDS at once (ROWS kernels: chunks of this many rows).
constexpr uint32_t kRowChunk = kMaxDecodeTokens;

// v[i] = src[min(tid + step i, chunks - 1)], and the matching store into
// LDS (chunks of rows staged by a workgroup; clamped indices keep every load
// unconditional).  Native vectors: the compiler keeps them in registers
// across the row-chunk loop, where copies of uint4 went to the stack.
template <int N>
__device__ __forceinline__ void load_chunks(u32x4 (&v)[N], const void* src, uint32_t tid,
                                            uint32_t step, uint32_t chunks) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] = reinterpret_cast<const u32x4*>(src)[min(tid + step * i, chunks - 1)];
}
template <int N>
__device__ __forceinline__ void store_chunks(const u32x4 (&v)[N], void* dst, uint32_t tid,
                                             uint32_t step, uint32_t chunks) {
#pragma unroll
    for (int i = 0; i < N; ++i) reinterpret_cast<u32x4*>(dst)[min(tid + step * i, chunks - 1)] = v[i];
}

// RB > 1: the workgroup takes RB consecutive 16-row blocks, each over
// kGuWaves / RB waves (the xn rows in LDS serve them all; for short K ranges,
// where a one-block unit's fixed cost would dominate).
// ROWS: a slot of any number of rows (the general path's verification
// windows): its rows pass through LDS kRowChunk at a time, tokens read from
// pair_token, while the wave's code tiles and scales stay in registers, so
// the weights stream once per slot.
template <int RB, bool ROWS = false>
__global__ __launch_bounds__(64 * kGuWaves) void decode_gateup_kernel(GateUpArgs a) {
    extern __shared__ uint4 s_x4[];  // [rows][H] bf16
    __shared__ f32x4 red[kGuWaves][2][64];
    constexpr uint32_t kWpr = kGuWaves / RB;  // waves per row block
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t per_expert = a.I / (16 * RB);
    const uint32_t ai = blockIdx.x / per_expert;
    const uint32_t rb = (blockIdx.x % per_expert) * RB + wave / kWpr, wv = wave % kWpr;
    // Status, active count and this slot's record in one round trip (the
    // record of an inactive slot is not used).
    const uint32_t st = prior_status(a.status);
    const uint32_t na = *a.n_active;
    const uint4 rec = a.arec[ai];  // ai < min(E, T*K): in bounds
    if (st || ai >= na) return;
    const uint32_t e = rec.x, cnt = rec.y, toks = rec.w;
    const uint32_t H = a.H, kt = a.kt;
    // 1. xn rows [m0, m0 + rows) of the slot (rows <= kRowChunk): chunk c of
    //    row r.
    const uint32_t rowc = H / 8;
    u32x4 v[kGuActLoads];
    auto load_rows = [&](uint32_t m0, uint32_t rows) __attribute__((always_inline)) {
        // Tokens of the rows, 8 bits each (ROWS: T <= kChunkedMaxTokens).
        uint32_t tk = toks;
        if constexpr (ROWS) {
            tk = 0;
#pragma unroll
            for (uint32_t r = 0; r < kRowChunk; ++r)
                tk |= a.pair_token[rec.z + m0 + min(r, rows - 1)] << (8 * r);
        }
        const uint32_t chunks = rows * rowc;
#pragma unroll
        for (int i = 0; i < kGuActLoads; ++i) {
            const uint32_t c = min(tid + 64 * kGuWaves * i, chunks - 1);
            const uint32_t r = (c >= rowc) + (c >= 2 * rowc) + (c >= 3 * rowc);
            const uint32_t tok = (tk >> (8 * r)) & 0xffu;
            v[i] = reinterpret_cast<const u32x4*>(a.xn + (size_t)tok * H)[c - r * rowc];
        }
    };
    uint32_t rows = ROWS ? min(cnt, kRowChunk) : cnt;
    load_rows(0, rows);
    // 2. This wave's K tiles [k0, k1) of the gate and up blocks, and the
    //    scale dwords of the (at most three) groups they touch.
    const uint32_t k0 = wv * kt / kWpr, k1 = (wv + 1) * kt / kWpr;
    const uint32_t N = k1 - k0;
    const uint4* codes = a.gu_codes + e * a.codes_per_expert + (size_t)rb * kt * 2 * 64 + lane;
    const uint32_t* scales = a.gu_scales + e * a.scales_per_expert + (size_t)rb * a.ks * 2 * 64 + lane;
    uint4 c0[kGuTiles], c1[kGuTiles];
    uint32_t s0[3], s1[3];
#pragma unroll
    for (int i = 0; i < kGuTiles; ++i) {
        const size_t k = min(k0 + i, kt - 1);  // tiles past k1 are loaded, not used
        c0[i] = ntl(codes + k * 128);
        c1[i] = ntl(codes + k * 128 + 64);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const size_t grp = min(k0 / 4 + i, a.ks - 1);
        s0[i] = ntl(scales + grp * 128);
        s1[i] = ntl(scales + grp * 128 + 64);
    }
    store_chunks(v, s_x4, tid, 64 * kGuWaves, rows * rowc);
    __syncthreads();
    const uint16_t* s_x = reinterpret_cast<const uint16_t*>(s_x4);
    for (uint32_t m0 = 0;;) {
        if constexpr (ROWS) {
            // The code tiles and scale dwords, as opaque values each pass:
            // their dequantised forms are not kept across passes (the
            // register file would not hold them).
#pragma unroll
            for (int i = 0; i < kGuTiles; ++i)
                asm volatile("" : "+v"(c0[i].x), "+v"(c0[i].y), "+v"(c0[i].z), "+v"(c0[i].w),
                                  "+v"(c1[i].x), "+v"(c1[i].y), "+v"(c1[i].z), "+v"(c1[i].w));
            asm volatile("" : "+v"(s0[0]), "+v"(s0[1]), "+v"(s0[2]), "+v"(s1[0]), "+v"(s1[1]),
                              "+v"(s1[2]));
        }
        const uint16_t* xrow = s_x + (size_t)(n < rows ? n : 0) * H + 32 * g;  // unused rows: row 0
        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int i = 0; i < kGuTiles; ++i) {
            if ((uint32_t)i < N) {
                const uint32_t k = k0 + i, gi = (k >> 2) - (k0 >> 2), sh = 8 * (k & 3);
                const uint32_t w0 = gi == 0 ? s0[0] : gi == 1 ? s0[1] : s0[2];
                const uint32_t w1 = gi == 0 ? s1[0] : gi == 1 ? s1[1] : s1[2];
                uint4 av[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    av[j] = *reinterpret_cast<const uint4*>(xrow + (size_t)k * 128 + 8 * j);
                acc[0] = mxfp4_tile(c0[i], e8m0_to_f32((w0 >> sh) & 0xffu), av, acc[0]);
                acc[1] = mxfp4_tile(c1[i], e8m0_to_f32((w1 >> sh) & 0xffu), av, acc[1]);
            }
        }
        red[wave][0][lane] = acc[0];
        red[wave][1][lane] = acc[1];
#pragma unroll
        for (uint32_t h = kWpr / 2; h >= 1; h /= 2) {
            __syncthreads();
            if (wv < h) {
                red[wave][0][lane] = red[wave][0][lane] + red[wave + h][0][lane];
                red[wave][1][lane] = red[wave][1][lane] + red[wave + h][1][lane];
            }
        }
        if (!ROWS && wv != 0) return;
        if (wv == 0) {
            const f32x4 gs = red[wave][0][lane], us = red[wave][1][lane];
            auto out = [&](int i) __attribute__((always_inline)) {
                const uint32_t row = 4 * g + i;
                if (row < rows) {
                    const float v = glu(gs[i], us[i], a.glu);
                    uint16_t* dst =
                        a.act + (size_t)(rec.z + m0 + row) * a.act_stride + rb * 16 + n;
                    const uint16_t hi = f32_to_bf16(v);
                    *dst = hi;
                    if (a.act_lo) dst[a.act_lo] = act_lo_bf16(v, hi);
                }
            };
            if constexpr (ROWS) {
                // One row at a time: the held weight registers leave no room
                // for four GLUs in flight.
#pragma unroll 1
                for (int i = 0; i < 4; ++i) out(i);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) out(i);
            }
        }
        if (!ROWS) return;
        m0 += rows;
        if (m0 >= cnt) return;  // block-uniform
        // The next rows, once every wave is past its reads of s_x and red.
        rows = min(cnt - m0, kRowChunk);
        load_rows(m0, rows);
        __syncthreads();
        store_chunks(v, s_x4, tid, 64 * kGuWaves, rows * rowc);
        __syncthreads();
    }
}

// One gate/up unit of the two-launch decode form (RB = 1): the whole block
// on 16-row block rb of active slot ai = blk / (I / 16), its K range split
// over the waves, every token's xn row already in LDS (s_x as [T][H]; row
// n of the slot is token (rec.w >> 8 n) & 0xff), the slot records in LDS.
// The loads, the MFMA steps, the wave tree and the GLU are those of
// decode_gateup_kernel<1>.
// A wave's code tiles and scale dwords of one gate/up unit (expert e, 16-row
// block rb): every load issued at once, none waited for here.
struct GuUnitRegs {
    uint4 c0[kGuTiles], c1[kGuTiles];
    uint32_t s0[3], s1[3];
};

__device__ __forceinline__ void gateup_unit_load(const GateUpArgs& a, uint32_t e, uint32_t rb,
                                                 GuUnitRegs& w) {
    const uint32_t lane = threadIdx.x & 63, wv = wave_id();
    const uint32_t kt = a.kt, k0 = wv * kt / kGuWaves;
    const uint4* codes = a.gu_codes + e * a.codes_per_expert + (size_t)rb * kt * 2 * 64 + lane;
    const uint32_t* scales = a.gu_scales + e * a.scales_per_expert + (size_t)rb * a.ks * 2 * 64 + lane;
#pragma unroll
    for (int i = 0; i < kGuTiles; ++i) {
        const size_t k = min(k0 + i, kt - 1);  // tiles past the wave's range are loaded, not used
        w.c0[i] = ntl(codes + k * 128);
        w.c1[i] = ntl(codes + k * 128 + 64);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const size_t grp = min(k0 / 4 + i, a.ks - 1);
        w.s0[i] = ntl(scales + grp * 128);
        w.s1[i] = ntl(scales + grp * 128 + 64);
    }
}

// The unit's products over the LDS xn rows of the slot record rec, the wave
// tree, GLU and the bf16 activation stores.
__device__ __forceinline__ void gateup_unit_compute(const GateUpArgs& a, uint32_t rb, uint4 rec,
                                                    const uint16_t* s_x, const GuUnitRegs& w,
                                                    f32x4 (&red)[kGuWaves][2][64]) {
    const uint32_t lane = threadIdx.x & 63, wave = wave_id();
    const uint32_t g = lane >> 4, n = lane & 15, wv = wave;
    const uint32_t rows = rec.y, toks = rec.w;
    const uint32_t H = a.H, kt = a.kt;
    const uint32_t k0 = wv * kt / kGuWaves, k1 = (wv + 1) * kt / kGuWaves;
    const uint32_t N = k1 - k0;
    // Plain local copies: a select between struct members would become a
    // load through a selected address and keep the struct in scratch.
    const uint32_t s0[3] = {w.s0[0], w.s0[1], w.s0[2]};
    const uint32_t s1[3] = {w.s1[0], w.s1[1], w.s1[2]};
    uint4 c0[kGuTiles], c1[kGuTiles];
#pragma unroll
    for (int i = 0; i < kGuTiles; ++i) {
        c0[i] = w.c0[i];
        c1[i] = w.c1[i];
    }
    const uint32_t tok = (toks >> (8 * (n < rows ? n : 0))) & 0xffu;  // unused rows: row 0's
    const uint16_t* xrow = s_x + (size_t)tok * H + 32 * g;
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < kGuTiles; ++i) {
        if ((uint32_t)i < N) {
            const uint32_t k = k0 + i, gi = (k >> 2) - (k0 >> 2), sh = 8 * (k & 3);
            const uint32_t w0 = gi == 0 ? s0[0] : gi == 1 ? s0[1] : s0[2];
            const uint32_t w1 = gi == 0 ? s1[0] : gi == 1 ? s1[1] : s1[2];
            uint4 av[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                av[j] = *reinterpret_cast<const uint4*>(xrow + (size_t)k * 128 + 8 * j);
            acc[0] = mxfp4_tile(c0[i], e8m0_to_f32((w0 >> sh) & 0xffu), av, acc[0]);
            acc[1] = mxfp4_tile(c1[i], e8m0_to_f32((w1 >> sh) & 0xffu), av, acc[1]);
        }
    }
    red[wave][0][lane] = acc[0];
    red[wave][1][lane] = acc[1];
#pragma unroll
    for (uint32_t h = kGuWaves / 2; h >= 1; h /= 2) {
        __syncthreads();
        if (wv < h) {
            red[wave][0][lane] = red[wave][0][lane] + red[wave + h][0][lane];
            red[wave][1][lane] = red[wave][1][lane] + red[wave + h][1][lane];
        }
    }
    if (wv != 0) return;
    const f32x4 gs = red[0][0][lane], us = red[0][1][lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = 4 * g + i;
        if (row < rows) {
            const float v = glu(gs[i], us[i], a.glu);
            uint16_t* dst = a.act + (size_t)(rec.z + row) * a.act_stride + rb * 16 + n;
            const uint16_t hi = f32_to_bf16(v);
            *dst = hi;
            if (a.act_lo) dst[a.act_lo] = act_lo_bf16(v, hi);
        }
    }
}

// Unit blk = (active slot, 16-row block) of the slot records lrec[0, lna).
__device__ __forceinline__ void gateup_unit_lds(const GateUpArgs& a, uint32_t blk,
                                                const uint16_t* s_x, const uint4* lrec,
                                                uint32_t lna, f32x4 (&red)[kGuWaves][2][64]) {
    const uint32_t per_expert = a.I / 16;
    const uint32_t ai = blk / per_expert, rb = blk % per_expert;
    if (ai >= lna) return;  // block-uniform
    const uint4 rec = lrec[ai];
    GuUnitRegs w;
    gateup_unit_load(a, rec.x, rb, w);
    gateup_unit_compute(a, rb, rec, s_x, w, red);
}

// ---------------------------------------------------------------------------
// Few experts (E <= kSmallMaxExperts, no shared expert): every workgroup of
// the routed gate/up launch finds the route itself -- xn, the E router rows
// (fp64, canonical order), Top-K and grouping, all in LDS, the same
// functions as the front and select kernels -- so that the route costs no
// launch of its own; block 0 also stores the route (ids, weights, CSR rows,
// active-slot records) for the down launch and xn and the logits for the
// taps.  A few router rows per wave are requested with the xn prologue's
// loads.
// ---------------------------------------------------------------------------
constexpr uint32_t kSmallMaxExperts = 2 * kFrontWaves;  // two router rows a wave at most
constexpr int kSmallRowLoads = 32;  // float4 router loads per lane, its rows together

// The route of a few experts (E <= 16, T <= 4) by one wave: lane 16 t + e
// holds expert e of token t.  The same keys, checks, exact ranking (rank r =
// number of larger keys; r < K is router slot r), slot-order
// renormalisation and CSR grouping as select_topk and select_group, which it
// replaces for these shapes.  With M the ballot of the selected lanes, every
// grouping quantity is a population count: the CSR row of a selected (t, e)
// is (pairs of experts below e) + (earlier tokens that picked e), and the
// active slots ascend by expert.  The slot records and their count go to
// LDS (sh.rec, sh.na, and sh.bad: nonzero when a check failed, the error
// latched as there); store: the route also goes to the global outputs.
__device__ void select_small(const SelectArgs& a, const float (&lgs)[kMaxDecodeTokens][16],
                             uint32_t lane, SelectShared& sh, bool store) {
    const uint32_t T = a.T, E = a.E, K = a.K;
    const uint32_t t = lane >> 4, e = lane & 15;
    const bool valid = t < T && e < E;
    const bool dbl = a.renorm == K3X_RENORM_DOUBLE;
    const float lg = lgs[min(t, T - 1)][min(e, E - 1)];
    const float b = a.bias[min(e, E - 1)];
    uint32_t err = 0;
    float s = 0.0f;
    uint64_t key = 0;
    if (valid) {
        if (dbl && (!__builtin_isfinite(lg) || !__builtin_isfinite(b))) err = K3X_ERR_INVALID_EXTENT;
        s = sigmoid_cr(lg);
        const float adj = __fadd_rn(s, b);
        if (!dbl && (!__builtin_isfinite(s) || s < 0.0f || s > 1.0f || !__builtin_isfinite(b) ||
                     !__builtin_isfinite(adj)))
            err = K3X_ERR_INVALID_STATE;
        key = topk_key(adj, e);
    }
    err = wave_max_u32(err);
    if (err) {
        if (lane == 0) {
            latch(a.status, err);
            sh.bad = 1;
        }
        return;
    }
    // Rank among the token's E keys (distinct: the low half holds the expert).
    const uint32_t row0 = lane & ~15u;
    uint32_t r = 0;
    for (uint32_t j = 0; j < E; ++j) {
        const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)key, (int)(row0 + j));
        const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(key >> 32), (int)(row0 + j));
        r += (((uint64_t)hi << 32) | lo) > key;
    }
    const bool sel = valid && r < K;
    // Denominator: the scores in slot order, summed in sequence.
    float den_f = 0.0f;
    double den_d = 0.0;
    for (uint32_t q = 0; q < K; ++q) {
        const uint64_t m = __ballot(valid && r == q);
        const uint32_t src = row0 + (uint32_t)__builtin_ctzll(((m >> row0) & 0xffffull) | 0x10000ull);
        const float x = __shfl(s, (int)min(src, 63u));
        den_f = __fadd_rn(den_f, x);
        den_d = __dadd_rn(den_d, (double)x);
    }
    const bool ok = dbl ? (__builtin_isfinite(den_d) && den_d > 0.0)
                        : (__builtin_isfinite(den_f) && den_f > 0.0f);
    if (__ballot(valid && !ok)) {
        if (lane == 0) {
            latch(a.status, dbl ? K3X_ERR_INVALID_EXTENT : K3X_ERR_INVALID_STATE);
            sh.bad = 1;
        }
        return;
    }
    // Grouping.  Bit 16 t' + e' of M: token t' picked expert e'.
    const uint64_t M = __ballot(sel);
    constexpr uint64_t kRows = 0x0001000100010001ull;
    const uint64_t col = kRows << e;
    const uint32_t below = (uint32_t)__popcll(M & (kRows * ((1ull << e) - 1)));
    const uint32_t rin = (uint32_t)__popcll(M & col & ((1ull << (16 * t)) - 1));
    const uint32_t cnt = (uint32_t)__popcll(M & col);
    const uint32_t act = (uint32_t)((M | M >> 16 | M >> 32 | M >> 48) & 0xffffu);
    if (t == 0 && (act >> e) & 1u) {  // one lane per active expert: its slot record
        const uint32_t ai = (uint32_t)__popc(act & ((1u << e) - 1));
        uint32_t toks = 0, j = 0;
        for (uint32_t tt = 0; tt < T; ++tt)
            if ((M >> (16 * tt + e)) & 1ull) toks |= tt << (8 * j++);
        const uint4 rec = make_uint4(e, cnt, below, toks);
        sh.rec[ai] = rec;
        if (store) a.arec[ai] = rec;
    }
    if (lane == 0) {
        sh.na = (uint32_t)__popc(act);
        sh.bad = 0;
        if (store) *a.n_active = (uint32_t)__popc(act);
    }
    if (!sel || !store) return;
    const float w = dbl ? __fmul_rn((float)__ddiv_rn((double)s, den_d), a.routed_scale)
                        : __fmul_rn(__fdiv_rn(s, den_f), a.routed_scale);
    const uint32_t p = t * K + r, row = below + rin;
    a.pair_token[row] = t;
    a.pair_slot[row] = r;
    a.ids[p] = e;
    a.weights[p] = w;
}

struct SmallArgs {
    const uint16_t* x;
    const float* gamma;
    const float* router_w;  // [E][H] fp32
    float eps;
    SelectArgs sel;         // shapes, bias, scale, renorm; block 0's route outputs
    GateUpArgs gu;
    uint16_t* xn;           // block 0: the xn copy
    float* logits;          // block 0: [T][E]
};

struct SmallLds {
    NormShared ns;
    SelectShared sel;
    float lg[kMaxDecodeTokens][kSmallMaxExperts];
    f32x4 red[kGuWaves][2][64];
};

// NE router rows per wave (experts wave + kFrontWaves i); TT bounds T.
// Workgroup b is unit (active slot, 16-row block), and routes by itself.
// ALL: every expert is active (E <= K), so slot s holds expert s (the slots
// ascend by expert) and its CSR rows are s T .. s T + T - 1, token by token
// (every token routes to every expert once): the units need no route.
// Workgroups [0, E I / 16) are then units that request their code tiles
// and scales with the x / gamma loads and go straight from xn to their
// products, and the one workgroup after them finds the route and stores it
// for the down launch (which alone reads it, for the slot order and the
// weights of the mix).
template <int TT, int NE, bool ALL>
__global__ __launch_bounds__(kFrontThreads) void small_route_gateup_kernel(SmallArgs a) {
    static_assert(kFrontThreads == 64 * kGuWaves, "one workgroup shape for route and gate/up");
    extern __shared__ uint4 dyn_lds[];  // xn [T][H] bf16, then gamma
    __shared__ SmallLds sh;
    const uint32_t lane = threadIdx.x & 63, wave = wave_id();
    const uint32_t T = a.sel.T, H = a.gu.H, E = a.sel.E, J = H / 256;
    const uint32_t per_expert = a.gu.I / 16;
    if constexpr (ALL) {
        if (blockIdx.x < E * per_expert) {
            const uint32_t e = blockIdx.x / per_expert, rb = blockIdx.x % per_expert;
            GuUnitRegs gw;
            // A non-finite x (or an earlier launch's error) ends every
            // workgroup here; the route workgroup latches it.
            if (!build_xn<kFrontThreads>(a.x, a.gamma, T, H, a.eps, dyn_lds, sh.ns, nullptr,
                                         nullptr, a.sel.status,
                                         [&]() { gateup_unit_load(a.gu, e, rb, gw); }, [] {}))
                return;
            uint32_t toks = 0;  // tokens of the slot's first four rows: 0, 1, ...
            for (uint32_t j = 1; j < min(T, 4u); ++j) toks |= j << (8 * j);
            gateup_unit_compute(a.gu, rb, make_uint4(e, T, e * T, toks),
                                reinterpret_cast<const uint16_t*>(dyn_lds), gw, sh.red);
            return;
        }
    }
    // The workgroup that stores the route (and xn and the logits).
    const bool store = ALL || blockIdx.x == 0;
    constexpr int kPer = kSmallRowLoads / NE;  // J <= kPer (checked on the host)
    float4 wb[NE][kPer];
    auto prefetch = [&]() {
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const uint32_t e = wave + kFrontWaves * i;
            const float* wr = a.router_w + (size_t)(e < E ? e : 0) * H + 4 * lane;
#pragma unroll
            for (int q = 0; q < kPer; ++q)
                wb[i][q] = *reinterpret_cast<const float4*>(wr + 256 * min((uint32_t)q, J - 1));
        }
    };
    if (!build_xn<kFrontThreads>(a.x, a.gamma, T, H, a.eps, dyn_lds, sh.ns,
                                 store ? a.xn : nullptr, a.sel.status, a.sel.status,
                                 prefetch, [] {}))
        return;
    // Logits of this wave's experts: partial 4 l + c sums j = 0, 1, ... in
    // sequence, then the canonical tree (router_block's order).
    const uint16_t* s_x = reinterpret_cast<const uint16_t*>(dyn_lds);
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const uint32_t e = wave + kFrontWaves * i;
        if (e >= E) continue;  // wave-uniform
        double p[TT][4];
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int c = 0; c < 4; ++c) p[t][c] = 0.0;
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            if ((uint32_t)q >= J) continue;
            const double wv[4] = {(double)wb[i][q].x, (double)wb[i][q].y, (double)wb[i][q].z,
                                  (double)wb[i][q].w};
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                if ((uint32_t)t >= T) continue;
                const uint2 xv =
                    *reinterpret_cast<const uint2*>(s_x + (size_t)t * H + 256 * q + 4 * lane);
                const float f[4] = {lo_bf16(xv.x), hi_bf16(xv.x), lo_bf16(xv.y), hi_bf16(xv.y)};
#pragma unroll
                for (int c = 0; c < 4; ++c) p[t][c] = __builtin_fma(wv[c], (double)f[c], p[t][c]);
            }
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if ((uint32_t)t >= T) continue;
            const float v = (float)canon_reduce(p[t]);
            if (lane == 0) {
                sh.lg[t][e] = v;
                if (store) a.logits[(size_t)t * E + e] = v;
            }
        }
    }
    // The route, by the first wave from the logits in LDS (this block's
    // copy of the slot records in LDS; the storing block stores it).
    __syncthreads();
    if (wave == 0) select_small(a.sel, sh.lg, lane, sh.sel, store);
    if constexpr (ALL) return;  // the route workgroup has no unit
    __syncthreads();
    if (sh.sel.bad) return;
    gateup_unit_lds(a.gu, blockIdx.x, reinterpret_cast<const uint16_t*>(dyn_lds), sh.sel.rec,
                    sh.sel.na, sh.red);
}

// ---------------------------------------------------------------------------
// Routed down projection -> per-pair rows; slot-ordered combine
// ---------------------------------------------------------------------------
struct DownArgs {
    const uint4* dn_codes;     // expert 0 base, tiles [H/16][I/128][64] x 16 B
    const uint32_t* dn_scales; // [H/16][ks][64]
    size_t codes_per_expert;
    size_t scales_per_expert;
    uint32_t kt, ks;           // I/128, scale groups
    uint32_t I, H, K;
    const uint16_t* act;       // [pairs][a_stride] CSR order (SPLIT: [hi | lo], lo at I)
    uint32_t a_stride;
    const uint32_t* n_active;
    const uint4* arec;         // per active slot {expert, rows, offset, row tokens}
    const uint32_t* pair_token;
    const uint32_t* pair_slot;
    float* y;                  // [T][K][H] per-pair outputs
    // Fused combine (decode_mix): router weights [T][K], shared expert
    // output [T][H] or null, the layer output, and the arrival counters
    // [T][H / 64] (zero between calls).  mix null: y only (the general
    // path's combine follows).
    const float* weights;
    const float* shared_y;
    uint16_t* out;
    float* out_f32;            // optional
    uint32_t* mix;
    uint32_t round_y;          // each y rounded to bf16 before its product
    const uint32_t* status;
};

// out[t][h] = bf16(sum over slots s in router order of w[t][s] * y[t][s][h]
// + shared[t][h]), float mul then float add per term
// (runtime/src/backend_cpu.cpp:295-301, runtime/src/model.cpp:1145), for
// the 64 columns h0 + lane of token t, by one wave.  The loads of a group of
// 16 slots are issued together (indices clamped, so there is no branch
// around them).
constexpr int kCombineBatch = 16;

// round_y: the official layer rounds each expert output to bf16 first
// (runtime/src/official_moe.cpp:99-101), as combine_kernel does.
__device__ inline void decode_mix(const float* y, const float* weights, const float* shared_y,
                                  uint32_t K, uint32_t H, uint32_t t, uint32_t h, uint16_t* out,
                                  float* out_f32, bool round_y) {
    const float* yr = y + (size_t)t * K * H + h;
    const float* wr = weights + (size_t)t * K;
    const float sh = shared_y ? shared_y[(size_t)t * H + h] : 0.0f;
    float mix = 0.0f;
    for (uint32_t s0 = 0; s0 < K; s0 += kCombineBatch) {
        float yv[kCombineBatch], wv[kCombineBatch];
#pragma unroll
        for (int u = 0; u < kCombineBatch; ++u) {
            const uint32_t s = min(s0 + u, K - 1);
            // Rows of other workgroups, stored device-scope in this launch:
            // device-scope loads (no stale cache line can answer them).
            yv[u] = __hip_atomic_load(yr + (size_t)s * H, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            wv[u] = wr[s];
        }
#pragma unroll
        for (int u = 0; u < kCombineBatch; ++u) {
            const float yu =
                round_y ? __uint_as_float((uint32_t)f32_to_bf16(yv[u]) << 16) : yv[u];
            if (s0 + u < K) mix = __fadd_rn(mix, __fmul_rn(wv[u], yu));
        }
    }
    const float v = shared_y ? __fadd_rn(mix, sh) : mix;
    out[(size_t)t * H + h] = f32_to_bf16(v);
    if (out_f32) out_f32[(size_t)t * H + h] = v;
}

// Workgroup = kDownWaves waves of one active slot ai, wave w taking 16-row
// block rb = (block % (H / 64)) * 4 + w.  The slot's activation rows (cnt
// rows of I bf16) are copied into LDS once by the whole block; their loads
// are issued first, then each wave's code tiles (the whole K range, I <=
// 2048) and scale dwords, all in flight together, so that a unit costs
// about one memory round trip.  Every load is unconditional (indices
// clamped; a clamped activation chunk is stored again with its own value),
// so the compiler keeps them all in flight.  The rows of the slot's pairs
// go to y.
// Then the combine, fused: per (token, 64-column group) a counter counts the
// workgroups that have stored their rows (one per router slot: an expert is
// routed at most once per token).  Wave w of the workgroup whose increment
// for the token of its row w completes the count (old value K - 1) mixes the
// token's 64 columns in router-slot order -- the same arithmetic whichever
// workgroup arrives last, so the result does not depend on the order -- and
// resets the counter for the next call.  The rows of y are stored, and read
// by the mixing wave, with device-scope atomic stores and loads, which are
// coherent across the XCDs' L2s without any cache write-back or
// invalidation; every store has completed before the workgroup's
// increments.  No workgroup waits for another.
constexpr int kDownWaves = 4;
// TILES: K tiles of the down projection held in registers (I <= 128 TILES);
// ACT: 16-byte activation loads per thread (cnt * a_stride / 8 <= 256 ACT);
// SPLIT: activation rows [hi | lo], two MFMAs per weight fragment.
constexpr int kDownTilesDecode = 16, kDownActDecode = 4;  // the decode path: I <= 2048
constexpr int kDownTilesFew = 24, kDownActFew = 12;       // general path: I <= 3072, split
// Split rows that fit half the loads (two tokens at I = 3072): 162 VGPRs,
// three workgroups a compute unit where the 12-load kernel fits two.
constexpr int kDownActFewHalf = kDownActFew / 2;

// ALL: every expert is active (E <= K), so slot ai holds expert ai (the
// slots ascend by expert) and the weights are requested before the slot
// record arrives.
template <int TILES, int ACT, bool SPLIT, bool ROWS = false, bool ALL = false>
__global__ __launch_bounds__(64 * kDownWaves) void decode_down_kernel(DownArgs a) {
    extern __shared__ uint4 s_act4[];  // [rows][a_stride] bf16
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t per_expert = a.H / (16 * kDownWaves);
    const uint32_t ai = blockIdx.x / per_expert;
    const uint32_t rb = (blockIdx.x % per_expert) * kDownWaves + wave;
    const uint32_t kt = a.kt;
    // Code tiles and scale dwords of this wave's 16-row block of expert e.
    uint4 c[TILES];
    uint32_t sw[TILES / 4];
    auto load_weights = [&](uint32_t e) {
        const uint4* codes = a.dn_codes + e * a.codes_per_expert + (size_t)rb * kt * 64 + lane;
        const uint32_t* scales =
            a.dn_scales + e * a.scales_per_expert + (size_t)rb * a.ks * 64 + lane;
#pragma unroll
        for (int i = 0; i < TILES; ++i) c[i] = ntl(codes + (size_t)min((uint32_t)i, kt - 1) * 64);
#pragma unroll
        for (int i = 0; i < TILES / 4; ++i)
            sw[i] = ntl(scales + (size_t)min((uint32_t)i, a.ks - 1) * 64);
    };
    const uint32_t st = prior_status(a.status);
    const uint32_t na = *a.n_active;
    const uint4 rec = a.arec[ai];  // ai < min(E, T*K): in bounds
    if constexpr (ALL) {
        load_weights(ai);
        // Keeps the loads ahead of the early return below (the compiler
        // would otherwise sink them past it, behind the record's arrival);
        // the three scalar loads above are issued before it.
        asm volatile("" ::: "memory");
    }
    if (st || ai >= na) return;
    const uint32_t e = rec.x, cnt = rec.y, off = rec.z;
    // 1. Activation rows [m0, m0 + rows) of the slot, contiguous in CSR
    //    order: chunks c < rows * a_stride / 8 (at most ACT per thread,
    //    checked by the host).  ROWS: kRowChunk rows at a time.
    u32x4 v[ACT];
#define K3X_DOWN_LOAD_ROWS(m0, rows)                                                           \
    load_chunks(v, a.act + (size_t)(off + (m0)) * a.a_stride, tid, 64 * kDownWaves,            \
                (rows) * (a.a_stride / 8))
#define K3X_DOWN_STORE_ROWS(rows) store_chunks(v, s_act4, tid, 64 * kDownWaves, (rows) * (a.a_stride / 8))
    // Pair rows of the outputs (needed at the end).
    uint32_t yrow[4];
#define K3X_DOWN_LOAD_YROWS(m0, rows)                                                          \
    {                                                                                          \
        _Pragma("unroll") for (int q = 0; q < 4; ++q) {                                        \
            const uint32_t r_ = off + (m0) + min(4 * g + q, (rows) - 1);                       \
            yrow[q] = a.pair_token[r_] * a.K + a.pair_slot[r_];                                \
        }                                                                                      \
    }
    uint32_t rows = ROWS ? min(cnt, kRowChunk) : cnt;
    K3X_DOWN_LOAD_ROWS(0, rows);
    // 2. The weights (unless requested already), then the pair rows.
    if constexpr (!ALL) load_weights(e);
    K3X_DOWN_LOAD_YROWS(0, rows);
    K3X_DOWN_STORE_ROWS(rows);
    __syncthreads();
    const uint16_t* s_act = reinterpret_cast<const uint16_t*>(s_act4);
    for (uint32_t m0 = 0;;) {
        const uint16_t* arow =
            s_act + (size_t)(n < rows ? n : 0) * a.a_stride + 32 * g;  // unused rows: row 0
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < TILES; ++i) {
            if ((uint32_t)i < kt) {
                uint4 av[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    av[j] = *reinterpret_cast<const uint4*>(arow + (size_t)i * 128 + 8 * j);
                const float sc = e8m0_to_f32((sw[i / 4] >> (8 * (i & 3))) & 0xffu);
                if constexpr (SPLIT) {
                    uint4 al[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        al[j] = *reinterpret_cast<const uint4*>(arow + a.I + (size_t)i * 128 + 8 * j);
                    acc = mxfp4_tile2(c[i], sc, av, al, acc);
                } else {
                    acc = mxfp4_tile(c[i], sc, av, acc);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (4 * g + q < rows)
                __hip_atomic_store(a.y + (size_t)yrow[q] * a.H + rb * 16 + n, acc[q],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if constexpr (!ROWS) {
            if (a.mix && a.K == 1) {
                // One router slot: each row's value is its token's whole
                // mix, formed here as decode_mix forms it (0 + w y, then the
                // shared row), with no counter (they stay zero) and no
                // reload of y.  yrow[q] is the token (slot 0).
                const uint32_t h = rb * 16 + n;
                float w[4], sh[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    w[q] = a.weights[yrow[q]];
                    sh[q] = a.shared_y ? a.shared_y[(size_t)yrow[q] * a.H + h] : 0.0f;
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (4 * g + q >= rows) continue;
                    const float yu = a.round_y
                                         ? __uint_as_float((uint32_t)f32_to_bf16(acc[q]) << 16)
                                         : acc[q];
                    const float mix = __fadd_rn(0.0f, __fmul_rn(w[q], yu));
                    const float v = a.shared_y ? __fadd_rn(mix, sh[q]) : mix;
                    a.out[(size_t)yrow[q] * a.H + h] = f32_to_bf16(v);
                    if (a.out_f32) a.out_f32[(size_t)yrow[q] * a.H + h] = v;
                }
                return;
            }
        }
        if (!ROWS) break;
        m0 += rows;
        if (m0 >= cnt) return;  // block-uniform; no mix (checked on the host)
        // The next rows, once every wave is past its reads of s_act.
        rows = min(cnt - m0, kRowChunk);
        K3X_DOWN_LOAD_ROWS(m0, rows);
        K3X_DOWN_LOAD_YROWS(m0, rows);
        __syncthreads();
        K3X_DOWN_STORE_ROWS(rows);
        __syncthreads();
    }
#undef K3X_DOWN_LOAD_ROWS
#undef K3X_DOWN_STORE_ROWS
#undef K3X_DOWN_LOAD_YROWS
    // The device-scope stores above are complete (so visible to every XCD)
    // once this wave's vector-memory counter is zero; the barrier extends
    // that to the workgroup before any increment.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (a.mix && wave < cnt) {  // wave-uniform; cnt <= T <= kDownWaves (checked on the host)
        const uint32_t hg = blockIdx.x % per_expert, t = a.pair_token[off + wave];
        uint32_t* ctr = a.mix + (size_t)t * per_expert + hg;
        uint32_t old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0);
        if (old == a.K - 1) {  // issued after the increment returned
            decode_mix(a.y, a.weights, a.shared_y, a.K, a.H, t, hg * 64 + lane, a.out,
                       a.out_f32, a.round_y != 0);
            if (lane == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace

namespace k3x_hip {

namespace {

size_t front_lds(uint32_t T, uint32_t H) { return xn_lds_bytes(T, H) + sizeof(FrontLds); }

// Pairs the decode path handles (T * K).
constexpr uint32_t kMaxDecodePairs = 256;

}  // namespace

// The two-launch form of the decode path (small_route_gateup_kernel): few
// experts whose router rows fit a wave's registers, no shared expert, no
// per-expert grouping taps; within decode_eligible's shapes.
bool small_route_eligible(const k3x_hip_ctx* ctx, const k3x_hip_bank* bank,
                          const k3x_hip_moe_params* p, bool group_taps) {
    const auto& d = bank->desc;
    const uint32_t ne = d.experts > (uint32_t)kFrontWaves ? 2 : 1;
    return !group_taps && d.shared_inter == 0 && d.experts <= kSmallMaxExperts &&
           d.hidden / 256 <= (uint32_t)kSmallRowLoads / ne &&
           xn_lds_bytes(p->tokens, d.hidden) + sizeof(SmallLds) <= ctx->max_lds_per_block;
}

bool decode_eligible(const k3x_hip_ctx* ctx, const k3x_hip_bank* bank,
                     const k3x_hip_moe_params* p, const void* x) {
    const auto& d = bank->desc;
    if (reinterpret_cast<uintptr_t>(x) % 16) return false;  // 16-byte input loads
    const size_t lds = front_lds(p->tokens, d.hidden);
    return p->tokens <= (uint32_t)kMaxDecodeTokens && lds <= ctx->max_lds_per_block &&
           d.hidden % 256 == 0 && d.experts <= (uint32_t)(kKeysPerLane * 64) &&
           p->top_k <= 64 && p->tokens * p->top_k <= (uint32_t)kMaxDecodePairs &&
           d.inter % 128 == 0 && d.inter <= 128 * kDownTilesDecode &&
           d.hidden <= 128 * kGuWaves * kGuTiles &&
           (size_t)p->tokens * d.hidden / 8 <= (size_t)64 * kGuWaves * kGuActLoads &&
           d.hidden % (16 * kDownWaves) == 0 && d.hidden / 64 <= kMixGroupsMax &&
           p->tokens <= (uint32_t)kDownWaves &&  // a slot's rows: one per mixing wave
           (size_t)p->tokens * d.inter / 8 <= (size_t)64 * kDownWaves * kDownActDecode &&
           d.shared_inter % 256 == 0;
}

// Five launches on the context stream.  The shared expert, which needs only
// xn, rides along as extra workgroups of the two latency-bound launches: its
// gate/up blocks beside the router blocks, its down blocks beside the Top-K
// block, so its ~90 MB stream while those steps wait on latency.
int decode_forward(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                   const LayerBuffers& b, const uint16_t* x, uint16_t* out, float* out_f32,
                   bool group_taps) {
    const auto& d = bank->desc;
    const uint32_t T = p->tokens, K = p->top_k, S = d.shared_inter;
    const GluParams glu{(int)p->glu, p->situ_beta, (int)p->has_situ_linear, p->situ_linear_beta};
    hipStream_t main = ctx->stream;

    FrontArgs f{};
    f.x = x;
    f.gamma = bank->gamma;
    f.router_w = bank->router_w;
    f.T = T;
    f.H = d.hidden;
    f.E = d.experts;
    f.S = S;
    f.eps = p->rms_epsilon;
    f.router_blocks = (d.experts + kRouterRows - 1) / kRouterRows;
    f.sh_gu = reinterpret_cast<const uint4*>(bank->sh_gu);
    f.glu = glu;
    f.xn = b.xn;
    f.logits = b.logits;
    f.sact = b.sact;
    f.status = ctx->status;
    const dim3 front_grid(f.router_blocks + S / 16);
    const size_t xn_lds = xn_lds_bytes(T, d.hidden);

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
    sa.group_taps = group_taps;
    sa.status = ctx->status;
    SharedDownArgs sd{};
    sd.sh_dn = reinterpret_cast<const uint4*>(bank->sh_dn);
    sd.sact = b.sact;
    sd.T = T;
    sd.H = d.hidden;
    sd.S = S;
    sd.sy = b.sy;
    sd.status = ctx->status;

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
    gu.act_stride = d.inter;
    gu.act_lo = 0;
    gu.glu = glu;
    gu.status = ctx->status;
    const uint32_t gu_blocks = max_active * (d.inter / 16);

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
    dn.a_stride = d.inter;
    dn.n_active = b.n_active;
    dn.arec = b.arec;
    dn.pair_token = b.pair_token;
    dn.pair_slot = b.pair_slot;
    dn.y = b.y;
    dn.weights = b.weights;
    dn.shared_y = S ? b.sy : nullptr;
    dn.out = out;
    dn.out_f32 = out_f32;
    dn.mix = b.mix;
    dn.status = ctx->status;

    int mark = 0;
    const bool small = small_route_eligible(ctx, bank, p, group_taps);
    if (small) {
        // Route + routed gate/up in one launch (every workgroup routes).
        SmallArgs sm{};
        sm.x = x;
        sm.gamma = bank->gamma;
        sm.router_w = bank->router_w;
        sm.eps = p->rms_epsilon;
        sm.sel = sa;
        sm.gu = gu;
        sm.xn = b.xn;
        sm.logits = b.logits;
        mark = begin_stage(ctx, K3X_STAGE_DECODE_GATE_UP);
        const bool two = d.experts > (uint32_t)kFrontWaves;
        // Every expert picked (E <= K): the weights stream beside the route.
        const bool all = d.experts <= K;
        // ALL: one more workgroup, the route's.
        const dim3 grid(gu_blocks + (all ? 1 : 0));
#define K3X_SMALL(TT_, NE_)                                                                 \
    do {                                                                                   \
        if (all)                                                                          \
            hipLaunchKernelGGL((small_route_gateup_kernel<TT_, NE_, true>), grid,          \
                               dim3(kFrontThreads), xn_lds, main, sm);                     \
        else                                                                               \
            hipLaunchKernelGGL((small_route_gateup_kernel<TT_, NE_, false>), grid,         \
                               dim3(kFrontThreads), xn_lds, main, sm);                     \
    } while (0)
        if (T <= 2 && !two)
            K3X_SMALL(2, 1);
        else if (T <= 2)
            K3X_SMALL(2, 2);
        else if (!two)
            K3X_SMALL(kMaxDecodeTokens, 1);
        else
            K3X_SMALL(kMaxDecodeTokens, 2);
#undef K3X_SMALL
        end_stage(ctx, mark);
    } else {
        mark = begin_stage(ctx, K3X_STAGE_DECODE_FRONT);
        if (T <= 2)
            hipLaunchKernelGGL((decode_front_kernel<2>), front_grid, dim3(kFrontThreads), xn_lds,
                               main, f);
        else
            hipLaunchKernelGGL((decode_front_kernel<kMaxDecodeTokens>), front_grid,
                               dim3(kFrontThreads), xn_lds, main, f);
        end_stage(ctx, mark);
        mark = begin_stage(ctx, K3X_STAGE_DECODE_SELECT);
        hipLaunchKernelGGL(decode_select_kernel, dim3(1 + (S ? d.hidden / 16 : 0)),
                           dim3(kFrontThreads), 0, main, sa, sd);
        end_stage(ctx, mark);
        mark = begin_stage(ctx, K3X_STAGE_DECODE_GATE_UP);
        hipLaunchKernelGGL(decode_gateup_kernel<1>, dim3(gu_blocks), dim3(64 * kGuWaves),
                           (size_t)T * d.hidden * 2, main, gu);
        end_stage(ctx, mark);
    }
    mark = begin_stage(ctx, K3X_STAGE_DECODE_DOWN);
    const dim3 dn_grid(max_active * (d.hidden / (16 * kDownWaves)));
    if (d.experts <= K)  // every expert active
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesDecode, kDownActDecode, false, false, true>),
                           dn_grid, dim3(64 * kDownWaves), (size_t)T * d.inter * 2, main, dn);
    else
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesDecode, kDownActDecode, false>), dn_grid,
                           dim3(64 * kDownWaves), (size_t)T * d.inter * 2, main, dn);
    end_stage(ctx, mark);
    ctx->kernel_launches += small ? 2 : 4;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

bool few_row_experts_eligible(const k3x_hip_ctx* ctx, const k3x_hip_bank* bank, uint32_t T,
                              bool split) {
    const auto& d = bank->desc;
    const uint32_t a_stride = split ? 2 * d.inter : d.inter;
    return T <= (uint32_t)kMaxDecodeTokens && d.hidden % 256 == 0 &&
           d.hidden <= 128 * kGuWaves * kGuTiles &&
           (size_t)T * d.hidden / 8 <= (size_t)64 * kGuWaves * kGuActLoads &&
           (size_t)T * d.hidden * 2 <= ctx->max_lds_per_block && d.inter % 128 == 0 &&
           d.inter <= 128 * kDownTilesFew && d.hidden % (16 * kDownWaves) == 0 &&
           (size_t)T * a_stride / 8 <= (size_t)64 * kDownWaves * kDownActFew &&
           (size_t)T * a_stride * 2 <= ctx->max_lds_per_block;
}

int launch_few_row_gate_up(k3x_hip_ctx* ctx, const k3x_hip_bank* bank, uint32_t T, uint32_t K,
                           const LayerBuffers& b, const uint16_t* xn, const GluParams& glu,
                           bool split, bool chunked) {
    const auto& d = bank->desc;
    // Row tokens travel as 8-bit fields (the records' packed tokens, or the
    // chunk's tokens packed in the kernel).
    if (T > (chunked ? kChunkedMaxTokens : (uint32_t)kMaxDecodeTokens) ||
        !few_row_experts_eligible(ctx, bank, chunked ? kRowChunk : T, split))
        return K3X_ERR_INVALID_EXTENT;
    GateUpArgs gu{};
    gu.gu_codes = reinterpret_cast<const uint4*>(bank->gu_codes);
    gu.gu_scales = bank->gu_scales;
    gu.codes_per_expert = bank->gu_codes_per_expert / 16;
    gu.scales_per_expert = bank->gu_scales_per_expert;
    gu.kt = bank->gate.kt;
    gu.ks = bank->gate.ks;
    gu.I = d.inter;
    gu.H = d.hidden;
    gu.xn = xn;
    gu.n_active = b.n_active;
    gu.arec = b.arec;
    gu.pair_token = b.pair_token;
    gu.act = b.act;
    gu.act_stride = split ? 2 * d.inter : d.inter;
    gu.act_lo = split ? d.inter : 0;
    gu.glu = glu;
    gu.status = ctx->status;
    const uint32_t max_active = std::min<uint32_t>(d.experts, T * K);
    const size_t lds = (size_t)(chunked ? kRowChunk : T) * d.hidden * 2;
    // Two row blocks a workgroup when each one's K range fits half the waves.
    const bool two = gu.kt <= (uint32_t)(kGuWaves / 2 * kGuTiles) && (d.inter / 16) % 2 == 0;
    const dim3 grid(max_active * (d.inter / (two ? 32 : 16))), block(64 * kGuWaves);
    if (two && chunked)
        hipLaunchKernelGGL((decode_gateup_kernel<2, true>), grid, block, lds, ctx->stream, gu);
    else if (two)
        hipLaunchKernelGGL((decode_gateup_kernel<2, false>), grid, block, lds, ctx->stream, gu);
    else if (chunked)
        hipLaunchKernelGGL((decode_gateup_kernel<1, true>), grid, block, lds, ctx->stream, gu);
    else
        hipLaunchKernelGGL((decode_gateup_kernel<1, false>), grid, block, lds, ctx->stream, gu);
    ctx->kernel_launches += 1;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

bool few_row_mix_eligible(const k3x_hip_bank* bank, uint32_t T) {
    return T <= (uint32_t)kDownWaves && bank->desc.hidden / 64 <= kMixGroupsMax;
}

int launch_few_row_down(k3x_hip_ctx* ctx, const k3x_hip_bank* bank, uint32_t T, uint32_t K,
                        const LayerBuffers& b, bool split, bool chunked, const FewRowMix* mix) {
    const auto& d = bank->desc;
    if (T > (chunked ? kChunkedMaxTokens : (uint32_t)kMaxDecodeTokens) ||
        !few_row_experts_eligible(ctx, bank, chunked ? kRowChunk : T, split))
        return K3X_ERR_INVALID_EXTENT;
    if (mix && (chunked || !few_row_mix_eligible(bank, T) || !b.mix || !mix->out))
        return K3X_ERR_INVALID_EXTENT;
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
    dn.a_stride = split ? 2 * d.inter : d.inter;
    dn.n_active = b.n_active;
    dn.arec = b.arec;
    dn.pair_token = b.pair_token;
    dn.pair_slot = b.pair_slot;
    dn.y = b.y;
    dn.mix = nullptr;  // without mix, the general path's combine follows
    if (mix) {
        dn.weights = mix->weights;
        dn.shared_y = mix->shared_y;
        dn.out = mix->out;
        dn.out_f32 = mix->out_f32;
        dn.round_y = mix->round_y ? 1u : 0u;
        dn.mix = b.mix;
    }
    dn.status = ctx->status;
    const uint32_t max_active = std::min<uint32_t>(d.experts, T * K);
    const uint32_t rows = chunked ? kRowChunk : T;
    const dim3 grid(max_active * (d.hidden / (16 * kDownWaves))), block(64 * kDownWaves);
    const size_t lds = (size_t)rows * dn.a_stride * 2;
    // The decode kernel's shape (16 tiles, 4 activation loads a thread)
    // where it holds the rows: fewer registers than the 24-tile one.
    const bool small = !split && d.inter <= 128u * kDownTilesDecode &&
                       (size_t)rows * dn.a_stride / 8 <= (size_t)64 * kDownWaves * kDownActDecode;
    if (small && chunked)
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesDecode, kDownActDecode, false, true>),
                           grid, block, lds, ctx->stream, dn);
    else if (small)
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesDecode, kDownActDecode, false, false>),
                           grid, block, lds, ctx->stream, dn);
    else if (split && chunked)
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesFew, kDownActFew, true, true>), grid,
                           block, lds, ctx->stream, dn);
    else if (split &&
             (size_t)rows * dn.a_stride / 8 <= (size_t)64 * kDownWaves * kDownActFewHalf)
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesFew, kDownActFewHalf, true, false>),
                           grid, block, lds, ctx->stream, dn);
    else if (split)
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesFew, kDownActFew, true, false>), grid,
                           block, lds, ctx->stream, dn);
    else if (chunked)
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesFew, kDownActFew, false, true>), grid,
                           block, lds, ctx->stream, dn);
    else
        hipLaunchKernelGGL((decode_down_kernel<kDownTilesFew, kDownActFew, false, false>), grid,
                           block, lds, ctx->stream, dn);
    ctx->kernel_launches += 1;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

}  // namespace k3x_hip
