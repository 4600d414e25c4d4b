// official.hip -- the official K3 MoE FFN (Stable LatentMoE) around a bank of
// experts at the latent width, after runtime/src/official_moe.cpp:156-344.
//
//   prepare   hidden = post_norm(bf16(p0 bf16(residual) + p1 bf16(prefix))),
//             p = softmax of the two sources' scores (official_prepare_kernel);
//             router logits over hidden (the layer's router kernels)
//   route     sigmoid + correction, natural Top-K, s / sum s (topk_kernel)
//   latent    bf16(routed_down . hidden)                 (dense GEMM + rounding)
//   experts   the bank's grouped MXFP4 path on latent; each expert output
//             rounded to bf16 before the slot-ordered mix; mixed rounded
//   norm      RMSNorm(mixed, routed_norm)                (rmsnorm_kernel)
//   routed    routed_up . norm; shared FFN on hidden     (dense GEMMs)
//   out       bf16(bf16(prefix) + bf16(bf16(routed) + bf16(shared)))
//
// Sums run in the layer's own orders (fp64 canonical for the norms and the
// router, fp32 MFMA for the projections), not the reference's sequential
// double ones; the reference's checks on this layer hold at 2e-2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "k3x_decode.hpp"
#include "k3x_device.hpp"
#include "k3x_gemm.hpp"
#include "k3x_internal.hpp"

using namespace k3x_dev;

struct k3x_hip_official {
    k3x_hip_ctx* ctx = nullptr;
    k3x_hip_bank* bank = nullptr;  // experts at the latent width
    uint32_t H = 0, L = 0, E = 0, I_s = 0;
    // Dense bf16 matrices in the bank's tile layout.
    uint4* routed_down = nullptr;  // [L/16][H/128][4][64]
    uint4* routed_up = nullptr;    // [H/16][L/128][4][64]
    uint4* shared_gu = nullptr;    // [Is/16][H/128][2][4][64]
    uint4* shared_dn = nullptr;    // [H/16][Is/128][4][64]
    // bf16 vectors and the router held as fp32 (exact).
    float* routed_norm = nullptr;    // [L]
    float* residual_norm = nullptr;  // [H]
    float* residual_proj = nullptr;  // [H]
    float* post_norm = nullptr;      // [H]
    float* router = nullptr;         // [E][H]
    float* router_wp = nullptr;      // residue-major copy (H <= 8192; matrix-core router)
    float* correction = nullptr;     // [E]
    bool ffn_ready = false, route_ready = false;
    // Per-call buffers (grow-only; the bank's forward uses the context scratch)
    // and the residue-major copy of hidden for the matrix-core router.
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    uint16_t* xp = nullptr;
    size_t xp_bytes = 0;
    // The latent projection and the shared FFN run on the context's side
    // stream between fork_ev and join_ev; latent_ev marks the latent done.
    hipEvent_t fork_ev = nullptr, join_ev = nullptr, latent_ev = nullptr;
};

namespace {

constexpr int kThreads = 256;
inline unsigned blocks_for(size_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

__device__ inline void latch(uint32_t* status, uint32_t code) { atomicCAS(status, 0u, code); }
__device__ inline float bf16_round(float v) { return __uint_as_float((uint32_t)f32_to_bf16(v) << 16); }

// Canonical fp64 block sum over 256 threads (xor butterfly in each wave, then
// (w0 + w1) + (w2 + w3)); every thread gets the result.
__device__ inline double block_sum(double v, double* red) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    const double r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

// One 256-thread block per token.  runtime/src/official_moe.cpp:156-209:
// both sources rounded to bf16; per source inv = 1 / sqrt(float(sum v^2 / H)
// + eps) and score = sum (double)(v * inv) * norm * proj; p = softmax of the
// two scores in float; mix = bf16(p0 v0 + p1 v1); hidden = bf16(mix * inv' *
// post_norm) with inv' from mix's own sum of squares (:61-80).  Sums of
// thread i run over k = i, i + 256, ... in order, then the canonical tree.
__global__ __launch_bounds__(kThreads) void official_prepare_kernel(
    const float* __restrict__ prefix, const float* __restrict__ residual,
    const float* __restrict__ res_norm, const float* __restrict__ res_proj,
    const float* __restrict__ post_norm, uint32_t H, float eps, uint16_t* __restrict__ hidden,
    uint32_t* status) {
    extern __shared__ float s_mix[];  // [H]
    __shared__ double red[4];
    if (*(volatile uint32_t*)status) return;
    const uint32_t tid = threadIdx.x;
    const float* src[2] = {residual + (size_t)blockIdx.x * H, prefix + (size_t)blockIdx.x * H};
    float inv[2], score[2];
    int bad = 0;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        double sq = 0.0;
        for (uint32_t k = tid; k < H; k += kThreads) {
            const float v = bf16_round(src[r][k]);
            bad |= !__builtin_isfinite(src[r][k]);
            sq = __builtin_fma((double)v, (double)v, sq);  // exact product: fused == separate
        }
        sq = block_sum(sq, red);
        inv[r] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)__ddiv_rn(sq, (double)H), eps)));
        double sc = 0.0;
        for (uint32_t k = tid; k < H; k += kThreads) {
            const float v = bf16_round(src[r][k]);
            const double term =
                ((double)__fmul_rn(v, inv[r]) * (double)res_norm[k]) * (double)res_proj[k];
            sc = sc + term;
        }
        score[r] = (float)block_sum(sc, red);
    }
    if (__syncthreads_or(bad)) {
        if (tid == 0) latch(status, K3X_ERR_INVALID_EXTENT);
        return;
    }
    const float mx = score[0] >= score[1] ? score[0] : score[1];
    float p0 = expf_cr(__fsub_rn(score[0], mx)), p1 = expf_cr(__fsub_rn(score[1], mx));
    const float den = __fadd_rn(p0, p1);
    p0 = __fdiv_rn(p0, den);
    p1 = __fdiv_rn(p1, den);
    double sq = 0.0;
    for (uint32_t k = tid; k < H; k += kThreads) {
        const float m = bf16_round(__fadd_rn(__fmul_rn(p0, bf16_round(src[0][k])),
                                             __fmul_rn(p1, bf16_round(src[1][k]))));
        s_mix[k] = m;
        sq = __builtin_fma((double)m, (double)m, sq);
    }
    sq = block_sum(sq, red);
    const float inv2 = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)__ddiv_rn(sq, (double)H), eps)));
    uint16_t* out = hidden + (size_t)blockIdx.x * H;
    for (uint32_t k = tid; k < H; k += kThreads)
        out[k] = f32_to_bf16(__fmul_rn(__fmul_rn(s_mix[k], inv2), post_norm[k]));
}

// The same computation with every row this thread touches in registers
// (H <= 8192: thread tid holds k = tid + 256 j, j < 32).  All loads are
// issued before the first sum; loads past the row read 0 through the buffer
// resource, and their zero terms come after the row's last term, leaving
// every sum unchanged.
constexpr uint32_t kPrepRegHidden = 8192;
// Up to this many tokens the prepare runs 1024 threads a token.
constexpr uint32_t kPrepWideTokens = 64;

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
void official_prepare_reg_kernel(
    const float* __restrict__ prefix, const float* __restrict__ residual,
    const float* __restrict__ res_norm, const float* __restrict__ res_proj,
    const float* __restrict__ post_norm, uint32_t H, float eps, uint16_t* __restrict__ hidden,
    uint32_t* status) {
    __shared__ double red[4];
    if (*(volatile uint32_t*)status) return;
    const uint32_t tid = threadIdx.x;
    auto rsrc = [&](const float* base) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, H * 4,
                                                 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t r0 = rsrc(residual + (size_t)blockIdx.x * H);
    const __amdgpu_buffer_rsrc_t r1 = rsrc(prefix + (size_t)blockIdx.x * H);
    const __amdgpu_buffer_rsrc_t rn = rsrc(res_norm), rp = rsrc(res_proj), pn = rsrc(post_norm);
    auto ld = [&](__amdgpu_buffer_rsrc_t r, int j) {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, tid * 4, j * 1024, 0));
    };
    auto lo = [](uint32_t w) { return __uint_as_float(w << 16); };
    auto hi = [](uint32_t w) { return __uint_as_float(w & 0xffff0000u); };
    // Both rows, rounded to bf16 as they arrive, held packed in LDS
    // (residual in the low half, prefix in the high half of word j, 32 KiB
    // a token; each thread reads only its own words); the weight vectors,
    // the same for every token, are read from the cache in batches where
    // they are used.  Four tokens then share a compute unit.
    __shared__ uint32_t s_pk[32][kThreads];
    int bad = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float a = ld(r0, j), b = ld(r1, j);
        bad |= !__builtin_isfinite(a) | !__builtin_isfinite(b);
        // Round to nearest even by the conversion instruction (f32_to_bf16's
        // rule for every finite value; a non-finite one fails the call).
        const bf16x2 h = {(__bf16)a, (__bf16)b};
        s_pk[j][tid] = __builtin_bit_cast(uint32_t, h);
    }
    // bad now, so that the raw values are not kept for it.
    asm volatile("" : "+v"(bad));
    constexpr int kB = 8;
    float inv[2], score[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        double sq = 0.0;
#pragma unroll 4
        for (int j = 0; j < 32; ++j) {
            const double f = (double)(r ? hi(s_pk[j][tid]) : lo(s_pk[j][tid]));
            sq = __builtin_fma(f, f, sq);
        }
        sq = block_sum(sq, red);
        inv[r] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)__ddiv_rn(sq, (double)H), eps)));
    }
    double sc[2] = {0.0, 0.0};
#pragma unroll 1
    for (int j0 = 0; j0 < 32; j0 += kB) {
        asm volatile("" ::: "memory");  // the batch's loads stay here
        float nw[kB], pw[kB];
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            nw[j] = ld(rn, j0 + j);
            pw[j] = ld(rp, j0 + j);
        }
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const uint32_t w = s_pk[j0 + j][tid];
            sc[0] = sc[0] + ((double)__fmul_rn(lo(w), inv[0]) * (double)nw[j]) * (double)pw[j];
            sc[1] = sc[1] + ((double)__fmul_rn(hi(w), inv[1]) * (double)nw[j]) * (double)pw[j];
        }
    }
    score[0] = (float)block_sum(sc[0], red);
    score[1] = (float)block_sum(sc[1], red);
    if (__syncthreads_or(bad)) {
        if (tid == 0) latch(status, K3X_ERR_INVALID_EXTENT);
        return;
    }
    const float mx = score[0] >= score[1] ? score[0] : score[1];
    float p0 = expf_cr(__fsub_rn(score[0], mx)), p1 = expf_cr(__fsub_rn(score[1], mx));
    const float den = __fadd_rn(p0, p1);
    p0 = __fdiv_rn(p0, den);
    p1 = __fdiv_rn(p1, den);
    // The mix replaces the pair in LDS (fp32 bits).
    double sq = 0.0;
#pragma unroll 4
    for (int j = 0; j < 32; ++j) {
        const uint32_t w = s_pk[j][tid];
        const float m = bf16_round(__fadd_rn(__fmul_rn(p0, lo(w)), __fmul_rn(p1, hi(w))));
        s_pk[j][tid] = __float_as_uint(m);
        sq = __builtin_fma((double)m, (double)m, sq);
    }
    sq = block_sum(sq, red);
    const float inv2 = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)__ddiv_rn(sq, (double)H), eps)));
    uint16_t* out = hidden + (size_t)blockIdx.x * H;
#pragma unroll 1
    for (int j0 = 0; j0 < 32; j0 += kB) {
        asm volatile("" ::: "memory");
        float g[kB];
#pragma unroll
        for (int j = 0; j < kB; ++j) g[j] = ld(pn, j0 + j);
#pragma unroll
        for (int j = 0; j < kB; ++j)
            if (tid + 256u * (j0 + j) < H)
                out[tid + 256 * (j0 + j)] = f32_to_bf16(
                    __fmul_rn(__fmul_rn(__uint_as_float(s_pk[j0 + j][tid]), inv2), g[j]));
    }
}

// Fp64 block sum over TPB threads in a fixed order: xor butterfly in each
// wave, then the balanced pairwise tree over the waves; every thread gets
// the result.
// red: TPB / 64 + 1 doubles.
template <int TPB>
__device__ inline double block_sum_tpb(double v, double* red) {
    constexpr int W = TPB / 64;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    if (wave == 0) {
        // Lane i < W holds wave i's sum; level h adds lane i + h into lane i
        // for i a multiple of 2 h.
        double w = red[lane < W ? lane : 0];
#pragma unroll
        for (int h = 1; h < W; h *= 2) {
            const double o = __shfl_down(w, h);
            if (lane % (2 * h) == 0) w = w + o;
        }
        if (lane == 0) red[W] = w;
    }
    __syncthreads();
    const double r = red[W];
    __syncthreads();
    return r;
}

// official_prepare_reg_kernel with TPB threads a token (thread tid holds k =
// tid + TPB j, j < 8192 / TPB): for few tokens, more threads issue a row's
// loads at once and run shorter sequential sums.  The same formulas; the
// sums' order is this kernel's own (per-thread sequential, then
// block_sum_tpb), within the contract's one bf16 ulp of the reference's
// sequential sums.
template <int TPB>
__global__ __launch_bounds__(TPB) void official_prepare_tpb_kernel(
    const float* __restrict__ prefix, const float* __restrict__ residual,
    const float* __restrict__ res_norm, const float* __restrict__ res_proj,
    const float* __restrict__ post_norm, uint32_t H, float eps, uint16_t* __restrict__ hidden,
    uint32_t* status) {
    constexpr int J = kPrepRegHidden / TPB;
    __shared__ double red[TPB / 64 + 1];
    if (*(volatile uint32_t*)status) return;
    const uint32_t tid = threadIdx.x;
    auto rsrc = [&](const float* base) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, H * 4,
                                                 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t r0 = rsrc(residual + (size_t)blockIdx.x * H);
    const __amdgpu_buffer_rsrc_t r1 = rsrc(prefix + (size_t)blockIdx.x * H);
    const __amdgpu_buffer_rsrc_t rn = rsrc(res_norm), rp = rsrc(res_proj), pn = rsrc(post_norm);
    // Loads past the row read 0 (their terms come after the row's last).
    auto ld = [&](__amdgpu_buffer_rsrc_t r, int j) {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, tid * 4, j * TPB * 4, 0));
    };
    float v[2][J], nw[J], pw[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        v[0][j] = ld(r0, j);
        v[1][j] = ld(r1, j);
        nw[j] = ld(rn, j);
        pw[j] = ld(rp, j);
    }
    int bad = 0;
    float inv[2], score[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        double sq = 0.0;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            bad |= !__builtin_isfinite(v[r][j]);
            v[r][j] = bf16_round(v[r][j]);
            sq = __builtin_fma((double)v[r][j], (double)v[r][j], sq);
        }
        sq = block_sum_tpb<TPB>(sq, red);
        inv[r] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)__ddiv_rn(sq, (double)H), eps)));
        double sc = 0.0;
#pragma unroll
        for (int j = 0; j < J; ++j)
            sc = sc + ((double)__fmul_rn(v[r][j], inv[r]) * (double)nw[j]) * (double)pw[j];
        score[r] = (float)block_sum_tpb<TPB>(sc, red);
    }
    if (__syncthreads_or(bad)) {
        if (tid == 0) latch(status, K3X_ERR_INVALID_EXTENT);
        return;
    }
    const float mx = score[0] >= score[1] ? score[0] : score[1];
    float p0 = expf_cr(__fsub_rn(score[0], mx)), p1 = expf_cr(__fsub_rn(score[1], mx));
    const float den = __fadd_rn(p0, p1);
    p0 = __fdiv_rn(p0, den);
    p1 = __fdiv_rn(p1, den);
    // The post-norm weights are requested only now (not hoisted above the
    // sums), so that they take no registers until then.
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < J; ++j) nw[j] = ld(pn, j);
    double sq = 0.0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        v[0][j] = bf16_round(__fadd_rn(__fmul_rn(p0, v[0][j]), __fmul_rn(p1, v[1][j])));
        sq = __builtin_fma((double)v[0][j], (double)v[0][j], sq);
    }
    sq = block_sum_tpb<TPB>(sq, red);
    const float inv2 = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)__ddiv_rn(sq, (double)H), eps)));
    uint16_t* out = hidden + (size_t)blockIdx.x * H;
#pragma unroll
    for (int j = 0; j < J; ++j)
        if (tid + (uint32_t)TPB * j < H)
            out[tid + TPB * j] = f32_to_bf16(__fmul_rn(__fmul_rn(v[0][j], inv2), nw[j]));
}

// fp32 values rounded to bf16 in place (synthetic bf16 weights held as fp32).
__global__ void round_in_place_kernel(float* __restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) p[i] = bf16_round(p[i]);
}

// bf16 bits of fp32 values.
__global__ void round_bf16_kernel(const float* __restrict__ in, size_t n,
                                  uint16_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(in[i]);
}

// out = bf16(bf16(prefix) + bf16(bf16(routed) + bf16(shared)))
// (runtime/src/official_moe.cpp:336-340; no shared FFN: shared = 0).
// Four elements per thread (16-byte loads, 8-byte store) when n % 4 == 0 and
// the rows are 16-byte aligned, else one.
template <int V>
__global__ void official_out_kernel(const float* __restrict__ prefix,
                                    const float* __restrict__ routed,
                                    const float* __restrict__ shared, size_t n,
                                    uint16_t* __restrict__ out, const uint32_t* status) {
    if (*(volatile const uint32_t*)status) return;
    const size_t i = ((size_t)blockIdx.x * kThreads + threadIdx.x) * V;
    if (i >= n) return;
    float pv[V], rv[V], sv[V];
    if constexpr (V == 4) {
        const float4 p4 = *reinterpret_cast<const float4*>(prefix + i);
        const float4 r4 = *reinterpret_cast<const float4*>(routed + i);
        const float4 s4 = shared ? *reinterpret_cast<const float4*>(shared + i) : make_float4(0, 0, 0, 0);
        pv[0] = p4.x; pv[1] = p4.y; pv[2] = p4.z; pv[3] = p4.w;
        rv[0] = r4.x; rv[1] = r4.y; rv[2] = r4.z; rv[3] = r4.w;
        sv[0] = s4.x; sv[1] = s4.y; sv[2] = s4.z; sv[3] = s4.w;
    } else {
        pv[0] = prefix[i];
        rv[0] = routed[i];
        sv[0] = shared ? shared[i] : 0.0f;
    }
    uint16_t o[V];
#pragma unroll
    for (int c = 0; c < V; ++c) {
        const float sh = shared ? bf16_round(sv[c]) : 0.0f;
        const float combined = bf16_round(__fadd_rn(bf16_round(rv[c]), sh));
        o[c] = f32_to_bf16(__fadd_rn(bf16_round(pv[c]), combined));
    }
    if constexpr (V == 4) {
        *reinterpret_cast<uint2*>(out + i) =
            make_uint2(o[0] | (uint32_t)o[1] << 16, o[2] | (uint32_t)o[3] << 16);
    } else {
        out[i] = o[0];
    }
}

// bf16 words -> fp32 on the host (exact).
std::vector<float> widen(const uint16_t* w, size_t n) {
    std::vector<float> f(n);
    for (size_t i = 0; i < n; ++i) {
        const uint32_t b = (uint32_t)w[i] << 16;
        std::memcpy(&f[i], &b, 4);
    }
    return f;
}

bool finite_bf16(const uint16_t* w, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if ((w[i] & 0x7f80u) == 0x7f80u) return false;
    return true;
}

template <typename T>
int alloc(T** p, size_t bytes) {
    if (!bytes) return K3X_OK;
    if (hipMalloc((void**)p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    return K3X_OK;
}

void free_all(k3x_hip_official* o) {
    for (void* p : {(void*)o->routed_down, (void*)o->routed_up, (void*)o->shared_gu,
                    (void*)o->shared_dn, (void*)o->routed_norm, (void*)o->residual_norm,
                    (void*)o->residual_proj, (void*)o->post_norm, (void*)o->router,
                    (void*)o->router_wp, (void*)o->correction, o->scratch, (void*)o->xp})
        if (p) (void)hipFree(p);
    if (o->fork_ev) (void)hipEventDestroy(o->fork_ev);
    if (o->join_ev) (void)hipEventDestroy(o->join_ev);
    if (o->latent_ev) (void)hipEventDestroy(o->latent_ev);
}

// Work of an earlier call may still use the per-call buffers on either stream.
int drain(k3x_hip_official* o) {
    k3x_hip_ctx* ctx = o->ctx;
    if (hipStreamSynchronize(ctx->stream) != hipSuccess ||
        (ctx->side_stream && hipStreamSynchronize(ctx->side_stream) != hipSuccess))
        return K3X_ERR_BACKEND_UNAVAILABLE;
    return K3X_OK;
}

// Router logits of hidden [T][H]: on the matrix cores through the
// residue-major copies from router_uses_mfma rows on, else the vector kernels
// (the same canonical fp64 logits either way).
int route_logits(k3x_hip_official* o, const uint16_t* hidden, uint32_t T, float* logits) {
    k3x_hip_ctx* ctx = o->ctx;
    const bool mfma = o->router_wp && k3x_hip::router_uses_mfma(o->H, T);
    if (mfma) {
        const size_t need = k3x_hip::router_xp_bytes(T);
        if (need > o->xp_bytes) {
            if (drain(o)) return K3X_ERR_BACKEND_UNAVAILABLE;
            if (o->xp) (void)hipFree(o->xp);
            o->xp = nullptr;
            o->xp_bytes = 0;
            if (alloc(&o->xp, need)) return K3X_ERR_BACKEND_UNAVAILABLE;
            o->xp_bytes = need;
        }
    }
    return k3x_hip::launch_router_logits(ctx, o->router, mfma ? o->router_wp : nullptr, hidden,
                                         o->xp, o->E, o->H, T, logits);
}

int permute(k3x_hip_official* o) {
    return o->router_wp ? k3x_hip::permute_router_matrix(o->ctx, o->router, o->E, o->H, o->router_wp)
                        : K3X_OK;
}

// Upload of a host bf16 matrix [rows][cols] into tiles (matrix `which` of S).
int upload_matrix(k3x_hip_official* o, const uint16_t* host, uint32_t rows, uint32_t cols,
                  uint32_t S, uint32_t which, uint4* dst) {
    k3x_hip_ctx* ctx = o->ctx;
    const size_t n = (size_t)rows * cols;
    uint16_t* staging = nullptr;
    if (alloc(&staging, n * 2)) return K3X_ERR_BACKEND_UNAVAILABLE;
    int st = hipMemcpyAsync(staging, host, n * 2, hipMemcpyHostToDevice, ctx->stream) == hipSuccess
                 ? K3X_OK
                 : K3X_ERR_BACKEND_UNAVAILABLE;
    if (!st) st = k3x_hip::retile_bf16_matrix(ctx, staging, 0, 0.0f, rows, cols, S, which, dst);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) st = K3X_ERR_BACKEND_UNAVAILABLE;
    (void)hipFree(staging);
    if (!st) ctx->weight_h2d_bytes += n * 2;
    return st;
}

int upload_vector(k3x_hip_official* o, const uint16_t* host, size_t n, float* dst) {
    const std::vector<float> f = widen(host, n);
    if (hipMemcpy(dst, f.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    o->ctx->weight_h2d_bytes += n * 2;
    return K3X_OK;
}

// Per-call buffer layout of k3x_hip_official_ffn; returns bytes (base null:
// measure only).
struct FfnBuffers {
    float* logits;        // [T][E] (device route)
    uint32_t* ids;        // [T][K]
    float* contrib;       // [T][K]
    float* latent_f32;    // [T][L]
    uint16_t* latent;     // [T][L]
    uint16_t* mixed;      // [T][L]
    uint16_t* normed;     // [T][L]
    float* routed;        // [T][H]
    uint16_t* sact;       // [T][2 Is] split [hi | lo] rows
    float* shared;        // [T][H]
};

size_t carve(uint8_t* base, const k3x_hip_official* o, uint32_t T, uint32_t K, FfnBuffers* b) {
    size_t at = 0;
    auto take = [&](size_t bytes) {
        uint8_t* p = base ? base + at : nullptr;
        at += (bytes + 255) & ~(size_t)255;
        return p;
    };
    b->logits = (float*)take((size_t)T * o->E * 4);
    b->ids = (uint32_t*)take((size_t)T * K * 4);
    b->contrib = (float*)take((size_t)T * K * 4);
    b->latent_f32 = (float*)take((size_t)T * o->L * 4);
    b->latent = (uint16_t*)take((size_t)T * o->L * 2);
    b->mixed = (uint16_t*)take((size_t)T * o->L * 2);
    b->normed = (uint16_t*)take((size_t)T * o->L * 2);
    b->routed = (float*)take((size_t)T * o->H * 4);
    b->sact = (uint16_t*)take((size_t)T * std::max(o->I_s, 1u) * 4);
    b->shared = (float*)take((size_t)T * o->H * 4);
    return at;
}

int ensure(k3x_hip_official* o, size_t bytes) {
    if (bytes <= o->scratch_bytes) return K3X_OK;
    if (drain(o)) return K3X_ERR_BACKEND_UNAVAILABLE;
    if (o->scratch) (void)hipFree(o->scratch);
    o->scratch = nullptr;
    o->scratch_bytes = 0;
    const size_t rounded = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    if (alloc(&o->scratch, rounded)) return K3X_ERR_BACKEND_UNAVAILABLE;
    o->scratch_bytes = rounded;
    return K3X_OK;
}

int copy_d2d(k3x_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!dst || dst == src) return K3X_OK;
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream) == hipSuccess
               ? K3X_OK
               : K3X_ERR_BACKEND_UNAVAILABLE;
}

int launched(k3x_hip_ctx* ctx, unsigned n) {
    ctx->kernel_launches += n;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

}  // namespace

extern "C" {

int k3x_hip_official_create(k3x_hip_ctx* ctx, k3x_hip_bank* experts,
                            const k3x_hip_official_desc* desc, k3x_hip_official** out) {
    if (!ctx || !desc || !out || (experts && experts->ctx != ctx)) return K3X_ERR_INVALID_EXTENT;
    *out = nullptr;
    // Without a bank: a route-only object (prepare and its router logits).
    const uint32_t H = desc->hidden, Is = desc->shared_inter, L = experts ? experts->desc.hidden : 0;
    const uint32_t E = experts ? experts->desc.experts : desc->router_experts;
    if (!H || H % 128 || Is % 128 || L % 128 || !E) return K3X_ERR_INVALID_EXTENT;
    if (experts ? desc->router_experts && desc->router_experts != E : Is != 0)
        return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    auto* o = new (std::nothrow) k3x_hip_official();
    if (!o) return K3X_ERR_BACKEND_UNAVAILABLE;
    o->ctx = ctx;
    o->bank = experts;
    o->H = H;
    o->L = L;
    o->E = E;
    o->I_s = Is;
    int st = K3X_OK;
    st = st ? st : alloc(&o->routed_down, (size_t)L * H * 2);
    st = st ? st : alloc(&o->routed_up, (size_t)H * L * 2);
    st = st ? st : alloc(&o->shared_gu, (size_t)2 * Is * H * 2);
    st = st ? st : alloc(&o->shared_dn, (size_t)H * Is * 2);
    st = st ? st : alloc(&o->routed_norm, (size_t)L * 4);
    st = st ? st : alloc(&o->residual_norm, (size_t)H * 4);
    st = st ? st : alloc(&o->residual_proj, (size_t)H * 4);
    st = st ? st : alloc(&o->post_norm, (size_t)H * 4);
    st = st ? st : alloc(&o->router, (size_t)o->E * H * 4);
    if (k3x_hip::router_mfma_eligible(H))
        st = st ? st : alloc(&o->router_wp, k3x_hip::router_wp_floats(o->E) * 4);
    st = st ? st : alloc(&o->correction, (size_t)o->E * 4);
    if (!st && (hipEventCreateWithFlags(&o->fork_ev, hipEventDisableTiming) != hipSuccess ||
                hipEventCreateWithFlags(&o->join_ev, hipEventDisableTiming) != hipSuccess ||
                hipEventCreateWithFlags(&o->latent_ev, hipEventDisableTiming) != hipSuccess))
        st = K3X_ERR_BACKEND_UNAVAILABLE;
    if (st) {
        free_all(o);
        delete o;
        return st;
    }
    ++ctx->live_banks;  // keeps the context alive as a bank would
    *out = o;
    return K3X_OK;
}

int k3x_hip_official_destroy(k3x_hip_official* o) {
    if (!o) return K3X_ERR_INVALID_EXTENT;
    (void)hipSetDevice(o->ctx->device);
    (void)drain(o);
    free_all(o);
    --o->ctx->live_banks;
    delete o;
    return K3X_OK;
}

int k3x_hip_official_upload_ffn(k3x_hip_official* o, const uint16_t* routed_down,
                                const uint16_t* routed_norm, const uint16_t* routed_up,
                                const uint16_t* shared_gate, const uint16_t* shared_up,
                                const uint16_t* shared_down) {
    if (!o || !routed_down || !routed_norm || !routed_up) return K3X_ERR_INVALID_EXTENT;
    if (!o->bank) return K3X_ERR_INVALID_STATE;
    const size_t HL = (size_t)o->H * o->L, HS = (size_t)o->H * o->I_s;
    if (o->I_s && (!shared_gate || !shared_up || !shared_down)) return K3X_ERR_INVALID_EXTENT;
    // Validation before any device write (the reference's views are finite bf16).
    if (!finite_bf16(routed_down, HL) || !finite_bf16(routed_up, HL) ||
        !finite_bf16(routed_norm, o->L) ||
        (o->I_s && (!finite_bf16(shared_gate, HS) || !finite_bf16(shared_up, HS) ||
                    !finite_bf16(shared_down, HS))))
        return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(o->ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    o->ffn_ready = false;
    int st = upload_matrix(o, routed_down, o->L, o->H, 1, 0, o->routed_down);
    st = st ? st : upload_matrix(o, routed_up, o->H, o->L, 1, 0, o->routed_up);
    st = st ? st : upload_vector(o, routed_norm, o->L, o->routed_norm);
    if (o->I_s) {
        st = st ? st : upload_matrix(o, shared_gate, o->I_s, o->H, 2, 0, o->shared_gu);
        st = st ? st : upload_matrix(o, shared_up, o->I_s, o->H, 2, 1, o->shared_gu);
        st = st ? st : upload_matrix(o, shared_down, o->H, o->I_s, 1, 0, o->shared_dn);
    }
    if (!st) o->ffn_ready = true;
    return st;
}

int k3x_hip_official_upload_route(k3x_hip_official* o, const uint16_t* residual_norm,
                                  const uint16_t* residual_proj, const uint16_t* post_norm,
                                  const uint16_t* router, const float* correction) {
    if (!o || !residual_norm || !residual_proj || !post_norm || !router || !correction)
        return K3X_ERR_INVALID_EXTENT;
    const size_t H = o->H, EH = (size_t)o->E * o->H;
    if (!finite_bf16(residual_norm, H) || !finite_bf16(residual_proj, H) ||
        !finite_bf16(post_norm, H) || !finite_bf16(router, EH))
        return K3X_ERR_INVALID_EXTENT;
    for (uint32_t e = 0; e < o->E; ++e)
        if (!std::isfinite(correction[e])) return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(o->ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    o->route_ready = false;
    int st = upload_vector(o, residual_norm, H, o->residual_norm);
    st = st ? st : upload_vector(o, residual_proj, H, o->residual_proj);
    st = st ? st : upload_vector(o, post_norm, H, o->post_norm);
    st = st ? st : upload_vector(o, router, EH, o->router);
    if (!st && hipMemcpy(o->correction, correction, (size_t)o->E * 4, hipMemcpyHostToDevice) !=
                   hipSuccess)
        st = K3X_ERR_BACKEND_UNAVAILABLE;
    st = st ? st : permute(o);
    if (hipStreamSynchronize(o->ctx->stream) != hipSuccess) st = K3X_ERR_BACKEND_UNAVAILABLE;
    if (!st) o->route_ready = true;
    return st;
}

int k3x_hip_official_fill_synthetic(k3x_hip_official* o, uint64_t seed, float sigma,
                                    float router_sigma, float proj_sigma,
                                    float correction_sigma) {
    if (!o) return K3X_ERR_INVALID_EXTENT;
    k3x_hip_ctx* ctx = o->ctx;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    auto key = [&](uint64_t stream) { return stream_key(seed, stream << 32); };
    // Streams of this generator: 1..4 dense, 5..7 vectors, 8 router, 9 correction.
    int st = K3X_OK;
    if (o->bank) {
        st = k3x_hip::retile_bf16_matrix(ctx, nullptr, key(1), sigma, o->L, o->H, 1, 0,
                                         o->routed_down);
        st = st ? st : k3x_hip::retile_bf16_matrix(ctx, nullptr, key(2), sigma, o->H, o->L, 1, 0,
                                                   o->routed_up);
        st = st ? st : k3x_hip::fill_const_f32_dev(ctx, o->L, 1.0f, o->routed_norm);
    }
    if (o->I_s) {
        st = st ? st : k3x_hip::retile_bf16_matrix(ctx, nullptr, key(3), sigma, o->I_s, o->H, 2,
                                                   0, o->shared_gu);
        st = st ? st : k3x_hip::retile_bf16_matrix(ctx, nullptr, key(4), sigma, o->I_s, o->H, 2,
                                                   1, o->shared_gu);
        st = st ? st : k3x_hip::retile_bf16_matrix(ctx, nullptr, key(5), sigma, o->H, o->I_s, 1,
                                                   0, o->shared_dn);
    }
    st = st ? st : k3x_hip::fill_const_f32_dev(ctx, o->H, 1.0f, o->residual_norm);
    st = st ? st : k3x_hip::fill_const_f32_dev(ctx, o->H, 1.0f, o->post_norm);
    st = st ? st : k3x_hip::fill_normal_f32_dev(ctx, key(6), o->H, proj_sigma, o->residual_proj);
    st = st ? st : k3x_hip::fill_normal_f32_dev(ctx, key(8), (size_t)o->E * o->H, router_sigma,
                                                 o->router);
    st = st ? st : k3x_hip::fill_normal_f32_dev(ctx, key(9), o->E, correction_sigma,
                                                 o->correction);
    // The router and residual_proj hold bf16 values in this layer.
    if (!st) {
        const size_t eh = (size_t)o->E * o->H;
        hipLaunchKernelGGL(round_in_place_kernel, dim3(blocks_for(eh)), dim3(kThreads), 0,
                           ctx->stream, o->router, eh);
        hipLaunchKernelGGL(round_in_place_kernel, dim3(blocks_for(o->H)), dim3(kThreads), 0,
                           ctx->stream, o->residual_proj, (size_t)o->H);
        st = launched(ctx, 2);
    }
    st = st ? st : permute(o);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) st = K3X_ERR_BACKEND_UNAVAILABLE;
    if (!st) {
        o->ffn_ready = o->bank != nullptr;
        o->route_ready = true;
    }
    return st;
}

int k3x_hip_official_prepare(k3x_hip_ctx* ctx, k3x_hip_official* o, uint32_t T, float eps,
                             const float* prefix, const float* block_residual, uint16_t* hidden,
                             float* logits) {
    if (!ctx || !o || o->ctx != ctx || !prefix || !block_residual || !hidden || !T)
        return K3X_ERR_INVALID_EXTENT;
    if (!std::isfinite(eps) || !(eps > 0.0f)) return K3X_ERR_INVALID_EXTENT;
    if (!o->route_ready) return K3X_ERR_INVALID_STATE;
    if (o->H > kPrepRegHidden && (size_t)o->H * 4 > ctx->max_lds_per_block)
        return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    if (o->H <= kPrepRegHidden && T <= kPrepWideTokens)
        hipLaunchKernelGGL(official_prepare_tpb_kernel<1024>, dim3(T), dim3(1024), 0, ctx->stream,
                           prefix, block_residual, o->residual_norm, o->residual_proj,
                           o->post_norm, o->H, eps, hidden, ctx->status);
    else if (o->H <= kPrepRegHidden)
        hipLaunchKernelGGL(official_prepare_reg_kernel, dim3(T), dim3(kThreads), 0, ctx->stream,
                           prefix, block_residual, o->residual_norm, o->residual_proj,
                           o->post_norm, o->H, eps, hidden, ctx->status);
    else
        hipLaunchKernelGGL(official_prepare_kernel, dim3(T), dim3(kThreads), (size_t)o->H * 4,
                           ctx->stream, prefix, block_residual, o->residual_norm,
                           o->residual_proj, o->post_norm, o->H, eps, hidden, ctx->status);
    int st = launched(ctx, 1);
    if (!st && logits) st = route_logits(o, hidden, T, logits);
    return st;
}

int k3x_hip_official_ffn(k3x_hip_ctx* ctx, k3x_hip_official* o, const k3x_hip_moe_params* p,
                         const uint16_t* hidden, const float* prefix, const uint32_t* ids,
                         const float* contributions, uint16_t* out,
                         const k3x_hip_official_taps* taps) {
    if (!ctx || !o || o->ctx != ctx || !p || !hidden || !prefix || !out)
        return K3X_ERR_INVALID_EXTENT;
    if ((ids == nullptr) != (contributions == nullptr)) return K3X_ERR_INVALID_EXTENT;
    const uint32_t T = p->tokens, K = p->top_k;
    if (!T || !K || K > 64 || K > o->E) return K3X_ERR_INVALID_EXTENT;
    if (!std::isfinite(p->rms_epsilon) || !(p->rms_epsilon > 0.0f)) return K3X_ERR_INVALID_EXTENT;
    if (!o->ffn_ready || (!ids && !o->route_ready)) return K3X_ERR_INVALID_STATE;
    // A route found on the device may pick any expert of the bank; a given
    // route needs only its own slots admitted (checked by the grouping).
    if (!ids)
        for (uint8_t r : o->bank->expert_ready)
            if (!r) return K3X_ERR_INVALID_STATE;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    FfnBuffers b;
    int st = ensure(o, carve(nullptr, o, T, K, &b));
    if (st) return st;
    carve(static_cast<uint8_t*>(o->scratch), o, T, K, &b);
    // Experts on the latent: the bank's grouped path with fp32 activations
    // into the down projection, each expert output rounded to bf16 before the
    // slot-ordered mix, the mix rounded (official_moe.cpp:82-103, :313-326).
    k3x_hip_moe_params ep = *p;
    ep.routed_scale = 1.0f;
    ep.renorm = K3X_RENORM_DOUBLE;
    ep.flags = K3X_FLAG_ROUND_EXPERT_OUT | K3X_FLAG_SPLIT_ACT;
    k3x_hip::LayerBuffers rs;
    // Its scratch is carved (and grown) before any launch of this call.
    if ((st = k3x_hip::routed_begin(ctx, o->bank, &ep, &rs))) return st;
    const GluParams glu{(int)p->glu, p->situ_beta, (int)p->has_situ_linear, p->situ_linear_beta};
    // Shared FFN on hidden (official_moe.cpp:105-117, :307): on the side
    // stream beside the route and the experts (few rows: the routed kernels
    // leave the device half idle; many rows: the latency-bound route steps
    // and the experts' tails do), joined before the output; in line when
    // its projections cannot leave the context stream.
    // Few tokens with the route found here: the route, the latent projection
    // and the shared FFN in two launches on the context stream (the
    // projections' workgroups beside the route's), no second stream.
    const bool fused = !ids && o->bank->desc.experts == o->E &&
                       k3x_hip::official_decode_eligible(o->E, o->H, o->L, o->I_s, K, T);
    const bool side = !fused && o->I_s && ctx->side_stream && !ctx->profiling &&
                      k3x_hip::dense_mlp_any_stream(o->I_s, o->H, T);
    // The latent projection needs hidden only: with the route found here it
    // goes first on the side stream, beside the route's latency-bound
    // launches, and the experts wait for it alone.
    const bool latent_side = !fused && !ids && ctx->side_stream && !ctx->profiling &&
                             k3x_hip::dense_down_any_stream(o->L, o->H, T);
    struct Join {
        k3x_hip_official* o;
        bool armed = false;
        int join() {
            if (!armed) return K3X_OK;
            armed = false;
            return hipStreamWaitEvent(o->ctx->stream, o->join_ev, 0) == hipSuccess
                       ? K3X_OK
                       : K3X_ERR_BACKEND_UNAVAILABLE;
        }
        ~Join() { (void)join(); }
    } joiner{o};
    // The shared gate and up are bf16 projections (rounded before the GLU)
    // and the activation enters the down projection at fp32 precision, as a
    // split [hi | lo] row.
    GluParams sglu = glu;
    sglu.round_in = 1;
    auto shared_ffn = [&](hipStream_t stream) {
        int r = k3x_hip::dense_gate_up(ctx, o->shared_gu, o->I_s, o->H, hidden, T, sglu, b.sact,
                                       stream, true);
        return r ? r : k3x_hip::dense_down(ctx, o->shared_dn, o->H, o->I_s, b.sact, T, b.shared,
                                           stream, nullptr, true);
    };
    // latent = bf16(routed_down . hidden) (official_moe.cpp:305); few rows
    // round in the GEMV's own epilogue.
    auto latent = [&](hipStream_t stream) {
        if (T <= k3x_hip::kDenseDirectTokens)
            return k3x_hip::dense_down(ctx, o->routed_down, o->L, o->H, hidden, T, nullptr, stream,
                                       b.latent);
        const int r = k3x_hip::dense_down(ctx, o->routed_down, o->L, o->H, hidden, T,
                                          b.latent_f32, stream);
        if (r) return r;
        hipLaunchKernelGGL(round_bf16_kernel, dim3(blocks_for((size_t)T * o->L)), dim3(kThreads),
                           0, stream, b.latent_f32, (size_t)T * o->L, b.latent);
        return launched(ctx, 1);
    };
    if (side || latent_side) {
        if (hipEventRecord(o->fork_ev, ctx->stream) != hipSuccess ||
            hipStreamWaitEvent(ctx->side_stream, o->fork_ev, 0) != hipSuccess)
            return K3X_ERR_BACKEND_UNAVAILABLE;
        int sst = latent_side ? latent(ctx->side_stream) : K3X_OK;
        if (!sst && latent_side && hipEventRecord(o->latent_ev, ctx->side_stream) != hipSuccess)
            sst = K3X_ERR_BACKEND_UNAVAILABLE;
        if (!sst && side) sst = shared_ffn(ctx->side_stream);
        if (hipEventRecord(o->join_ev, ctx->side_stream) != hipSuccess) {
            (void)hipStreamSynchronize(ctx->side_stream);
            return K3X_ERR_BACKEND_UNAVAILABLE;
        }
        joiner.armed = true;
        if (sst) return sst;
    }
    // Route (official_moe.cpp:211-269): logits over hidden, sigmoid +
    // correction, natural Top-K, contributions s / sum s in double.
    if (fused) {
        const k3x_hip::OfficialDecode od{o->router,      o->correction, o->E,       o->H,
                                         o->L,           o->I_s,        K,          T,
                                         hidden,         o->routed_down, b.latent,  o->shared_gu,
                                         o->shared_dn,   sglu,          b.sact,     b.shared,
                                         b.logits,       b.ids,         b.contrib,
                                         o->bank->ready_dev};
        st = k3x_hip::launch_official_front(ctx, od);
        st = st ? st : k3x_hip::launch_official_select(ctx, od, rs);
        if (st) return st;
        rs.grouped = true;
        ids = b.ids;
        contributions = b.contrib;
    } else if (!ids) {
        // Few pairs: the Top-K groups the route into the routed call's
        // buffers in the same launch (the routed call skips its grouping).
        rs.grouped = o->bank->desc.experts == o->E && k3x_hip::topk_group_eligible(o->E, K, T);
        st = route_logits(o, hidden, T, b.logits);
        if (rs.grouped)
            st = st ? st : k3x_hip::launch_topk_group(ctx, b.logits, o->correction, o->E, K, T,
                                                      1.0f, K3X_RENORM_DOUBLE, b.ids, b.contrib,
                                                      o->bank->ready_dev, rs);
        else
            st = st ? st : k3x_hip::launch_topk(ctx, b.logits, o->correction, o->E, K, T, 1.0f,
                                                K3X_RENORM_DOUBLE, b.ids, b.contrib);
        if (st) return st;
        ids = b.ids;
        contributions = b.contrib;
    }
    if (latent_side) {
        if (hipStreamWaitEvent(ctx->stream, o->latent_ev, 0) != hipSuccess)
            return K3X_ERR_BACKEND_UNAVAILABLE;
    } else if (!fused && (st = latent(ctx->stream))) {
        return st;
    }
    k3x_hip_moe_taps et{};
    if (taps) et.expert_out = taps->expert_out;
    st = k3x_hip::routed_finish(ctx, o->bank, &ep, rs, b.latent, ids, contributions, b.mixed,
                                taps ? &et : nullptr);
    if (st) return st;
    // routed = routed_up . RMSNorm(mixed, routed_norm) (official_moe.cpp:327-333).
    // Up to four tokens, one launch: every routed_up workgroup normalises the
    // mixed rows itself.
    const bool norm_out = k3x_hip::dense_norm_output_ok(o->H, o->L, T) &&
                          reinterpret_cast<uintptr_t>(b.mixed) % 16 == 0 &&
                          reinterpret_cast<uintptr_t>(o->routed_norm) % 16 == 0;
    if (!norm_out)
        st = k3x_hip::launch_rmsnorm(ctx, b.mixed, o->routed_norm, T, o->L, p->rms_epsilon,
                                     b.normed);
    const size_t n = (size_t)T * o->H;
    if (norm_out) {
        if (!st && o->I_s && !side && !fused) st = shared_ffn(ctx->stream);
        st = st ? st : joiner.join();
        st = st ? st : k3x_hip::dense_norm_output(ctx, o->routed_up, o->H, o->L, b.mixed,
                                                  o->routed_norm, p->rms_epsilon, T, prefix,
                                                  o->I_s ? b.shared : nullptr, b.routed, out);
        if (st) return st;
    } else if (T <= k3x_hip::kDenseDirectTokens) {
        // Few rows: the output formula in the routed_up GEMV's epilogue, after
        // the shared FFN (long finished on the side stream by now).
        if (!st && o->I_s && !side && !fused) st = shared_ffn(ctx->stream);
        st = st ? st : joiner.join();
        st = st ? st : k3x_hip::dense_down_output(ctx, o->routed_up, o->H, o->L, b.normed, T,
                                                  prefix, o->I_s ? b.shared : nullptr, b.routed,
                                                  out);
        if (st) return st;
    } else {
        st = st ? st : k3x_hip::dense_down(ctx, o->routed_up, o->H, o->L, b.normed, T, b.routed,
                                           ctx->stream);
        if (!st && o->I_s && !side && !fused) st = shared_ffn(ctx->stream);
        st = st ? st : joiner.join();
        if (st) return st;
        const bool vec = n % 4 == 0 && reinterpret_cast<uintptr_t>(prefix) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(out) % 8 == 0;
        if (vec)
            hipLaunchKernelGGL(official_out_kernel<4>, dim3(blocks_for(n / 4)), dim3(kThreads), 0,
                               ctx->stream, prefix, b.routed, o->I_s ? b.shared : nullptr, n, out,
                               ctx->status);
        else
            hipLaunchKernelGGL(official_out_kernel<1>, dim3(blocks_for(n)), dim3(kThreads), 0,
                               ctx->stream, prefix, b.routed, o->I_s ? b.shared : nullptr, n, out,
                               ctx->status);
        if ((st = launched(ctx, 1))) return st;
    }
    if (taps) {
        st = copy_d2d(ctx, taps->ids, ids, (size_t)T * K * 4);
        st = st ? st : copy_d2d(ctx, taps->contributions, contributions, (size_t)T * K * 4);
        if (!st && taps->logits && ids == b.ids)
            st = copy_d2d(ctx, taps->logits, b.logits, (size_t)T * o->E * 4);
        st = st ? st : copy_d2d(ctx, taps->latent, b.latent, (size_t)T * o->L * 2);
        st = st ? st : copy_d2d(ctx, taps->mixed, b.mixed, (size_t)T * o->L * 2);
        st = st ? st : copy_d2d(ctx, taps->routed, b.routed, n * 4);
        if (!st && taps->shared) {
            st = o->I_s ? copy_d2d(ctx, taps->shared, b.shared, n * 4)
                        : k3x_hip::fill_const_f32_dev(ctx, n, 0.0f, taps->shared);
        }
    }
    return st;
}

}  // extern "C"
