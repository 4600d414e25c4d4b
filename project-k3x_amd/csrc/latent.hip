// latent.hip -- the fp32 side of the backend interface: dense fp32 and
// row-major MXFP4 matrix-vector products with double accumulation, the fp32
// SiTU MLP, and the resident latent MoE layer
// (runtime/src/backend_cpu.cpp:22-122, :305-339) around the bank's grouped
// expert path.
//
// Every product here is HBM-bound (one token, or a few, per weight byte), so
// the kernels stream each weight row once with 16-byte loads per lane and
// keep the reference's arithmetic: each product formed exactly in double
// (fp32 x fp32, or fp32 x an MXFP4 value of two significant bits) and summed
// in double, one rounding to fp32 at the end.  Only the summation order
// differs from the reference's sequential loop (a lane-strided sum and a
// butterfly), which moves the double sum by a few units in its last place,
// far below the fp32 rounding that follows.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "k3x_device.hpp"
#include "k3x_internal.hpp"

using namespace k3x_dev;

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr uint32_t kMaxTokens = 4;  // tokens per weight pass

__device__ inline double wave_sum(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ inline float situ(float g, float u, float beta, int has_linear, float linear) {
    // runtime/src/ops.cpp:20-30 in fp32 with the library's expf / tanhf.
    const float sig = 1.0f / (1.0f + expf(-g));
    const float bg = beta * tanhf(g / beta) * sig;
    const float bu = has_linear ? linear * tanhf(u / linear) : u;
    return bg * bu;
}

// One output row per wave, T <= kMaxTokens tokens per pass (x rows
// [T][x_stride]); VEC: 16-byte loads (cols % 4 == 0, rows 16-byte aligned).
// OUT: 0 y = Wx; 1 y = Wx + add (fp32 add, as routed[row] += shared[row]);
// 2 y = Wx and the split copy ys = [bf16 hi | bf16 lo] rows of 2 rows_total;
// 3 y = situ(W x, W2 x) (the gate / up pair of an MLP).
struct GemvArgs {
    const float* W;
    const float* W2;      // OUT 3: the up matrix
    uint32_t rows, cols;
    const float* x;
    uint32_t x_stride;
    uint32_t T;
    float* y;
    uint32_t y_stride;
    const float* add;     // OUT 1, [T][y_stride]
    uint16_t* ys;         // OUT 2, [T][2 * y_stride]
    float beta, linear;
    int has_linear;
    const uint32_t* status;
};

template <int OUT, bool VEC>
__global__ __launch_bounds__(kThreads) void f32_gemv_kernel(GemvArgs a) {
    if (*(volatile const uint32_t*)a.status) return;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t r = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (r >= a.rows) return;
    constexpr int M = OUT == 3 ? 2 : 1;
    const float* wr[M];
    wr[0] = a.W + (size_t)r * a.cols;
    if constexpr (M == 2) wr[1] = a.W2 + (size_t)r * a.cols;
    for (uint32_t t0 = 0; t0 < a.T; t0 += kMaxTokens) {
        const uint32_t nt = min(a.T - t0, kMaxTokens);
        double acc[M][kMaxTokens];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (uint32_t t = 0; t < kMaxTokens; ++t) acc[m][t] = 0.0;
        if constexpr (VEC) {
            // Four 16-byte loads per lane in flight (4 KiB per wave).
            constexpr uint32_t kStep = 64 * 4 * 4;
            for (uint32_t c0 = 0; c0 < a.cols; c0 += kStep) {
                float4 w[M][4];
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t c = c0 + (q * 64 + lane) * 4;
                        w[m][q] = c < a.cols ? *reinterpret_cast<const float4*>(wr[m] + c)
                                             : make_float4(0.f, 0.f, 0.f, 0.f);
                    }
#pragma unroll
                for (uint32_t t = 0; t < kMaxTokens; ++t) {
                    if (t >= nt) break;
                    const float* xr = a.x + (size_t)(t0 + t) * a.x_stride;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t c = c0 + (q * 64 + lane) * 4;
                        if (c >= a.cols) continue;
                        const float4 xv = *reinterpret_cast<const float4*>(xr + c);
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            acc[m][t] = __builtin_fma((double)w[m][q].x, (double)xv.x, acc[m][t]);
                            acc[m][t] = __builtin_fma((double)w[m][q].y, (double)xv.y, acc[m][t]);
                            acc[m][t] = __builtin_fma((double)w[m][q].z, (double)xv.z, acc[m][t]);
                            acc[m][t] = __builtin_fma((double)w[m][q].w, (double)xv.w, acc[m][t]);
                        }
                    }
                }
            }
        } else {
            for (uint32_t c = lane; c < a.cols; c += 64) {
                float w[M];
#pragma unroll
                for (int m = 0; m < M; ++m) w[m] = wr[m][c];
#pragma unroll
                for (uint32_t t = 0; t < kMaxTokens; ++t) {
                    if (t >= nt) break;
                    const double xv = (double)a.x[(size_t)(t0 + t) * a.x_stride + c];
#pragma unroll
                    for (int m = 0; m < M; ++m)
                        acc[m][t] = __builtin_fma((double)w[m], xv, acc[m][t]);
                }
            }
        }
#pragma unroll
        for (uint32_t t = 0; t < kMaxTokens; ++t) {
            if (t >= nt) break;
            float v[M];
#pragma unroll
            for (int m = 0; m < M; ++m) v[m] = (float)wave_sum(acc[m][t]);
            if (lane != 0) continue;
            const size_t at = (size_t)(t0 + t) * a.y_stride + r;
            if constexpr (OUT == 0) {
                a.y[at] = v[0];
            } else if constexpr (OUT == 1) {
                a.y[at] = __fadd_rn(a.add[at], v[0]);
            } else if constexpr (OUT == 2) {
                a.y[at] = v[0];
                const uint16_t hi = f32_to_bf16(v[0]);
                uint16_t* ys = a.ys + (size_t)(t0 + t) * 2 * a.y_stride;
                ys[r] = hi;
                ys[a.y_stride + r] = act_lo_bf16(v[0], hi);
            } else {
                a.y[at] = situ(v[0], v[M - 1], a.beta, a.has_linear, a.linear);
            }
        }
    }
}

// One MXFP4 row per wave in the K3X layout (packed [rows][cols / 2], low
// nibble = even column; E8M0 scales [rows][cols / 32]); lane l takes the
// 32-element groups l, l + 64, ...  The 32 products of a group are exact in
// fp32 only up to their alignment, so each one is formed in double
// (runtime/src/ops.cpp:57-76).
__global__ __launch_bounds__(kThreads) void mxfp4_gemv_kernel(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ scales, uint32_t rows,
    uint32_t cols, const float* __restrict__ x, uint32_t T, float* __restrict__ y,
    const uint32_t* status) {
    if (*(volatile const uint32_t*)status) return;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t r = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (r >= rows) return;
    const uint32_t groups = cols / 32;
    const uint4* pr = reinterpret_cast<const uint4*>(packed + (size_t)r * cols / 2);
    const uint8_t* sr = scales + (size_t)r * groups;
    for (uint32_t t0 = 0; t0 < T; t0 += kMaxTokens) {
        const uint32_t nt = min(T - t0, kMaxTokens);
        double acc[kMaxTokens];
#pragma unroll
        for (uint32_t t = 0; t < kMaxTokens; ++t) acc[t] = 0.0;
        for (uint32_t gi = lane; gi < groups; gi += 64) {
            const uint4 c = pr[gi];
            const float sc = e8m0_to_f32(sr[gi]);
            const uint32_t words[4] = {c.x, c.y, c.z, c.w};
            float wv[32];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // Eight bf16 values, element 2i in the low half of dword i.
                const uint4 d = __builtin_bit_cast(uint4, dequant8(words[j], sc));
                const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    wv[8 * j + 2 * i] = __uint_as_float(dw[i] << 16);
                    wv[8 * j + 2 * i + 1] = __uint_as_float(dw[i] & 0xffff0000u);
                }
            }
#pragma unroll
            for (uint32_t t = 0; t < kMaxTokens; ++t) {
                if (t >= nt) break;
                const float4* xr =
                    reinterpret_cast<const float4*>(x + (size_t)(t0 + t) * cols + (size_t)gi * 32);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 xv = xr[q];
                    acc[t] = __builtin_fma((double)wv[4 * q + 0], (double)xv.x, acc[t]);
                    acc[t] = __builtin_fma((double)wv[4 * q + 1], (double)xv.y, acc[t]);
                    acc[t] = __builtin_fma((double)wv[4 * q + 2], (double)xv.z, acc[t]);
                    acc[t] = __builtin_fma((double)wv[4 * q + 3], (double)xv.w, acc[t]);
                }
            }
        }
#pragma unroll
        for (uint32_t t = 0; t < kMaxTokens; ++t) {
            if (t >= nt) break;
            const float v = (float)wave_sum(acc[t]);
            if (lane == 0) y[(size_t)(t0 + t) * rows + r] = v;
        }
    }
}

// RMSNorm of fp32 rows (runtime/src/ops.cpp:10-18): double sum of squares,
// inverse = 1 / sqrt(float(sum / n) + eps) in fp32, out = x * inverse * w.
__global__ __launch_bounds__(kThreads) void rmsnorm_f32_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ w,
                                                               uint32_t n, uint32_t n_div,
                                                               float eps,
                                                               float* __restrict__ out,
                                                               const uint32_t* status) {
    __shared__ double part[kWaves];
    if (*(volatile const uint32_t*)status) return;
    const float* xr = x + (size_t)blockIdx.x * n;
    double sq = 0.0;
    for (uint32_t i = threadIdx.x; i < n; i += kThreads) sq = __builtin_fma((double)xr[i], (double)xr[i], sq);
    sq = wave_sum(sq);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sq;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) tot += part[i];
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn((float)(tot / (double)n_div), eps)));
    float* orow = out + (size_t)blockIdx.x * n;
    for (uint32_t i = threadIdx.x; i < n; i += kThreads)
        orow[i] = __fmul_rn(__fmul_rn(xr[i], inv), w[i]);
}

int launched(k3x_hip_ctx* ctx, unsigned n) {
    ctx->kernel_launches += n;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <int OUT>
int launch_gemv(k3x_hip_ctx* ctx, GemvArgs a, hipStream_t stream) {
    const bool vec = a.cols % 4 == 0 && aligned16(a.W) && aligned16(a.x) && a.x_stride % 4 == 0 &&
                     (OUT != 3 || aligned16(a.W2));
    const dim3 grid((a.rows + kWaves - 1) / kWaves);
    a.status = ctx->status;
    if (vec)
        hipLaunchKernelGGL((f32_gemv_kernel<OUT, true>), grid, dim3(kThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((f32_gemv_kernel<OUT, false>), grid, dim3(kThreads), 0, stream, a);
    return launched(ctx, 1);
}

bool dims_ok(uint32_t rows, uint32_t cols, uint32_t T) {
    return rows && cols && T && rows <= (1u << 24) && cols <= (1u << 24) && T <= (1u << 16);
}

// Device scratch of the latent layer, grow-only, apart from the layer
// scratch the grouped expert call carves.
int ensure_latent(k3x_hip_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->latent_bytes) return K3X_OK;
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    if (ctx->latent_scratch) (void)hipFree(ctx->latent_scratch);
    ctx->latent_scratch = nullptr;
    ctx->latent_bytes = 0;
    const size_t rounded = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    if (hipMalloc(&ctx->latent_scratch, rounded) != hipSuccess) {
        (void)hipGetLastError();
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    ctx->latent_bytes = rounded;
    return K3X_OK;
}

}  // namespace

extern "C" {

int k3x_hip_dense_f32_matvec(k3x_hip_ctx* ctx, const float* W, uint32_t rows, uint32_t cols,
                             const float* x, uint32_t tokens, float* y) {
    if (!ctx || !W || !x || !y || !dims_ok(rows, cols, tokens)) return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    GemvArgs a{};
    a.W = W;
    a.rows = rows;
    a.cols = cols;
    a.x = x;
    a.x_stride = cols;
    a.T = tokens;
    a.y = y;
    a.y_stride = rows;
    return launch_gemv<0>(ctx, a, ctx->stream);
}

int k3x_hip_mxfp4_matvec(k3x_hip_ctx* ctx, const uint8_t* packed, const uint8_t* scales,
                         uint32_t rows, uint32_t cols, const float* x, uint32_t tokens, float* y) {
    if (!ctx || !packed || !scales || !x || !y || !dims_ok(rows, cols, tokens) || cols % 32)
        return K3X_ERR_INVALID_EXTENT;
    if (!aligned16(packed) || !aligned16(x)) return K3X_ERR_INVALID_EXTENT;  // 16-byte loads
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    hipLaunchKernelGGL(mxfp4_gemv_kernel, dim3((rows + kWaves - 1) / kWaves), dim3(kThreads), 0,
                       ctx->stream, packed, scales, rows, cols, x, tokens, y, ctx->status);
    return launched(ctx, 1);
}

int k3x_hip_dense_situ_mlp(k3x_hip_ctx* ctx, const float* gate, const float* up,
                           const float* down, uint32_t hidden, uint32_t inter, uint32_t out_rows,
                           float situ_beta, int has_situ_linear, float situ_linear_beta,
                           const float* x, uint32_t tokens, float* act, float* y) {
    if (!ctx || !gate || !up || !down || !x || !act || !y || !dims_ok(inter, hidden, tokens) ||
        !dims_ok(out_rows, inter, tokens))
        return K3X_ERR_INVALID_EXTENT;
    // The betas are used as given, as situ_glu does (no checks there).
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    GemvArgs g{};
    g.W = gate;
    g.W2 = up;
    g.rows = inter;
    g.cols = hidden;
    g.x = x;
    g.x_stride = hidden;
    g.T = tokens;
    g.y = act;
    g.y_stride = inter;
    g.beta = situ_beta;
    g.has_linear = has_situ_linear != 0;
    g.linear = situ_linear_beta;
    int st = launch_gemv<3>(ctx, g, ctx->stream);
    if (st) return st;
    GemvArgs d{};
    d.W = down;
    d.rows = out_rows;
    d.cols = inter;
    d.x = act;
    d.x_stride = inter;
    d.T = tokens;
    d.y = y;
    d.y_stride = out_rows;
    return launch_gemv<0>(ctx, d, ctx->stream);
}

int k3x_hip_resident_moe_layer(k3x_hip_ctx* ctx, k3x_hip_bank* bank,
                               const k3x_hip_latent_weights* w, const k3x_hip_moe_params* p,
                               const float* x, const uint32_t* ids, const float* contributions,
                               const uint32_t* host_ids, const float* host_contributions,
                               float* out, float* mixed_out) {
    if (!ctx || !bank || !w || !p || !x || !ids || !contributions || !out || bank->ctx != ctx)
        return K3X_ERR_INVALID_EXTENT;
    const uint32_t H = w->hidden, L = w->latent, S = w->shared_inter, T = p->tokens;
    const uint32_t Ln = w->latent_norm ? w->latent_norm : L;  // RMSNorm divisor
    if (!w->routed_down || !w->routed_norm || !w->routed_up || !w->shared_gate ||
        !w->shared_up || !w->shared_down || !dims_ok(L, H, T) || !dims_ok(S, H, T) ||
        bank->desc.hidden != L || bank->desc.shared_inter != 0 || p->flags || Ln > L)
        return K3X_ERR_INVALID_EXTENT;
    if (p->glu != K3X_GLU_SITU || !std::isfinite(p->rms_epsilon) || !(p->rms_epsilon > 0.0f))
        return K3X_ERR_INVALID_MXFP4;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    // Per-call buffers: latent [T][L] fp32 and its split bf16 rows [T][2 L],
    // the expert mix [T][L] fp32 (+ its bf16 cast), its RMSNorm [T][L], the
    // routed projection [T][H] and the shared activation [T][S].
    const size_t f_lat = (size_t)T * L * 4, f_hid = (size_t)T * H * 4, f_sh = (size_t)T * S * 4;
    auto up256 = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t need = up256(f_lat) * 3 + up256(f_lat) + up256((size_t)T * L * 2) +
                        up256(f_hid) + up256(f_sh);
    int st = ensure_latent(ctx, need);
    if (st) return st;
    uint8_t* base = static_cast<uint8_t*>(ctx->latent_scratch);
    size_t at = 0;
    auto take = [&](size_t b) {
        uint8_t* q = base + at;
        at += up256(b);
        return q;
    };
    float* latent = (float*)take(f_lat);
    uint16_t* latent_split = (uint16_t*)take(f_lat);  // [T][2 L] bf16
    float* mixed = mixed_out ? mixed_out : (float*)take(f_lat);
    float* normed = (float*)take(f_lat);
    uint16_t* mixed_bf16 = (uint16_t*)take((size_t)T * L * 2);
    float* routed = (float*)take(f_hid);
    float* sact = (float*)take(f_sh);
    // latent = routed_down . x (backend_cpu.cpp:317), with its split copy.
    GemvArgs a{};
    a.W = w->routed_down;
    a.rows = L;
    a.cols = H;
    a.x = x;
    a.x_stride = H;
    a.T = T;
    a.y = latent;
    a.y_stride = L;
    a.ys = latent_split;
    if ((st = launch_gemv<2>(ctx, a, ctx->stream))) return st;
    // The experts on the latent, mixed in slot order in fp32
    // (backend_cpu.cpp:318-325): the bank's grouped path with fp32 input and
    // activations.
    k3x_hip_moe_params ep = *p;
    ep.flags = K3X_FLAG_SPLIT_INPUT | K3X_FLAG_SPLIT_ACT;
    k3x_hip_moe_taps taps{};
    taps.out_f32 = mixed;
    if ((st = k3x_hip_moe_forward_routed(ctx, bank, &ep, latent_split, ids, contributions,
                                         host_ids, host_contributions, mixed_bf16, &taps)))
        return st;
    // normalized = rms_norm(mixed, routed_norm) (backend_cpu.cpp:327-328).
    hipLaunchKernelGGL(rmsnorm_f32_kernel, dim3(T), dim3(kThreads), 0, ctx->stream, mixed,
                       w->routed_norm, L, Ln, p->rms_epsilon, normed, ctx->status);
    if ((st = launched(ctx, 1))) return st;
    // routed = routed_up . normalized (backend_cpu.cpp:329-330).
    GemvArgs r{};
    r.W = w->routed_up;
    r.rows = H;
    r.cols = L;
    r.x = normed;
    r.x_stride = L;
    r.T = T;
    r.y = routed;
    r.y_stride = H;
    if ((st = launch_gemv<0>(ctx, r, ctx->stream))) return st;
    // shared = dense_situ_mlp(x) (backend_cpu.cpp:331-332); out = routed +
    // shared (:333-335) in the down projection's epilogue.
    GemvArgs g{};
    g.W = w->shared_gate;
    g.W2 = w->shared_up;
    g.rows = S;
    g.cols = H;
    g.x = x;
    g.x_stride = H;
    g.T = T;
    g.y = sact;
    g.y_stride = S;
    g.beta = p->situ_beta;
    g.has_linear = p->has_situ_linear != 0;
    g.linear = p->situ_linear_beta;
    if ((st = launch_gemv<3>(ctx, g, ctx->stream))) return st;
    GemvArgs d{};
    d.W = w->shared_down;
    d.rows = H;
    d.cols = S;
    d.x = sact;
    d.x_stride = S;
    d.T = T;
    d.y = out;
    d.y_stride = H;
    d.add = routed;
    return launch_gemv<1>(ctx, d, ctx->stream);
}

}  // extern "C"
