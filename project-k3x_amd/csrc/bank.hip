// bank.hip -- context, resident expert bank (tile layout, admission,
// synthetic fill, dequantised read-back).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <iterator>
#include <new>

#include "k3x_decode.hpp"
#include "k3x_device.hpp"
#include "k3x_internal.hpp"

using namespace k3x_dev;

namespace {

constexpr int kThreads = 256;

inline unsigned blocks_for(size_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

// ---------------------------------------------------------------------------
// Re-tiling kernels.  Source is either the K3X reference layout in device
// memory (src != nullptr) or the seeded generator (src == nullptr, key).
// ---------------------------------------------------------------------------

// MXFP4 codes -> tiles [rb][kt][S][64] x 16 B (S = 2 for interleaved gate/up).
__global__ void retile_fp4_codes(const uint8_t* __restrict__ src, uint64_t key,
                                 uint32_t rows, uint32_t cols, uint32_t kt,
                                 uint32_t S, uint32_t which, uint4* __restrict__ dst) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)(rows / 16) * kt * 64;
    if (t >= total) return;
    const uint32_t lane = t % 64;
    const uint32_t k = (uint32_t)((t / 64) % kt);
    const size_t rb = t / (64 * (size_t)kt);
    const size_t row = rb * 16 + (lane & 15);
    const size_t col0 = (size_t)k * 128 + 32 * (lane >> 4);
    const size_t p0 = row * (cols / 2) + col0 / 2;  // first packed byte, multiple of 16
    uint4 v;
    if (src) {
        v = *reinterpret_cast<const uint4*>(src + p0);
    } else {
        const uint64_t w0 = word_at(key, p0 >> 3);
        const uint64_t w1 = word_at(key, (p0 >> 3) + 1);
        v = make_uint4((uint32_t)w0, (uint32_t)(w0 >> 32), (uint32_t)w1, (uint32_t)(w1 >> 32));
    }
    dst[((rb * kt + k) * S + which) * 64 + lane] = v;
}

// E8M0 scales -> dwords [rb][ks][S][64]; byte b of a dword is K-tile 4q+b.
__global__ void retile_fp4_scales(const uint8_t* __restrict__ src, uint64_t key,
                                  uint32_t lo, uint32_t span, uint32_t rows,
                                  uint32_t cols, uint32_t kt, uint32_t ks, uint32_t S,
                                  uint32_t which, uint32_t* __restrict__ dst) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)(rows / 16) * ks * 64;
    if (t >= total) return;
    const uint32_t lane = t % 64;
    const uint32_t q = (uint32_t)((t / 64) % ks);
    const size_t rb = t / (64 * (size_t)ks);
    const size_t row = rb * 16 + (lane & 15);
    const uint32_t g = lane >> 4;
    const size_t blocks = cols / 32;
    uint32_t packed = 0;
    for (uint32_t b = 0; b < 4; ++b) {
        const uint32_t k = 4 * q + b;
        uint32_t s = 127;
        if (k < kt) {
            const size_t idx = row * blocks + 4 * (size_t)k + g;
            s = src ? src[idx] : lo + (uint32_t)(word_at(key, idx) % span);
        }
        packed |= s << (8 * b);
    }
    dst[((rb * ks + q) * S + which) * 64 + lane] = packed;
}

// bf16 matrix -> tiles [rb][kt][S][4][64] x 16 B (8 bf16 per lane per MFMA).
__global__ void retile_bf16(const uint16_t* __restrict__ src, uint64_t key, float sigma,
                            uint32_t rows, uint32_t cols, uint32_t kt, uint32_t S,
                            uint32_t which, uint4* __restrict__ dst) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)(rows / 16) * kt * 4 * 64;
    if (t >= total) return;
    const uint32_t lane = t % 64;
    const uint32_t j = (uint32_t)((t / 64) % 4);
    const uint32_t k = (uint32_t)((t / 256) % kt);
    const size_t rb = t / (256 * (size_t)kt);
    const size_t row = rb * 16 + (lane & 15);
    const size_t col = (size_t)k * 128 + 32 * (lane >> 4) + 8 * j;
    const size_t e0 = row * cols + col;
    uint4 v;
    if (src) {
        v = *reinterpret_cast<const uint4*>(src + e0);
    } else {
        uint32_t w[4];
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo16 = f32_to_bf16(normal_at(key, e0 + 2 * i, sigma));
            const uint32_t hi16 = f32_to_bf16(normal_at(key, e0 + 2 * i + 1, sigma));
            w[i] = lo16 | (hi16 << 16);
        }
        v = make_uint4(w[0], w[1], w[2], w[3]);
    }
    dst[(((rb * kt + k) * S + which) * 4 + j) * 64 + lane] = v;
}

__global__ void fill_normal_f32(uint64_t key, size_t n, float sigma, float* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = normal_at(key, i, sigma);
}

__global__ void fill_normal_bf16(uint64_t key, size_t n, float sigma, uint16_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(normal_at(key, i, sigma));
}

__global__ void fill_const_f32(size_t n, float v, float* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = v;
}

// Read-back of rows [row0, row0+nrows) as fp32 through dequant8, the same
// conversion the GEMM kernels feed to the MFMA.  One thread per 32-column
// block.
// Streaming read: workgroup b reads the contiguous span [b per, (b + 1) per)
// of 16-byte words, U words a thread in flight per step (indices clamped,
// so no load sits behind a branch), and every wave XORs its words into
// *fold once.  8192 workgroups of 512 threads, U = 4: the best of a sweep
// over 256..8192 workgroups and 4..16 words in flight on MI355X.  The loads
// are non-temporal (data read once, not kept in the L2 / MALL): 6.80 TB/s
// against 6.27 TB/s for plain loads on 4 GiB.
constexpr uint32_t kStreamReadBlocks = 8192, kStreamReadThreads = 512;
__global__ __launch_bounds__(kStreamReadThreads) void stream_read_kernel(
    const uint4* __restrict__ p, size_t n16, size_t per_block, uint32_t* fold) {
    constexpr int U = 4;
    const size_t b0 = (size_t)blockIdx.x * per_block;
    const size_t b1 = min(b0 + per_block, n16);
    uint32_t acc = 0;
    for (size_t i = b0 + threadIdx.x; i < b1; i += (size_t)kStreamReadThreads * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const u32x4 w = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(p + min(i + (size_t)kStreamReadThreads * u, b1 - 1)));
            v[u] = make_uint4(w[0], w[1], w[2], w[3]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (i + (size_t)kStreamReadThreads * u < b1) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) acc ^= __shfl_xor(acc, d);
    if ((threadIdx.x & 63) == 0 && acc) atomicXor(fold, acc);
}

__global__ void dequant_rows(const uint4* __restrict__ codes, const uint32_t* __restrict__ scales,
                             uint32_t cols, uint32_t kt, uint32_t ks, uint32_t S,
                             uint32_t which, uint32_t row0, uint32_t nrows,
                             float* __restrict__ out) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t blocks = cols / 32;
    if (t >= (size_t)nrows * blocks) return;
    const uint32_t r = row0 + (uint32_t)(t / blocks);
    const uint32_t b = (uint32_t)(t % blocks);
    const uint32_t rb = r / 16, n = r % 16, k = b / 4, g = b % 4;
    const uint32_t lane = n + 16 * g;
    const uint4 c = codes[((size_t)(rb * kt + k) * S + which) * 64 + lane];
    const uint32_t sw = scales[((size_t)(rb * ks + k / 4) * S + which) * 64 + lane];
    const float scale = e8m0_to_f32((sw >> (8 * (k % 4))) & 0xffu);
    const uint32_t words[4] = {c.x, c.y, c.z, c.w};
    float* dst = out + (size_t)(r - row0) * cols + 32 * (size_t)b;
    for (int j = 0; j < 4; ++j) {
        const bf16x8 v = dequant8(words[j], scale);
        for (int i = 0; i < 8; ++i) dst[8 * j + i] = (float)v[i];
    }
}

MatrixGeom geom(uint32_t rows, uint32_t cols) {
    MatrixGeom g;
    g.rows = rows;
    g.cols = cols;
    g.kt = cols / 128;
    g.ks = (g.kt + 3) / 4;
    return g;
}

int check_launch(k3x_hip_ctx* ctx, unsigned launches = 1) {
    ctx->kernel_launches += launches;
    return hipGetLastError() == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE;
}

void free_bank_memory(k3x_hip_bank* b) {
    for (void* p : {(void*)b->gu_codes, (void*)b->gu_scales, (void*)b->dn_codes,
                    (void*)b->dn_scales, (void*)b->sh_gu, (void*)b->sh_dn, (void*)b->router_w,
                    (void*)b->router_wp, (void*)b->router_bias, (void*)b->gamma,
                    (void*)b->ready_dev})
        if (p) (void)hipFree(p);
}

template <typename T>
int alloc(T** p, size_t bytes, uint64_t* total) {
    if (!bytes) return K3X_OK;
    if (hipMalloc((void**)p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    *total += bytes;
    return K3X_OK;
}

// Launches the four re-tile kernels of one routed expert.
int retile_expert(k3x_hip_bank* b, uint32_t e, const uint8_t* src[6], uint64_t seed,
                  uint32_t lo, uint32_t span) {
    k3x_hip_ctx* ctx = b->ctx;
    const MatrixGeom& G = b->gate;
    const MatrixGeom& D = b->down;
    uint4* gu = reinterpret_cast<uint4*>(b->gu_codes + e * b->gu_codes_per_expert);
    uint32_t* gus = b->gu_scales + e * b->gu_scales_per_expert;
    uint4* dn = reinterpret_cast<uint4*>(b->dn_codes + e * b->dn_codes_per_expert);
    uint32_t* dns = b->dn_scales + e * b->dn_scales_per_expert;
    const uint64_t ex = e;
    auto key = [&](uint64_t kind) { return stream_key(seed, (kind << 32) | ex); };
    const size_t gcodes = (size_t)(G.rows / 16) * G.kt * 64;
    const size_t gscales = (size_t)(G.rows / 16) * G.ks * 64;
    for (uint32_t which = 0; which < 2; ++which) {
        const uint64_t ck = which ? K3X_STREAM_UP_CODES : K3X_STREAM_GATE_CODES;
        const uint64_t sk = which ? K3X_STREAM_UP_SCALES : K3X_STREAM_GATE_SCALES;
        hipLaunchKernelGGL(retile_fp4_codes, dim3(blocks_for(gcodes)), dim3(kThreads), 0,
                           ctx->stream, src[2 * which], key(ck), G.rows, G.cols, G.kt, 2u,
                           which, gu);
        hipLaunchKernelGGL(retile_fp4_scales, dim3(blocks_for(gscales)), dim3(kThreads), 0,
                           ctx->stream, src[2 * which + 1], key(sk), lo, span, G.rows, G.cols,
                           G.kt, G.ks, 2u, which, gus);
    }
    const size_t dcodes = (size_t)(D.rows / 16) * D.kt * 64;
    const size_t dscales = (size_t)(D.rows / 16) * D.ks * 64;
    hipLaunchKernelGGL(retile_fp4_codes, dim3(blocks_for(dcodes)), dim3(kThreads), 0,
                       ctx->stream, src[4], key(K3X_STREAM_DOWN_CODES), D.rows, D.cols, D.kt,
                       1u, 0u, dn);
    hipLaunchKernelGGL(retile_fp4_scales, dim3(blocks_for(dscales)), dim3(kThreads), 0,
                       ctx->stream, src[5], key(K3X_STREAM_DOWN_SCALES), lo, span, D.rows,
                       D.cols, D.kt, D.ks, 1u, 0u, dns);
    return check_launch(ctx, 6);
}

int retile_shared(k3x_hip_bank* b, const uint16_t* src[3], uint64_t seed, float sigma) {
    k3x_hip_ctx* ctx = b->ctx;
    const MatrixGeom& G = b->sgate;
    const MatrixGeom& D = b->sdown;
    const size_t gn = (size_t)(G.rows / 16) * G.kt * 256;
    for (uint32_t which = 0; which < 2; ++which) {
        const uint64_t k = stream_key(seed, (uint64_t)(which ? K3X_STREAM_SHARED_UP
                                                             : K3X_STREAM_SHARED_GATE) << 32);
        hipLaunchKernelGGL(retile_bf16, dim3(blocks_for(gn)), dim3(kThreads), 0, ctx->stream,
                           src[which], k, sigma, G.rows, G.cols, G.kt, 2u, which,
                           reinterpret_cast<uint4*>(b->sh_gu));
    }
    const size_t dn = (size_t)(D.rows / 16) * D.kt * 256;
    const uint64_t kd = stream_key(seed, (uint64_t)K3X_STREAM_SHARED_DOWN << 32);
    hipLaunchKernelGGL(retile_bf16, dim3(blocks_for(dn)), dim3(kThreads), 0, ctx->stream,
                       src[2], kd, sigma, D.rows, D.cols, D.kt, 1u, 0u,
                       reinterpret_cast<uint4*>(b->sh_dn));
    return check_launch(ctx, 3);
}

}  // namespace

namespace k3x_hip {

int set_expert_ready(k3x_hip_bank* b, uint32_t e, bool ready) {
    b->expert_ready[e] = ready ? 1 : 0;
    return hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(b->ready_dev + e), ready ? 1 : 0, 1,
                             b->ctx->stream) == hipSuccess
               ? K3X_OK
               : K3X_ERR_BACKEND_UNAVAILABLE;
}

int retile_expert_device(k3x_hip_bank* b, uint32_t e, const uint8_t* const src[6]) {
    const uint8_t* s[6];
    for (int i = 0; i < 6; ++i) s[i] = src[i];
    return retile_expert(b, e, s, 0, 0, 1);
}

int retile_bf16_matrix(k3x_hip_ctx* ctx, const uint16_t* src, uint64_t key, float sigma,
                       uint32_t rows, uint32_t cols, uint32_t S, uint32_t which, uint4* dst) {
    const size_t n = (size_t)(rows / 16) * (cols / 128) * 256;
    hipLaunchKernelGGL(retile_bf16, dim3(blocks_for(n)), dim3(kThreads), 0, ctx->stream, src, key,
                       sigma, rows, cols, cols / 128, S, which, dst);
    return check_launch(ctx);
}

int fill_normal_f32_dev(k3x_hip_ctx* ctx, uint64_t key, size_t n, float sigma, float* out) {
    hipLaunchKernelGGL(fill_normal_f32, dim3(blocks_for(n)), dim3(kThreads), 0, ctx->stream, key, n,
                       sigma, out);
    return check_launch(ctx);
}

int fill_const_f32_dev(k3x_hip_ctx* ctx, size_t n, float v, float* out) {
    hipLaunchKernelGGL(fill_const_f32, dim3(blocks_for(n)), dim3(kThreads), 0, ctx->stream, n, v, out);
    return check_launch(ctx);
}

int ensure_scratch(k3x_hip_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->scratch_bytes) return K3X_OK;
    // The old scratch may still be read by enqueued kernels (on either stream).
    if (hipStreamSynchronize(ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->side_stream) != hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
    const size_t rounded = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    if (hipMalloc(&ctx->scratch, rounded) != hipSuccess) {
        (void)hipGetLastError();
        ctx->scratch = nullptr;
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    ctx->scratch_bytes = rounded;
    return K3X_OK;
}

namespace {

hipEvent_t take_event(k3x_hip_ctx* ctx) {
    if (!ctx->free_events.empty()) {
        hipEvent_t e = ctx->free_events.back();
        ctx->free_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

}  // namespace

// Marks kept pending before a forced read-back (bounds the event pool).
constexpr size_t kMaxPendingMarks = 1u << 16;

int begin_stage(k3x_hip_ctx* ctx, uint32_t stage) {
    if (!ctx->profiling || stage >= K3X_STAGE_COUNT) return -1;
    if (ctx->pending.size() >= kMaxPendingMarks && drain_stage_marks(ctx) != K3X_OK) return -1;
    StageMark m{stage, take_event(ctx), take_event(ctx)};
    if (!m.start || !m.stop || hipEventRecord(m.start, ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        if (m.start) ctx->free_events.push_back(m.start);
        if (m.stop) ctx->free_events.push_back(m.stop);
        return -1;
    }
    ctx->pending.push_back(m);
    return (int)ctx->pending.size() - 1;
}

void end_stage(k3x_hip_ctx* ctx, int mark) {
    if (mark < 0 || (size_t)mark >= ctx->pending.size()) return;
    if (hipEventRecord(ctx->pending[mark].stop, ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        StageMark m = ctx->pending[mark];
        ctx->pending.erase(ctx->pending.begin() + mark);
        ctx->free_events.push_back(m.start);
        ctx->free_events.push_back(m.stop);
    }
}

int drain_stage_marks(k3x_hip_ctx* ctx) {
    if (ctx->pending.empty()) return K3X_OK;
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    int st = K3X_OK;
    for (const StageMark& m : ctx->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, m.start, m.stop) == hipSuccess) {
            ctx->stage_ms[m.stage] += ms;
            ctx->stage_launches[m.stage] += 1;
        } else {
            (void)hipGetLastError();
            st = K3X_ERR_BACKEND_UNAVAILABLE;
        }
        ctx->free_events.push_back(m.start);
        ctx->free_events.push_back(m.stop);
    }
    ctx->pending.clear();
    return st;
}

}  // namespace k3x_hip

extern "C" {

const char* k3x_hip_status_name(int status) {
    switch (status) {
        case K3X_OK: return "OK";
        case K3X_ERR_INVALID_EXTENT: return "INVALID_EXTENT";
        case K3X_ERR_TENSOR_NOT_FOUND: return "TENSOR_NOT_FOUND";
        case K3X_ERR_INVALID_MXFP4: return "INVALID_MXFP4";
        case K3X_ERR_INVALID_STATE: return "INVALID_STATE";
        case K3X_ERR_BACKEND_UNAVAILABLE: return "BACKEND_UNAVAILABLE";
        default: return "UNKNOWN";
    }
}

int k3x_hip_ctx_create(int device, k3x_hip_ctx** out) {
    if (!out) return K3X_ERR_INVALID_EXTENT;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
        (void)hipGetLastError();
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    if (hipSetDevice(device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    auto* ctx = new (std::nothrow) k3x_hip_ctx();
    if (!ctx) return K3X_ERR_BACKEND_UNAVAILABLE;
    ctx->device = device;
    int lds = 0, cus = 0;
    if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->side_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->join_ev, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->class_fork_ev, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->class_join_ev, hipEventDisableTiming) != hipSuccess ||
        hipMalloc((void**)&ctx->status, 256) != hipSuccess ||
        hipMemset(ctx->status, 0, 256) != hipSuccess ||
        hipMalloc((void**)&ctx->mix_counts, k3x_hip::kDecodeMixBytes + 256) != hipSuccess ||
        hipMemset(ctx->mix_counts, 0, k3x_hip::kDecodeMixBytes + 256) != hipSuccess ||
        hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device) !=
            hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
        (void)hipGetLastError();
        if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
        if (ctx->side_stream) (void)hipStreamDestroy(ctx->side_stream);
        if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
        if (ctx->join_ev) (void)hipEventDestroy(ctx->join_ev);
        if (ctx->class_fork_ev) (void)hipEventDestroy(ctx->class_fork_ev);
        if (ctx->class_join_ev) (void)hipEventDestroy(ctx->class_join_ev);
        if (ctx->status) (void)hipFree(ctx->status);
        if (ctx->mix_counts) (void)hipFree(ctx->mix_counts);
        delete ctx;
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    ctx->route_counter = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(ctx->mix_counts) +
                                                     k3x_hip::kDecodeMixBytes);
    ctx->max_lds_per_block = (size_t)lds;
    ctx->cu_count = (uint32_t)cus;
    ctx->stream = ctx->own_stream;
    // The no-allocation entry point's fixed scratch on this device (device
    // current); without it that entry point reports backend_unavailable and
    // the rest of the library is unaffected.
    if (k3x_hip::noalloc_scratch(device, &ctx->noalloc_scratch) != K3X_OK)
        ctx->noalloc_scratch = nullptr;
    *out = ctx;
    return K3X_OK;
}

int k3x_hip_ctx_destroy(k3x_hip_ctx* ctx) {
    if (!ctx) return K3X_ERR_INVALID_EXTENT;
    if (ctx->live_banks) return K3X_ERR_INVALID_STATE;  // destroy the banks first
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamSynchronize(ctx->side_stream);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->latent_scratch) (void)hipFree(ctx->latent_scratch);
    if (ctx->status) (void)hipFree(ctx->status);
    if (ctx->mix_counts) (void)hipFree(ctx->mix_counts);
    k3x_hip::free_crc(ctx);
    for (const StageMark& m : ctx->pending) {
        (void)hipEventDestroy(m.start);
        (void)hipEventDestroy(m.stop);
    }
    for (hipEvent_t e : ctx->free_events) (void)hipEventDestroy(e);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    if (ctx->side_stream) (void)hipStreamDestroy(ctx->side_stream);
    if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
    if (ctx->join_ev) (void)hipEventDestroy(ctx->join_ev);
    if (ctx->class_fork_ev) (void)hipEventDestroy(ctx->class_fork_ev);
    if (ctx->class_join_ev) (void)hipEventDestroy(ctx->class_join_ev);
    delete ctx;
    return K3X_OK;
}

int k3x_hip_ctx_set_profiling(k3x_hip_ctx* ctx, int enabled) {
    if (!ctx) return K3X_ERR_INVALID_EXTENT;
    ctx->profiling = enabled != 0;
    return K3X_OK;
}

int k3x_hip_ctx_stage_times(k3x_hip_ctx* ctx, double* ms, uint64_t* launches, int reset) {
    if (!ctx || !ms || !launches) return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    const int st = k3x_hip::drain_stage_marks(ctx);
    for (int i = 0; i < K3X_STAGE_COUNT; ++i) {
        ms[i] = ctx->stage_ms[i];
        launches[i] = ctx->stage_launches[i];
        if (reset) {
            ctx->stage_ms[i] = 0.0;
            ctx->stage_launches[i] = 0;
        }
    }
    return st;
}

int k3x_hip_ctx_set_stream(k3x_hip_ctx* ctx, void* hip_stream) {
    if (!ctx) return K3X_ERR_INVALID_EXTENT;
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    return K3X_OK;
}

int k3x_hip_ctx_use_own_stream(k3x_hip_ctx* ctx) {
    if (!ctx) return K3X_ERR_INVALID_EXTENT;
    ctx->stream = ctx->own_stream;
    return K3X_OK;
}

void* k3x_hip_ctx_stream(k3x_hip_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int k3x_hip_ctx_synchronize(k3x_hip_ctx* ctx) {
    if (!ctx) return K3X_ERR_INVALID_EXTENT;
    uint32_t status = 0;
    if (hipMemcpyAsync(&status, ctx->status, sizeof(status), hipMemcpyDeviceToHost,
                       ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    if (status) {
        // A latched error leaves every later launch of the calls in flight
        // idle; the arrival counters are cleared with the word, whatever
        // state such a call left them in.
        if (hipMemsetAsync(ctx->status, 0, sizeof(uint32_t), ctx->stream) != hipSuccess ||
            hipMemsetAsync(ctx->mix_counts, 0, k3x_hip::kDecodeMixBytes + 256, ctx->stream) !=
                hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess)
            return K3X_ERR_BACKEND_UNAVAILABLE;
        return (int)status;
    }
    return K3X_OK;
}

int k3x_hip_ctx_stats(k3x_hip_ctx* ctx, k3x_hip_stats* out) {
    if (!ctx || !out) return K3X_ERR_INVALID_EXTENT;
    std::memset(out, 0, sizeof(*out));
    out->forward_calls = ctx->forward_calls;
    out->kernel_launches = ctx->kernel_launches;
    out->scratch_bytes = ctx->scratch_bytes;
    out->weight_h2d_bytes = ctx->weight_h2d_bytes;
    return K3X_OK;
}

int k3x_hip_bank_create(k3x_hip_ctx* ctx, const k3x_hip_layer_desc* desc, k3x_hip_bank** out) {
    if (!ctx || !desc || !out) return K3X_ERR_INVALID_EXTENT;
    *out = nullptr;
    const auto& d = *desc;
    if (!d.hidden || !d.inter || !d.experts || d.hidden % 128 || d.inter % 128 ||
        d.group_size != 32 || d.shared_inter % 128 || d.experts > 4096)
        return K3X_ERR_INVALID_MXFP4;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    auto* b = new (std::nothrow) k3x_hip_bank();
    if (!b) return K3X_ERR_BACKEND_UNAVAILABLE;
    b->ctx = ctx;
    b->desc = d;
    b->gate = geom(d.inter, d.hidden);
    b->down = geom(d.hidden, d.inter);
    b->gu_codes_per_expert = (size_t)(d.inter / 16) * b->gate.kt * 2 * 64 * 16;
    b->gu_scales_per_expert = (size_t)(d.inter / 16) * b->gate.ks * 2 * 64;
    b->dn_codes_per_expert = (size_t)(d.hidden / 16) * b->down.kt * 64 * 16;
    b->dn_scales_per_expert = (size_t)(d.hidden / 16) * b->down.ks * 64;
    const size_t E = d.experts;
    int st = K3X_OK;
    st = st ? st : alloc(&b->gu_codes, E * b->gu_codes_per_expert, &b->device_bytes);
    st = st ? st : alloc(&b->gu_scales, E * b->gu_scales_per_expert * 4, &b->device_bytes);
    st = st ? st : alloc(&b->dn_codes, E * b->dn_codes_per_expert, &b->device_bytes);
    st = st ? st : alloc(&b->dn_scales, E * b->dn_scales_per_expert * 4, &b->device_bytes);
    st = st ? st : alloc(&b->router_w, E * d.hidden * sizeof(float), &b->device_bytes);
    if (k3x_hip::router_mfma_eligible(d.hidden))
        st = st ? st : alloc(&b->router_wp, k3x_hip::router_wp_floats(d.experts) * sizeof(float),
                             &b->device_bytes);
    st = st ? st : alloc(&b->router_bias, E * sizeof(float), &b->device_bytes);
    st = st ? st : alloc(&b->gamma, (size_t)d.hidden * sizeof(float), &b->device_bytes);
    st = st ? st : alloc(&b->ready_dev, E * sizeof(uint32_t), &b->device_bytes);
    if (!st && hipMemset(b->ready_dev, 0, E * sizeof(uint32_t)) != hipSuccess)
        st = K3X_ERR_BACKEND_UNAVAILABLE;
    if (d.shared_inter) {
        b->sgate = geom(d.shared_inter, d.hidden);
        b->sdown = geom(d.hidden, d.shared_inter);
        st = st ? st : alloc(&b->sh_gu, (size_t)2 * d.shared_inter * d.hidden * 2, &b->device_bytes);
        st = st ? st : alloc(&b->sh_dn, (size_t)d.hidden * d.shared_inter * 2, &b->device_bytes);
    }
    if (st) {
        free_bank_memory(b);
        delete b;
        return st;
    }
    b->expert_ready.assign(E, 0);
    ++ctx->live_banks;
    *out = b;
    return K3X_OK;
}

int k3x_hip_bank_destroy(k3x_hip_bank* bank) {
    if (!bank) return K3X_ERR_INVALID_EXTENT;
    (void)hipSetDevice(bank->ctx->device);
    (void)hipStreamSynchronize(bank->ctx->stream);
    free_bank_memory(bank);
    --bank->ctx->live_banks;
    delete bank;
    return K3X_OK;
}

uint64_t k3x_hip_bank_bytes(const k3x_hip_bank* bank) { return bank ? bank->device_bytes : 0; }

int k3x_hip_bank_upload_expert(k3x_hip_bank* bank, uint32_t expert, const uint64_t tensor_ids[3],
                               const uint8_t* gate_packed, const uint8_t* gate_scales,
                               const uint8_t* up_packed, const uint8_t* up_scales,
                               const uint8_t* down_packed, const uint8_t* down_scales) {
    if (!bank || !tensor_ids || !gate_packed || !gate_scales || !up_packed || !up_scales ||
        !down_packed || !down_scales)
        return K3X_ERR_INVALID_MXFP4;
    const auto& d = bank->desc;
    if (expert >= d.experts) return K3X_ERR_INVALID_MXFP4;
    // Residency identities: non-zero, distinct, not owned by another slot
    // (runtime/cuda/backend_cuda.cu:1847-1883).
    for (int m = 0; m < 3; ++m) {
        if (!tensor_ids[m]) return K3X_ERR_INVALID_MXFP4;
        for (int q = 0; q < m; ++q)
            if (tensor_ids[q] == tensor_ids[m]) return K3X_ERR_INVALID_MXFP4;
        auto it = bank->tensor_ids.find(tensor_ids[m]);
        if (it != bank->tensor_ids.end() && it->second != expert * 4 + (uint32_t)m)
            return K3X_ERR_INVALID_MXFP4;
    }
    const size_t n = (size_t)d.inter * d.hidden;  // elements per matrix
    const size_t pbytes = n / 2, sbytes = n / 32;
    for (const uint8_t* s : {gate_scales, up_scales, down_scales})
        for (size_t i = 0; i < sbytes; ++i)
            if (s[i] == 0xffu) return K3X_ERR_INVALID_MXFP4;
    k3x_hip_ctx* ctx = bank->ctx;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    // The slot is about to be overwritten: whatever it held is no longer
    // resident (its ids stop resolving to it, even if the upload fails).
    if (int st = k3x_hip::set_expert_ready(bank, expert, false)) return st;
    for (auto it = bank->tensor_ids.begin(); it != bank->tensor_ids.end();)
        it = it->second / 4 == expert ? bank->tensor_ids.erase(it) : std::next(it);
    // Staging buffer holding the six source arrays, each 256-byte aligned so
    // the re-tile kernels can read 16-byte vectors.
    const uint8_t* host[6] = {gate_packed, gate_scales, up_packed, up_scales, down_packed,
                              down_scales};
    size_t offset[6];
    size_t need = 0;
    for (int i = 0; i < 6; ++i) {
        offset[i] = need;
        need += (((i % 2) ? sbytes : pbytes) + 255) & ~(size_t)255;
    }
    uint8_t* staging = nullptr;
    if (hipMalloc((void**)&staging, need) != hipSuccess) {
        (void)hipGetLastError();
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    const uint8_t* dev[6];
    int st = K3X_OK;
    for (int i = 0; i < 6 && !st; ++i) {
        dev[i] = staging + offset[i];
        if (hipMemcpyAsync(staging + offset[i], host[i], (i % 2) ? sbytes : pbytes,
                           hipMemcpyHostToDevice, ctx->stream) != hipSuccess)
            st = K3X_ERR_BACKEND_UNAVAILABLE;
    }
    if (!st) st = retile_expert(bank, expert, dev, 0, 0, 1);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) st = K3X_ERR_BACKEND_UNAVAILABLE;
    if (staging) (void)hipFree(staging);
    if (st) return st;
    for (int m = 0; m < 3; ++m) bank->tensor_ids[tensor_ids[m]] = expert * 4 + (uint32_t)m;
    if ((st = k3x_hip::set_expert_ready(bank, expert, true))) return st;
    ctx->weight_h2d_bytes += 3 * (pbytes + sbytes);
    return K3X_OK;
}

int k3x_hip_bank_upload_expert_device(k3x_hip_bank* bank, uint32_t expert,
                                      const uint64_t tensor_ids[3],
                                      const uint8_t* const extents[6], const uint32_t crc32c[6]) {
    if (!bank || !tensor_ids || !extents) return K3X_ERR_INVALID_MXFP4;
    const auto& d = bank->desc;
    if (expert >= d.experts) return K3X_ERR_INVALID_MXFP4;
    for (int i = 0; i < 6; ++i)
        if (!extents[i] || reinterpret_cast<uintptr_t>(extents[i]) % 16) return K3X_ERR_INVALID_EXTENT;
    for (int m = 0; m < 3; ++m) {
        if (!tensor_ids[m]) return K3X_ERR_INVALID_MXFP4;
        for (int q = 0; q < m; ++q)
            if (tensor_ids[q] == tensor_ids[m]) return K3X_ERR_INVALID_MXFP4;
        auto it = bank->tensor_ids.find(tensor_ids[m]);
        if (it != bank->tensor_ids.end() && it->second != expert * 4 + (uint32_t)m)
            return K3X_ERR_INVALID_MXFP4;
    }
    k3x_hip_ctx* ctx = bank->ctx;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    const size_t n = (size_t)d.inter * d.hidden;
    const size_t len[6] = {n / 2, n / 32, n / 2, n / 32, n / 2, n / 32};
    // Integrity and validity before the slot is touched.
    for (int i = 0; i < 6; ++i) {
        if (crc32c) {
            uint32_t c = 0;
            if (int st = k3x_hip::crc32c_device(ctx, extents[i], len[i], &c)) return st;
            if (c != crc32c[i])
                return i % 2 ? K3X_ERR_AUXILIARY_CRC_MISMATCH : K3X_ERR_DATA_CRC_MISMATCH;
        }
        if (i % 2) {
            bool ff = false;
            if (int st = k3x_hip::any_ff_device(ctx, extents[i], len[i], &ff)) return st;
            if (ff) return K3X_ERR_INVALID_MXFP4;
        }
    }
    int st = k3x_hip::set_expert_ready(bank, expert, false);
    if (st) return st;
    for (auto it = bank->tensor_ids.begin(); it != bank->tensor_ids.end();)
        it = it->second / 4 == expert ? bank->tensor_ids.erase(it) : std::next(it);
    st = k3x_hip::retile_expert_device(bank, expert, extents);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) st = K3X_ERR_BACKEND_UNAVAILABLE;
    if (st) return st;
    for (int m = 0; m < 3; ++m) bank->tensor_ids[tensor_ids[m]] = expert * 4 + (uint32_t)m;
    return k3x_hip::set_expert_ready(bank, expert, true);
}

int k3x_hip_bank_find(k3x_hip_bank* bank, uint64_t tensor_id, uint32_t* expert, uint32_t* matrix) {
    if (!bank || !expert || !matrix) return K3X_ERR_INVALID_EXTENT;
    auto it = bank->tensor_ids.find(tensor_id);
    if (it == bank->tensor_ids.end()) return K3X_ERR_TENSOR_NOT_FOUND;
    *expert = it->second / 4;
    *matrix = it->second % 4;
    return K3X_OK;
}

int k3x_hip_bank_upload_shared(k3x_hip_bank* bank, const uint16_t* gate, const uint16_t* up,
                               const uint16_t* down) {
    if (!bank || !gate || !up || !down) return K3X_ERR_INVALID_EXTENT;
    const auto& d = bank->desc;
    if (!d.shared_inter) return K3X_ERR_INVALID_STATE;
    const size_t n = (size_t)d.shared_inter * d.hidden;
    for (const uint16_t* m : {gate, up, down})
        for (size_t i = 0; i < n; ++i)
            if ((m[i] & 0x7f80u) == 0x7f80u) return K3X_ERR_INVALID_EXTENT;  // non-finite
    k3x_hip_ctx* ctx = bank->ctx;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    uint16_t* staging = nullptr;
    if (hipMalloc((void**)&staging, 3 * n * 2) != hipSuccess) {
        (void)hipGetLastError();
        return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    int st = K3X_OK;
    const uint16_t* host[3] = {gate, up, down};
    const uint16_t* dev[3];
    for (int i = 0; i < 3 && !st; ++i) {
        dev[i] = staging + i * n;
        if (hipMemcpyAsync(staging + i * n, host[i], n * 2, hipMemcpyHostToDevice, ctx->stream) !=
            hipSuccess)
            st = K3X_ERR_BACKEND_UNAVAILABLE;
    }
    if (!st) st = retile_shared(bank, dev, 0, 0.0f);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) st = K3X_ERR_BACKEND_UNAVAILABLE;
    (void)hipFree(staging);
    if (st) return st;
    bank->shared_ready = true;
    ctx->weight_h2d_bytes += 3 * n * 2;
    return K3X_OK;
}

int k3x_hip_bank_upload_router(k3x_hip_bank* bank, const float* weight, const float* bias,
                               const float* gamma) {
    if (!bank || !weight || !bias || !gamma) return K3X_ERR_INVALID_EXTENT;
    const auto& d = bank->desc;
    const size_t wn = (size_t)d.experts * d.hidden;
    auto finite = [](const float* p, size_t n) {
        for (size_t i = 0; i < n; ++i)
            if (!(p[i] - p[i] == 0.0f)) return false;
        return true;
    };
    if (!finite(weight, wn) || !finite(bias, d.experts) || !finite(gamma, d.hidden))
        return K3X_ERR_INVALID_EXTENT;
    k3x_hip_ctx* ctx = bank->ctx;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    if (hipMemcpyAsync(bank->router_w, weight, wn * 4, hipMemcpyHostToDevice, ctx->stream) ||
        hipMemcpyAsync(bank->router_bias, bias, d.experts * 4, hipMemcpyHostToDevice,
                       ctx->stream) ||
        hipMemcpyAsync(bank->gamma, gamma, d.hidden * 4, hipMemcpyHostToDevice, ctx->stream) ||
        k3x_hip::permute_router(bank) || hipStreamSynchronize(ctx->stream))
        return K3X_ERR_BACKEND_UNAVAILABLE;
    bank->router_ready = true;
    return K3X_OK;
}

int k3x_hip_bank_set_router_device(k3x_hip_bank* bank, const float* weight, const float* bias,
                                   const float* gamma) {
    if (!bank || !weight || !bias || !gamma) return K3X_ERR_INVALID_EXTENT;
    const auto& d = bank->desc;
    k3x_hip_ctx* ctx = bank->ctx;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    if (hipMemcpyAsync(bank->router_w, weight, (size_t)d.experts * d.hidden * 4,
                       hipMemcpyDeviceToDevice, ctx->stream) ||
        hipMemcpyAsync(bank->router_bias, bias, d.experts * 4, hipMemcpyDeviceToDevice,
                       ctx->stream) ||
        hipMemcpyAsync(bank->gamma, gamma, d.hidden * 4, hipMemcpyDeviceToDevice, ctx->stream) ||
        k3x_hip::permute_router(bank))
        return K3X_ERR_BACKEND_UNAVAILABLE;
    bank->router_ready = true;
    return K3X_OK;
}

int k3x_hip_bank_fill_synthetic(k3x_hip_bank* bank, const k3x_hip_synth_desc* s) {
    if (!bank || !s) return K3X_ERR_INVALID_EXTENT;
    if (s->scale_lo > s->scale_hi || s->scale_hi >= 255) return K3X_ERR_INVALID_MXFP4;
    k3x_hip_ctx* ctx = bank->ctx;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    const auto& d = bank->desc;
    const uint8_t* none[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    int st = K3X_OK;
    for (uint32_t e = 0; e < d.experts && !st; ++e)
        st = retile_expert(bank, e, none, s->seed, s->scale_lo, s->scale_hi - s->scale_lo + 1);
    if (st) return st;
    const size_t wn = (size_t)d.experts * d.hidden;
    hipLaunchKernelGGL(fill_normal_f32, dim3(blocks_for(wn)), dim3(kThreads), 0, ctx->stream,
                       stream_key(s->seed, (uint64_t)K3X_STREAM_ROUTER << 32), wn,
                       s->router_sigma, bank->router_w);
    hipLaunchKernelGGL(fill_normal_f32, dim3(blocks_for(d.experts)), dim3(kThreads), 0,
                       ctx->stream, stream_key(s->seed, (uint64_t)K3X_STREAM_BIAS << 32),
                       (size_t)d.experts, s->bias_sigma, bank->router_bias);
    hipLaunchKernelGGL(fill_const_f32, dim3(blocks_for(d.hidden)), dim3(kThreads), 0,
                       ctx->stream, (size_t)d.hidden, s->gamma_value, bank->gamma);
    st = check_launch(ctx, 3);
    st = st ? st : k3x_hip::permute_router(bank);
    if (!st && d.shared_inter) {
        const uint16_t* none3[3] = {nullptr, nullptr, nullptr};
        st = retile_shared(bank, none3, s->seed, s->shared_sigma);
    }
    if (!st && hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(bank->ready_dev), 1,
                                 d.experts, ctx->stream) != hipSuccess)
        st = K3X_ERR_BACKEND_UNAVAILABLE;
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) st = K3X_ERR_BACKEND_UNAVAILABLE;
    if (st) return st;
    std::fill(bank->expert_ready.begin(), bank->expert_ready.end(), 1);
    bank->router_ready = true;
    bank->shared_ready = d.shared_inter != 0;
    return K3X_OK;
}

int k3x_hip_stream_read(k3x_hip_ctx* ctx, const void* data, size_t bytes, uint32_t* fold) {
    if (!ctx || !data || !fold || !bytes || bytes % 16 || reinterpret_cast<uintptr_t>(data) % 16)
        return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    const size_t n16 = bytes / 16;
    const uint32_t blocks = (uint32_t)std::min<size_t>(kStreamReadBlocks,
                                                       (n16 + kStreamReadThreads - 1) /
                                                           kStreamReadThreads);
    const size_t per_block = (n16 + blocks - 1) / blocks;
    hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(kStreamReadThreads), 0, ctx->stream,
                       static_cast<const uint4*>(data), n16, per_block, fold);
    return check_launch(ctx);
}

int k3x_hip_synth_normal_bf16(k3x_hip_ctx* ctx, uint64_t seed, uint64_t stream, float sigma,
                              size_t n, uint16_t* out) {
    if (!ctx || !out || !n) return K3X_ERR_INVALID_EXTENT;
    hipLaunchKernelGGL(fill_normal_bf16, dim3(blocks_for(n)), dim3(kThreads), 0, ctx->stream,
                       stream_key(seed, stream), n, sigma, out);
    return check_launch(ctx);
}

int k3x_hip_bank_dequant_rows(k3x_hip_bank* bank, uint32_t expert, uint32_t matrix, uint32_t row0,
                              uint32_t nrows, float* out) {
    if (!bank || !out || expert >= bank->desc.experts || matrix > 2 || !nrows)
        return K3X_ERR_INVALID_EXTENT;
    const MatrixGeom& G = matrix == K3X_MATRIX_DOWN ? bank->down : bank->gate;
    if ((uint64_t)row0 + nrows > G.rows) return K3X_ERR_INVALID_EXTENT;
    const bool gu = matrix != K3X_MATRIX_DOWN;
    const uint4* codes = reinterpret_cast<const uint4*>(
        gu ? bank->gu_codes + expert * bank->gu_codes_per_expert
           : bank->dn_codes + expert * bank->dn_codes_per_expert);
    const uint32_t* scales = gu ? bank->gu_scales + expert * bank->gu_scales_per_expert
                                : bank->dn_scales + expert * bank->dn_scales_per_expert;
    const size_t work = (size_t)nrows * (G.cols / 32);
    hipLaunchKernelGGL(dequant_rows, dim3(blocks_for(work)), dim3(kThreads), 0,
                       bank->ctx->stream, codes, scales, G.cols, G.kt, G.ks, gu ? 2u : 1u,
                       gu ? matrix : 0u, row0, nrows, out);
    return check_launch(bank->ctx);
}

}  // extern "C"
