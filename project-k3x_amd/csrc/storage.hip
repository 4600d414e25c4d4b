// storage.hip -- CRC32C of device bytes, for K3X storage extents checked once
// they are in HBM (the value of runtime/src/crc32c.cpp:22-28).
//
// CRC32C is linear over GF(2).  Write raw(A) for the register after A from a
// zero register; then the register after A || B from r is adv(r, |B|) ^
// raw(B), where adv(r, m) advances r over m zero bytes.  So:
//   * each lane takes 64 contiguous bytes of a 4 KiB chunk and forms their
//     raw CRC four bytes at a time (slicing-by-4 tables in LDS);
//   * a wave folds its 64 lane values into the chunk's raw CRC in a binary
//     tree, adv(left, 64 * 2^k) ^ right at level k, with adv by a fixed
//     length tabulated as four 256-entry byte tables (adv is linear);
//   * the host folds the chunks from the preset register 0xFFFFFFFF with
//     adv(., 4096), runs the tail (< 4 KiB) byte by byte, and inverts.
// Each wave folds 16 sub-chunks itself (one value per 64 KiB reaches the
// host).  The kernel is bound by LDS table lookups (about 1.4 per byte).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <vector>

#include "k3x_device.hpp"
#include "k3x_internal.hpp"
#include "k3x_reader.hpp"

using namespace k3x_dev;

namespace {

constexpr uint32_t kPoly = 0x82f63b78u;  // reflected Castagnoli polynomial
constexpr size_t kChunk = 4096;          // bytes per wave
constexpr int kLevels = 6;               // wave tree: 64 B .. 2 KiB halves
constexpr int kTables = 2 + kLevels;     // slicing, the tree levels, advance by 4 KiB
constexpr int kSub = 16;                 // 4 KiB sub-chunks a wave folds (64 KiB chunks)
constexpr int kCrcThreads = 256;

// Host tables: T[k][256] slicing-by-4, and advance tables A_m[4][256] with
// adv(r, m) = A_m[0][r & 255] ^ A_m[1][(r >> 8) & 255] ^ ...
struct CrcTables {
    uint32_t slice[4][256];
    uint32_t adv[kLevels + 5][4][256];  // m = 64 * 2^k, k = 0..10 (4 KiB at 6, 64 KiB at 10)
};

uint32_t adv_apply(const uint32_t (&a)[4][256], uint32_t r) {
    return a[0][r & 255] ^ a[1][(r >> 8) & 255] ^ a[2][(r >> 16) & 255] ^ a[3][r >> 24];
}

const CrcTables& host_tables() {
    static const CrcTables t = [] {
        CrcTables c{};
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t r = i;
            for (int b = 0; b < 8; ++b) r = (r >> 1) ^ (kPoly & (0u - (r & 1u)));
            c.slice[0][i] = r;
        }
        for (int k = 1; k < 4; ++k)
            for (uint32_t i = 0; i < 256; ++i)
                c.slice[k][i] = (c.slice[k - 1][i] >> 8) ^ c.slice[0][c.slice[k - 1][i] & 255];
        // adv over 64 zero bytes, directly; then doubling: adv_2m = adv_m o adv_m.
        for (int b = 0; b < 4; ++b)
            for (uint32_t x = 0; x < 256; ++x) {
                uint32_t r = x << (8 * b);
                for (int m = 0; m < 64; ++m) r = c.slice[0][r & 255] ^ (r >> 8);
                c.adv[0][b][x] = r;
            }
        for (int k = 1; k <= kLevels + 4; ++k)
            for (int b = 0; b < 4; ++b)
                for (uint32_t x = 0; x < 256; ++x)
                    c.adv[k][b][x] = adv_apply(c.adv[k - 1], c.adv[k - 1][b][x]);
        return c;
    }();
    return t;
}

// One wave per chunk of SUB 4 KiB sub-chunks (grid-stride over the
// chunks); tables in LDS: [0] slicing, [1 + k] advance by 64 * 2^k bytes,
// [1 + kLevels] advance by 4 KiB.  Each sub-chunk's raw CRC comes out of the
// lane tree; lane 0 folds them in order: acc = adv(acc, 4 KiB) ^ sub.
template <int SUB>
__global__ __launch_bounds__(kCrcThreads) void crc32c_chunks_kernel(
    const uint8_t* __restrict__ data, size_t chunks, const uint32_t* __restrict__ tables,
    uint32_t* __restrict__ out) {
    __shared__ uint32_t t[kTables][1024];
    for (uint32_t i = threadIdx.x; i < kTables * 1024; i += kCrcThreads) (&t[0][0])[i] = tables[i];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (size_t c = (size_t)blockIdx.x * 4 + wave; c < chunks; c += (size_t)gridDim.x * 4) {
      uint32_t acc = 0;
      for (int sc = 0; sc < SUB; ++sc) {
        const u32x4* p =
            reinterpret_cast<const u32x4*>(data + (c * SUB + sc) * kChunk + lane * 64);
        u32x4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = p[i];
        uint32_t r = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                r ^= v[i][j];
                r = t[0][768 + (r & 255)] ^ t[0][512 + ((r >> 8) & 255)] ^
                    t[0][256 + ((r >> 16) & 255)] ^ t[0][r >> 24];
            }
#pragma unroll
        for (int k = 0; k < kLevels; ++k) {
            const uint32_t right = __shfl_down(r, 1u << k);
            r = t[1 + k][r & 255] ^ t[1 + k][256 + ((r >> 8) & 255)] ^
                t[1 + k][512 + ((r >> 16) & 255)] ^ t[1 + k][768 + (r >> 24)] ^ right;
        }
        const uint32_t* a = t[1 + kLevels];
        acc = (a[acc & 255] ^ a[256 + ((acc >> 8) & 255)] ^ a[512 + ((acc >> 16) & 255)] ^
               a[768 + (acc >> 24)]) ^ r;
      }
      if (lane == 0) out[c] = acc;
    }
}

// Sets *flag when a 16-byte group holds a 0xFF byte (haszero of ~w).
__global__ __launch_bounds__(256) void any_ff_kernel(const uint8_t* __restrict__ data, size_t n16,
                                                     uint32_t* flag) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) {
        const u32x4 v = reinterpret_cast<const u32x4*>(data)[i];
        uint32_t hit = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t w = ~v[j];
            hit |= (w - 0x01010101u) & ~w & 0x80808080u;
        }
        if (hit) atomicOr(flag, 1u);
    }
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t n, uint32_t v) {
    if (threadIdx.x < n) p[threadIdx.x] = v;
}

int ensure_crc(k3x_hip_ctx* ctx, size_t chunks) {
    if (!ctx->crc_tables) {
        const CrcTables& h = host_tables();
        std::vector<uint32_t> dev(kTables * 1024);
        std::memcpy(dev.data(), h.slice, 4096);
        for (int k = 0; k <= kLevels; ++k) std::memcpy(dev.data() + (1 + k) * 1024, h.adv[k], 4096);
        if (hipMalloc((void**)&ctx->crc_tables, dev.size() * 4) != hipSuccess) {
            (void)hipGetLastError();
            ctx->crc_tables = nullptr;
            return K3X_ERR_BACKEND_UNAVAILABLE;
        }
        if (hipMemcpy(ctx->crc_tables, dev.data(), dev.size() * 4, hipMemcpyHostToDevice) !=
            hipSuccess)
            return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    const size_t need = std::max<size_t>(chunks, 1);
    if (need > ctx->crc_chunk_cap) {
        if (ctx->crc_chunks) (void)hipFree(ctx->crc_chunks);
        ctx->crc_chunks = nullptr;
        ctx->crc_chunk_cap = 0;
        if (hipMalloc((void**)&ctx->crc_chunks, need * 4) != hipSuccess) {
            (void)hipGetLastError();
            return K3X_ERR_BACKEND_UNAVAILABLE;
        }
        ctx->crc_chunk_cap = need;
    }
    return K3X_OK;
}

}  // namespace

namespace k3x_hip {

void free_crc(k3x_hip_ctx* ctx) {
    if (ctx->crc_tables) (void)hipFree(ctx->crc_tables);
    if (ctx->crc_chunks) (void)hipFree(ctx->crc_chunks);
    ctx->crc_tables = ctx->crc_chunks = nullptr;
    ctx->crc_chunk_cap = 0;
}

int crc32c_device(k3x_hip_ctx* ctx, const void* data, size_t bytes, uint32_t* crc) {
    if (!ctx || (!data && bytes) || !crc) return K3X_ERR_INVALID_EXTENT;
    if (reinterpret_cast<uintptr_t>(data) % 16) return K3X_ERR_INVALID_EXTENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    // Whole 64 KiB chunks, then the remaining whole 4 KiB chunks, then the
    // byte tail on the host.
    const size_t big = bytes / (kChunk * kSub);
    const size_t chunks = (bytes - big * kChunk * kSub) / kChunk;
    const size_t tail = bytes % kChunk;
    if (int st = ensure_crc(ctx, big + chunks)) return st;
    const auto* src = static_cast<const uint8_t*>(data);
    std::vector<uint32_t> part(big + chunks);
    std::array<uint8_t, kChunk> tail_bytes{};
    auto grid = [&](size_t n) {
        return dim3((unsigned)std::min<size_t>((n + 3) / 4, (size_t)ctx->cu_count * 8));
    };
    if (big)
        hipLaunchKernelGGL(crc32c_chunks_kernel<kSub>, grid(big), dim3(kCrcThreads), 0,
                           ctx->stream, src, big, ctx->crc_tables, ctx->crc_chunks);
    if (chunks)
        hipLaunchKernelGGL(crc32c_chunks_kernel<1>, grid(chunks), dim3(kCrcThreads), 0,
                           ctx->stream, src + big * kChunk * kSub, chunks, ctx->crc_tables,
                           ctx->crc_chunks + big);
    if (big + chunks) {
        ctx->kernel_launches += (big != 0) + (chunks != 0);
        if (hipGetLastError() != hipSuccess ||
            hipMemcpyAsync(part.data(), ctx->crc_chunks, (big + chunks) * 4,
                           hipMemcpyDeviceToHost, ctx->stream) != hipSuccess)
            return K3X_ERR_BACKEND_UNAVAILABLE;
    }
    if (tail && hipMemcpyAsync(tail_bytes.data(), src + (big * kSub + chunks) * kChunk, tail,
                               hipMemcpyDeviceToHost, ctx->stream) != hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    const CrcTables& h = host_tables();
    uint32_t r = 0xffffffffu;
    for (size_t c = 0; c < big; ++c) r = adv_apply(h.adv[kLevels + 4], r) ^ part[c];
    for (size_t c = 0; c < chunks; ++c) r = adv_apply(h.adv[kLevels], r) ^ part[big + c];
    for (size_t i = 0; i < tail; ++i) r = h.slice[0][(r ^ tail_bytes[i]) & 255] ^ (r >> 8);
    *crc = ~r;
    return K3X_OK;
}

int any_ff_device(k3x_hip_ctx* ctx, const void* data, size_t bytes, bool* found) {
    if (reinterpret_cast<uintptr_t>(data) % 16 || bytes % 16) return K3X_ERR_INVALID_EXTENT;
    if (int st = ensure_crc(ctx, 1)) return st;
    uint32_t flag = 0;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, ctx->stream, ctx->crc_chunks, 1u, 0u);
    const size_t n16 = bytes / 16;
    if (n16)
        hipLaunchKernelGGL(any_ff_kernel,
                           dim3((unsigned)std::min<size_t>((n16 + 255) / 256, ctx->cu_count * 8)),
                           dim3(256), 0, ctx->stream, static_cast<const uint8_t*>(data), n16,
                           ctx->crc_chunks);
    ctx->kernel_launches += 2;
    if (hipGetLastError() != hipSuccess ||
        hipMemcpyAsync(&flag, ctx->crc_chunks, 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    *found = flag != 0;
    return K3X_OK;
}

}  // namespace k3x_hip

extern "C" int k3x_hip_crc32c(k3x_hip_ctx* ctx, const void* data, size_t bytes, uint32_t* crc) {
    return k3x_hip::crc32c_device(ctx, data, bytes, crc);
}

// ---------------------------------------------------------------------------
// K3X storage objects: the reader's checked directory (k3x_reader.cpp) and
// the expert load of load_storage_expert, feeding the bank through one pinned
// staging buffer and one device staging buffer per storage object.
// ---------------------------------------------------------------------------
#include <string>

struct k3x_hip_storage {
    k3x_reader::Directory dir;   // the checked directory (k3x_reader.cpp)
    uint8_t* pinned = nullptr;   // hipHostMalloc
    size_t pinned_bytes = 0;
    uint8_t* staging = nullptr;  // device
    size_t staging_bytes = 0;
    int staging_device = -1;
};

namespace {

void close_storage(k3x_hip_storage* s) {
    k3x_reader::close(&s->dir);
    if (s->pinned) (void)hipHostFree(s->pinned);
    if (s->staging) {
        (void)hipSetDevice(s->staging_device);
        (void)hipFree(s->staging);
    }
}

}  // namespace

extern "C" {

int k3x_hip_storage_open(const char* path, k3x_hip_storage** out) {
    if (!path || !out) return K3X_ERR_INVALID_EXTENT;
    *out = nullptr;
    auto* s = new (std::nothrow) k3x_hip_storage();
    if (!s) return K3X_ERR_BACKEND_UNAVAILABLE;
    const int st = k3x_reader::open_checked(&s->dir, path);
    if (st) {
        close_storage(s);
        delete s;
        return st;
    }
    *out = s;
    return K3X_OK;
}

int k3x_hip_storage_close(k3x_hip_storage* s) {
    if (!s) return K3X_ERR_INVALID_EXTENT;
    close_storage(s);
    delete s;
    return K3X_OK;
}

int k3x_hip_storage_verify(k3x_hip_storage* s) {
    if (!s) return K3X_ERR_INVALID_EXTENT;
    return k3x_reader::verify_checksums(s->dir);
}

int k3x_hip_storage_upload_expert(k3x_hip_storage* s, k3x_hip_bank* bank, uint32_t expert,
                                  uint32_t layer_id, uint32_t expert_id, uint64_t* bytes_read,
                                  uint8_t* ordered_sha256) {
    if (!s || !bank) return K3X_ERR_INVALID_EXTENT;
    if (!(s->dir.optional_features & 1u)) return K3X_ERR_INVALID_EXTENT;  // not a storage fixture
    const auto& d = bank->desc;
    const std::string base = "model.layers." + std::to_string(layer_id) +
                             ".feed_forward.experts." + std::to_string(expert_id) + ".";
    const char* roles[3] = {"gate", "up", "down"};
    const uint64_t shape[3][2] = {{d.inter, d.hidden}, {d.inter, d.hidden}, {d.hidden, d.inter}};
    const k3x_reader::TensorRecord* rec[3];
    for (int m = 0; m < 3; ++m) {
        const uint64_t id = k3x_reader::fnv1a64(base + roles[m]);
        rec[m] = nullptr;
        for (const auto& t : s->dir.tensors)
            if (t.id == id) rec[m] = &t;
        if (!rec[m]) return K3X_ERR_TENSOR_NOT_FOUND;
        const auto& t = *rec[m];
        const uint64_t n = shape[m][0] * shape[m][1];
        // valid_native_matrix (runtime/src/storage_slice.cpp:19-33).
        if (t.dtype != 2 || t.quant != 1 || t.rank != 2 || t.layer != (int32_t)layer_id ||
            t.expert != (int32_t)expert_id || t.dims[0] != shape[m][0] ||
            t.dims[1] != shape[m][1] || t.dims[2] || t.dims[3] || t.data_length != n / 2 ||
            t.aux_length != n / 32)
            return K3X_ERR_INVALID_MXFP4;
    }
    uint64_t off[6], len[6], at[6];
    uint32_t crc[6];
    size_t total = 0;
    for (int m = 0; m < 3; ++m) {
        off[2 * m] = rec[m]->data_offset;
        len[2 * m] = rec[m]->data_length;
        crc[2 * m] = rec[m]->data_crc;
        off[2 * m + 1] = rec[m]->aux_offset;
        len[2 * m + 1] = rec[m]->aux_length;
        crc[2 * m + 1] = rec[m]->aux_crc;
    }
    for (int i = 0; i < 6; ++i) {
        at[i] = total;
        total += (len[i] + 255) & ~(uint64_t)255;
    }
    if (expert >= bank->desc.experts) return K3X_ERR_INVALID_MXFP4;
    k3x_hip_ctx* ctx = bank->ctx;
    if (hipSetDevice(ctx->device) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    if (total > s->pinned_bytes) {
        if (s->pinned) (void)hipHostFree(s->pinned);
        s->pinned = nullptr;
        s->pinned_bytes = 0;
        if (hipHostMalloc((void**)&s->pinned, total, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            return K3X_ERR_BACKEND_UNAVAILABLE;
        }
        s->pinned_bytes = total;
    }
    if (total > s->staging_bytes || s->staging_device != ctx->device) {
        if (s->staging) {
            (void)hipSetDevice(s->staging_device);
            (void)hipFree(s->staging);
            (void)hipSetDevice(ctx->device);
        }
        s->staging = nullptr;
        s->staging_bytes = 0;
        if (hipMalloc((void**)&s->staging, total) != hipSuccess) {
            (void)hipGetLastError();
            return K3X_ERR_BACKEND_UNAVAILABLE;
        }
        s->staging_bytes = total;
        s->staging_device = ctx->device;
    }
    for (int i = 0; i < 6; ++i)
        if (!k3x_reader::read_at(s->dir.fd, off[i], len[i], s->pinned + at[i]))
            return K3X_ERR_TRUNCATED_FILE;
    if (hipMemcpyAsync(s->staging, s->pinned, total, hipMemcpyHostToDevice, ctx->stream) !=
        hipSuccess)
        return K3X_ERR_BACKEND_UNAVAILABLE;
    const uint8_t* ext[6];
    for (int i = 0; i < 6; ++i) ext[i] = s->staging + at[i];
    const uint64_t ids[3] = {rec[0]->id, rec[1]->id, rec[2]->id};
    const int st = k3x_hip_bank_upload_expert_device(bank, expert, ids, ext, crc);
    // A rejection may return before the copy above has been waited for:
    // drain it, so that no later call refills the pinned or staging buffer
    // while this copy still reads or writes it.
    if (st && hipStreamSynchronize(ctx->stream) != hipSuccess) return K3X_ERR_BACKEND_UNAVAILABLE;
    if (!st && bytes_read) *bytes_read = len[0] + len[1] + len[2] + len[3] + len[4] + len[5];
    if (!st && ordered_sha256) {
        // The digest load_storage_expert returns (storage_slice.cpp:80-90):
        // the six extents in order, from the bytes read into pinned memory.
        k3x_reader::Sha256 h;
        for (int i = 0; i < 6; ++i) h.update(s->pinned + at[i], len[i]);
        h.finish(ordered_sha256);
    }
    return st;
}

}  // extern "C"
