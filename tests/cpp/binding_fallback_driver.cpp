// binding_fallback_driver.cpp -- host-only check of the reference-side
// binding's error contract (project-k3x_amd/host/binding/backend_hip.cpp),
// built by tests/test_binding.py against the reference's own headers and CPU
// sources (runtime/src/backend_cpu.cpp and its dependencies) where that tree
// is present.  The device backend is created with no device attached
// (k3x_amd::HipBackendOptions::kNoDevice), so nothing here touches a GPU:
//   1. a shape the device path does not run (a down projection whose rows
//      differ from the hidden width) is declined by the library's checks
//      and computed by the reference CPU backend, bit for bit its result,
//      and counted in runtime_stats().resident_grid_fallbacks;
//   2. a shape the device path runs reaches the device, which is absent:
//      the call fails with backend_unavailable and is NOT recomputed on the
//      CPU (the CUDA backend's contract, runtime/cuda/backend_cuda.cu:
//      1806-1883; the caller raises, runtime/src/model.cpp:1034-1037);
//   3. invalid arguments fail with invalid_mxfp4 on either shape;
//   4. the Profiler given to the factory receives the CPU backend's events
//      for the declined call.
// Exit code 0 when every check holds; prints one line per check.
#include "k3x/backend.hpp"
#include "k3x_hip_backend.hpp"

#include <cstdio>
#include <cstring>
#include <memory>
#include <vector>

namespace k3x {
Result<std::unique_ptr<ComputeBackend>> make_hip_backend(const BackendOptions& options,
                                                         Profiler* profiler,
                                                         const k3x_amd::HipBackendOptions& o);
}

namespace {

struct Matrix {
    std::vector<std::byte> packed, scales;
    std::size_t rows, cols;
    k3x::Mxfp4WeightView view(std::uint64_t id) const {
        return {id, packed, scales, rows, cols, 32};
    }
};

// Deterministic codes (every nibble value) and scales in 2^-6 .. 2^-2.
Matrix make(std::size_t rows, std::size_t cols, unsigned seed) {
    Matrix m{std::vector<std::byte>(rows * cols / 2), std::vector<std::byte>(rows * cols / 32),
             rows, cols};
    unsigned s = seed * 2654435761u + 12345u;
    for (auto& b : m.packed) {
        s = s * 1103515245u + 12345u;
        b = std::byte((s >> 16) & 0xff);
    }
    for (auto& b : m.scales) {
        s = s * 1103515245u + 12345u;
        b = std::byte(121 + ((s >> 16) % 5));
    }
    return m;
}

bool same(const std::vector<std::vector<float>>& a, const std::vector<std::vector<float>>& b) {
    if (a.size() != b.size()) return false;
    for (std::size_t i = 0; i < a.size(); ++i)
        if (a[i].size() != b[i].size() ||
            std::memcmp(a[i].data(), b[i].data(), a[i].size() * sizeof(float)) != 0)
            return false;
    return true;
}

}  // namespace

int main() {
    k3x::BackendOptions options;
    k3x_amd::HipBackendOptions ho;
    ho.device = k3x_amd::HipBackendOptions::kNoDevice;
    ho.resident_experts = 4;
    k3x::Profiler profiler;
    auto made = k3x::make_hip_backend(options, &profiler, ho);
    if (!made) {
        std::printf("factory failed: %d\n", (int)made.error());
        return 1;
    }
    k3x::ComputeBackend& be = *made.value();
    auto cpu = k3x::make_cpu_backend();
    const float beta = 4.0f;
    const std::optional<float> linear = 25.0f;

    // 1. Declined: hidden 128, intermediate 128, down rows 64 (not square).
    const std::size_t H = 128, I = 128;
    const Matrix g = make(I, H, 1), u = make(I, H, 2), d_ns = make(64, I, 3), d_sq = make(H, I, 4);
    const k3x::Mxfp4MlpView ns[1] = {{g.view(11), u.view(12), d_ns.view(13)}};
    std::vector<float> x(H);
    for (std::size_t i = 0; i < H; ++i) x[i] = (float)((int)(i % 17) - 8) / 8.0f;
    auto r1 = be.mxfp4_situ_mlp_group(x, ns, beta, linear, 0, k3x::ProfilePhase::decode);
    auto c1 = cpu->mxfp4_situ_mlp_group(x, ns, beta, linear, 0, k3x::ProfilePhase::decode);
    if (!r1 || !c1 || !same(r1.value(), c1.value())) {
        std::printf("declined shape: not the CPU backend's result\n");
        return 2;
    }
    if (be.runtime_stats().resident_grid_fallbacks != 1) {
        std::printf("declined shape: fallback not counted\n");
        return 3;
    }
    std::printf("declined shape: CPU backend's result, counted: ok\n");
    const std::size_t declined_events = profiler.events().size();
    if (declined_events == 0) {
        std::printf("declined shape: no profile events recorded\n");
        return 8;
    }

    // 2. A shape the device runs, no device: the failure is returned.
    const k3x::Mxfp4MlpView sq[1] = {{g.view(21), u.view(22), d_sq.view(23)}};
    auto r2 = be.mxfp4_situ_mlp_group(x, sq, beta, linear, 0, k3x::ProfilePhase::decode);
    if (r2 || r2.error() != k3x::ErrorCode::backend_unavailable) {
        std::printf("device shape without a device: expected backend_unavailable\n");
        return 4;
    }
    auto r2b = be.mxfp4_situ_moe(x, sq, std::vector<float>{1.0f}, beta, linear, 0,
                                 k3x::ProfilePhase::decode);
    if (r2b || r2b.error() != k3x::ErrorCode::backend_unavailable) {
        std::printf("device shape without a device (mix): expected backend_unavailable\n");
        return 5;
    }
    if (be.runtime_stats().resident_grid_fallbacks != 1) {
        std::printf("device failure was recomputed on the CPU\n");
        return 6;
    }
    std::printf("device failure returned, not recomputed: ok\n");

    // 3. Invalid arguments: invalid_mxfp4 before anything else.
    std::vector<float> short_x(H - 32, 1.0f);
    for (const auto* e : {&ns[0], &sq[0]}) {
        auto r3 = be.mxfp4_situ_mlp_group(short_x, std::span<const k3x::Mxfp4MlpView>(e, 1), beta,
                                          linear, 0, k3x::ProfilePhase::decode);
        if (r3 || r3.error() != k3x::ErrorCode::invalid_mxfp4) {
            std::printf("invalid input width: expected invalid_mxfp4\n");
            return 7;
        }
    }
    std::printf("invalid arguments: invalid_mxfp4: ok\n");
    std::printf("profiler: %zu events of the declined call: ok\n", declined_events);
    return 0;
}
