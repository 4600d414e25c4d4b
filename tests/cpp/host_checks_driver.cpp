// host_checks_driver.cpp -- host-only checks of k3x_amd::HipMoeBackend's
// argument and shape contract, on a backend with no device attached
// (HipBackendOptions::kNoDevice): nothing here touches a GPU, so it runs on
// any host (tests/test_host_backend.py).
//   * a shape the device path does not run is declined (backend_unavailable
//     with declined() set) by the checks, before any device work, and
//     counted in runtime_stats().declined_shapes;
//   * a shape the device path runs reaches the (absent) device and fails
//     with backend_unavailable, not declined: a device failure is never
//     reported as a shape the caller may compute elsewhere;
//   * one tensor id given to two different tensors of one call is
//     rejected before anything is uploaded -- invalid_extent in
//     dense_situ_mlp, invalid_mxfp4 in the resident latent layer (its
//     reference validation rejects any repeated id,
//     runtime/src/backend_cpu.cpp:441-497) -- so the device path never frees
//     a buffer the same call is using.
#include "k3x_hip_backend.hpp"

#include <cstdio>
#include <vector>

using namespace k3x_amd;

namespace {

int fail(int code, const char* what) {
    std::printf("FAIL %s\n", what);
    return code;
}

}  // namespace

int main() {
    HipBackendOptions o;
    o.device = HipBackendOptions::kNoDevice;
    o.resident_experts = 4;
    auto made = make_hip_backend(o);
    if (!made) return fail(1, "factory without a device");
    HipMoeBackend& be = *made.value();

    // Declined: a down projection of 64 rows under hidden 128.
    const std::size_t H = 128, I = 128;
    std::vector<std::byte> p(I * H / 2, std::byte{0x21}), sc(I * H / 32, std::byte{125});
    std::vector<std::byte> pd(64 * I / 2, std::byte{0x21}), sd(64 * I / 32, std::byte{125});
    std::vector<std::byte> pq(H * I / 2, std::byte{0x21}), sq(H * I / 32, std::byte{125});
    const Mxfp4MlpView ns[1] = {{{11, p, sc, I, H, 32}, {12, p, sc, I, H, 32}, {13, pd, sd, 64, I, 32}}};
    const Mxfp4MlpView ok[1] = {{{21, p, sc, I, H, 32}, {22, p, sc, I, H, 32}, {23, pq, sq, H, I, 32}}};
    std::vector<float> x(H, 0.5f);
    auto r1 = be.mxfp4_situ_mlp_group(x, ns, 4.0f, 25.0f, 0, ProfilePhase::decode);
    if (r1 || r1.error() != ErrorCode::backend_unavailable || !r1.declined())
        return fail(2, "non-square expert: declined");
    auto r1b = be.mxfp4_situ_moe(x, ns, std::vector<float>{1.0f}, 4.0f, 25.0f, 0, ProfilePhase::decode);
    if (r1b || !r1b.declined()) return fail(3, "non-square expert mix: declined");
    if (be.runtime_stats().declined_shapes != 2) return fail(4, "declined shapes counted");
    std::printf("declined shapes: ok\n");

    // A shape the device runs, no device: a failure, not declined.
    auto r2 = be.mxfp4_situ_mlp_group(x, ok, 4.0f, 25.0f, 0, ProfilePhase::decode);
    if (r2 || r2.error() != ErrorCode::backend_unavailable || r2.declined())
        return fail(5, "device shape without a device: failure, not declined");
    // Invalid arguments come first, on either shape.
    std::vector<float> xs(H - 32, 0.5f);
    if (be.mxfp4_situ_mlp_group(xs, ns, 4.0f, 25.0f, 0, ProfilePhase::decode).error() !=
        ErrorCode::invalid_mxfp4)
        return fail(6, "invalid width before the shape decision");
    std::printf("device failure is not declined: ok\n");

    // dense_situ_mlp: gate and down under one id, different tensors.
    const std::size_t S = 8;
    std::vector<float> g(S * H, 0.01f), u(S * H, 0.02f), d(H * S, 0.03f);
    const DenseMlpView shared_id{{701, g, S, H}, {702, u, S, H}, {701, d, H, S}};
    auto r3 = be.dense_situ_mlp(x, shared_id, 4.0f, 25.0f, 0, ProfilePhase::decode);
    if (r3 || r3.error() != ErrorCode::invalid_extent)
        return fail(7, "dense_situ_mlp: one id for two tensors is invalid_extent");
    const DenseMlpView same_tensor{{703, g, S, H}, {703, g, S, H}, {704, d, H, S}};
    auto r4 = be.dense_situ_mlp(x, same_tensor, 4.0f, 25.0f, 0, ProfilePhase::decode);
    if (r4 || r4.error() != ErrorCode::backend_unavailable || r4.declined())
        return fail(8, "dense_situ_mlp: one tensor under one id is valid (then no device)");
    std::printf("dense_situ_mlp tensor ids: ok\n");

    // The resident latent layer: routed_up and the shared down under one id.
    const std::size_t L = 128;
    std::vector<float> rd(L * H, 0.01f), rn(L, 1.0f), ru(H * L, 0.01f);
    std::vector<float> in(H, 0.25f);
    const ResidentMoeLayerView lv{{801, rd, L, H}, {802, rn}, {803, ru, H, L},
                                  {{804, g, S, H}, {805, u, S, H}, {803, d, H, S}}};
    const Mxfp4MlpView lx[1] = {{{31, p, sc, I, L, 32}, {32, p, sc, I, L, 32}, {33, pq, sq, L, I, 32}}};
    auto r5 = be.resident_mxfp4_moe_layer(in, lv, lx, std::vector<float>{1.0f}, 1e-6f, 4.0f, 25.0f,
                                          0, ProfilePhase::decode);
    if (r5 || r5.error() != ErrorCode::invalid_mxfp4)
        return fail(9, r5 ? "latent layer: succeeded without a device"
                          : error_code_name(r5.error()));
    std::printf("latent layer tensor ids: ok\n");
    return 0;
}
