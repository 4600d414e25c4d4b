// backend_hip.cpp -- the reference-side binding of the MI355X backend: a
// k3x::ComputeBackend (runtime/include/k3x/backend.hpp:326-462) over
// k3x_amd::HipMoeBackend, for a maintainer to add as runtime/src/
// backend_hip.cpp beside make_cuda_backend (backend.hpp:465-466).
//
// It compiles against the reference's own headers (tests/test_binding.py
// builds it with -I runtime/include where that tree is present); this
// repository does not link or run it.
//
//   * The expert-path methods run on the MI355X: the MXFP4 expert MLP group,
//     batch, grid and slot-ordered mix, the resident latent layer, the
//     official layer's four methods, the fp32 dense / MXFP4 matrix-vector
//     products and the fp32 SiTU MLP.  A shape the device path does not run
//     -- a result the library marks declined(), returned by its argument
//     checks before any upload or launch -- is computed by the reference's
//     CPU backend instead and counted (runtime_stats().resident_grid_fallbacks;
//     the latent layer's also in resident_moe_layer_fallbacks).  Every other
//     failure, device, allocation and launch failures included, is returned
//     as the failure it is, as the CUDA backend returns them
//     (runtime/cuda/backend_cuda.cu:1806-1883) for the caller to raise
//     (runtime/src/model.cpp:1034-1037).
//   * Every other method -- the prefetch trio, official_kda and the layer
//     front / tail -- forwards to make_cpu_backend(), the reference's exact
//     path.
// Views convert member by member (the structs hold the same members) and
// error codes by value (the enumerations list the same codes in the same
// order).  With a Profiler, every device method's operations are recorded
// into it as ProfileEvents (stage device times where the library stages
// the call), beside the CPU backend's own for the calls it runs.
#include "k3x/backend.hpp"
#include "k3x_hip_backend.hpp"

#include <algorithm>
#include <memory>
#include <utility>
#include <vector>

namespace k3x {
namespace {

namespace hip = k3x_amd;

hip::ProfilePhase to_hip(ProfilePhase p) {
    return p == ProfilePhase::prefill ? hip::ProfilePhase::prefill : hip::ProfilePhase::decode;
}
hip::Mxfp4WeightView to_hip(const Mxfp4WeightView& w) {
    return {w.tensor_id, w.packed, w.scales, w.rows, w.cols, w.group_size};
}
hip::Mxfp4MlpView to_hip(const Mxfp4MlpView& e) { return {to_hip(e.gate), to_hip(e.up), to_hip(e.down)}; }
hip::DenseWeightView to_hip(const DenseWeightView& w) {
    return {w.tensor_id, w.values, w.rows, w.cols};
}
hip::DenseMlpView to_hip(const DenseMlpView& m) { return {to_hip(m.gate), to_hip(m.up), to_hip(m.down)}; }
hip::ResidentMoeLayerView to_hip(const ResidentMoeLayerView& v) {
    return {to_hip(v.routed_down), {v.routed_norm.tensor_id, v.routed_norm.values},
            to_hip(v.routed_up), to_hip(v.shared)};
}
hip::Bf16WeightView to_hip(const Bf16WeightView& w) { return {w.values, w.rows, w.cols, w.tensor_id}; }
hip::Bf16VectorView to_hip(const Bf16VectorView& v) { return {v.values, v.tensor_id}; }
hip::Bf16MlpView to_hip(const Bf16MlpView& m) { return {to_hip(m.gate), to_hip(m.up), to_hip(m.down)}; }
hip::OfficialMoeFfnView to_hip(const OfficialMoeFfnView& v) {
    return {to_hip(v.routed_down), to_hip(v.routed_norm), to_hip(v.routed_up), to_hip(v.shared)};
}
hip::OfficialMoeRoutePrepareView to_hip(const OfficialMoeRoutePrepareView& v) {
    return {to_hip(v.residual_norm), to_hip(v.residual_proj), to_hip(v.post_norm),
            to_hip(v.router)};
}
hip::OfficialMoePreparedToken to_hip(OfficialMoePreparedToken t) { return {t.owner, t.generation}; }

template <class V>
auto to_hip_all(std::span<const V> views) {
    std::vector<decltype(to_hip(views.front()))> out;
    out.reserve(views.size());
    for (const V& v : views) out.push_back(to_hip(v));
    return out;
}

ErrorCode code(hip::ErrorCode c) { return static_cast<ErrorCode>(c); }

OfficialMoeFfnResult from_hip(hip::OfficialMoeFfnResult&& r) {
    return {r.executed, std::move(r.output), std::move(r.selected_expert_ids)};
}
OfficialMoeRoutePrepareResult from_hip(hip::OfficialMoeRoutePrepareResult&& r) {
    return {r.executed, {r.prepared.owner, r.prepared.generation}, std::move(r.router_logits)};
}
ResidentMoeLayerResult from_hip(hip::ResidentMoeLayerResult&& r) {
    return {r.executed, std::move(r.output)};
}
template <class T>
T from_hip(T&& v) {
    return std::move(v);
}

// The library's result as the reference's; where the library declined the
// shape (before any device work), the CPU backend's, counted in *declined.
template <class H, class F>
auto or_cpu(hip::Result<H>&& r, std::uint64_t* declined, F&& cpu) -> decltype(cpu()) {
    using R = decltype(cpu());
    if (r) return R::success(from_hip(std::move(r.value())));
    if (r.declined()) {
        ++*declined;
        return cpu();
    }
    return R::failure(code(r.error()), r.message());
}

class HipBackend final : public ComputeBackend {
public:
    HipBackend(std::unique_ptr<hip::HipMoeBackend> be, BackendOptions options, Profiler* profiler)
        : be_(std::move(be)), cpu_(make_cpu_backend(profiler)), options_(options) {
        // The device methods' operations reach the same Profiler as the CPU
        // backend's (the enumerations list the same members in the same
        // order), as the CUDA backend records them (backend_cuda.cu:2505-2542).
        if (profiler)
            be_->set_profile_sink([profiler](const hip::ProfileEvent& e) {
                profiler->record(ProfileEvent{
                    e.phase == hip::ProfilePhase::prefill ? ProfilePhase::prefill
                                                          : ProfilePhase::decode,
                    static_cast<ProfileOperation>(e.operation),
                    static_cast<NumericPrecision>(e.precision), e.layer, e.wall_nanoseconds,
                    e.device_nanoseconds, e.logical_bytes, e.transfer_bytes, e.success});
            });
    }

    BackendKind kind() const noexcept override { return options_.kind; }
    const BackendOptions& options() const noexcept override { return options_; }
    BackendRuntimeStats runtime_stats() const noexcept override {
        const hip::HipBackendStats s = be_->runtime_stats();
        BackendRuntimeStats r{};
        r.weight_h2d_bytes = s.weight_h2d_bytes;
        r.weight_cache_hits = s.residency_hits;
        r.weight_cache_misses = s.experts_admitted + s.dense_uploads;
        r.resident_moe_layer_fallbacks = s.resident_layer_fallbacks + layer_declined_;
        r.resident_grid_kernel_launches = s.kernel_launches;
        // Calls the device path declined by shape, computed by the CPU
        // backend instead.
        r.resident_grid_fallbacks = declined_;
        r.resident_weight_bytes = s.device_bytes;
        r.peak_resident_weight_bytes = s.peak_device_bytes;
        return r;
    }

    Result<std::vector<float>> dense_matvec(std::span<const float> input, DenseWeightView weight,
                                            std::uint32_t layer, ProfilePhase phase) override {
        return or_cpu(be_->dense_matvec(input, to_hip(weight), layer, to_hip(phase)), &declined_,
                      [&] { return cpu_->dense_matvec(input, weight, layer, phase); });
    }
    Result<std::vector<float>> mxfp4_matvec(std::span<const float> input, Mxfp4WeightView weight,
                                            std::uint32_t layer, ProfilePhase phase) override {
        return or_cpu(be_->mxfp4_matvec(input, to_hip(weight), layer, to_hip(phase)), &declined_,
                      [&] { return cpu_->mxfp4_matvec(input, weight, layer, phase); });
    }
    Result<std::vector<std::vector<float>>> dense_matvec_group(
        std::span<const float> input, std::span<const DenseWeightView> weights,
        std::uint32_t layer, ProfilePhase phase) override {
        const auto w = to_hip_all(weights);
        return or_cpu(be_->dense_matvec_group(input, w, layer, to_hip(phase)), &declined_,
                      [&] { return cpu_->dense_matvec_group(input, weights, layer, phase); });
    }
    Result<std::vector<std::vector<float>>> mxfp4_matvec_group(
        std::span<const float> input, std::span<const Mxfp4WeightView> weights,
        std::uint32_t layer, ProfilePhase phase) override {
        const auto w = to_hip_all(weights);
        return or_cpu(be_->mxfp4_matvec_group(input, w, layer, to_hip(phase)), &declined_,
                      [&] { return cpu_->mxfp4_matvec_group(input, weights, layer, phase); });
    }
    Result<std::vector<float>> dense_situ_mlp(std::span<const float> input, DenseMlpView weights,
                                              float situ_beta, std::optional<float> situ_linear,
                                              std::uint32_t layer, ProfilePhase phase) override {
        return or_cpu(
            be_->dense_situ_mlp(input, to_hip(weights), situ_beta, situ_linear, layer,
                                to_hip(phase)), &declined_,
            [&] { return cpu_->dense_situ_mlp(input, weights, situ_beta, situ_linear, layer, phase); });
    }
    Result<std::vector<std::vector<float>>> mxfp4_situ_mlp_group(
        std::span<const float> input, std::span<const Mxfp4MlpView> experts, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase) override {
        const auto e = to_hip_all(experts);
        return or_cpu(be_->mxfp4_situ_mlp_group(input, e, situ_beta, situ_linear, layer,
                                                to_hip(phase)), &declined_,
                      [&] {
                          return cpu_->mxfp4_situ_mlp_group(input, experts, situ_beta, situ_linear,
                                                            layer, phase);
                      });
    }
    Result<std::vector<std::vector<float>>> mxfp4_situ_mlp_batch(
        std::span<const float> inputs, std::size_t batch_size, Mxfp4MlpView expert,
        float situ_beta, std::optional<float> situ_linear, std::uint32_t layer,
        ProfilePhase phase) override {
        return or_cpu(be_->mxfp4_situ_mlp_batch(inputs, batch_size, to_hip(expert), situ_beta,
                                                situ_linear, layer, to_hip(phase)), &declined_,
                      [&] {
                          return cpu_->mxfp4_situ_mlp_batch(inputs, batch_size, expert, situ_beta,
                                                            situ_linear, layer, phase);
                      });
    }
    Result<std::vector<std::vector<float>>> mxfp4_situ_mlp_grid(
        std::span<const float> inputs, std::size_t token_count,
        std::span<const Mxfp4MlpView> experts, float situ_beta, std::optional<float> situ_linear,
        std::uint32_t layer, ProfilePhase phase) override {
        const auto e = to_hip_all(experts);
        return or_cpu(be_->mxfp4_situ_mlp_grid(inputs, token_count, e, situ_beta, situ_linear,
                                               layer, to_hip(phase)), &declined_,
                      [&] {
                          return cpu_->mxfp4_situ_mlp_grid(inputs, token_count, experts, situ_beta,
                                                           situ_linear, layer, phase);
                      });
    }
    Result<std::vector<float>> mxfp4_situ_moe(std::span<const float> input,
                                              std::span<const Mxfp4MlpView> experts,
                                              std::span<const float> contributions,
                                              float situ_beta, std::optional<float> situ_linear,
                                              std::uint32_t layer, ProfilePhase phase) override {
        const auto e = to_hip_all(experts);
        return or_cpu(be_->mxfp4_situ_moe(input, e, contributions, situ_beta, situ_linear, layer,
                                          to_hip(phase)), &declined_,
                      [&] {
                          return cpu_->mxfp4_situ_moe(input, experts, contributions, situ_beta,
                                                      situ_linear, layer, phase);
                      });
    }
    Result<ResidentMoeLayerResult> resident_mxfp4_moe_layer(
        std::span<const float> input, ResidentMoeLayerView weights,
        std::span<const Mxfp4MlpView> experts, std::span<const float> contributions,
        float epsilon, float situ_beta, std::optional<float> situ_linear, std::uint32_t layer,
        ProfilePhase phase) override {
        const auto e = to_hip_all(experts);
        return or_cpu(be_->resident_mxfp4_moe_layer(input, to_hip(weights), e, contributions,
                                                    epsilon, situ_beta, situ_linear, layer,
                                                    to_hip(phase)), &declined_,
                      [&] {
                          ++layer_declined_;
                          return cpu_->resident_mxfp4_moe_layer(input, weights, experts,
                                                                contributions, epsilon, situ_beta,
                                                                situ_linear, layer, phase);
                      });
    }
    Result<OfficialMoeFfnResult> official_mxfp4_moe_ffn(
        std::span<const float> hidden, std::span<const float> prefix, OfficialMoeFfnView weights,
        std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
        std::span<const float> contributions, float epsilon, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase) override {
        const auto e = to_hip_all(experts);
        return or_cpu(be_->official_mxfp4_moe_ffn(hidden, prefix, to_hip(weights), e, expert_ids,
                                                  contributions, epsilon, situ_beta, situ_linear,
                                                  layer, to_hip(phase)), &declined_,
                      [&] {
                          return cpu_->official_mxfp4_moe_ffn(hidden, prefix, weights, experts,
                                                              expert_ids, contributions, epsilon,
                                                              situ_beta, situ_linear, layer, phase);
                      });
    }
    Result<OfficialMoeRoutePrepareResult> prepare_official_moe_route(
        std::span<const float> prefix, std::span<const float> block_residual,
        OfficialMoeRoutePrepareView weights, float epsilon, std::uint32_t layer,
        ProfilePhase phase) override {
        return or_cpu(be_->prepare_official_moe_route(prefix, block_residual, to_hip(weights),
                                                      epsilon, layer, to_hip(phase)), &declined_,
                      [&] {
                          return cpu_->prepare_official_moe_route(prefix, block_residual, weights,
                                                                  epsilon, layer, phase);
                      });
    }
    Result<OfficialMoeFfnResult> official_mxfp4_moe_ffn_prepared(
        OfficialMoePreparedToken prepared, OfficialMoeFfnView weights,
        std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
        std::span<const float> contributions, float epsilon, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase) override {
        const auto e = to_hip_all(experts);
        // A token this backend prepared on the device; the CPU backend holds
        // none of its tokens, so no fallback here.
        auto r = be_->official_mxfp4_moe_ffn_prepared(to_hip(prepared), to_hip(weights), e,
                                                      expert_ids, contributions, epsilon,
                                                      situ_beta, situ_linear, layer, to_hip(phase));
        if (!r) return Result<OfficialMoeFfnResult>::failure(code(r.error()), r.message());
        return Result<OfficialMoeFfnResult>::success(from_hip(std::move(r.value())));
    }
    Result<bool> discard_official_moe_prepared(OfficialMoePreparedToken prepared) override {
        auto r = be_->discard_official_moe_prepared(to_hip(prepared));
        if (!r) return Result<bool>::failure(code(r.error()), r.message());
        return Result<bool>::success(r.value());
    }

    // Off the device path: the reference CPU backend.
    Result<OfficialKdaCudaResult> official_kda(std::span<const float> input,
                                               OfficialKdaCudaView weights,
                                               OfficialKdaCudaStateView state,
                                               OfficialKdaCudaConfig config, std::uint32_t layer,
                                               ProfilePhase phase,
                                               OfficialKdaStateControl control) override {
        return cpu_->official_kda(input, weights, state, config, layer, phase, control);
    }
    Result<bool> discard_official_kda_device_state(OfficialKdaDeviceStateToken token) override {
        return cpu_->discard_official_kda_device_state(token);
    }
    Result<OfficialLayerFrontResult> official_layer_front(
        std::span<const float> input, std::span<const float> residual,
        OfficialLayerHiddenToken hidden, OfficialLayerFrontWeights weights,
        OfficialKdaCudaStateView state, OfficialKdaCudaConfig config, std::uint32_t layer,
        ProfilePhase phase, OfficialKdaStateControl control) override {
        return cpu_->official_layer_front(input, residual, hidden, weights, state, config, layer,
                                          phase, control);
    }
    Result<OfficialLayerTailResult> official_layer_tail(
        OfficialMoePreparedToken prepared, OfficialMoeFfnView weights,
        std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
        std::span<const float> contributions, float epsilon, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase,
        bool publish) override {
        return cpu_->official_layer_tail(prepared, weights, experts, expert_ids, contributions,
                                         epsilon, situ_beta, situ_linear, layer, phase, publish);
    }
    Result<bool> discard_official_layer_hidden(OfficialLayerHiddenToken token) override {
        return cpu_->discard_official_layer_hidden(token);
    }
    Result<Mxfp4PrefetchToken> prefetch_mxfp4_situ_mlp_group(std::span<const Mxfp4MlpView> experts,
                                                            std::uint64_t use_sequence,
                                                            std::uint32_t layer,
                                                            ProfilePhase phase) override {
        return cpu_->prefetch_mxfp4_situ_mlp_group(experts, use_sequence, layer, phase);
    }
    Result<std::vector<std::vector<float>>> mxfp4_situ_mlp_group_prepared(
        std::span<const float> input, Mxfp4PrefetchToken token, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase) override {
        return cpu_->mxfp4_situ_mlp_group_prepared(input, token, situ_beta, situ_linear, layer,
                                                   phase);
    }
    Result<std::vector<float>> mxfp4_situ_moe_prepared(std::span<const float> input,
                                                       Mxfp4PrefetchToken token,
                                                       std::span<const float> contributions,
                                                       float situ_beta,
                                                       std::optional<float> situ_linear,
                                                       std::uint32_t layer,
                                                       ProfilePhase phase) override {
        return cpu_->mxfp4_situ_moe_prepared(input, token, contributions, situ_beta, situ_linear,
                                             layer, phase);
    }

    // The device bytes this backend holds now (banks, resident dense
    // weights, scratch, per-call buffers) and their peak.
    BackendMemoryStats memory_stats() const noexcept override {
        const hip::HipBackendStats s = be_->runtime_stats();
        return {s.device_bytes, s.peak_device_bytes};
    }
    std::string_view device_name() const noexcept override { return be_->device_name(); }

private:
    std::unique_ptr<hip::HipMoeBackend> be_;
    std::unique_ptr<ComputeBackend> cpu_;
    BackendOptions options_;
    std::uint64_t declined_ = 0;        // calls declined by shape, run on the CPU backend
    std::uint64_t layer_declined_ = 0;  // of them, resident_mxfp4_moe_layer calls
};

}  // namespace

// The factory with the device-side options given explicitly (device index,
// bank slots, resident byte budget; HipBackendOptions::kNoDevice gives a
// backend with no device, whose declined shapes still run on the CPU
// backend and whose other calls fail with backend_unavailable).
Result<std::unique_ptr<ComputeBackend>> make_hip_backend(const BackendOptions& options,
                                                         Profiler* profiler,
                                                         const k3x_amd::HipBackendOptions& o) {
    auto be = hip::make_hip_backend(o);
    if (!be) {
        return Result<std::unique_ptr<ComputeBackend>>::failure(code(be.error()), be.message());
    }
    return Result<std::unique_ptr<ComputeBackend>>::success(
        std::make_unique<HipBackend>(std::move(be.value()), options, profiler));
}

// The factory a maintainer declares beside make_cuda_backend
// (backend.hpp:465-466).  Slots: every routed expert of a K3-shaped layer
// (384) resident.
Result<std::unique_ptr<ComputeBackend>> make_hip_backend(const BackendOptions& options,
                                                         Profiler* profiler) {
    hip::HipBackendOptions o;
    o.device = 0;
    o.resident_experts = 384;
    if (options.cuda_resident_bytes) o.resident_dense_bytes = options.cuda_resident_bytes;
    return make_hip_backend(options, profiler, o);
}

}  // namespace k3x
