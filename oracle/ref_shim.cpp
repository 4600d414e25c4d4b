// ref_shim.cpp -- C entry points over the reference's own CPU sources.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together
// with the reference's unmodified CPU sources (runtime/src/{ops,
// routing_policy,expert_major,official_moe,backend_cpu,profile}.cpp, read
// in place under /root/reference) into oracle/_ref/libk3x_ref.so.  Tests use
// it to pin the C restatement in k3x_oracle.c, on the build machine only:
// oracle/_ref is excluded from what is copied to GPU machines, and nothing
// there loads or times it.  Nothing from the reference is copied into this
// repository.
#include "k3x/checksums.hpp"
#include "k3x/backend.hpp"
#include "k3x/expert_major.hpp"
#include "k3x/official_moe.hpp"
#include "k3x/ops.hpp"
#include "k3x/routing_policy.hpp"

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <memory>
#include <optional>
#include <span>
#include <vector>

namespace {

std::optional<float> linear_of(int has_linear, float linear_beta) {
    if (has_linear) return linear_beta;
    return std::nullopt;
}

std::span<const std::byte> bytes(const std::uint8_t* data, std::size_t n) {
    return {reinterpret_cast<const std::byte*>(data), n};
}

k3x::ComputeBackend& cpu_backend() {
    static std::unique_ptr<k3x::ComputeBackend> backend = k3x::make_cpu_backend();
    return *backend;
}

// One expert in the K3X reference layout: packed [rows][cols/2] (low nibble
// first) and scales [rows][cols/32] for gate, up and down.
struct ExpertBytes {
    const std::uint8_t* gate_packed;
    const std::uint8_t* gate_scales;
    const std::uint8_t* up_packed;
    const std::uint8_t* up_scales;
    const std::uint8_t* down_packed;
    const std::uint8_t* down_scales;
};

k3x::Mxfp4MlpView expert_view(const ExpertBytes& e, std::size_t hidden,
                              std::size_t inter, std::uint64_t id_base) {
    const auto gate_n = inter * hidden;
    return {
        {id_base + 1, bytes(e.gate_packed, gate_n / 2),
         bytes(e.gate_scales, gate_n / 32), inter, hidden, 32},
        {id_base + 2, bytes(e.up_packed, gate_n / 2),
         bytes(e.up_scales, gate_n / 32), inter, hidden, 32},
        {id_base + 3, bytes(e.down_packed, gate_n / 2),
         bytes(e.down_scales, gate_n / 32), hidden, inter, 32},
    };
}

}  // namespace

extern "C" {

// runtime/src/crc32c.cpp:22-28.
std::uint32_t k3xr_crc32c(const std::uint8_t* data, std::size_t n) {
    return k3x::crc32c(std::as_bytes(std::span<const std::uint8_t>(data, n)));
}

}  // extern "C"

extern "C" {

int k3xr_decode_mxfp4(const std::uint8_t* packed, std::size_t packed_len,
                      const std::uint8_t* scales, std::size_t scales_len,
                      std::size_t rows, std::size_t cols, std::size_t group,
                      float* out) {
    auto result = k3x::decode_mxfp4(bytes(packed, packed_len),
                                    bytes(scales, scales_len), rows, cols, group);
    if (!result) return static_cast<int>(result.error());
    std::memcpy(out, result.value().data(), result.value().size() * sizeof(float));
    return 0;
}

int k3xr_mxfp4_matvec(const float* input, std::size_t input_len,
                      const std::uint8_t* packed, std::size_t packed_len,
                      const std::uint8_t* scales, std::size_t scales_len,
                      std::size_t rows, std::size_t cols, std::size_t group,
                      float* out) {
    auto result = k3x::mxfp4_matmul({input, input_len}, bytes(packed, packed_len),
                                    bytes(scales, scales_len), rows, cols, group);
    if (!result) return static_cast<int>(result.error());
    std::memcpy(out, result.value().data(), rows * sizeof(float));
    return 0;
}

void k3xr_rms_norm(float* out, const float* in, const float* weight,
                   std::size_t n, float epsilon) {
    k3x::rms_norm({out, n}, {in, n}, {weight, n}, epsilon);
}

void k3xr_situ_glu(float* out, const float* gate, const float* up,
                   std::size_t n, float beta, int has_linear,
                   float linear_beta) {
    k3x::situ_glu({out, n}, {gate, n}, {up, n}, beta,
                  linear_of(has_linear, linear_beta));
}

int k3xr_route_official_logits(const float* logits, const float* correction,
                               std::size_t experts, std::size_t top_k,
                               std::uint32_t* ids, float* contributions,
                               float* scores) {
    auto route = k3x::route_official_moe_logits({logits, experts},
                                                {correction, experts}, top_k);
    if (!route) return static_cast<int>(route.error());
    for (std::size_t i = 0; i < top_k; ++i) {
        ids[i] = route.value().expert_ids[i];
        contributions[i] = route.value().contributions[i];
    }
    std::memcpy(scores, route.value().scores.data(), experts * sizeof(float));
    return 0;
}

int k3xr_select_routing_natural(const float* scores, const float* bias,
                                std::size_t experts, std::size_t top_k,
                                std::uint32_t* ids, float* weights) {
    auto decision = k3x::select_routing(
        {scores, experts}, {bias, experts}, top_k,
        k3x::RoutingPolicyConfig{.mode = k3x::RoutingMode::natural});
    if (!decision) return static_cast<int>(decision.error());
    for (std::size_t i = 0; i < top_k; ++i) {
        ids[i] = static_cast<std::uint32_t>(decision.value().expert_ids[i]);
        weights[i] = decision.value().normalized_weights[i];
    }
    return 0;
}

int k3xr_expert_major_plan(const std::uint32_t* ids, const float* contributions,
                           std::size_t tokens, std::size_t top_k,
                           std::size_t* n_groups, std::uint32_t* group_expert,
                           std::uint32_t* group_start,
                           std::uint32_t* assign_token,
                           std::uint32_t* assign_slot,
                           float* assign_contribution) {
    std::vector<k3x::ExpertMajorTokenRoute> routes(tokens);
    for (std::size_t t = 0; t < tokens; ++t) {
        routes[t].expert_ids.assign(ids + t * top_k, ids + (t + 1) * top_k);
        routes[t].contributions.assign(contributions + t * top_k,
                                       contributions + (t + 1) * top_k);
    }
    auto plan = k3x::build_expert_major_plan(routes);
    if (!plan) return static_cast<int>(plan.error());
    std::size_t at = 0;
    group_start[0] = 0;
    for (std::size_t g = 0; g < plan.value().groups.size(); ++g) {
        const auto& group = plan.value().groups[g];
        group_expert[g] = group.expert_id;
        for (const auto& a : group.assignments) {
            assign_token[at] = static_cast<std::uint32_t>(a.token_index);
            assign_slot[at] = static_cast<std::uint32_t>(a.router_slot);
            assign_contribution[at] = a.contribution;
            ++at;
        }
        group_start[g + 1] = static_cast<std::uint32_t>(at);
    }
    *n_groups = plan.value().groups.size();
    return 0;
}

// CpuBackend::dense_matvec (runtime/src/backend_cpu.cpp:23-46).
int k3xr_dense_matvec(const float* input, const float* weight, std::size_t rows,
                      std::size_t cols, float* out) {
    auto r = cpu_backend().dense_matvec({input, cols},
                                        k3x::DenseWeightView{7, {weight, rows * cols}, rows, cols},
                                        0, k3x::ProfilePhase::decode);
    if (!r) return static_cast<int>(r.error());
    std::memcpy(out, r.value().data(), rows * sizeof(float));
    return 0;
}

// CpuBackend::mxfp4_situ_mlp_group for a list of experts sharing one input
// (runtime/src/backend_cpu.cpp:124-154).  Output: [n_experts][hidden].
int k3xr_mxfp4_situ_mlp_group(const float* input, std::size_t hidden,
                              std::size_t inter, const ExpertBytes* experts,
                              std::size_t n_experts, float beta,
                              int has_linear, float linear_beta, float* out) {
    std::vector<k3x::Mxfp4MlpView> views;
    for (std::size_t e = 0; e < n_experts; ++e)
        views.push_back(expert_view(experts[e], hidden, inter, 16 * (e + 1)));
    auto r = cpu_backend().mxfp4_situ_mlp_group(
        {input, hidden}, views, beta, linear_of(has_linear, linear_beta), 0,
        k3x::ProfilePhase::decode);
    if (!r) return static_cast<int>(r.error());
    for (std::size_t e = 0; e < n_experts; ++e)
        std::memcpy(out + e * hidden, r.value()[e].data(), hidden * sizeof(float));
    return 0;
}

// CpuBackend::mxfp4_situ_moe (runtime/src/backend_cpu.cpp:266-303).
int k3xr_mxfp4_situ_moe(const float* input, std::size_t hidden,
                        std::size_t inter, const ExpertBytes* experts,
                        const float* contributions, std::size_t n_experts,
                        float beta, int has_linear, float linear_beta,
                        float* out) {
    std::vector<k3x::Mxfp4MlpView> views;
    for (std::size_t e = 0; e < n_experts; ++e)
        views.push_back(expert_view(experts[e], hidden, inter, 16 * (e + 1)));
    auto r = cpu_backend().mxfp4_situ_moe(
        {input, hidden}, views, {contributions, n_experts}, beta,
        linear_of(has_linear, linear_beta), 0, k3x::ProfilePhase::decode);
    if (!r) return static_cast<int>(r.error());
    std::memcpy(out, r.value().data(), hidden * sizeof(float));
    return 0;
}

// Routing of T tokens through the reference's functions: rms_norm
// (ops.cpp:10-18), optionally rounded to bf16 as the official path rounds its
// normalised hidden (official_moe.cpp:61-80; the rounding rule is
// official_moe.cpp:18-26, whose function is file-local, so it is restated
// here), router dense_matvec (model.cpp:919-921), the float sigmoid of
// model.cpp:60 / :924, select_routing natural (routing_policy.cpp) and
// contributions * routed_scale (model.cpp:1004-1009).  Outputs [T][K].
int k3xr_route_tokens(const float* x, std::size_t tokens, const float* gamma,
                      float epsilon, const float* router, const float* bias,
                      std::size_t n_experts, std::size_t hidden,
                      std::size_t top_k, float routed_scale, int round_normed,
                      std::uint32_t* ids_out, float* weights_out) {
    std::vector<float> normed(hidden);
    for (std::size_t t = 0; t < tokens; ++t) {
        k3x::rms_norm(normed, {x + t * hidden, hidden}, {gamma, hidden}, epsilon);
        if (round_normed) {
            for (auto& v : normed) {
                std::uint32_t b;
                std::memcpy(&b, &v, 4);
                if ((b & 0x7f800000U) == 0x7f800000U) {
                    if (b & 0x007fffffU) b |= 0x00400000U;
                } else {
                    b += 0x7fffU + ((b >> 16U) & 1U);
                }
                b &= 0xffff0000U;
                std::memcpy(&v, &b, 4);
            }
        }
        auto logits = cpu_backend().dense_matvec(
            normed, k3x::DenseWeightView{5, {router, n_experts * hidden}, n_experts, hidden},
            0, k3x::ProfilePhase::decode);
        if (!logits) return static_cast<int>(logits.error());
        std::vector<float> scores(n_experts);
        for (std::size_t e = 0; e < n_experts; ++e)
            scores[e] = 1.0F / (1.0F + std::exp(-logits.value()[e]));
        auto decision = k3x::select_routing(
            scores, {bias, n_experts}, top_k,
            k3x::RoutingPolicyConfig{.mode = k3x::RoutingMode::natural});
        if (!decision) return static_cast<int>(decision.error());
        for (std::size_t k = 0; k < top_k; ++k) {
            ids_out[t * top_k + k] =
                static_cast<std::uint32_t>(decision.value().expert_ids[k]);
            weights_out[t * top_k + k] =
                decision.value().normalized_weights[k] * routed_scale;
        }
    }
    return 0;
}

// The reference CPU composition of one token of the latent-free layer:
// rms_norm (ops.cpp:10-18) -> router dense_matvec (model.cpp:919-921) ->
// sigmoid (model.cpp:60) -> select_routing natural (routing_policy.cpp) ->
// contributions * routed_scale (model.cpp:1004-1009) -> mxfp4_situ_moe
// (backend_cpu.cpp:266-303) + dense_situ_mlp shared expert
// (backend_cpu.cpp:107-122), added as in model.cpp:1145.
// `experts` is indexed by expert id.  Returns the routed ids as well.
int k3xr_moe_layer_token(const float* x, const float* gamma, float epsilon,
                         const float* router, const float* bias,
                         std::size_t n_experts, std::size_t hidden,
                         std::size_t inter, std::size_t top_k,
                         float routed_scale, const ExpertBytes* experts,
                         const float* shared_gate, const float* shared_up,
                         const float* shared_down, std::size_t shared_inter,
                         float beta, int has_linear, float linear_beta,
                         std::uint32_t* ids_out, float* out) {
    std::vector<float> normed(hidden);
    k3x::rms_norm(normed, {x, hidden}, {gamma, hidden}, epsilon);
    auto logits = cpu_backend().dense_matvec(
        normed, k3x::DenseWeightView{5, {router, n_experts * hidden}, n_experts, hidden},
        0, k3x::ProfilePhase::decode);
    if (!logits) return static_cast<int>(logits.error());
    std::vector<float> scores(n_experts);
    for (std::size_t e = 0; e < n_experts; ++e)
        scores[e] = 1.0F / (1.0F + std::exp(-logits.value()[e]));
    auto decision = k3x::select_routing(
        scores, {bias, n_experts}, top_k,
        k3x::RoutingPolicyConfig{.mode = k3x::RoutingMode::natural});
    if (!decision) return static_cast<int>(decision.error());
    std::vector<k3x::Mxfp4MlpView> views;
    std::vector<float> contributions;
    for (std::size_t slot = 0; slot < top_k; ++slot) {
        const auto id = decision.value().expert_ids[slot];
        ids_out[slot] = static_cast<std::uint32_t>(id);
        views.push_back(expert_view(experts[id], hidden, inter, 16 * (slot + 1)));
        contributions.push_back(decision.value().normalized_weights[slot] * routed_scale);
    }
    auto mixed = cpu_backend().mxfp4_situ_moe(
        normed, views, contributions, beta, linear_of(has_linear, linear_beta),
        0, k3x::ProfilePhase::decode);
    if (!mixed) return static_cast<int>(mixed.error());
    std::vector<float> zero_out(hidden);
    if (shared_inter) {
        const k3x::DenseMlpView shared{
            {1001, {shared_gate, shared_inter * hidden}, shared_inter, hidden},
            {1002, {shared_up, shared_inter * hidden}, shared_inter, hidden},
            {1003, {shared_down, hidden * shared_inter}, hidden, shared_inter},
        };
        auto s = cpu_backend().dense_situ_mlp(
            normed, shared, beta, linear_of(has_linear, linear_beta), 0,
            k3x::ProfilePhase::decode);
        if (!s) return static_cast<int>(s.error());
        zero_out = std::move(s.value());
    }
    for (std::size_t h = 0; h < hidden; ++h) out[h] = mixed.value()[h] + zero_out[h];
    return 0;
}

// Official K3 MoE FFN for one token (runtime/src/official_moe.cpp:271-344):
// the reference prepares the hidden from (prefix, block residual), routes it
// through the bf16 router with the correction, and runs the latent experts.
// Widths: H hidden, L latent (experts' hidden), I expert inter, Is shared
// inter, E experts (experts[] holds E ExpertBytes of hidden L).  Outputs:
// hidden [H], ids/contributions [K], latent [L], expert_out [K][L],
// mixed [L], routed [H], shared [H], out [H].
int k3xr_official_moe(const float* prefix, const float* block_residual, std::size_t hidden,
                      std::size_t latent, std::size_t inter, std::size_t shared_inter,
                      std::size_t experts_n, std::size_t top_k,
                      const std::uint16_t* residual_norm, const std::uint16_t* residual_proj,
                      const std::uint16_t* post_norm, const std::uint16_t* router,
                      const float* correction, const std::uint16_t* routed_down,
                      const std::uint16_t* routed_norm, const std::uint16_t* routed_up,
                      const std::uint16_t* shared_gate, const std::uint16_t* shared_up,
                      const std::uint16_t* shared_down, const ExpertBytes* experts,
                      float epsilon, float beta, int has_linear, float linear_beta,
                      float* hidden_out, std::uint32_t* ids, float* contributions,
                      float* latent_out, float* expert_out, float* mixed_out,
                      float* routed_out, float* shared_out, float* out) {
    std::vector<k3x::OfficialExpertView> views;
    views.reserve(experts_n);
    for (std::size_t e = 0; e < experts_n; ++e)
        views.push_back({static_cast<std::uint32_t>(e),
                         expert_view(experts[e], latent, inter, 100 * (e + 1))});
    const k3x::OfficialMoeWeights weights{
        {{residual_norm, hidden}},
        {{residual_proj, hidden}, 1, hidden},
        {{post_norm, hidden}},
        {{router, experts_n * hidden}, experts_n, hidden},
        {correction, experts_n},
        {{routed_down, latent * hidden}, latent, hidden},
        {{routed_norm, latent}},
        {{routed_up, hidden * latent}, hidden, latent},
        {{{shared_gate, shared_inter * hidden}, shared_inter, hidden},
         {{shared_up, shared_inter * hidden}, shared_inter, hidden},
         {{shared_down, hidden * shared_inter}, hidden, shared_inter}},
        views,
    };
    k3x::OfficialMoeInput input{{prefix, prefix + hidden},
                                {block_residual, block_residual + hidden}};
    auto h = k3x::prepare_official_moe_input(input, weights, epsilon);
    if (!h) return static_cast<int>(h.error());
    auto route = k3x::route_official_moe(h.value(), weights.router, weights.correction, top_k);
    if (!route) return static_cast<int>(route.error());
    auto result = k3x::official_moe_cpu(input, weights, route.value(), epsilon, beta,
                                        linear_of(has_linear, linear_beta));
    if (!result) return static_cast<int>(result.error());
    const auto& r = result.value();
    std::memcpy(hidden_out, r.hidden.data(), hidden * sizeof(float));
    for (std::size_t k = 0; k < top_k; ++k) {
        ids[k] = route.value().expert_ids[k];
        contributions[k] = route.value().contributions[k];
        std::memcpy(expert_out + k * latent, r.expert_outputs[k].data(), latent * sizeof(float));
    }
    std::memcpy(latent_out, r.latent.data(), latent * sizeof(float));
    std::memcpy(mixed_out, r.mixed_latent.data(), latent * sizeof(float));
    std::memcpy(routed_out, r.routed.data(), hidden * sizeof(float));
    std::memcpy(shared_out, r.shared.data(), hidden * sizeof(float));
    std::memcpy(out, r.output.data(), hidden * sizeof(float));
    return 0;
}

// CpuBackend::dense_situ_mlp (runtime/src/backend_cpu.cpp:108-122).
int k3xr_dense_situ_mlp(const float* input, std::size_t hidden, std::size_t inter,
                        std::size_t out_rows, const float* gate, const float* up,
                        const float* down, float beta, int has_linear, float linear_beta,
                        float* out) {
    const k3x::DenseMlpView mlp{{21, {gate, inter * hidden}, inter, hidden},
                                {22, {up, inter * hidden}, inter, hidden},
                                {23, {down, out_rows * inter}, out_rows, inter}};
    auto r = cpu_backend().dense_situ_mlp({input, hidden}, mlp, beta,
                                          linear_of(has_linear, linear_beta), 0,
                                          k3x::ProfilePhase::decode);
    if (!r) return static_cast<int>(r.error());
    std::memcpy(out, r.value().data(), out_rows * sizeof(float));
    return 0;
}

// CpuBackend::resident_mxfp4_moe_layer (runtime/src/backend_cpu.cpp:
// 305-339) for one token; experts in the K3X layout at the latent width.
// Returns the error code, or 0 with out [hidden] and *executed.
int k3xr_resident_layer(const float* input, std::size_t hidden, std::size_t latent,
                        std::size_t inter, std::size_t shared_inter, const float* routed_down,
                        const float* routed_norm, const float* routed_up,
                        const float* shared_gate, const float* shared_up,
                        const float* shared_down, const ExpertBytes* experts,
                        const float* contributions, std::size_t n_experts, float epsilon,
                        float beta, int has_linear, float linear_beta, int* executed,
                        float* out) {
    const k3x::ResidentMoeLayerView view{
        {31, {routed_down, latent * hidden}, latent, hidden},
        {32, {routed_norm, latent}},
        {33, {routed_up, hidden * latent}, hidden, latent},
        {{34, {shared_gate, shared_inter * hidden}, shared_inter, hidden},
         {35, {shared_up, shared_inter * hidden}, shared_inter, hidden},
         {36, {shared_down, hidden * shared_inter}, hidden, shared_inter}}};
    std::vector<k3x::Mxfp4MlpView> views;
    for (std::size_t e = 0; e < n_experts; ++e)
        views.push_back(expert_view(experts[e], latent, inter, 64 * (e + 1)));
    auto r = cpu_backend().resident_mxfp4_moe_layer(
        {input, hidden}, view, views, {contributions, n_experts}, epsilon, beta,
        linear_of(has_linear, linear_beta), 0, k3x::ProfilePhase::decode);
    if (!r) return static_cast<int>(r.error());
    *executed = r.value().executed ? 1 : 0;
    std::memcpy(out, r.value().output.data(), r.value().output.size() * sizeof(float));
    return 0;
}

}  // extern "C"
