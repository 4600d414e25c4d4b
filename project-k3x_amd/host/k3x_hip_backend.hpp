// k3x_hip_backend.hpp -- C++20 host side of the MI355X MoE layer: the
// expert-execution methods of the K3X runtime's ComputeBackend
// (runtime/include/k3x/backend.hpp:326-462) with the same names, argument
// meaning and error behaviour, running on libk3x_hip_moe.so through its C ABI
// (include/k3x_hip_moe.h).
//
// Contract, as the reference's backends:
//   * inputs are borrowed host spans, valid for the call; results come back
//     by value after the device work has finished (every method is
//     synchronous);
//   * no exceptions cross the interface: failures are Result::failure with an
//     ErrorCode, and argument checks run before anything is uploaded or
//     launched;
//   * experts are resident: the first use of an expert (keyed by the
//     tensor_id of its three matrices) admits it into a bank slot of its
//     layer; later uses find it there (ResidentWeightTable::acquire,
//     runtime/cuda/resident_weights.cu:107-166).  When every slot is taken,
//     the least recently used expert not needed by the current call is
//     replaced.
// Numerics: the layer's rounding points -- the input and the GLU output are
// rounded to bf16 (round to nearest even), matrix products accumulate in
// fp32, the per-expert outputs and the slot-ordered mix stay fp32 -- where
// the reference CPU backend keeps fp32 inputs and double sums.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <optional>
#include <span>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace k3x_amd {

// Same enumerators in the same order (hence the same values) as
// k3x::ErrorCode (runtime/include/k3x/status.hpp:9-31); the C ABI's status
// codes are these values.
enum class ErrorCode {
    ok,
    io_error,
    bad_magic,
    unsupported_version,
    unsupported_required_feature,
    non_executable_artifact,
    superblock_crc_mismatch,
    truncated_file,
    invalid_directory,
    invalid_extent,
    data_crc_mismatch,
    auxiliary_crc_mismatch,
    directory_sha256_mismatch,
    root_sha256_mismatch,
    tensor_not_found,
    invalid_mxfp4,
    invalid_state,
    backend_unavailable,
    storage_unavailable,
    unsupported_architecture,
};

const char* error_code_name(ErrorCode code);

// A value or an error code with a message (the interface of k3x::Result,
// status.hpp:58-76).
template <typename T>
class Result {
public:
    static Result success(T value) { return Result(std::move(value)); }
    static Result failure(ErrorCode code, std::string message = {}) {
        return Result(code, std::move(message));
    }
    // A shape (or size) the device path does not run, found by the argument
    // checks before anything was uploaded or launched: error() is
    // backend_unavailable, as for a device failure, and declined() tells the
    // two apart (a caller may compute a declined call elsewhere; a device
    // failure is a failure).
    static Result declined_shape(std::string message = {}) {
        Result r(ErrorCode::backend_unavailable, std::move(message));
        r.declined_ = true;
        return r;
    }
    explicit operator bool() const { return value_.has_value(); }
    T& value() { return *value_; }
    const T& value() const { return *value_; }
    ErrorCode error() const { return error_; }
    const std::string& message() const { return message_; }
    bool declined() const { return declined_; }

private:
    explicit Result(T value) : value_(std::move(value)) {}
    Result(ErrorCode code, std::string message) : error_(code), message_(std::move(message)) {}
    std::optional<T> value_;
    ErrorCode error_{ErrorCode::ok};
    std::string message_;
    bool declined_ = false;
};

enum class ProfilePhase { prefill, decode };  // runtime/include/k3x/profile.hpp:11

// Same enumerators in the same order as k3x::ProfileOperation and
// k3x::NumericPrecision (runtime/include/k3x/profile.hpp:13-27).
enum class ProfileOperation {
    tensor_read,
    dense_matvec,
    mxfp4_matvec,
    situ_glu,
    moe_mix,
    rms_norm,
    residual_add,
    host_to_device,
    weight_host_to_device,
    activation_host_to_device,
    device_to_host,
};
enum class NumericPrecision { none, fp32, bf16_rounded, mxfp4_e2m1_e8m0 };

// One operation of a method call, the members of k3x::ProfileEvent
// (profile.hpp:32-42).  device_nanoseconds comes from the library's stage
// events (hipEvent pairs on the context stream) where the call's kernels are
// staged, and is the host-measured launch-to-completion time of the call
// otherwise; logical_bytes are the bytes the operation reads by definition
// (weights and activations), transfer_bytes the bytes a copy moved.
struct ProfileEvent {
    ProfilePhase phase;
    ProfileOperation operation;
    NumericPrecision precision;
    std::uint32_t layer;
    std::uint64_t wall_nanoseconds;
    std::uint64_t device_nanoseconds;
    std::uint64_t logical_bytes;
    std::uint64_t transfer_bytes;
    bool success;
};
using ProfileSink = std::function<void(const ProfileEvent&)>;

// One MXFP4 matrix in the K3X layout: packed [rows][cols/2] (low nibble =
// even column), scales [rows][cols/group_size] E8M0 (backend.hpp:150-157).
struct Mxfp4WeightView {
    std::uint64_t tensor_id;
    std::span<const std::byte> packed;
    std::span<const std::byte> scales;
    std::size_t rows;
    std::size_t cols;
    std::size_t group_size;
};

// fp32 dense views (backend.hpp:131-136, :204-207, :165-169): values
// row-major [rows][cols].
struct DenseWeightView {
    std::uint64_t tensor_id;
    std::span<const float> values;
    std::size_t rows;
    std::size_t cols;
};

struct DenseVectorView {
    std::uint64_t tensor_id;
    std::span<const float> values;
};

struct DenseMlpView {
    DenseWeightView gate;
    DenseWeightView up;
    DenseWeightView down;
};

// The resident latent layer's dense weights and result (backend.hpp:
// 302-312).
struct ResidentMoeLayerView {
    DenseWeightView routed_down;
    DenseVectorView routed_norm;
    DenseWeightView routed_up;
    DenseMlpView shared;
};

struct ResidentMoeLayerResult {
    bool executed{};
    std::vector<float> output;
};

// gate [I x H], up [I x H], down [out x I] (backend.hpp:315-319).
struct Mxfp4MlpView {
    Mxfp4WeightView gate;
    Mxfp4WeightView up;
    Mxfp4WeightView down;
};

// bf16 views of the official layer (backend.hpp:138-148, :165-176, :184-189):
// values are bf16 words, row-major [rows][cols].
struct Bf16WeightView {
    std::span<const std::uint16_t> values;
    std::size_t rows{};
    std::size_t cols{};
    std::uint64_t tensor_id{};
};

struct Bf16VectorView {
    std::span<const std::uint16_t> values;
    std::uint64_t tensor_id{};
};

struct Bf16MlpView {
    Bf16WeightView gate;
    Bf16WeightView up;
    Bf16WeightView down;
};

struct OfficialMoeFfnView {
    Bf16WeightView routed_down;
    Bf16VectorView routed_norm;
    Bf16WeightView routed_up;
    Bf16MlpView shared;
};

struct OfficialMoeFfnResult {
    bool executed{};
    std::vector<float> output;
    std::vector<std::uint32_t> selected_expert_ids;
};

struct OfficialMoeRoutePrepareView {
    Bf16VectorView residual_norm;
    Bf16WeightView residual_proj;
    Bf16VectorView post_norm;
    Bf16WeightView router;
};

struct OfficialMoePreparedToken {
    std::uint64_t owner{};
    std::uint64_t generation{};
    bool operator==(const OfficialMoePreparedToken&) const = default;
};

struct OfficialMoeRoutePrepareResult {
    bool executed{};
    OfficialMoePreparedToken prepared;
    std::vector<float> router_logits;
};

// Same members as k3x::ExpertMajorTokenRoute (expert_major.hpp:12-15).
struct ExpertMajorTokenRoute {
    std::vector<std::uint32_t> expert_ids;
    std::vector<float> contributions;
};

struct ExpertMajorBlockMoe {
    std::vector<float> mixed;          // [positions][width]
    std::uint64_t unique_experts = 0;  // groups of the block's expert-major plan
    std::uint64_t assignments = 0;     // (position, slot) pairs
    std::uint64_t layer_calls = 0;     // grouped layer calls made
};

struct HipBackendOptions {
    // HIP device index; kNoDevice builds a backend with no device attached,
    // whose methods run their argument and shape checks and then fail with
    // backend_unavailable (not declined) where they would touch the device
    // (host-only tests of the checks and of the declined-shape contract).
    static constexpr int kNoDevice = -1;
    int device = 0;
    // Bank slots per (layer, hidden, intermediate) shape; each slot holds
    // one expert (hidden * intermediate * 3 * 17 / 32 bytes, 23.4 MB at
    // 7168 x 2048).
    std::uint32_t resident_experts = 64;
    // Device bytes for resident fp32 dense weights and single MXFP4
    // matrices (the matvec methods and the latent layer's dense weights),
    // least recently used first out; a matrix that does not fit runs from a
    // transient upload (matvec methods) or bypasses the latent layer.
    std::uint64_t resident_dense_bytes = 8ull << 30;
};

struct HipBackendStats {
    std::uint64_t calls = 0;             // method calls that reached the device
    std::uint64_t layer_calls = 0;       // library layer calls they made
    std::uint64_t kernel_launches = 0;
    std::uint64_t experts_admitted = 0;  // slot uploads
    std::uint64_t residency_hits = 0;    // experts found resident
    std::uint64_t weight_h2d_bytes = 0;
    std::uint64_t dense_uploads = 0;             // dense / single-matrix uploads
    std::uint64_t resident_layer_fallbacks = 0;  // latent layer calls returned executed=false
    std::uint64_t declined_shapes = 0;   // calls declined by shape before any device work
    // Device memory this backend holds now (banks, resident dense weights,
    // the context's scratch, the per-call buffers) and its peak.
    std::uint64_t device_bytes = 0;
    std::uint64_t peak_device_bytes = 0;
};

class HipMoeBackend {
public:
    ~HipMoeBackend();
    HipMoeBackend(const HipMoeBackend&) = delete;
    HipMoeBackend& operator=(const HipMoeBackend&) = delete;

    // One token through each expert: outputs[e] = down(GLU(gate x, up x))
    // (backend.hpp:348-351, backend_cpu.cpp:124-154).
    Result<std::vector<std::vector<float>>> mxfp4_situ_mlp_group(
        std::span<const float> input, std::span<const Mxfp4MlpView> experts, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase);
    // batch_size tokens (rows of inputs) through one expert: outputs[t]
    // (backend.hpp:352-356, backend_cpu.cpp:156-189).
    Result<std::vector<std::vector<float>>> mxfp4_situ_mlp_batch(
        std::span<const float> inputs, std::size_t batch_size, Mxfp4MlpView expert,
        float situ_beta, std::optional<float> situ_linear, std::uint32_t layer,
        ProfilePhase phase);
    // token_count tokens through every expert: outputs[e] = the token_count
    // outputs of expert e, concatenated (backend.hpp:357-363,
    // backend_cpu.cpp:191-264).
    Result<std::vector<std::vector<float>>> mxfp4_situ_mlp_grid(
        std::span<const float> inputs, std::size_t token_count,
        std::span<const Mxfp4MlpView> experts, float situ_beta, std::optional<float> situ_linear,
        std::uint32_t layer, ProfilePhase phase);
    // One token: sum over slots, in slot order, of contributions[k] *
    // expert k's output (backend.hpp:364-368, backend_cpu.cpp:266-303).
    Result<std::vector<float>> mxfp4_situ_moe(std::span<const float> input,
                                              std::span<const Mxfp4MlpView> experts,
                                              std::span<const float> contributions,
                                              float situ_beta, std::optional<float> situ_linear,
                                              std::uint32_t layer, ProfilePhase phase);
    // mxfp4_situ_moe for token_count tokens in one layer call: token t mixes
    // experts[routes[t * top_k + k]] with contributions[t * top_k + k],
    // k = 0 .. top_k - 1 (no expert twice in one token); returns
    // [token_count][hidden].  The batched call the reference's expert-major
    // verification block makes one group at a time (model.cpp:313-356).
    Result<std::vector<float>> mxfp4_situ_moe_tokens(
        std::span<const float> inputs, std::size_t token_count, std::size_t top_k,
        std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> routes,
        std::span<const float> contributions, float situ_beta, std::optional<float> situ_linear,
        std::uint32_t layer, ProfilePhase phase);

    // The official K3 MoE FFN (Stable LatentMoE) for one token: hidden
    // (the prepared, bf16-valued hidden; other values are rounded to bf16)
    // -> routed_down -> the routed experts at the latent width, mixed in
    // slot order -> routed_norm -> routed_up, plus the shared FFN and the
    // prefix add (backend.hpp:376-383, official_moe.cpp:271-344).  Any
    // pending prepared token is dropped.
    Result<OfficialMoeFfnResult> official_mxfp4_moe_ffn(
        std::span<const float> hidden, std::span<const float> prefix, OfficialMoeFfnView weights,
        std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
        std::span<const float> contributions, float rms_epsilon, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase);
    // Route preparation (backend.hpp:384-389, official_moe.cpp:156-209,
    // :247-269): the two-source mix and post-norm of prefix and
    // block_residual into the hidden, kept on the device for the prepared
    // FFN, and the router logits over it (canonical fp64 sums).  The token
    // names that hidden until it is consumed, discarded or replaced.
    Result<OfficialMoeRoutePrepareResult> prepare_official_moe_route(
        std::span<const float> prefix, std::span<const float> block_residual,
        OfficialMoeRoutePrepareView weights, float rms_epsilon, std::uint32_t layer,
        ProfilePhase phase);
    // The FFN on the prepared hidden and prefix (backend.hpp:390-395);
    // consumes the token.
    Result<OfficialMoeFfnResult> official_mxfp4_moe_ffn_prepared(
        OfficialMoePreparedToken prepared, OfficialMoeFfnView weights,
        std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
        std::span<const float> contributions, float rms_epsilon, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase);
    // Drops the prepared hidden (backend.hpp:396-399): invalid_state unless
    // the token is the pending one.
    Result<bool> discard_official_moe_prepared(OfficialMoePreparedToken prepared);

    // The routed experts of one layer of an expert-major verification block
    // (model.cpp:278-345): position p's latent through the experts of
    // routes[p], mixed in slot order with routes[p].contributions.
    //   * The reference builds the block's expert-major plan and makes one
    //     mxfp4_situ_mlp_batch per group. Here the block takes one grouped
    //     layer call per distinct route width (normally exactly one).
    //   * experts[id] is the view of expert id.
    //   * Routes are checked as build_expert_major_plan checks them
    //     (expert_major.cpp:10-54): invalid_extent for an empty block or
    //     route, invalid_state for a non-finite contribution or an expert
    //     twice in one route.
    //   * unique_experts and assignments are the plan's group and
    //     assignment counts (model.cpp:279-283).
    Result<ExpertMajorBlockMoe> expert_major_block_moe(
        std::span<const float> latents, std::size_t positions,
        std::span<const ExpertMajorTokenRoute> routes, std::span<const Mxfp4MlpView> experts,
        float situ_beta, std::optional<float> situ_linear, std::uint32_t layer,
        ProfilePhase phase);

    // y = W x in fp32 with double sums (backend.hpp:333-335,
    // backend_cpu.cpp:22-45); invalid_extent when the extents disagree.
    Result<std::vector<float>> dense_matvec(std::span<const float> input, DenseWeightView weight,
                                            std::uint32_t layer, ProfilePhase phase);
    // y = W x for one MXFP4 matrix (backend.hpp:336-338, backend_cpu.cpp:
    // 47-59); invalid_mxfp4 for a malformed matrix (a 0xFF scale included),
    // backend_unavailable for a group size other than 32.
    Result<std::vector<float>> mxfp4_matvec(std::span<const float> input, Mxfp4WeightView weight,
                                            std::uint32_t layer, ProfilePhase phase);
    // Every weight checked first, then one product each (backend.hpp:339-344,
    // backend_cpu.cpp:61-106).
    Result<std::vector<std::vector<float>>> dense_matvec_group(
        std::span<const float> input, std::span<const DenseWeightView> weights,
        std::uint32_t layer, ProfilePhase phase);
    Result<std::vector<std::vector<float>>> mxfp4_matvec_group(
        std::span<const float> input, std::span<const Mxfp4WeightView> weights,
        std::uint32_t layer, ProfilePhase phase);
    // down(situ(gate x, up x)) in fp32 (backend.hpp:345-348, backend_cpu.cpp:
    // 108-122).
    Result<std::vector<float>> dense_situ_mlp(std::span<const float> input, DenseMlpView weights,
                                              float situ_beta, std::optional<float> situ_linear,
                                              std::uint32_t layer, ProfilePhase phase);
    // The resident latent MoE layer for one token (backend.hpp:369-375):
    // latent = routed_down x, the experts on the fp32 latent mixed in slot
    // order, RMSNorm with routed_norm, routed_up, plus the fp32 SiTU shared
    // MLP of x (backend_cpu.cpp:305-339).  Arguments are checked as
    // valid_resident_moe_layer (backend_cpu.cpp:441-497, invalid_mxfp4).
    // When the experts or the dense weights cannot all be resident (more
    // experts than bank slots, dense weights over resident_dense_bytes) the
    // call succeeds with executed = false and no output, for the caller's
    // split path (backend_cuda.cu:1995-2003).
    Result<ResidentMoeLayerResult> resident_mxfp4_moe_layer(
        std::span<const float> input, ResidentMoeLayerView weights,
        std::span<const Mxfp4MlpView> experts, std::span<const float> contributions,
        float epsilon, float situ_beta, std::optional<float> situ_linear, std::uint32_t layer,
        ProfilePhase phase);

    HipBackendStats runtime_stats() const noexcept;
    std::string_view device_name() const noexcept;
    // Every later method call reports its operations to `sink` (the
    // reference backends' Profiler::record, backend_cuda.cu:2505-2542); the
    // library's stage timing is on while a sink is set.  An empty sink turns
    // it off.
    void set_profile_sink(ProfileSink sink);

    struct Impl;

private:
    Result<OfficialMoeFfnResult> official_ffn(
        std::span<const float> hidden, std::span<const float> prefix,
        std::optional<OfficialMoePreparedToken> prepared, const OfficialMoeFfnView& weights,
        std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
        std::span<const float> contributions, float rms_epsilon, float situ_beta,
        std::optional<float> situ_linear, std::uint32_t layer);
    friend Result<std::unique_ptr<HipMoeBackend>> make_hip_backend(const HipBackendOptions&);
    explicit HipMoeBackend(std::unique_ptr<Impl> impl);
    std::unique_ptr<Impl> impl_;
};

// The factory beside make_cuda_backend (backend.hpp:465-466).
Result<std::unique_ptr<HipMoeBackend>> make_hip_backend(const HipBackendOptions& options = {});

}  // namespace k3x_amd
