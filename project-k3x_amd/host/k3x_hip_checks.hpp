// k3x_hip_checks.hpp -- argument checks of HipMoeBackend's methods over the
// caller's views, before anything is uploaded or launched.  Host code only
// (no HIP), so a sanitizer build can drive them on the CPU
// (tests/cpp/sanitize_driver.cpp).  Each check cites the reference check it
// follows.
#pragma once

#include <algorithm>
#include <cmath>
#include <initializer_list>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <optional>
#include <span>
#include <vector>

#include "k3x_hip_backend.hpp"

namespace k3x_amd::checks {

inline bool mul_fits(std::size_t a, std::size_t b) {
    return b == 0 || a <= std::numeric_limits<std::size_t>::max() / b;
}

// backend_cpu.cpp:384-402 (valid_mxfp4).
inline bool valid_mxfp4(std::size_t input_size, const Mxfp4WeightView& w) {
    if (input_size != w.cols || !w.rows || !w.cols || !w.group_size || w.cols % w.group_size ||
        w.cols % 2 || !mul_fits(w.rows, w.cols))
        return false;
    const std::size_t elements = w.rows * w.cols;
    if (w.packed.size() != elements / 2 || w.scales.size() != elements / w.group_size)
        return false;
    for (const std::byte s : w.scales)
        if (s == std::byte{0xff}) return false;
    return true;
}

// backend_cpu.cpp:427-433 (valid_mxfp4_mlp).
inline bool valid_mxfp4_mlp(std::size_t input_size, const Mxfp4MlpView& e) {
    return valid_mxfp4(input_size, e.gate) && valid_mxfp4(input_size, e.up) &&
           e.gate.rows == e.up.rows && valid_mxfp4(e.gate.rows, e.down);
}

inline bool valid_situ(float beta, std::optional<float> linear) {
    return std::isfinite(beta) && beta > 0.0f &&
           (!linear || (std::isfinite(*linear) && *linear > 0.0f));
}

// backend_cpu.cpp:365-374 (valid_dense).
inline bool valid_dense(std::size_t input_size, const DenseWeightView& w) {
    if (input_size != w.cols || w.rows > w.values.size() ||
        (w.cols != 0 && w.rows > w.values.size() / w.cols))
        return false;
    return w.values.size() == w.rows * w.cols;
}

// backend_cpu.cpp:410-420 (valid_dense_size: non-empty as well).
inline bool valid_dense_size(std::size_t input_size, const DenseWeightView& w) {
    return w.rows && w.cols && valid_dense(input_size, w);
}

// backend_cpu.cpp:403-408 (valid_dense_mlp).
inline bool valid_dense_mlp(std::size_t input_size, const DenseMlpView& m) {
    return valid_dense(input_size, m.gate) && valid_dense(input_size, m.up) && m.gate.rows != 0 &&
           m.gate.rows == m.up.rows && valid_dense_size(m.gate.rows, m.down);
}

// Tensor ids name one tensor each: views of one call that share a nonzero id
// must be the same tensor (same data, same shape), as the reference's
// resident table keys them (runtime/cuda/resident_weights.cu:107-114).
inline bool consistent_ids(std::initializer_list<const DenseWeightView*> views) {
    for (auto a = views.begin(); a != views.end(); ++a)
        for (auto b = views.begin(); b != a; ++b)
            if ((*a)->tensor_id && (*a)->tensor_id == (*b)->tensor_id &&
                ((*a)->values.data() != (*b)->values.data() ||
                 (*a)->values.size() != (*b)->values.size() || (*a)->rows != (*b)->rows ||
                 (*a)->cols != (*b)->cols))
                return false;
    return true;
}

inline bool all_finite(std::span<const float> v) {
    for (float x : v)
        if (!std::isfinite(x)) return false;
    return true;
}

// valid_resident_moe_layer (backend_cpu.cpp:441-497) without the finiteness
// of the dense weights, which the backend checks when it uploads them.
inline bool valid_resident_layer(std::span<const float> input, const ResidentMoeLayerView& w,
                                 std::span<const Mxfp4MlpView> experts,
                                 std::span<const float> contributions, float epsilon,
                                 float situ_beta, std::optional<float> situ_linear) {
    if (input.empty() || experts.empty() || experts.size() != contributions.size() ||
        !std::isfinite(epsilon) || epsilon <= 0.0f || !valid_situ(situ_beta, situ_linear) ||
        !all_finite(input) || !all_finite(contributions) ||
        !valid_dense(input.size(), w.routed_down) || !valid_dense_mlp(input.size(), w.shared))
        return false;
    const std::size_t H = input.size(), L = w.routed_down.rows, W = experts.front().down.rows;
    if (L == 0 || W == 0 || w.routed_norm.values.size() != W ||
        !valid_dense_size(W, w.routed_up) || w.routed_up.rows != H || w.shared.down.rows != H)
        return false;
    std::vector<std::uint64_t> ids;
    auto insert_id = [&](std::uint64_t id) {
        if (id == 0 || std::find(ids.begin(), ids.end(), id) != ids.end()) return false;
        ids.push_back(id);
        return true;
    };
    if (!insert_id(w.routed_down.tensor_id) || !insert_id(w.routed_norm.tensor_id) ||
        !insert_id(w.routed_up.tensor_id) || !insert_id(w.shared.gate.tensor_id) ||
        !insert_id(w.shared.up.tensor_id) || !insert_id(w.shared.down.tensor_id))
        return false;
    const std::size_t I = experts.front().gate.rows;
    for (const auto& e : experts)
        if (!valid_mxfp4_mlp(L, e) || e.gate.rows != I || e.down.rows != W ||
            e.gate.group_size != 32 || e.up.group_size != 32 || e.down.group_size != 32 ||
            !insert_id(e.gate.tensor_id) || !insert_id(e.up.tensor_id) ||
            !insert_id(e.down.tensor_id))
            return false;
    return true;
}

}  // namespace k3x_amd::checks
