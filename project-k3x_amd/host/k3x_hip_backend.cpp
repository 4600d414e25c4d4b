// k3x_hip_backend.cpp -- HipMoeBackend: the reference's expert-execution
// methods over the C ABI of libk3x_hip_moe.so.  Argument checks follow
// runtime/src/backend_cpu.cpp (valid_mxfp4 :384-402, valid_mxfp4_mlp
// :427-433, the per-method checks of :124-303); the group size 32 rule is
// the CUDA backend's (runtime/cuda/backend_cuda.cu:1865-1867).
#include "k3x_hip_backend.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <tuple>

#include "k3x_hip_moe.h"

namespace k3x_amd {

const char* error_code_name(ErrorCode code) { return k3x_hip_status_name(static_cast<int>(code)); }

namespace {

using Outputs = std::vector<std::vector<float>>;

constexpr std::size_t kMaxSlotsPerToken = 64;  // top_k limit of one layer call
constexpr std::size_t kTokensPerCall = 4096;   // bounds the per-pair output buffer

ErrorCode code_of(int status) { return static_cast<ErrorCode>(status); }

bool mul_fits(std::size_t a, std::size_t b) {
    return b == 0 || a <= std::numeric_limits<std::size_t>::max() / b;
}

// backend_cpu.cpp:384-402.
bool valid_mxfp4(std::size_t input_size, const Mxfp4WeightView& w) {
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

// backend_cpu.cpp:427-433.
bool valid_mxfp4_mlp(std::size_t input_size, const Mxfp4MlpView& e) {
    return valid_mxfp4(input_size, e.gate) && valid_mxfp4(input_size, e.up) &&
           e.gate.rows == e.up.rows && valid_mxfp4(e.gate.rows, e.down);
}

bool valid_situ(float beta, std::optional<float> linear) {
    return std::isfinite(beta) && beta > 0.0f &&
           (!linear || (std::isfinite(*linear) && *linear > 0.0f));
}

bool same_expert(const Mxfp4MlpView& a, const Mxfp4MlpView& b) {
    return a.gate.tensor_id == b.gate.tensor_id && a.up.tensor_id == b.up.tensor_id &&
           a.down.tensor_id == b.down.tensor_id;
}

// fp32 -> bf16 bits, round to nearest even (quiet NaN kept a NaN).
std::uint16_t to_bf16(float f) {
    std::uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (std::uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (std::uint16_t)(u >> 16);
}

const std::uint8_t* bytes(std::span<const std::byte> s) {
    return reinterpret_cast<const std::uint8_t*>(s.data());
}

}  // namespace

struct HipMoeBackend::Impl {
    HipBackendOptions opt;
    k3x_hip_ctx* ctx = nullptr;
    std::string name;
    struct Slot {
        std::uint64_t ids[3] = {0, 0, 0};
        std::uint64_t last_use = 0;
    };
    struct Bank {
        k3x_hip_bank* bank = nullptr;
        std::vector<Slot> slots;
    };
    std::map<std::tuple<std::uint32_t, std::size_t, std::size_t>, Bank> banks;
    std::uint64_t tick = 0;
    HipBackendStats stats;
    struct Dev {
        void* p = nullptr;
        std::size_t bytes = 0;
    };
    Dev xn, ids, w, out, out_f32, pairs;

    ~Impl() {
        for (auto& kv : banks) k3x_hip_bank_destroy(kv.second.bank);
        for (Dev* d : {&xn, &ids, &w, &out, &out_f32, &pairs})
            if (d->p) (void)hipFree(d->p);
        if (ctx) k3x_hip_ctx_destroy(ctx);
    }

    ErrorCode ensure(Dev& d, std::size_t n) {
        if (d.bytes >= n) return ErrorCode::ok;
        if (d.p) (void)hipFree(d.p);
        d.p = nullptr;
        d.bytes = 0;
        if (hipMalloc(&d.p, n) != hipSuccess) {
            (void)hipGetLastError();
            return ErrorCode::backend_unavailable;
        }
        d.bytes = n;
        return ErrorCode::ok;
    }

    // The layer's shapes this library runs: group size 32 (as the CUDA
    // backend), hidden and intermediate multiples of 128, a square layer
    // (down rows = hidden).
    static ErrorCode supported(const Mxfp4MlpView& e) {
        for (const Mxfp4WeightView* m : {&e.gate, &e.up, &e.down})
            if (m->group_size != 32) return ErrorCode::invalid_mxfp4;
        const std::size_t H = e.gate.cols, I = e.gate.rows;
        if (H % 128 || I % 128 || e.down.rows != H || H > (1u << 20) || I > (1u << 20))
            return ErrorCode::backend_unavailable;
        return ErrorCode::ok;
    }

    Result<Bank*> bank_for(std::uint32_t layer, std::size_t H, std::size_t I) {
        auto key = std::make_tuple(layer, H, I);
        auto it = banks.find(key);
        if (it != banks.end()) return Result<Bank*>::success(&it->second);
        k3x_hip_layer_desc d{};
        d.hidden = (std::uint32_t)H;
        d.inter = (std::uint32_t)I;
        d.experts = opt.resident_experts;
        d.group_size = 32;
        d.shared_inter = 0;
        Bank b;
        const int st = k3x_hip_bank_create(ctx, &d, &b.bank);
        if (st) return Result<Bank*>::failure(code_of(st), "bank_create");
        b.slots.resize(opt.resident_experts);
        auto ins = banks.emplace(key, std::move(b));
        return Result<Bank*>::success(&ins.first->second);
    }

    // Maps every expert to a bank slot, admitting the missing ones.
    ErrorCode admit(Bank& b, std::span<const Mxfp4MlpView> experts, std::vector<std::uint32_t>& slot) {
        const std::size_t n = b.slots.size();
        std::vector<char> pinned(n, 0);
        slot.assign(experts.size(), UINT32_MAX);
        auto holds = [&](std::size_t s, const Mxfp4MlpView& e) {
            return b.slots[s].ids[0] == e.gate.tensor_id && b.slots[s].ids[1] == e.up.tensor_id &&
                   b.slots[s].ids[2] == e.down.tensor_id;
        };
        for (std::size_t i = 0; i < experts.size(); ++i)
            for (std::size_t s = 0; s < n; ++s)
                if (holds(s, experts[i])) {
                    slot[i] = (std::uint32_t)s;
                    pinned[s] = 1;
                    ++stats.residency_hits;
                    break;
                }
        for (std::size_t i = 0; i < experts.size(); ++i) {
            if (slot[i] != UINT32_MAX) continue;
            const Mxfp4MlpView& e = experts[i];
            // A duplicate of an expert admitted earlier in this call.
            bool dup = false;
            for (std::size_t s = 0; s < n && !dup; ++s)
                if (pinned[s] && holds(s, e)) {
                    slot[i] = (std::uint32_t)s;
                    dup = true;
                }
            if (dup) continue;
            // A slot holding one of these tensor ids with other companions
            // must be the one replaced (ids are unique within a bank).
            std::size_t victim = n;
            for (std::size_t s = 0; s < n && victim == n; ++s)
                for (std::uint64_t id : b.slots[s].ids)
                    if (id && (id == e.gate.tensor_id || id == e.up.tensor_id ||
                               id == e.down.tensor_id))
                        victim = s;
            if (victim != n && pinned[victim]) return ErrorCode::invalid_mxfp4;
            if (victim == n) {
                std::uint64_t oldest = UINT64_MAX;
                for (std::size_t s = 0; s < n; ++s)
                    if (!pinned[s] && b.slots[s].last_use < oldest) {
                        oldest = b.slots[s].last_use;
                        victim = s;
                    }
            }
            if (victim == n) return ErrorCode::backend_unavailable;  // more experts than slots
            const std::uint64_t tid[3] = {e.gate.tensor_id, e.up.tensor_id, e.down.tensor_id};
            const int st = k3x_hip_bank_upload_expert(
                b.bank, (std::uint32_t)victim, tid, bytes(e.gate.packed), bytes(e.gate.scales),
                bytes(e.up.packed), bytes(e.up.scales), bytes(e.down.packed), bytes(e.down.scales));
            if (st) {
                // Rejected arguments leave the slot as it was; a failure
                // after the slot was touched leaves it empty.
                std::uint32_t at = 0, m = 0;
                if (b.slots[victim].ids[0] &&
                    (k3x_hip_bank_find(b.bank, b.slots[victim].ids[0], &at, &m) != 0 || at != victim))
                    b.slots[victim] = Slot{};
                return code_of(st);
            }
            std::copy(tid, tid + 3, b.slots[victim].ids);
            pinned[victim] = 1;
            slot[i] = (std::uint32_t)victim;
            ++stats.experts_admitted;
            stats.weight_h2d_bytes += e.gate.packed.size() + e.gate.scales.size() +
                                      e.up.packed.size() + e.up.scales.size() +
                                      e.down.packed.size() + e.down.scales.size();
        }
        ++tick;
        for (std::size_t s = 0; s < n; ++s)
            if (pinned[s]) b.slots[s].last_use = tick;
        return ErrorCode::ok;
    }

    // One layer call: T tokens, K slots each, routes index `experts`
    // (distinct within a token), weights = contributions (or 1).  Fills
    // pairs_out [T][K][H] and/or mix_out [T][H].
    ErrorCode run(std::uint32_t layer, std::span<const float> inputs, std::size_t T,
                  std::size_t K, std::span<const Mxfp4MlpView> experts,
                  std::span<const std::uint32_t> routes, std::span<const float> contributions,
                  float beta, std::optional<float> linear, std::vector<float>* pairs_out,
                  std::vector<float>* mix_out) {
        const std::size_t H = experts.front().gate.cols, I = experts.front().gate.rows;
        auto bank = bank_for(layer, H, I);
        if (!bank) return bank.error();
        std::vector<std::uint32_t> slot;
        if (ErrorCode c = admit(*bank.value(), experts, slot); c != ErrorCode::ok) return c;
        std::vector<std::uint32_t> hid(T * K);
        std::vector<float> hw(T * K, 1.0f);
        for (std::size_t p = 0; p < T * K; ++p) {
            hid[p] = slot[routes[p]];
            if (!contributions.empty()) hw[p] = contributions[p];
        }
        std::vector<std::uint16_t> xb(T * H);
        for (std::size_t i = 0; i < T * H; ++i) xb[i] = to_bf16(inputs[i]);
        for (auto [d, n] : {std::pair<Dev*, std::size_t>{&xn, T * H * 2}, {&ids, T * K * 4},
                            {&w, T * K * 4}, {&out, T * H * 2}})
            if (ErrorCode c = ensure(*d, n); c != ErrorCode::ok) return c;
        if (mix_out)
            if (ErrorCode c = ensure(out_f32, T * H * 4); c != ErrorCode::ok) return c;
        if (pairs_out)
            if (ErrorCode c = ensure(pairs, T * K * H * 4); c != ErrorCode::ok) return c;
        if (hipMemcpy(xn.p, xb.data(), T * H * 2, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(ids.p, hid.data(), T * K * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(w.p, hw.data(), T * K * 4, hipMemcpyHostToDevice) != hipSuccess)
            return ErrorCode::backend_unavailable;
        k3x_hip_moe_params p{};
        p.tokens = (std::uint32_t)T;
        p.top_k = (std::uint32_t)K;
        p.routed_scale = 1.0f;
        p.rms_epsilon = 1e-6f;
        p.glu = K3X_GLU_SITU;
        p.situ_beta = beta;
        p.has_situ_linear = linear.has_value();
        p.situ_linear_beta = linear.value_or(0.0f);
        p.renorm = K3X_RENORM_FLOAT;
        k3x_hip_moe_taps taps{};
        taps.expert_out = pairs_out ? static_cast<float*>(pairs.p) : nullptr;
        taps.out_f32 = mix_out ? static_cast<float*>(out_f32.p) : nullptr;
        int st = k3x_hip_moe_forward_routed(
            ctx, bank.value()->bank, &p, static_cast<const std::uint16_t*>(xn.p),
            static_cast<const std::uint32_t*>(ids.p), static_cast<const float*>(w.p), hid.data(),
            hw.data(), static_cast<std::uint16_t*>(out.p), &taps);
        if (!st) st = k3x_hip_ctx_synchronize(ctx);
        if (st) return code_of(st);
        ++stats.layer_calls;
        if (pairs_out) {
            pairs_out->resize(T * K * H);
            if (hipMemcpy(pairs_out->data(), pairs.p, T * K * H * 4, hipMemcpyDeviceToHost) !=
                hipSuccess)
                return ErrorCode::backend_unavailable;
        }
        if (mix_out) {
            mix_out->resize(T * H);
            if (hipMemcpy(mix_out->data(), out_f32.p, T * H * 4, hipMemcpyDeviceToHost) !=
                hipSuccess)
                return ErrorCode::backend_unavailable;
        }
        return ErrorCode::ok;
    }

    // Per-expert outputs of T tokens through every expert of `experts`
    // (distinct), in chunks of at most 64 experts and kTokensPerCall tokens:
    // out[e][t * H + h].
    ErrorCode grid(std::uint32_t layer, std::span<const float> inputs, std::size_t T,
                   std::span<const Mxfp4MlpView> experts, float beta,
                   std::optional<float> linear, Outputs& out) {
        const std::size_t H = experts.front().gate.cols;
        out.assign(experts.size(), std::vector<float>(T * H));
        for (std::size_t e0 = 0; e0 < experts.size(); e0 += kMaxSlotsPerToken) {
            const std::size_t K = std::min(kMaxSlotsPerToken, experts.size() - e0);
            const auto chunk = experts.subspan(e0, K);
            for (std::size_t t0 = 0; t0 < T; t0 += kTokensPerCall) {
                const std::size_t Tc = std::min(kTokensPerCall, T - t0);
                std::vector<std::uint32_t> routes(Tc * K);
                for (std::size_t t = 0; t < Tc; ++t)
                    for (std::size_t k = 0; k < K; ++k) routes[t * K + k] = (std::uint32_t)k;
                std::vector<float> pairs_out;
                if (ErrorCode c = run(layer, inputs.subspan(t0 * H, Tc * H), Tc, K, chunk, routes,
                                      {}, beta, linear, &pairs_out, nullptr);
                    c != ErrorCode::ok)
                    return c;
                for (std::size_t t = 0; t < Tc; ++t)
                    for (std::size_t k = 0; k < K; ++k)
                        std::copy_n(pairs_out.data() + (t * K + k) * H, H,
                                    out[e0 + k].data() + (t0 + t) * H);
            }
        }
        return ErrorCode::ok;
    }
};

HipMoeBackend::HipMoeBackend(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
HipMoeBackend::~HipMoeBackend() = default;

Result<std::unique_ptr<HipMoeBackend>> make_hip_backend(const HipBackendOptions& options) {
    using R = Result<std::unique_ptr<HipMoeBackend>>;
    if (!options.resident_experts) return R::failure(ErrorCode::invalid_extent, "resident_experts");
    auto impl = std::make_unique<HipMoeBackend::Impl>();
    impl->opt = options;
    if (int st = k3x_hip_ctx_create(options.device, &impl->ctx)) {
        impl->ctx = nullptr;
        return R::failure(code_of(st), "k3x_hip_ctx_create");
    }
    hipDeviceProp_t prop{};
    if (hipGetDeviceProperties(&prop, options.device) == hipSuccess)
        impl->name = prop.name[0] ? prop.name : prop.gcnArchName;  // no marketing-name table
    return R::success(std::unique_ptr<HipMoeBackend>(new HipMoeBackend(std::move(impl))));
}

Result<Outputs> HipMoeBackend::mxfp4_situ_mlp_group(std::span<const float> input,
                                                    std::span<const Mxfp4MlpView> experts,
                                                    float situ_beta,
                                                    std::optional<float> situ_linear,
                                                    std::uint32_t layer, ProfilePhase) {
    for (const auto& e : experts)
        if (!valid_mxfp4_mlp(input.size(), e)) return Result<Outputs>::failure(ErrorCode::invalid_mxfp4);
    if (experts.empty()) return Result<Outputs>::success({});
    for (const auto& e : experts)
        if (ErrorCode c = Impl::supported(e); c != ErrorCode::ok) return Result<Outputs>::failure(c);
    for (const auto& e : experts)
        if (e.gate.cols != experts.front().gate.cols || e.gate.rows != experts.front().gate.rows)
            return Result<Outputs>::failure(ErrorCode::backend_unavailable, "mixed shapes");
    // Each distinct expert once (a layer call takes an expert once per token).
    std::vector<Mxfp4MlpView> uniq;
    std::vector<std::size_t> of(experts.size());
    for (std::size_t i = 0; i < experts.size(); ++i) {
        std::size_t u = 0;
        while (u < uniq.size() && !same_expert(uniq[u], experts[i])) ++u;
        if (u == uniq.size()) uniq.push_back(experts[i]);
        of[i] = u;
    }
    Outputs per;
    if (ErrorCode c = impl_->grid(layer, input, 1, uniq, situ_beta, situ_linear, per); c != ErrorCode::ok)
        return Result<Outputs>::failure(c);
    ++impl_->stats.calls;
    Outputs out(experts.size());
    for (std::size_t i = 0; i < experts.size(); ++i) out[i] = per[of[i]];
    return Result<Outputs>::success(std::move(out));
}

Result<Outputs> HipMoeBackend::mxfp4_situ_mlp_batch(std::span<const float> inputs,
                                                    std::size_t batch_size, Mxfp4MlpView expert,
                                                    float situ_beta,
                                                    std::optional<float> situ_linear,
                                                    std::uint32_t layer, ProfilePhase) {
    // backend_cpu.cpp:161-171.
    if (batch_size == 0 || expert.gate.cols == 0 || !mul_fits(batch_size, expert.gate.cols) ||
        inputs.size() != batch_size * expert.gate.cols || !valid_situ(situ_beta, situ_linear) ||
        !valid_mxfp4_mlp(expert.gate.cols, expert))
        return Result<Outputs>::failure(ErrorCode::invalid_mxfp4);
    if (ErrorCode c = Impl::supported(expert); c != ErrorCode::ok) return Result<Outputs>::failure(c);
    Outputs per;
    const Mxfp4MlpView one[1] = {expert};
    if (ErrorCode c = impl_->grid(layer, inputs, batch_size, one, situ_beta, situ_linear, per);
        c != ErrorCode::ok)
        return Result<Outputs>::failure(c);
    ++impl_->stats.calls;
    const std::size_t H = expert.down.rows;
    Outputs out(batch_size);
    for (std::size_t t = 0; t < batch_size; ++t)
        out[t].assign(per[0].begin() + t * H, per[0].begin() + (t + 1) * H);
    return Result<Outputs>::success(std::move(out));
}

Result<Outputs> HipMoeBackend::mxfp4_situ_mlp_grid(std::span<const float> inputs,
                                                   std::size_t token_count,
                                                   std::span<const Mxfp4MlpView> experts,
                                                   float situ_beta,
                                                   std::optional<float> situ_linear,
                                                   std::uint32_t layer, ProfilePhase) {
    // backend_cpu.cpp:197-246.
    using R = Result<Outputs>;
    if (token_count == 0 || experts.empty() || experts.front().gate.cols == 0 ||
        !mul_fits(token_count, experts.front().gate.cols) ||
        inputs.size() != token_count * experts.front().gate.cols ||
        !valid_situ(situ_beta, situ_linear))
        return R::failure(ErrorCode::invalid_mxfp4);
    const std::size_t in_w = experts.front().gate.cols, mid_w = experts.front().gate.rows,
                      out_w = experts.front().down.rows;
    std::vector<std::uint64_t> seen;
    for (const auto& e : experts) {
        if (e.gate.cols != in_w || e.gate.rows != mid_w || e.up.cols != in_w ||
            e.up.rows != mid_w || e.down.cols != mid_w || e.down.rows != out_w ||
            !valid_mxfp4_mlp(in_w, e))
            return R::failure(ErrorCode::invalid_mxfp4);
        for (std::uint64_t id : {e.gate.tensor_id, e.up.tensor_id, e.down.tensor_id}) {
            if (id == 0 || std::find(seen.begin(), seen.end(), id) != seen.end())
                return R::failure(ErrorCode::invalid_mxfp4);
            seen.push_back(id);
        }
    }
    if (!mul_fits(token_count, out_w)) return R::failure(ErrorCode::invalid_mxfp4);
    if (ErrorCode c = Impl::supported(experts.front()); c != ErrorCode::ok) return R::failure(c);
    Outputs out;
    if (ErrorCode c = impl_->grid(layer, inputs, token_count, experts, situ_beta, situ_linear, out);
        c != ErrorCode::ok)
        return R::failure(c);
    ++impl_->stats.calls;
    return R::success(std::move(out));
}

Result<std::vector<float>> HipMoeBackend::mxfp4_situ_moe(std::span<const float> input,
                                                         std::span<const Mxfp4MlpView> experts,
                                                         std::span<const float> contributions,
                                                         float situ_beta,
                                                         std::optional<float> situ_linear,
                                                         std::uint32_t layer, ProfilePhase phase) {
    // backend_cpu.cpp:271-288.
    using R = Result<std::vector<float>>;
    if (experts.empty() || experts.size() != contributions.size())
        return R::failure(ErrorCode::invalid_mxfp4);
    for (float c : contributions)
        if (!std::isfinite(c)) return R::failure(ErrorCode::invalid_mxfp4);
    const std::size_t out_rows = experts.front().down.rows;
    for (const auto& e : experts)
        if (!valid_mxfp4_mlp(input.size(), e) || e.down.rows != out_rows)
            return R::failure(ErrorCode::invalid_mxfp4);
    bool distinct = experts.size() <= kMaxSlotsPerToken;
    for (std::size_t i = 0; i < experts.size() && distinct; ++i)
        for (std::size_t j = 0; j < i && distinct; ++j) distinct = !same_expert(experts[i], experts[j]);
    if (!distinct) {
        // An expert twice (or more slots than one layer call takes): the
        // per-expert outputs, mixed here in slot order as backend_cpu.cpp
        // :294-301 does.
        auto outs = mxfp4_situ_mlp_group(input, experts, situ_beta, situ_linear, layer, phase);
        if (!outs) return R::failure(outs.error(), outs.message());
        std::vector<float> mixed(out_rows, 0.0f);
        for (std::size_t e = 0; e < experts.size(); ++e)
            for (std::size_t r = 0; r < out_rows; ++r)
                mixed[r] = mixed[r] + contributions[e] * outs.value()[e][r];
        return R::success(std::move(mixed));
    }
    for (const auto& e : experts)
        if (ErrorCode c = Impl::supported(e); c != ErrorCode::ok) return R::failure(c);
    for (const auto& e : experts)
        if (e.gate.cols != experts.front().gate.cols || e.gate.rows != experts.front().gate.rows)
            return R::failure(ErrorCode::backend_unavailable, "mixed shapes");
    if (!valid_situ(situ_beta, situ_linear)) return R::failure(ErrorCode::invalid_mxfp4);
    std::vector<std::uint32_t> routes(experts.size());
    for (std::size_t k = 0; k < routes.size(); ++k) routes[k] = (std::uint32_t)k;
    std::vector<float> mixed;
    if (ErrorCode c = impl_->run(layer, input, 1, experts.size(), experts, routes, contributions,
                                 situ_beta, situ_linear, nullptr, &mixed);
        c != ErrorCode::ok)
        return R::failure(c);
    ++impl_->stats.calls;
    return R::success(std::move(mixed));
}

Result<std::vector<float>> HipMoeBackend::mxfp4_situ_moe_tokens(
    std::span<const float> inputs, std::size_t token_count, std::size_t top_k,
    std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> routes,
    std::span<const float> contributions, float situ_beta, std::optional<float> situ_linear,
    std::uint32_t layer, ProfilePhase) {
    using R = Result<std::vector<float>>;
    if (token_count == 0 || top_k == 0 || top_k > kMaxSlotsPerToken || experts.empty() ||
        !mul_fits(token_count, top_k) || routes.size() != token_count * top_k ||
        contributions.size() != token_count * top_k || !valid_situ(situ_beta, situ_linear))
        return R::failure(ErrorCode::invalid_mxfp4);
    const std::size_t H = experts.front().gate.cols, I = experts.front().gate.rows;
    if (!mul_fits(token_count, H) || inputs.size() != token_count * H)
        return R::failure(ErrorCode::invalid_mxfp4);
    for (const auto& e : experts)
        if (!valid_mxfp4_mlp(H, e) || e.gate.rows != I || e.down.rows != experts.front().down.rows)
            return R::failure(ErrorCode::invalid_mxfp4);
    for (float c : contributions)
        if (!std::isfinite(c)) return R::failure(ErrorCode::invalid_mxfp4);
    // Routes: in range, no expert twice in one token (expert_major.cpp:30-35).
    for (std::size_t t = 0; t < token_count; ++t)
        for (std::size_t k = 0; k < top_k; ++k) {
            const std::uint32_t r = routes[t * top_k + k];
            if (r >= experts.size()) return R::failure(ErrorCode::invalid_state);
            for (std::size_t q = 0; q < k; ++q)
                if (same_expert(experts[routes[t * top_k + q]], experts[r]))
                    return R::failure(ErrorCode::invalid_state);
        }
    if (ErrorCode c = Impl::supported(experts.front()); c != ErrorCode::ok) return R::failure(c);
    std::vector<float> out(token_count * H);
    for (std::size_t t0 = 0; t0 < token_count; t0 += kTokensPerCall) {
        const std::size_t Tc = std::min(kTokensPerCall, token_count - t0);
        std::vector<float> mixed;
        if (ErrorCode c = impl_->run(layer, inputs.subspan(t0 * H, Tc * H), Tc, top_k, experts,
                                     routes.subspan(t0 * top_k, Tc * top_k),
                                     contributions.subspan(t0 * top_k, Tc * top_k), situ_beta,
                                     situ_linear, nullptr, &mixed);
            c != ErrorCode::ok)
            return R::failure(c);
        std::copy(mixed.begin(), mixed.end(), out.begin() + t0 * H);
    }
    ++impl_->stats.calls;
    return R::success(std::move(out));
}

HipBackendStats HipMoeBackend::runtime_stats() const noexcept {
    HipBackendStats s = impl_->stats;
    k3x_hip_stats cs{};
    if (k3x_hip_ctx_stats(impl_->ctx, &cs) == 0) s.kernel_launches = cs.kernel_launches;
    return s;
}

std::string_view HipMoeBackend::device_name() const noexcept { return impl_->name; }

}  // namespace k3x_amd
