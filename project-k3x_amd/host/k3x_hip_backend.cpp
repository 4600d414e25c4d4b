// k3x_hip_backend.cpp -- HipMoeBackend: the reference's expert-execution
// methods over the C ABI of libk3x_hip_moe.so.  Argument checks follow
// runtime/src/backend_cpu.cpp (valid_mxfp4 :384-402, valid_mxfp4_mlp
// :427-433, the per-method checks of :124-303); the group size 32 rule is
// the CUDA backend's (runtime/cuda/backend_cuda.cu:1865-1867).
#include "k3x_hip_backend.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <tuple>

#include "k3x_hip_checks.hpp"
#include "k3x_hip_moe.h"

namespace k3x_amd {

const char* error_code_name(ErrorCode code) { return k3x_hip_status_name(static_cast<int>(code)); }

namespace {

using Outputs = std::vector<std::vector<float>>;

constexpr std::size_t kMaxSlotsPerToken = 64;  // top_k limit of one layer call
constexpr std::size_t kTokensPerCall = 4096;   // bounds the per-pair output buffer

ErrorCode code_of(int status) { return static_cast<ErrorCode>(status); }

using checks::mul_fits;
using checks::valid_dense;
using checks::valid_dense_mlp;
using checks::valid_dense_size;
using checks::valid_mxfp4;
using checks::valid_mxfp4_mlp;
using checks::valid_situ;
using checks::all_finite;

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

// Widths of the bank's tile layout: multiples of 128 (one MFMA tile of K).
std::size_t pad128(std::size_t n) { return (n + 127) / 128 * 128; }

// An MXFP4 matrix [rows][cols] in the reference layout (cols % 32 == 0) as
// [prows][pcols]: zero codes in the added rows and columns (+0.0 whatever
// the scale) and scale byte 127 (1.0) in their blocks.
void pad_mxfp4(const Mxfp4WeightView& m, std::size_t prows, std::size_t pcols,
               std::vector<std::uint8_t>& packed, std::vector<std::uint8_t>& scales) {
    packed.assign(prows * pcols / 2, 0);
    scales.assign(prows * pcols / 32, 127);
    for (std::size_t r = 0; r < m.rows; ++r) {
        std::memcpy(packed.data() + r * pcols / 2, bytes(m.packed) + r * m.cols / 2, m.cols / 2);
        std::memcpy(scales.data() + r * pcols / 32, bytes(m.scales) + r * m.cols / 32, m.cols / 32);
    }
}

// fp32 row-major [rows][cols] as [prows][pcols], zeros added.
std::vector<float> pad_dense(std::span<const float> v, std::size_t rows, std::size_t cols,
                             std::size_t prows, std::size_t pcols) {
    std::vector<float> out(prows * pcols, 0.0f);
    for (std::size_t r = 0; r < rows; ++r)
        std::memcpy(out.data() + r * pcols, v.data() + r * cols, cols * sizeof(float));
    return out;
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
    // One bank per (layer, hidden, intermediate): widths padded to
    // multiples of 128 (hp, ip) when the layer's are not; the padded rows
    // and columns hold zero codes, and callers pad activations with zeros.
    struct Bank {
        k3x_hip_bank* bank = nullptr;
        std::vector<Slot> slots;
        std::size_t h = 0, i = 0, hp = 0, ip = 0;
        bool padded() const { return h != hp || i != ip; }
    };
    std::map<std::tuple<std::uint32_t, std::size_t, std::size_t>, Bank> banks;
    std::uint64_t tick = 0;
    HipBackendStats stats;
    struct Dev {
        void* p = nullptr;
        std::size_t bytes = 0;
    };
    Dev xn, ids, w, out, out_f32, pairs;

    // Resident single matrices (fp32 dense weights, row-major MXFP4
    // matrices), keyed by tensor id; identity = host data, bytes and shape,
    // and a changed identity is uploaded again.  Least recently used first
    // out within opt.resident_dense_bytes; entries used by the current call
    // (last_use == dense_tick) stay.
    struct Resident {
        void* p = nullptr;
        std::size_t bytes = 0;
        const void* host = nullptr;
        std::size_t host_bytes = 0, rows = 0, cols = 0;
        std::uint64_t last_use = 0;
    };
    std::map<std::uint64_t, Resident> resident;
    std::uint64_t resident_total = 0;
    std::uint64_t dense_tick = 0;
    Dev transient[3], vin, vout, vact, vids, vc;

    // Official layer: per layer, a route-only object for the preparation;
    // per (layer, H, L, I, Is), the FFN object over a bank of latent experts.
    // Dense weights are uploaded again when a tensor id or its host data
    // changes.
    struct WeightKey {
        std::uint64_t id = 0;
        const void* data = nullptr;
        bool operator==(const WeightKey&) const = default;
    };
    struct OfficialRoute {
        k3x_hip_official* obj = nullptr;
        std::size_t H = 0, E = 0;
        WeightKey keys[4];
    };
    struct OfficialFfn {
        Bank bank;
        k3x_hip_official* obj = nullptr;
        WeightKey keys[6];
    };
    std::map<std::uint32_t, OfficialRoute> official_routes;
    std::map<std::tuple<std::uint32_t, std::size_t, std::size_t, std::size_t, std::size_t>,
             OfficialFfn>
        official_ffns;
    // The pending prepared token and its device hidden (bf16) and prefix.
    bool prepared_active = false;
    std::uint64_t prepared_generation = 0;
    std::uint32_t prepared_layer = 0;
    std::size_t prepared_width = 0;
    Dev prep_prefix, prep_block, prep_hidden, prep_logits, o_hidden, o_prefix, o_ids, o_contrib,
        o_out;

    // Device bytes held now: the banks (routed and official), the resident
    // single matrices, the per-call buffers and the context's scratch.
    std::uint64_t device_bytes(std::uint64_t ctx_scratch) const {
        std::uint64_t n = ctx_scratch + resident_total;
        for (const auto& kv : banks) n += k3x_hip_bank_bytes(kv.second.bank);
        for (const auto& kv : official_ffns) n += k3x_hip_bank_bytes(kv.second.bank.bank);
        for (const Dev* d : {&xn, &ids, &w, &out, &out_f32, &pairs, &prep_prefix, &prep_block,
                             &prep_hidden, &prep_logits, &o_hidden, &o_prefix, &o_ids, &o_contrib,
                             &o_out, &transient[0], &transient[1], &transient[2], &vin, &vout,
                             &vact, &vids, &vc})
            n += d->bytes;
        return n;
    }

    ~Impl() {
        for (auto& kv : official_ffns) {
            k3x_hip_official_destroy(kv.second.obj);
            k3x_hip_bank_destroy(kv.second.bank.bank);
        }
        for (auto& kv : official_routes) k3x_hip_official_destroy(kv.second.obj);
        for (auto& kv : banks) k3x_hip_bank_destroy(kv.second.bank);
        for (Dev* d : {&xn, &ids, &w, &out, &out_f32, &pairs, &prep_prefix, &prep_block,
                       &prep_hidden, &prep_logits, &o_hidden, &o_prefix, &o_ids, &o_contrib,
                       &o_out, &transient[0], &transient[1], &transient[2], &vin, &vout, &vact,
                       &vids, &vc})
            if (d->p) (void)hipFree(d->p);
        for (auto& kv : resident) (void)hipFree(kv.second.p);
        if (ctx) k3x_hip_ctx_destroy(ctx);
    }

    std::uint64_t owner() const { return reinterpret_cast<std::uintptr_t>(this); }

    // Profile events of the current call (set_profile_sink).
    ProfileSink sink;
    ProfilePhase call_phase = ProfilePhase::decode;
    using Clock = std::chrono::steady_clock;
    static std::uint64_t ns_since(Clock::time_point t0) {
        return (std::uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now() - t0)
            .count();
    }
    void emit(ProfileOperation op, NumericPrecision pr, std::uint32_t layer, std::uint64_t wall,
              std::uint64_t device, std::uint64_t logical, std::uint64_t transfer, bool ok = true) {
        if (sink) sink(ProfileEvent{call_phase, op, pr, layer, wall, device, logical, transfer, ok});
    }
    // One call without stage events: its launch-to-completion time on its
    // main operation (op, the bytes it reads), then the rest of its
    // operations' bytes with no time of their own.
    struct OpBytes {
        ProfileOperation op;
        NumericPrecision precision;
        std::uint64_t bytes;
    };
    void emit_call(std::uint32_t layer, Clock::time_point t0, std::initializer_list<OpBytes> ops) {
        if (!sink) return;
        const std::uint64_t t = ns_since(t0);
        bool first = true;
        for (const OpBytes& o : ops) {
            emit(o.op, o.precision, layer, t, first ? t : 0, o.bytes, 0);
            first = false;
        }
    }
    // The library's stage totals since the last read, cleared.
    void take_stage_ms(double (&ms)[K3X_STAGE_COUNT]) {
        std::uint64_t n[K3X_STAGE_COUNT];
        if (!ctx || k3x_hip_ctx_stage_times(ctx, ms, n, 1) != 0)
            for (double& v : ms) v = 0.0;
    }
    // Events of one layer call from its stages: routed gate/up (+ the fused
    // GLU) and down as mxfp4_matvec over the distinct experts' weights, the
    // slot-ordered combine as moe_mix, the decode front as rms_norm.
    void emit_layer_stages(std::uint32_t layer, std::uint64_t wall, std::size_t experts,
                           std::size_t T, std::size_t K, std::size_t H, std::size_t I) {
        double ms[K3X_STAGE_COUNT];
        take_stage_ms(ms);
        const std::uint64_t gu = experts * 2 * (I * H / 2 + I * H / 32) + T * H * 2;
        const std::uint64_t dn = experts * (H * I / 2 + H * I / 32) + T * K * I * 2;
        auto ns = [&](int a, int b) { return (std::uint64_t)((ms[a] + ms[b]) * 1e6); };
        const auto fp4 = NumericPrecision::mxfp4_e2m1_e8m0;
        if (ms[K3X_STAGE_DECODE_FRONT] > 0 || ms[K3X_STAGE_ROUTE] > 0)
            emit(ProfileOperation::rms_norm, NumericPrecision::bf16_rounded, layer, wall,
                 ns(K3X_STAGE_DECODE_FRONT, K3X_STAGE_ROUTE), T * H * 2, 0);
        emit(ProfileOperation::mxfp4_matvec, fp4, layer, wall,
             ns(K3X_STAGE_GATE_UP, K3X_STAGE_DECODE_GATE_UP), gu, 0);
        emit(ProfileOperation::mxfp4_matvec, fp4, layer, wall,
             ns(K3X_STAGE_DOWN, K3X_STAGE_DECODE_DOWN), dn, 0);
        if (ms[K3X_STAGE_COMBINE] > 0)
            emit(ProfileOperation::moe_mix, NumericPrecision::fp32, layer, wall,
                 (std::uint64_t)(ms[K3X_STAGE_COMBINE] * 1e6), T * K * H * 4 + T * K * 4, 0);
    }

    // A shape the device path does not run, found before any device work.
    template <class R>
    R decline(const char* what) {
        ++stats.declined_shapes;
        return R::declined_shape(what);
    }
    // supported()'s answer as a method result: backend_unavailable is a
    // declined shape, anything else a failure.
    template <class R>
    R shape_failure(ErrorCode c, const char* what) {
        return c == ErrorCode::backend_unavailable ? decline<R>(what) : R::failure(c);
    }

    ErrorCode ensure(Dev& d, std::size_t n) {
        if (!ctx) return ErrorCode::backend_unavailable;  // no device attached
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

    // One matrix as device bytes: its host segments (data, bytes) placed
    // 256-byte aligned one after the other.  `check` (may be null) runs on
    // the host data before any upload and rejects it with its error code.
    // Returns the device base, or nullptr with ok when the resident budget
    // cannot hold it (then `fallback`, if given, receives a transient copy).
    // `identity` (default: the first segment's data) is the host tensor the
    // entry stands for, when the segments are a padded copy of it.
    struct Segment {
        const void* data;
        std::size_t bytes;
    };
    template <typename Check>
    ErrorCode acquire(std::uint64_t id, std::initializer_list<Segment> segs, std::size_t rows,
                      std::size_t cols, Check check, Dev* fallback, const void** out,
                      const void* identity = nullptr) {
        *out = nullptr;
        std::size_t total = 0;
        for (const Segment& g : segs) total += (g.bytes + 255) & ~(std::size_t)255;
        const Segment first{identity ? identity : segs.begin()->data, segs.begin()->bytes};
        // Tensor id 0 names no tensor (the reference's convenience overloads
        // pass it): always a transient copy.
        auto it = id ? resident.find(id) : resident.end();
        if (it != resident.end() && it->second.host == first.data &&
            it->second.host_bytes == total && it->second.rows == rows && it->second.cols == cols) {
            it->second.last_use = dense_tick;
            *out = it->second.p;
            return ErrorCode::ok;
        }
        if (ErrorCode c = check(); c != ErrorCode::ok) return c;
        if (it != resident.end()) {
            // Tensor ids name one tensor: another shape under a resident id
            // is rejected, as the reference table's compatible() does
            // (runtime/cuda/resident_weights.cu:110-114); and an entry this
            // call already uses is never freed under it (one id given for two
            // different host tensors in one call).
            if (it->second.rows != rows || it->second.cols != cols ||
                it->second.host_bytes != total || it->second.last_use == dense_tick)
                return ErrorCode::invalid_extent;
        }
        if (!ctx) return ErrorCode::backend_unavailable;  // no device attached
        if (it != resident.end()) {  // same id and shape, other host data: replaced
            (void)hipFree(it->second.p);
            resident_total -= it->second.bytes;
            resident.erase(it);
        }
        void* dst = nullptr;
        const bool fits_budget = id != 0 && total <= opt.resident_dense_bytes;
        while (fits_budget && resident_total + total > opt.resident_dense_bytes) {
            auto victim = resident.end();
            for (auto r = resident.begin(); r != resident.end(); ++r)
                if (r->second.last_use != dense_tick &&
                    (victim == resident.end() || r->second.last_use < victim->second.last_use))
                    victim = r;
            if (victim == resident.end()) break;
            (void)hipFree(victim->second.p);
            resident_total -= victim->second.bytes;
            resident.erase(victim);
        }
        if (fits_budget && resident_total + total <= opt.resident_dense_bytes) {
            if (hipMalloc(&dst, total) != hipSuccess) {
                (void)hipGetLastError();
                dst = nullptr;
            }
        }
        if (!dst) {
            if (!fallback) return ErrorCode::ok;  // not resident: the caller bypasses
            if (ErrorCode c = ensure(*fallback, total); c != ErrorCode::ok) return c;
            dst = fallback->p;
        }
        std::size_t at = 0;
        for (const Segment& g : segs) {
            if (g.bytes && hipMemcpy(static_cast<std::uint8_t*>(dst) + at, g.data, g.bytes,
                                     hipMemcpyHostToDevice) != hipSuccess)
                return ErrorCode::backend_unavailable;
            at += (g.bytes + 255) & ~(std::size_t)255;
        }
        stats.weight_h2d_bytes += total;
        ++stats.dense_uploads;
        if (!fallback || dst != fallback->p) {
            Resident r;
            r.p = dst;
            r.bytes = total;
            r.host = first.data;
            r.host_bytes = total;
            r.rows = rows;
            r.cols = cols;
            r.last_use = dense_tick;
            resident[id] = r;
            resident_total += total;
        }
        *out = dst;
        return ErrorCode::ok;
    }

    ErrorCode upload(Dev& d, const void* host, std::size_t bytes) {
        if (ErrorCode c = ensure(d, std::max<std::size_t>(bytes, 16)); c != ErrorCode::ok) return c;
        return hipMemcpy(d.p, host, bytes, hipMemcpyHostToDevice) == hipSuccess
                   ? ErrorCode::ok
                   : ErrorCode::backend_unavailable;
    }

    ErrorCode finish(const Dev& d, std::vector<float>& out, std::size_t n) {
        if (int st = k3x_hip_ctx_synchronize(ctx)) return code_of(st);
        out.resize(n);
        return hipMemcpy(out.data(), d.p, n * 4, hipMemcpyDeviceToHost) == hipSuccess
                   ? ErrorCode::ok
                   : ErrorCode::backend_unavailable;
    }

    // The layer's shapes this library runs: group size 32 (as the CUDA
    // backend; another is invalid_mxfp4), any hidden and intermediate the
    // MXFP4 format allows (multiples of 32; the bank pads them to multiples
    // of 128 with zero codes), a square layer (down rows = hidden); other
    // shapes are backend_unavailable, which the methods return as declined.
    static ErrorCode supported(const Mxfp4MlpView& e) {
        for (const Mxfp4WeightView* m : {&e.gate, &e.up, &e.down})
            if (m->group_size != 32) return ErrorCode::invalid_mxfp4;
        const std::size_t H = e.gate.cols, I = e.gate.rows;
        if (H % 32 || I % 32 || e.down.rows != H || H > (1u << 20) || I > (1u << 20))
            return ErrorCode::backend_unavailable;
        return ErrorCode::ok;
    }

    Result<Bank*> bank_for(std::uint32_t layer, std::size_t H, std::size_t I) {
        auto key = std::make_tuple(layer, H, I);
        auto it = banks.find(key);
        if (it != banks.end()) return Result<Bank*>::success(&it->second);
        if (!ctx) return Result<Bank*>::failure(ErrorCode::backend_unavailable, "no device");
        k3x_hip_layer_desc d{};
        d.hidden = (std::uint32_t)pad128(H);
        d.inter = (std::uint32_t)pad128(I);
        d.experts = opt.resident_experts;
        d.group_size = 32;
        d.shared_inter = 0;
        Bank b;
        b.h = H;
        b.i = I;
        b.hp = d.hidden;
        b.ip = d.inter;
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
            int st;
            if (b.padded()) {
                std::vector<std::uint8_t> p[6];
                pad_mxfp4(e.gate, b.ip, b.hp, p[0], p[1]);
                pad_mxfp4(e.up, b.ip, b.hp, p[2], p[3]);
                pad_mxfp4(e.down, b.hp, b.ip, p[4], p[5]);
                st = k3x_hip_bank_upload_expert(b.bank, (std::uint32_t)victim, tid, p[0].data(),
                                                p[1].data(), p[2].data(), p[3].data(),
                                                p[4].data(), p[5].data());
            } else {
                st = k3x_hip_bank_upload_expert(
                    b.bank, (std::uint32_t)victim, tid, bytes(e.gate.packed), bytes(e.gate.scales),
                    bytes(e.up.packed), bytes(e.up.scales), bytes(e.down.packed),
                    bytes(e.down.scales));
            }
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
    // pairs_out [T][K][H] and/or mix_out [T][H].  On a padded bank the rows
    // of x are padded with zeros to the bank's hidden width (the padded
    // codes are zero, so the padded activations are GLU(0, 0) = 0 and the
    // products are those of the unpadded layer) and the outputs cropped.
    ErrorCode run(std::uint32_t layer, std::span<const float> inputs, std::size_t T,
                  std::size_t K, std::span<const Mxfp4MlpView> experts,
                  std::span<const std::uint32_t> routes, std::span<const float> contributions,
                  float beta, std::optional<float> linear, std::vector<float>* pairs_out,
                  std::vector<float>* mix_out) {
        const std::size_t H = experts.front().gate.cols, I = experts.front().gate.rows;
        const auto t_call = Clock::now();
        auto bank = bank_for(layer, H, I);
        if (!bank) return bank.error();
        std::vector<std::uint32_t> slot;
        const std::uint64_t h2d0 = stats.weight_h2d_bytes;
        if (ErrorCode c = admit(*bank.value(), experts, slot); c != ErrorCode::ok) return c;
        if (sink && stats.weight_h2d_bytes != h2d0)
            emit(ProfileOperation::weight_host_to_device, NumericPrecision::mxfp4_e2m1_e8m0, layer,
                 ns_since(t_call), 0, 0, stats.weight_h2d_bytes - h2d0);
        double stale[K3X_STAGE_COUNT];
        if (sink) take_stage_ms(stale);  // this call's stages only
        std::vector<std::uint32_t> hid(T * K);
        std::vector<float> hw(T * K, 1.0f);
        for (std::size_t p = 0; p < T * K; ++p) {
            hid[p] = slot[routes[p]];
            if (!contributions.empty()) hw[p] = contributions[p];
        }
        const std::size_t Hp = bank.value()->hp;
        std::vector<std::uint16_t> xb(T * Hp, 0);
        for (std::size_t t = 0; t < T; ++t)
            for (std::size_t i = 0; i < H; ++i) xb[t * Hp + i] = to_bf16(inputs[t * H + i]);
        for (auto [d, n] : {std::pair<Dev*, std::size_t>{&xn, T * Hp * 2}, {&ids, T * K * 4},
                            {&w, T * K * 4}, {&out, T * Hp * 2}})
            if (ErrorCode c = ensure(*d, n); c != ErrorCode::ok) return c;
        if (mix_out)
            if (ErrorCode c = ensure(out_f32, T * Hp * 4); c != ErrorCode::ok) return c;
        if (pairs_out)
            if (ErrorCode c = ensure(pairs, T * K * Hp * 4); c != ErrorCode::ok) return c;
        if (hipMemcpy(xn.p, xb.data(), T * Hp * 2, hipMemcpyHostToDevice) != hipSuccess ||
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
        if (sink) {
            std::vector<std::uint32_t> u(hid);
            std::sort(u.begin(), u.end());
            const std::size_t distinct = (std::size_t)(std::unique(u.begin(), u.end()) - u.begin());
            emit(ProfileOperation::activation_host_to_device, NumericPrecision::bf16_rounded, layer,
                 ns_since(t_call), 0, 0, T * Hp * 2 + T * K * 8);
            emit_layer_stages(layer, ns_since(t_call), distinct, T, K, Hp, bank.value()->ip);
        }
        const auto t_d2h = Clock::now();
        // Rows of Hp values on the device, H of each kept.
        auto fetch = [&](std::vector<float>& dst, const void* src, std::size_t rows) {
            dst.resize(rows * H);
            return hipMemcpy2D(dst.data(), H * 4, src, Hp * 4, H * 4, rows,
                               hipMemcpyDeviceToHost) == hipSuccess;
        };
        if (pairs_out && !fetch(*pairs_out, pairs.p, T * K)) return ErrorCode::backend_unavailable;
        if (mix_out && !fetch(*mix_out, out_f32.p, T)) return ErrorCode::backend_unavailable;
        if (sink)
            emit(ProfileOperation::device_to_host, NumericPrecision::fp32, layer, ns_since(t_d2h), 0,
                 0, ((pairs_out ? T * K : 0) + (mix_out ? T : 0)) * H * 4);
        return ErrorCode::ok;
    }

    // Per-expert outputs of T tokens through every expert of `experts`
    // (distinct), in chunks of at most 64 experts (and at most the layer's
    // bank slots, so that more experts than slots run chunk after chunk,
    // each admitted over the last) and kTokensPerCall tokens:
    // out[e][t * H + h].
    ErrorCode grid(std::uint32_t layer, std::span<const float> inputs, std::size_t T,
                   std::span<const Mxfp4MlpView> experts, float beta,
                   std::optional<float> linear, Outputs& out) {
        const std::size_t H = experts.front().gate.cols;
        out.assign(experts.size(), std::vector<float>(T * H));
        const std::size_t chunk = std::min<std::size_t>(kMaxSlotsPerToken, opt.resident_experts);
        for (std::size_t e0 = 0; e0 < experts.size(); e0 += chunk) {
            const std::size_t K = std::min(chunk, experts.size() - e0);
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
    if (options.device == HipBackendOptions::kNoDevice) {
        impl->name = "none (no device attached)";
        return R::success(std::unique_ptr<HipMoeBackend>(new HipMoeBackend(std::move(impl))));
    }
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
                                                    std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    for (const auto& e : experts)
        if (!valid_mxfp4_mlp(input.size(), e)) return Result<Outputs>::failure(ErrorCode::invalid_mxfp4);
    if (experts.empty()) return Result<Outputs>::success({});
    for (const auto& e : experts)
        if (ErrorCode c = Impl::supported(e); c != ErrorCode::ok)
            return impl_->shape_failure<Result<Outputs>>(c, "expert shape");
    for (const auto& e : experts)
        if (e.gate.cols != experts.front().gate.cols || e.gate.rows != experts.front().gate.rows)
            return impl_->decline<Result<Outputs>>("mixed shapes");
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
                                                    std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    // backend_cpu.cpp:161-171.
    if (batch_size == 0 || expert.gate.cols == 0 || !mul_fits(batch_size, expert.gate.cols) ||
        inputs.size() != batch_size * expert.gate.cols || !valid_situ(situ_beta, situ_linear) ||
        !valid_mxfp4_mlp(expert.gate.cols, expert))
        return Result<Outputs>::failure(ErrorCode::invalid_mxfp4);
    if (ErrorCode c = Impl::supported(expert); c != ErrorCode::ok)
        return impl_->shape_failure<Result<Outputs>>(c, "expert shape");
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
                                                   std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
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
    if (ErrorCode c = Impl::supported(experts.front()); c != ErrorCode::ok)
        return impl_->shape_failure<R>(c, "expert shape");
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
    impl_->call_phase = phase;
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
    // One layer call takes each expert once, at most 64 slots and at most the
    // bank's slots; otherwise the per-expert outputs (run chunk by chunk) are
    // mixed here.
    bool distinct = experts.size() <= std::min<std::size_t>(kMaxSlotsPerToken,
                                                            impl_->opt.resident_experts);
    for (std::size_t i = 0; i < experts.size() && distinct; ++i)
        for (std::size_t j = 0; j < i && distinct; ++j) distinct = !same_expert(experts[i], experts[j]);
    if (!distinct) {
        // An expert twice, or more experts than one layer call or the bank
        // takes: the per-expert outputs, mixed here in slot order as
        // backend_cpu.cpp:294-301 does.
        auto outs = mxfp4_situ_mlp_group(input, experts, situ_beta, situ_linear, layer, phase);
        if (!outs) return R::failure(outs.error(), outs.message());
        std::vector<float> mixed(out_rows, 0.0f);
        for (std::size_t e = 0; e < experts.size(); ++e)
            for (std::size_t r = 0; r < out_rows; ++r)
                mixed[r] = mixed[r] + contributions[e] * outs.value()[e][r];
        return R::success(std::move(mixed));
    }
    for (const auto& e : experts)
        if (ErrorCode c = Impl::supported(e); c != ErrorCode::ok)
            return impl_->shape_failure<R>(c, "expert shape");
    for (const auto& e : experts)
        if (e.gate.cols != experts.front().gate.cols || e.gate.rows != experts.front().gate.rows)
            return impl_->decline<R>("mixed shapes");
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
    std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
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
    if (ErrorCode c = Impl::supported(experts.front()); c != ErrorCode::ok)
        return impl_->shape_failure<R>(c, "expert shape");
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

// ---- expert-major verification block -----------------------------------------

Result<ExpertMajorBlockMoe> HipMoeBackend::expert_major_block_moe(
    std::span<const float> latents, std::size_t positions,
    std::span<const ExpertMajorTokenRoute> routes, std::span<const Mxfp4MlpView> experts,
    float situ_beta, std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    using R = Result<ExpertMajorBlockMoe>;
    if (routes.empty() || routes.size() != positions) return R::failure(ErrorCode::invalid_extent);
    ExpertMajorBlockMoe res;
    std::vector<std::uint32_t> seen;  // distinct experts of the block (the plan's groups)
    for (const auto& r : routes) {
        if (r.expert_ids.empty() || r.expert_ids.size() != r.contributions.size())
            return R::failure(ErrorCode::invalid_extent);
        for (std::size_t k = 0; k < r.expert_ids.size(); ++k) {
            if (!std::isfinite(r.contributions[k]) ||
                std::count(r.expert_ids.begin(), r.expert_ids.begin() + k, r.expert_ids[k]))
                return R::failure(ErrorCode::invalid_state);
            if (r.expert_ids[k] >= experts.size()) return R::failure(ErrorCode::invalid_extent);
            if (std::find(seen.begin(), seen.end(), r.expert_ids[k]) == seen.end())
                seen.push_back(r.expert_ids[k]);
            ++res.assignments;
        }
    }
    res.unique_experts = seen.size();
    const std::size_t width_in = experts[seen.front()].gate.cols;
    const std::size_t width_out = experts[seen.front()].down.rows;
    if (!mul_fits(positions, width_in) || latents.size() != positions * width_in)
        return R::failure(ErrorCode::invalid_mxfp4);
    res.mixed.assign(positions * width_out, 0.0f);
    // One grouped call per route width: positions of that width, their
    // experts as a local list, routes as indices into it.
    std::vector<std::size_t> widths;
    for (const auto& r : routes)
        if (std::find(widths.begin(), widths.end(), r.expert_ids.size()) == widths.end())
            widths.push_back(r.expert_ids.size());
    for (const std::size_t K : widths) {
        std::vector<std::size_t> pos;
        std::vector<Mxfp4MlpView> local;
        std::vector<std::uint32_t> local_id, idx;
        std::vector<float> contrib, in;
        for (std::size_t p = 0; p < positions; ++p) {
            if (routes[p].expert_ids.size() != K) continue;
            pos.push_back(p);
            in.insert(in.end(), latents.begin() + p * width_in,
                      latents.begin() + (p + 1) * width_in);
            for (std::size_t k = 0; k < K; ++k) {
                const std::uint32_t id = routes[p].expert_ids[k];
                auto at = std::find(local_id.begin(), local_id.end(), id);
                if (at == local_id.end()) {
                    local_id.push_back(id);
                    local.push_back(experts[id]);
                    at = local_id.end() - 1;
                }
                idx.push_back((std::uint32_t)(at - local_id.begin()));
                contrib.push_back(routes[p].contributions[k]);
            }
        }
        auto mixed = mxfp4_situ_moe_tokens(in, pos.size(), K, local, idx, contrib, situ_beta,
                                           situ_linear, layer, phase);
        if (!mixed) return R::failure(mixed.error(), mixed.message());
        ++res.layer_calls;
        for (std::size_t i = 0; i < pos.size(); ++i)
            std::copy_n(mixed.value().data() + i * width_out, width_out,
                        res.mixed.data() + pos[i] * width_out);
    }
    return R::success(std::move(res));
}

// ---- official K3 MoE FFN ----------------------------------------------------

namespace {

bool finite_all(std::span<const float> v) {
    return std::all_of(v.begin(), v.end(), [](float x) { return std::isfinite(x); });
}

bool finite_bf16_words(std::span<const std::uint16_t> v) {
    return std::all_of(v.begin(), v.end(), [](std::uint16_t w) { return (w & 0x7f80u) != 0x7f80u; });
}

// backend_cuda.cu:3763-3768 / :3490-3495.
bool valid_bf16(const Bf16WeightView& v) {
    return v.tensor_id && v.rows && v.cols && mul_fits(v.rows, v.cols) &&
           v.values.size() == v.rows * v.cols;
}

float bf16_word_to_f32(std::uint16_t w) {
    const std::uint32_t u = (std::uint32_t)w << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

Result<OfficialMoeRoutePrepareResult> HipMoeBackend::prepare_official_moe_route(
    std::span<const float> prefix, std::span<const float> block, OfficialMoeRoutePrepareView wv,
    float epsilon, std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    using R = Result<OfficialMoeRoutePrepareResult>;
    Impl& m = *impl_;
    const std::size_t H = prefix.size();
    // backend_cuda.cu:3498-3512, :3520-3528, :3561-3568.
    auto valid_h = [&](const Bf16WeightView& v, std::size_t rows) {
        return valid_bf16(v) && v.rows == rows && v.cols == H;
    };
    if (prefix.empty() || prefix.size() != block.size() || !finite_all(prefix) ||
        !finite_all(block) || !std::isfinite(epsilon) || epsilon <= 0.0f ||
        !wv.residual_norm.tensor_id || wv.residual_norm.values.size() != H ||
        !valid_h(wv.residual_proj, 1) || !wv.post_norm.tensor_id ||
        wv.post_norm.values.size() != H || !valid_h(wv.router, wv.router.rows))
        return R::failure(ErrorCode::invalid_extent);
    const std::uint64_t tids[4] = {wv.residual_norm.tensor_id, wv.residual_proj.tensor_id,
                                   wv.post_norm.tensor_id, wv.router.tensor_id};
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < i; ++j)
            if (tids[i] == tids[j]) return R::failure(ErrorCode::invalid_extent);
    if (!finite_bf16_words(wv.residual_norm.values) || !finite_bf16_words(wv.residual_proj.values) ||
        !finite_bf16_words(wv.post_norm.values) || !finite_bf16_words(wv.router.values))
        return R::failure(ErrorCode::invalid_extent);
    const std::size_t E = wv.router.rows;
    if (H % 128 || H > (1u << 20) || E > (1u << 20)) return m.decline<R>("hidden / router shape");
    if (!m.ctx) return R::failure(ErrorCode::backend_unavailable, "no device");
    // A new preparation replaces a pending one (backend_cuda.cu:3609-3616).
    m.prepared_active = false;
    auto& rt = m.official_routes[layer];
    if (rt.obj && (rt.H != H || rt.E != E)) {
        k3x_hip_official_destroy(rt.obj);
        rt = Impl::OfficialRoute{};
    }
    if (!rt.obj) {
        k3x_hip_official_desc d{};
        d.hidden = (std::uint32_t)H;
        d.router_experts = (std::uint32_t)E;
        if (int st = k3x_hip_official_create(m.ctx, nullptr, &d, &rt.obj)) {
            rt.obj = nullptr;
            return R::failure(code_of(st), "official_create");
        }
        rt.H = H;
        rt.E = E;
    }
    const Impl::WeightKey keys[4] = {{tids[0], wv.residual_norm.values.data()},
                                     {tids[1], wv.residual_proj.values.data()},
                                     {tids[2], wv.post_norm.values.data()},
                                     {tids[3], wv.router.values.data()}};
    if (!std::equal(keys, keys + 4, rt.keys)) {
        const std::vector<float> zero_correction(E, 0.0f);  // the route itself is the caller's
        std::fill(rt.keys, rt.keys + 4, Impl::WeightKey{});
        if (int st = k3x_hip_official_upload_route(rt.obj, wv.residual_norm.values.data(),
                                                   wv.residual_proj.values.data(),
                                                   wv.post_norm.values.data(),
                                                   wv.router.values.data(), zero_correction.data()))
            return R::failure(code_of(st), "official_upload_route");
        std::copy(keys, keys + 4, rt.keys);
        m.stats.weight_h2d_bytes += (3 * H + E * H) * 2;
    }
    for (auto [d, n] : {std::pair<Impl::Dev*, std::size_t>{&m.prep_prefix, H * 4},
                        {&m.prep_block, H * 4}, {&m.prep_hidden, H * 2}, {&m.prep_logits, E * 4}})
        if (ErrorCode c = m.ensure(*d, n); c != ErrorCode::ok) return R::failure(c);
    if (hipMemcpy(m.prep_prefix.p, prefix.data(), H * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m.prep_block.p, block.data(), H * 4, hipMemcpyHostToDevice) != hipSuccess)
        return R::failure(ErrorCode::backend_unavailable);
    const auto t_launch = Impl::Clock::now();
    int st = k3x_hip_official_prepare(m.ctx, rt.obj, 1, epsilon,
                                      static_cast<const float*>(m.prep_prefix.p),
                                      static_cast<const float*>(m.prep_block.p),
                                      static_cast<std::uint16_t*>(m.prep_hidden.p),
                                      static_cast<float*>(m.prep_logits.p));
    if (!st) st = k3x_hip_ctx_synchronize(m.ctx);
    if (st) return R::failure(code_of(st));
    m.emit_call(layer, t_launch,
                {{ProfileOperation::rms_norm, NumericPrecision::bf16_rounded, (3 * H + H * H) * 2},
                 {ProfileOperation::dense_matvec, NumericPrecision::bf16_rounded, E * H * 2}});
    OfficialMoeRoutePrepareResult r;
    r.executed = true;
    r.router_logits.resize(E);
    if (hipMemcpy(r.router_logits.data(), m.prep_logits.p, E * 4, hipMemcpyDeviceToHost) !=
            hipSuccess ||
        !finite_all(r.router_logits))
        return R::failure(ErrorCode::backend_unavailable);
    if (!++m.prepared_generation) ++m.prepared_generation;
    m.prepared_active = true;
    m.prepared_layer = layer;
    m.prepared_width = H;
    r.prepared = {m.owner(), m.prepared_generation};
    ++m.stats.calls;
    return R::success(std::move(r));
}

Result<bool> HipMoeBackend::discard_official_moe_prepared(OfficialMoePreparedToken token) {
    Impl& m = *impl_;
    if (!m.prepared_active || token.owner != m.owner() || token.generation != m.prepared_generation)
        return Result<bool>::failure(ErrorCode::invalid_state);
    m.prepared_active = false;
    return Result<bool>::success(true);
}

Result<OfficialMoeFfnResult> HipMoeBackend::official_mxfp4_moe_ffn(
    std::span<const float> hidden, std::span<const float> prefix, OfficialMoeFfnView weights,
    std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
    std::span<const float> contributions, float epsilon, float situ_beta,
    std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    impl_->prepared_active = false;  // backend_cuda.cu:3723-3731
    return official_ffn(hidden, prefix, std::nullopt, weights, experts, expert_ids, contributions,
                        epsilon, situ_beta, situ_linear, layer);
}

Result<OfficialMoeFfnResult> HipMoeBackend::official_mxfp4_moe_ffn_prepared(
    OfficialMoePreparedToken prepared, OfficialMoeFfnView weights,
    std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
    std::span<const float> contributions, float epsilon, float situ_beta,
    std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    return official_ffn({}, {}, prepared, weights, experts, expert_ids, contributions, epsilon,
                        situ_beta, situ_linear, layer);
}

// Checks as backend_cuda.cu:3769-3880 (invalid_mxfp4 for every rejected
// argument); shapes the kernels do not run are backend_unavailable.
Result<OfficialMoeFfnResult> HipMoeBackend::official_ffn(
    std::span<const float> hidden, std::span<const float> prefix,
    std::optional<OfficialMoePreparedToken> prepared, const OfficialMoeFfnView& wv,
    std::span<const Mxfp4MlpView> experts, std::span<const std::uint32_t> expert_ids,
    std::span<const float> contributions, float epsilon, float beta, std::optional<float> linear,
    std::uint32_t layer) {
    using R = Result<OfficialMoeFfnResult>;
    Impl& m = *impl_;
    const auto bad = [] { return R::failure(ErrorCode::invalid_mxfp4); };
    if ((!prepared && (hidden.empty() || hidden.size() != prefix.size())) ||
        (prepared && (!m.prepared_active || prepared->owner != m.owner() ||
                      prepared->generation != m.prepared_generation ||
                      m.prepared_layer != layer || !m.prepared_width)) ||
        experts.empty() || experts.size() > 65535 || experts.size() != expert_ids.size() ||
        experts.size() != contributions.size() ||
        (!prepared && (!finite_all(hidden) || !finite_all(prefix))) ||
        !finite_all(contributions) || !std::isfinite(epsilon) || epsilon <= 0.0f ||
        !valid_situ(beta, linear) || !valid_bf16(wv.routed_down) || !valid_bf16(wv.routed_up) ||
        !valid_bf16(wv.shared.gate) || !valid_bf16(wv.shared.up) || !valid_bf16(wv.shared.down) ||
        !wv.routed_norm.tensor_id || wv.routed_norm.values.empty())
        return bad();
    const std::size_t H = prepared ? m.prepared_width : hidden.size();
    const std::size_t L = wv.routed_down.rows, I = experts.front().gate.rows,
                      out_w = experts.front().down.rows, Is = wv.shared.gate.rows;
    if (wv.routed_down.cols != H || wv.routed_norm.values.size() != out_w ||
        wv.routed_up.rows != H || wv.routed_up.cols != out_w || wv.shared.gate.cols != H ||
        wv.shared.up.rows != Is || wv.shared.up.cols != H || wv.shared.down.rows != H ||
        wv.shared.down.cols != Is)
        return bad();
    std::vector<std::uint64_t> tensor_ids;
    auto insert = [&](std::uint64_t id) {
        if (!id || std::find(tensor_ids.begin(), tensor_ids.end(), id) != tensor_ids.end())
            return false;
        tensor_ids.push_back(id);
        return true;
    };
    if (!insert(wv.routed_down.tensor_id) || !insert(wv.routed_norm.tensor_id) ||
        !insert(wv.routed_up.tensor_id) || !insert(wv.shared.gate.tensor_id) ||
        !insert(wv.shared.up.tensor_id) || !insert(wv.shared.down.tensor_id))
        return bad();
    double sum = 0.0;
    for (std::size_t k = 0; k < experts.size(); ++k) {
        const Mxfp4MlpView& e = experts[k];
        if (std::count(expert_ids.begin(), expert_ids.begin() + k, expert_ids[k]) ||
            contributions[k] <= 0.0f || e.gate.cols != L || e.gate.rows != I || e.up.cols != L ||
            e.up.rows != I || e.down.cols != I || e.down.rows != out_w || e.gate.group_size != 32 ||
            e.up.group_size != 32 || e.down.group_size != 32 || !valid_mxfp4(L, e.gate) ||
            !valid_mxfp4(L, e.up) || !valid_mxfp4(I, e.down) || !insert(e.gate.tensor_id) ||
            !insert(e.up.tensor_id) || !insert(e.down.tensor_id))
            return bad();
        sum += contributions[k];
    }
    if (std::abs(sum - 1.0) > 1.0e-5) return bad();
    // The official composition's routed width is the latent (official_moe.cpp:327-333).
    if (out_w != L) return bad();
    if (H % 128 || L % 128 || I % 128 || Is % 128 || experts.size() > kMaxSlotsPerToken ||
        experts.size() > m.opt.resident_experts)
        return m.decline<R>("official layer shape");
    if (!finite_bf16_words(wv.routed_down.values) || !finite_bf16_words(wv.routed_up.values) ||
        !finite_bf16_words(wv.routed_norm.values) || !finite_bf16_words(wv.shared.gate.values) ||
        !finite_bf16_words(wv.shared.up.values) || !finite_bf16_words(wv.shared.down.values))
        return bad();
    if (!m.ctx) return R::failure(ErrorCode::backend_unavailable, "no device");
    if (prepared) m.prepared_active = false;  // consumed (backend_cuda.cu:3875-3878)
    // The FFN object and its latent experts.
    const auto key = std::make_tuple(layer, H, L, I, Is);
    auto it = m.official_ffns.find(key);
    if (it == m.official_ffns.end()) {
        Impl::OfficialFfn f;
        k3x_hip_layer_desc d{};
        d.hidden = (std::uint32_t)L;
        d.inter = (std::uint32_t)I;
        d.experts = m.opt.resident_experts;
        d.group_size = 32;
        if (int st = k3x_hip_bank_create(m.ctx, &d, &f.bank.bank))
            return R::failure(code_of(st), "bank_create");
        f.bank.slots.resize(m.opt.resident_experts);
        k3x_hip_official_desc od{};
        od.hidden = (std::uint32_t)H;
        od.shared_inter = (std::uint32_t)Is;
        if (int st = k3x_hip_official_create(m.ctx, f.bank.bank, &od, &f.obj)) {
            k3x_hip_bank_destroy(f.bank.bank);
            return R::failure(code_of(st), "official_create");
        }
        it = m.official_ffns.emplace(key, std::move(f)).first;
    }
    Impl::OfficialFfn& f = it->second;
    const Impl::WeightKey keys[6] = {
        {wv.routed_down.tensor_id, wv.routed_down.values.data()},
        {wv.routed_norm.tensor_id, wv.routed_norm.values.data()},
        {wv.routed_up.tensor_id, wv.routed_up.values.data()},
        {wv.shared.gate.tensor_id, wv.shared.gate.values.data()},
        {wv.shared.up.tensor_id, wv.shared.up.values.data()},
        {wv.shared.down.tensor_id, wv.shared.down.values.data()}};
    if (!std::equal(keys, keys + 6, f.keys)) {
        std::fill(f.keys, f.keys + 6, Impl::WeightKey{});
        if (int st = k3x_hip_official_upload_ffn(
                f.obj, wv.routed_down.values.data(), wv.routed_norm.values.data(),
                wv.routed_up.values.data(), wv.shared.gate.values.data(),
                wv.shared.up.values.data(), wv.shared.down.values.data()))
            return R::failure(code_of(st), "official_upload_ffn");
        std::copy(keys, keys + 6, f.keys);
        m.stats.weight_h2d_bytes += (2 * L * H + L + 3 * Is * H) * 2;
    }
    std::vector<std::uint32_t> slot;
    if (ErrorCode c = m.admit(f.bank, experts, slot); c != ErrorCode::ok) return R::failure(c);
    const std::size_t K = experts.size();
    for (auto [d, n] : {std::pair<Impl::Dev*, std::size_t>{&m.o_ids, K * 4}, {&m.o_contrib, K * 4},
                        {&m.o_out, H * 2}, {&m.o_hidden, H * 2}, {&m.o_prefix, H * 4}})
        if (ErrorCode c = m.ensure(*d, n); c != ErrorCode::ok) return R::failure(c);
    const void* hid = m.prep_hidden.p;
    const void* pre = m.prep_prefix.p;
    if (!prepared) {
        std::vector<std::uint16_t> hb(H);
        for (std::size_t i = 0; i < H; ++i) hb[i] = to_bf16(hidden[i]);
        if (hipMemcpy(m.o_hidden.p, hb.data(), H * 2, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(m.o_prefix.p, prefix.data(), H * 4, hipMemcpyHostToDevice) != hipSuccess)
            return R::failure(ErrorCode::backend_unavailable);
        hid = m.o_hidden.p;
        pre = m.o_prefix.p;
    }
    if (hipMemcpy(m.o_ids.p, slot.data(), K * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m.o_contrib.p, contributions.data(), K * 4, hipMemcpyHostToDevice) != hipSuccess)
        return R::failure(ErrorCode::backend_unavailable);
    k3x_hip_moe_params p{};
    p.tokens = 1;
    p.top_k = (std::uint32_t)K;
    p.routed_scale = 1.0f;
    p.rms_epsilon = epsilon;
    p.glu = K3X_GLU_SITU;
    p.situ_beta = beta;
    p.has_situ_linear = linear.has_value();
    p.situ_linear_beta = linear.value_or(0.0f);
    p.renorm = K3X_RENORM_DOUBLE;
    const auto t_launch = Impl::Clock::now();
    int st = k3x_hip_official_ffn(m.ctx, f.obj, &p, static_cast<const std::uint16_t*>(hid),
                                  static_cast<const float*>(pre),
                                  static_cast<const std::uint32_t*>(m.o_ids.p),
                                  static_cast<const float*>(m.o_contrib.p),
                                  static_cast<std::uint16_t*>(m.o_out.p), nullptr);
    if (!st) st = k3x_hip_ctx_synchronize(m.ctx);
    if (st) return R::failure(code_of(st));
    m.emit_call(layer, t_launch,
                {{ProfileOperation::mxfp4_matvec, NumericPrecision::mxfp4_e2m1_e8m0,
                  K * 3 * (I * L / 2 + I * L / 32)},
                 {ProfileOperation::dense_matvec, NumericPrecision::bf16_rounded,
                  (2 * L * H + 3 * Is * H) * 2},
                 {ProfileOperation::rms_norm, NumericPrecision::bf16_rounded, L * 2 + L * 2},
                 {ProfileOperation::moe_mix, NumericPrecision::bf16_rounded, K * L * 2}});
    std::vector<std::uint16_t> ob(H);
    if (hipMemcpy(ob.data(), m.o_out.p, H * 2, hipMemcpyDeviceToHost) != hipSuccess)
        return R::failure(ErrorCode::backend_unavailable);
    OfficialMoeFfnResult r;
    r.executed = true;
    r.output.resize(H);
    for (std::size_t i = 0; i < H; ++i) r.output[i] = bf16_word_to_f32(ob[i]);
    r.selected_expert_ids.assign(expert_ids.begin(), expert_ids.end());
    ++m.stats.calls;
    ++m.stats.layer_calls;
    return R::success(std::move(r));
}

namespace {

std::span<const float> as_span(const float* p, std::size_t n) { return {p, n}; }

}  // namespace

Result<std::vector<float>> HipMoeBackend::dense_matvec(std::span<const float> input,
                                                       DenseWeightView weight, std::uint32_t layer,
                                                       ProfilePhase phase) {
    impl_->call_phase = phase;
    using R = Result<std::vector<float>>;
    if (!valid_dense(input.size(), weight)) return R::failure(ErrorCode::invalid_extent);
    if (!weight.rows || !weight.cols) return R::success(std::vector<float>(weight.rows, 0.0f));
    if (weight.rows > (1u << 24) || weight.cols > (1u << 24))
        return impl_->decline<R>("matrix size");
    Impl& m = *impl_;
    ++m.dense_tick;
    const void* W = nullptr;
    auto none = [] { return ErrorCode::ok; };
    if (ErrorCode c = m.acquire(weight.tensor_id, {{weight.values.data(), weight.values.size_bytes()}},
                                weight.rows, weight.cols, none, &m.transient[0], &W);
        c != ErrorCode::ok)
        return R::failure(c);
    if (ErrorCode c = m.upload(m.vin, input.data(), input.size_bytes()); c != ErrorCode::ok)
        return R::failure(c);
    if (ErrorCode c = m.ensure(m.vout, weight.rows * 4); c != ErrorCode::ok) return R::failure(c);
    const auto t_launch = Impl::Clock::now();
    if (int st = k3x_hip_dense_f32_matvec(m.ctx, static_cast<const float*>(W),
                                          (std::uint32_t)weight.rows, (std::uint32_t)weight.cols,
                                          static_cast<const float*>(m.vin.p), 1,
                                          static_cast<float*>(m.vout.p)))
        return R::failure(code_of(st));
    std::vector<float> out;
    if (ErrorCode c = m.finish(m.vout, out, weight.rows); c != ErrorCode::ok) return R::failure(c);
    m.emit_call(layer, t_launch,
                {{ProfileOperation::dense_matvec, NumericPrecision::fp32, weight.values.size_bytes()}});
    ++m.stats.calls;
    return R::success(std::move(out));
}

Result<std::vector<float>> HipMoeBackend::mxfp4_matvec(std::span<const float> input,
                                                       Mxfp4WeightView weight, std::uint32_t layer,
                                                       ProfilePhase phase) {
    impl_->call_phase = phase;
    using R = Result<std::vector<float>>;
    // mxfp4_matmul and decode_mxfp4 (runtime/src/ops.cpp:32-76): extents
    // first, then the scale bytes (at upload; a resident copy was checked).
    if (input.size() != weight.cols || !weight.rows || !weight.cols || !weight.group_size ||
        weight.cols % weight.group_size || weight.cols % 2 || !mul_fits(weight.rows, weight.cols) ||
        weight.packed.size() != weight.rows * weight.cols / 2 ||
        weight.scales.size() != weight.rows * weight.cols / weight.group_size)
        return R::failure(ErrorCode::invalid_mxfp4);
    if (weight.group_size != 32 || weight.rows > (1u << 24) || weight.cols > (1u << 24))
        return impl_->decline<R>("group size 32 only");
    Impl& m = *impl_;
    ++m.dense_tick;
    auto scales_ok = [&] {
        for (const std::byte b : weight.scales)
            if (b == std::byte{0xff}) return ErrorCode::invalid_mxfp4;
        return ErrorCode::ok;
    };
    const void* W = nullptr;
    if (ErrorCode c = m.acquire(weight.tensor_id,
                                {{weight.packed.data(), weight.packed.size()},
                                 {weight.scales.data(), weight.scales.size()}},
                                weight.rows, weight.cols, scales_ok, &m.transient[0], &W);
        c != ErrorCode::ok)
        return R::failure(c);
    const std::uint8_t* packed = static_cast<const std::uint8_t*>(W);
    const std::uint8_t* scales = packed + ((weight.packed.size() + 255) & ~(std::size_t)255);
    if (ErrorCode c = m.upload(m.vin, input.data(), input.size_bytes()); c != ErrorCode::ok)
        return R::failure(c);
    if (ErrorCode c = m.ensure(m.vout, weight.rows * 4); c != ErrorCode::ok) return R::failure(c);
    const auto t_launch = Impl::Clock::now();
    if (int st = k3x_hip_mxfp4_matvec(m.ctx, packed, scales, (std::uint32_t)weight.rows,
                                      (std::uint32_t)weight.cols,
                                      static_cast<const float*>(m.vin.p), 1,
                                      static_cast<float*>(m.vout.p)))
        return R::failure(code_of(st));
    std::vector<float> out;
    if (ErrorCode c = m.finish(m.vout, out, weight.rows); c != ErrorCode::ok) return R::failure(c);
    m.emit_call(layer, t_launch, {{ProfileOperation::mxfp4_matvec, NumericPrecision::mxfp4_e2m1_e8m0,
                                   weight.packed.size() + weight.scales.size()}});
    ++m.stats.calls;
    return R::success(std::move(out));
}

Result<Outputs> HipMoeBackend::dense_matvec_group(std::span<const float> input,
                                                  std::span<const DenseWeightView> weights,
                                                  std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    for (const auto& w : weights)
        if (!valid_dense(input.size(), w)) return Result<Outputs>::failure(ErrorCode::invalid_extent);
    Outputs out;
    out.reserve(weights.size());
    for (const auto& w : weights) {
        auto r = dense_matvec(input, w, layer, phase);
        if (!r) return Result<Outputs>::failure(r.error(), r.message());
        out.push_back(std::move(r.value()));
    }
    return Result<Outputs>::success(std::move(out));
}

Result<Outputs> HipMoeBackend::mxfp4_matvec_group(std::span<const float> input,
                                                  std::span<const Mxfp4WeightView> weights,
                                                  std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    for (const auto& w : weights)
        if (!valid_mxfp4(input.size(), w)) return Result<Outputs>::failure(ErrorCode::invalid_mxfp4);
    Outputs out;
    out.reserve(weights.size());
    for (const auto& w : weights) {
        auto r = mxfp4_matvec(input, w, layer, phase);
        if (!r) return Result<Outputs>::failure(r.error(), r.message());
        out.push_back(std::move(r.value()));
    }
    return Result<Outputs>::success(std::move(out));
}

Result<std::vector<float>> HipMoeBackend::dense_situ_mlp(std::span<const float> input,
                                                         DenseMlpView weights, float situ_beta,
                                                         std::optional<float> situ_linear,
                                                         std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    using R = Result<std::vector<float>>;
    if (!valid_dense_mlp(input.size(), weights) ||
        !checks::consistent_ids({&weights.gate, &weights.up, &weights.down}))
        return R::failure(ErrorCode::invalid_extent);
    const std::size_t H = input.size(), I = weights.gate.rows, O = weights.down.rows;
    if (!H || H > (1u << 24) || I > (1u << 24) || O > (1u << 24))
        return impl_->decline<R>("matrix size");
    Impl& m = *impl_;
    ++m.dense_tick;
    auto none = [] { return ErrorCode::ok; };
    const void* W[3] = {};
    const DenseWeightView* v[3] = {&weights.gate, &weights.up, &weights.down};
    for (int i = 0; i < 3; ++i)
        if (ErrorCode c = m.acquire(v[i]->tensor_id, {{v[i]->values.data(), v[i]->values.size_bytes()}},
                                    v[i]->rows, v[i]->cols, none, &m.transient[i], &W[i]);
            c != ErrorCode::ok)
            return R::failure(c);
    if (ErrorCode c = m.upload(m.vin, input.data(), input.size_bytes()); c != ErrorCode::ok)
        return R::failure(c);
    if (ErrorCode c = m.ensure(m.vact, I * 4); c != ErrorCode::ok) return R::failure(c);
    if (ErrorCode c = m.ensure(m.vout, O * 4); c != ErrorCode::ok) return R::failure(c);
    const auto t_launch = Impl::Clock::now();
    if (int st = k3x_hip_dense_situ_mlp(
            m.ctx, static_cast<const float*>(W[0]), static_cast<const float*>(W[1]),
            static_cast<const float*>(W[2]), (std::uint32_t)H, (std::uint32_t)I, (std::uint32_t)O,
            situ_beta, situ_linear.has_value(), situ_linear.value_or(0.0f),
            static_cast<const float*>(m.vin.p), 1, static_cast<float*>(m.vact.p),
            static_cast<float*>(m.vout.p)))
        return R::failure(code_of(st));
    std::vector<float> out;
    if (ErrorCode c = m.finish(m.vout, out, O); c != ErrorCode::ok) return R::failure(c);
    m.emit_call(layer, t_launch,
                {{ProfileOperation::dense_matvec, NumericPrecision::fp32,
                  weights.gate.values.size_bytes() + weights.up.values.size_bytes() +
                      weights.down.values.size_bytes()},
                 {ProfileOperation::situ_glu, NumericPrecision::fp32, I * 8}});
    ++m.stats.calls;
    return R::success(std::move(out));
}

Result<ResidentMoeLayerResult> HipMoeBackend::resident_mxfp4_moe_layer(
    std::span<const float> input, ResidentMoeLayerView weights,
    std::span<const Mxfp4MlpView> experts, std::span<const float> contributions, float epsilon,
    float situ_beta, std::optional<float> situ_linear, std::uint32_t layer, ProfilePhase phase) {
    impl_->call_phase = phase;
    using R = Result<ResidentMoeLayerResult>;
    const auto bad = [] { return R::failure(ErrorCode::invalid_mxfp4); };
    // valid_resident_moe_layer (backend_cpu.cpp:441-497); the finiteness of
    // the dense weights is checked when they are uploaded (a resident copy
    // was checked then).
    if (!checks::valid_resident_layer(input, weights, experts, contributions, epsilon, situ_beta,
                                      situ_linear))
        return bad();
    const std::size_t H = input.size(), L = weights.routed_down.rows,
                      W = experts.front().down.rows, I = experts.front().gate.rows;
    // (valid_resident_layer rejects a tensor id given twice, as the
    // reference does, so no resident entry is replaced under this call.)
    const DenseWeightView norm_view{weights.routed_norm.tensor_id, weights.routed_norm.values, 1,
                                    weights.routed_norm.values.size()};
    // Shapes the device path runs: routed width = latent (a square expert
    // bank), widths multiples of 128, one layer call of at most 64 slots.
    if (W != L || experts.size() > kMaxSlotsPerToken || H > (1u << 24) ||
        weights.shared.gate.rows > (1u << 24))
        return impl_->decline<R>("latent layer shape");
    if (ErrorCode c = Impl::supported(experts.front()); c != ErrorCode::ok)
        return impl_->shape_failure<R>(c, "expert shape");
    Impl& m = *impl_;
    auto bypass = [&] {
        ++m.stats.resident_layer_fallbacks;
        return R::success(ResidentMoeLayerResult{false, {}});
    };
    // Experts into the bank's slots: more distinct experts than slots is the
    // capacity bypass.
    auto bank = m.bank_for(layer, L, I);
    if (!bank) return R::failure(bank.error(), bank.message());
    if (experts.size() > bank.value()->slots.size()) return bypass();
    std::vector<std::uint32_t> slot;
    if (ErrorCode c = m.admit(*bank.value(), experts, slot); c != ErrorCode::ok) return R::failure(c);
    // The six dense weights resident, or the bypass.
    ++m.dense_tick;
    const DenseWeightView* dv[6] = {&weights.routed_down, &norm_view,          &weights.routed_up,
                                    &weights.shared.gate, &weights.shared.up, &weights.shared.down};
    const void* dp[6] = {};
    // On a padded bank (latent Lp = a multiple of 128 above L) the latent's
    // dense weights are padded with zeros to match: routed_down [Lp][H],
    // routed_norm [Lp], routed_up [H][Lp]; the RMSNorm divides by L.
    const std::size_t Lp = bank.value()->hp;
    std::vector<float> padded[3];
    if (Lp != L) {
        padded[0] = pad_dense(weights.routed_down.values, L, H, Lp, H);
        padded[1] = pad_dense(weights.routed_norm.values, 1, L, 1, Lp);
        padded[2] = pad_dense(weights.routed_up.values, H, L, H, Lp);
    }
    for (int i = 0; i < 6; ++i) {
        const DenseWeightView& v = *dv[i];
        auto finite = [&] {
            return all_finite(as_span(v.values.data(), v.values.size())) ? ErrorCode::ok
                                                                          : ErrorCode::invalid_mxfp4;
        };
        const bool pad = i < 3 && Lp != L;
        const float* data = pad ? padded[i].data() : v.values.data();
        const std::size_t nbytes = pad ? padded[i].size() * sizeof(float) : v.values.size_bytes();
        if (ErrorCode c = m.acquire(v.tensor_id, {{data, nbytes}}, v.rows, v.cols, finite, nullptr,
                                    &dp[i], v.values.data());
            c != ErrorCode::ok)
            return R::failure(c);
        if (!dp[i]) return bypass();
    }
    const std::size_t K = experts.size();
    if (ErrorCode c = m.upload(m.vin, input.data(), input.size_bytes()); c != ErrorCode::ok)
        return R::failure(c);
    if (ErrorCode c = m.upload(m.vids, slot.data(), K * 4); c != ErrorCode::ok) return R::failure(c);
    if (ErrorCode c = m.upload(m.vc, contributions.data(), K * 4); c != ErrorCode::ok)
        return R::failure(c);
    if (ErrorCode c = m.ensure(m.vout, H * 4); c != ErrorCode::ok) return R::failure(c);
    k3x_hip_latent_weights lw{};
    lw.routed_down = static_cast<const float*>(dp[0]);
    lw.routed_norm = static_cast<const float*>(dp[1]);
    lw.routed_up = static_cast<const float*>(dp[2]);
    lw.shared_gate = static_cast<const float*>(dp[3]);
    lw.shared_up = static_cast<const float*>(dp[4]);
    lw.shared_down = static_cast<const float*>(dp[5]);
    lw.hidden = (std::uint32_t)H;
    lw.latent = (std::uint32_t)Lp;
    lw.shared_inter = (std::uint32_t)weights.shared.gate.rows;
    lw.latent_norm = (std::uint32_t)L;
    k3x_hip_moe_params p{};
    p.tokens = 1;
    p.top_k = (std::uint32_t)K;
    p.routed_scale = 1.0f;
    p.rms_epsilon = epsilon;
    p.glu = K3X_GLU_SITU;
    p.situ_beta = situ_beta;
    p.has_situ_linear = situ_linear.has_value();
    p.situ_linear_beta = situ_linear.value_or(0.0f);
    p.renorm = K3X_RENORM_FLOAT;
    const auto t_launch = Impl::Clock::now();
    if (int st = k3x_hip_resident_moe_layer(
            m.ctx, bank.value()->bank, &lw, &p, static_cast<const float*>(m.vin.p),
            static_cast<const std::uint32_t*>(m.vids.p), static_cast<const float*>(m.vc.p),
            slot.data(), contributions.data(), static_cast<float*>(m.vout.p), nullptr))
        return R::failure(code_of(st));
    ResidentMoeLayerResult res{true, {}};
    if (ErrorCode c = m.finish(m.vout, res.output, H); c != ErrorCode::ok) return R::failure(c);
    m.emit_call(layer, t_launch,
                {{ProfileOperation::mxfp4_matvec, NumericPrecision::mxfp4_e2m1_e8m0,
                  K * 3 * (I * L / 2 + I * L / 32)},
                 {ProfileOperation::dense_matvec, NumericPrecision::fp32,
                  (2 * L * H + 3 * weights.shared.gate.rows * H) * 4},
                 {ProfileOperation::moe_mix, NumericPrecision::fp32, K * L * 4},
                 {ProfileOperation::rms_norm, NumericPrecision::fp32, L * 8},
                 {ProfileOperation::residual_add, NumericPrecision::fp32, H * 8}});
    ++m.stats.calls;
    ++m.stats.layer_calls;
    return R::success(std::move(res));
}

HipBackendStats HipMoeBackend::runtime_stats() const noexcept {
    Impl& m = *impl_;
    HipBackendStats s = m.stats;
    k3x_hip_stats cs{};
    if (m.ctx && k3x_hip_ctx_stats(m.ctx, &cs) == 0) s.kernel_launches = cs.kernel_launches;
    s.device_bytes = m.device_bytes(cs.scratch_bytes);
    m.stats.peak_device_bytes = std::max(m.stats.peak_device_bytes, s.device_bytes);
    s.peak_device_bytes = m.stats.peak_device_bytes;
    return s;
}

std::string_view HipMoeBackend::device_name() const noexcept { return impl_->name; }

void HipMoeBackend::set_profile_sink(ProfileSink sink) {
    impl_->sink = std::move(sink);
    if (impl_->ctx) (void)k3x_hip_ctx_set_profiling(impl_->ctx, impl_->sink ? 1 : 0);
}

}  // namespace k3x_amd
