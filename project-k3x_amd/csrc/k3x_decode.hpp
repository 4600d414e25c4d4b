// k3x_decode.hpp -- the decode path (T <= kMaxDecodeTokens) of the layer.
#pragma once

#include "k3x_device.hpp"
#include "k3x_internal.hpp"

namespace k3x_hip {

constexpr int kMaxDecodeTokens = 4;
// Arrival counters of the decode down kernel's fused combine: one per
// (token, 64-column group of H), H <= 64 * kMixGroupsMax.
constexpr uint32_t kMixGroupsMax = 1024;
constexpr size_t kDecodeMixBytes = (size_t)kMaxDecodeTokens * kMixGroupsMax * 4;

// Whether the four-launch decode path handles this call.
bool decode_eligible(const k3x_hip_ctx* ctx, const k3x_hip_bank* bank,
                     const k3x_hip_moe_params* p, const void* x);

// RMSNorm, routing, grouping, experts, shared expert and combine of one
// decode call; x is the raw bf16 input [T][H].  The per-expert grouping
// arrays (counts, offsets, first_use, active_asc, active_fu), which no decode
// kernel reads, are written only with group_taps.  b.mix: kDecodeMixBytes
// of counters, zero before the call and left zero by it.  Asynchronous.
int decode_forward(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                   const LayerBuffers& b, const uint16_t* x, uint16_t* out, float* out_f32,
                   bool group_taps);

// The routed experts of a general-path call on the decode path's gate/up
// and down kernels: b.arec holds the active slots' records {expert, rows, CSR
// offset, tokens} (the grouping writes them), act rows [P][I] or, split,
// [P][2 I] as [hi | lo]; y receives the per-pair rows.  Few tokens (T <=
// kMaxDecodeTokens): a slot's rows at once, tokens from the record.
// chunked: slots of any size (T <= kChunkedMaxTokens), their rows through LDS
// kMaxDecodeTokens at a time with the weights held in registers, tokens from
// b.pair_token.  Whether the bank's shapes fit those kernels (T: the rows in
// LDS at once):
constexpr uint32_t kChunkedMaxTokens = 64;
bool few_row_experts_eligible(const k3x_hip_ctx* ctx, const k3x_hip_bank* bank, uint32_t T,
                              bool split);
int launch_few_row_gate_up(k3x_hip_ctx* ctx, const k3x_hip_bank* bank, uint32_t T, uint32_t K,
                           const LayerBuffers& b, const uint16_t* xn,
                           const k3x_dev::GluParams& glu, bool split, bool chunked = false);
// mix (optional): the combine fused into the down launch, as on the decode
// path (b.mix's counters, zero before and after): out = bf16(sum over slots
// in router order of w * y (y rounded to bf16 first with round_y) +
// shared_y), out_f32 (may be null) the same sum in fp32.  Few tokens only
// (few_row_mix_eligible), not chunked.
struct FewRowMix {
    const float* weights;   // [T][K]
    const float* shared_y;  // [T][H] or null
    uint16_t* out;          // [T][H]
    float* out_f32;
    bool round_y;
};
bool few_row_mix_eligible(const k3x_hip_bank* bank, uint32_t T);
int launch_few_row_down(k3x_hip_ctx* ctx, const k3x_hip_bank* bank, uint32_t T, uint32_t K,
                        const LayerBuffers& b, bool split, bool chunked = false,
                        const FewRowMix* mix = nullptr);

// out[t][h] = bf16(sum over slots in router order of w[t][s] * y[t][s][h]
// + shared[t][h]) on the context stream (the combine of both paths).
int launch_combine(k3x_hip_ctx* ctx, const float* y, const float* weights, const float* shared,
                   uint32_t K, uint32_t H, uint32_t T, uint16_t* out, float* out_f32,
                   bool round_y = false);

}  // namespace k3x_hip
