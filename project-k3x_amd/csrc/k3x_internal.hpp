// k3x_internal.hpp -- host-side state behind the C ABI handles.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <unordered_map>
#include <vector>

#include "../../include/k3x_hip_moe.h"
#include "k3x_device.hpp"

// One timed stage launch: a hipEvent pair recorded around it.
struct StageMark {
    uint32_t stage;
    hipEvent_t start;
    hipEvent_t stop;
};

struct k3x_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipStream_t own_stream = nullptr;
    // Second stream for the shared expert's wide GEMMs (default priority),
    // forked from and joined back into `stream` with these events.
    hipStream_t side_stream = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    // The wide path's smaller size classes run on side_stream beside the
    // full chunks: forked after the grouping, joined after their down GEMMs.
    hipEvent_t class_fork_ev = nullptr, class_join_ev = nullptr;
    uint32_t* status = nullptr;  // device word, latched kernel errors
    size_t max_lds_per_block = 65536;
    uint32_t cu_count = 256;
    // Grow-only scratch (replaces runtime/cuda/device_memory.cuh:44-61).
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // Grow-only scratch of the latent layer (k3x_hip_resident_moe_layer).
    void* latent_scratch = nullptr;
    size_t latent_bytes = 0;
    // Device address of the fixed scratch of k3x_hip_moe_forward_noalloc on
    // this context's device (null when it could not be taken).
    void* noalloc_scratch = nullptr;
    // Decode combine counters of k3x_hip_moe_forward (zeroed at creation,
    // left zero by every call).
    uint32_t* mix_counts = nullptr;
    // Arrival counter of the fused Top-K and grouping launch (zeroed at
    // creation, left zero by every launch).
    uint32_t* route_counter = nullptr;
    uint64_t forward_calls = 0;
    uint64_t kernel_launches = 0;
    uint64_t weight_h2d_bytes = 0;
    uint32_t live_banks = 0;  // banks created on this context and not destroyed
    // Stage profiling (k3x_hip_ctx_set_profiling).
    bool profiling = false;
    std::vector<StageMark> pending;      // recorded, not yet read back
    std::vector<hipEvent_t> free_events;
    double stage_ms[K3X_STAGE_COUNT] = {};
    uint64_t stage_launches[K3X_STAGE_COUNT] = {};
    // CRC32C: device tables (uploaded at first use), chunk results, flag.
    uint32_t* crc_tables = nullptr;
    uint32_t* crc_chunks = nullptr;
    size_t crc_chunk_cap = 0;
};

// Geometry of the tile layout for one matrix family of the bank.
struct MatrixGeom {
    uint32_t rows = 0;    // output rows
    uint32_t cols = 0;    // K
    uint32_t kt = 0;      // cols / 128
    uint32_t ks = 0;      // ceil(kt / 4) scale dword groups
};

struct k3x_hip_bank {
    k3x_hip_ctx* ctx = nullptr;
    k3x_hip_layer_desc desc{};
    MatrixGeom gate;  // [inter x hidden]; gate and up share one interleaved layout
    MatrixGeom down;  // [hidden x inter]
    MatrixGeom sgate; // shared [shared_inter x hidden]
    MatrixGeom sdown; // shared [hidden x shared_inter]
    // Routed experts, expert-major.  Gate/up codes: [I/16][H/128][2][64] x16B.
    // Gate/up scales: [I/16][ks][2][64] dwords.  Down codes: [H/16][I/128][64]
    // x16B; down scales: [H/16][ks][64] dwords.
    uint8_t* gu_codes = nullptr;
    uint32_t* gu_scales = nullptr;
    uint8_t* dn_codes = nullptr;
    uint32_t* dn_scales = nullptr;
    size_t gu_codes_per_expert = 0;   // bytes
    size_t gu_scales_per_expert = 0;  // dwords
    size_t dn_codes_per_expert = 0;   // bytes
    size_t dn_scales_per_expert = 0;  // dwords
    // Shared expert bf16.  Gate/up: [S/16][H/128][2][4][64] x16B;
    // down: [H/16][S/128][4][64] x16B.
    uint8_t* sh_gu = nullptr;
    uint8_t* sh_dn = nullptr;
    float* router_w = nullptr;   // [E][H]
    float* router_wp = nullptr;  // [E/16][256][16][4][8] tile/residue-major router_w (H <= 8192)
    float* router_bias = nullptr;
    float* gamma = nullptr;
    bool router_ready = false;
    bool shared_ready = false;
    std::vector<uint8_t> expert_ready;
    // Device copy of expert_ready ([E] words, 1 = admitted), kept in step on
    // the context stream: the grouping rejects a device-given route to a slot
    // that holds no admitted expert.
    uint32_t* ready_dev = nullptr;
    std::unordered_map<uint64_t, uint32_t> tensor_ids;  // id -> expert*4+matrix
    uint64_t device_bytes = 0;
};

namespace k3x_hip {

// Per-call device buffers of one forward call, carved from the context
// scratch.  Shapes: T tokens, K slots, P = T*K pairs, E experts, H hidden,
// I expert inter, S shared inter.
struct LayerBuffers {
    uint16_t* xn;          // [T][H] bf16, normalised input
    float* logits;         // [T][E]
    uint32_t* ids;         // [T][K]
    float* weights;        // [T][K]
    uint32_t* counts;      // [E]
    uint32_t* offsets;     // [E+1]
    uint32_t* pair_token;  // [P] CSR rows
    uint32_t* pair_slot;   // [P]
    uint32_t* first_use;   // [E]
    uint32_t* n_active;    // [1]
    uint32_t* active_asc;  // [E]
    uint32_t* active_fu;   // [E]
    uint16_t* act;         // [P][I] bf16, CSR row order
    float* y;              // [T][K][H] per-pair down projections
    uint16_t* sact;        // [T][S] bf16 shared activation
    float* sy;             // [T][H] shared expert output
    uint4* arec;           // [E] decode path: per active slot {expert, rows, CSR offset,
                           //     tokens of the rows, 8 bits each}
    uint32_t* witems;      // wide GEMM work items (expert << 16 | 128-row chunk)
    uint32_t* n_witems;    // [1 + kWideClasses]: all items, then each size class's
    uint8_t* gscratch;     // grouping: per-chunk counts and first uses, pair ranks
    uint16_t* xp;          // [T/16][256][16][4][8] bf16 tile/residue-major xn (in y's bytes)
    // K3X_FLAG_SCALED_FP4 only (else null): q8 rows of xn and act, and their
    // scale dword pairs per 128-element tile.
    uint16_t* qx;          // [T][H] 16-bit units
    uint32_t* qxs;         // [T][H/128][2]
    uint16_t* qact;        // [P][I] 16-bit units
    uint32_t* qacts;       // [P][I/128][2]
    // Decode path: arrival counters of the fused combine (kDecodeMixBytes,
    // zero between calls); set by the entry point, not by the carve.
    uint32_t* mix;
    // The route was grouped into these buffers already (the fused Top-K and
    // grouping launch); the routed call skips its own grouping.
    bool grouped = false;
};

inline int fail_hip(hipError_t e) { return e == hipSuccess ? K3X_OK : K3X_ERR_BACKEND_UNAVAILABLE; }

// The routed call of k3x_hip_moe_forward_routed in two halves, for a caller
// that groups the route itself in between (the official layer's fused
// Top-K and grouping): routed_begin checks the parameters and carves the
// call's scratch into *s; routed_finish groups the route (unless
// s.grouped), runs the experts and the combine, and copies the taps.
int routed_begin(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                 LayerBuffers* s);
int routed_finish(k3x_hip_ctx* ctx, k3x_hip_bank* bank, const k3x_hip_moe_params* p,
                  const LayerBuffers& s, const uint16_t* xn, const uint32_t* ids,
                  const float* weights, uint16_t* out, const k3x_hip_moe_taps* taps);
// Whether the Top-K of T tokens over E experts and the grouping of its
// T * K pairs run as one launch (topk_group_kernel): the threshold Top-K's
// expert counts (256 < E <= 1024), the pairs within one grouping workgroup,
// fewer tokens than the wide GEMM takes.
bool topk_group_eligible(uint32_t E, uint32_t K, uint32_t T);
// That launch: ids and weights of the route, and the grouping into s's
// buffers (counts, offsets, CSR rows, first uses, active lists, active-slot
// records); ready (may be null) as launch_group.
int launch_topk_group(k3x_hip_ctx* ctx, const float* logits, const float* bias, uint32_t E,
                      uint32_t K, uint32_t T, float routed_scale, uint32_t renorm, uint32_t* ids,
                      float* weights, const uint32_t* ready, const LayerBuffers& s);

// The official layer's route, latent projection and shared FFN for a few
// tokens in two launches on the context stream (the shared FFN's weight
// streams beside the route's latency-bound steps):
//   front   logits = router . hidden (fp64, canonical order), latent =
//           bf16(latent_tiles . hidden), sact = GLU(shared gate/up . hidden)
//           as split [hi | lo] rows of 2 I_s;
//   select  the Top-K (sigmoid + correction, double contributions, scale 1)
//           grouped into s's buffers as launch_topk_group, and shared =
//           shared_dn . sact (fp32).
// I_s = 0: no shared FFN.
struct OfficialDecode {
    const float* router;
    const float* correction;
    uint32_t E, H, L, I_s, K, T;
    const uint16_t* hidden;    // [T][H]
    const uint4* latent_tiles; // L x H
    uint16_t* latent;          // [T][L]
    const uint4* shared_gu;    // 2 I_s x H (gate, up)
    const uint4* shared_dn;    // H x I_s
    k3x_dev::GluParams glu;
    uint16_t* sact;            // [T][2 I_s]
    float* shared;             // [T][H]
    float* logits;             // [T][E]
    uint32_t* ids;             // [T][K]
    float* weights;            // [T][K]
    const uint32_t* ready;     // the bank's admitted-slot words
};
bool official_decode_eligible(uint32_t E, uint32_t H, uint32_t L, uint32_t I_s, uint32_t K,
                              uint32_t T);
int launch_official_front(k3x_hip_ctx* ctx, const OfficialDecode& d);
int launch_official_select(k3x_hip_ctx* ctx, const OfficialDecode& d, const LayerBuffers& s);

// Makes sure ctx->scratch holds at least `bytes`; grow-only.
int ensure_scratch(k3x_hip_ctx* ctx, size_t bytes);

// Device address of the fixed no-allocation scratch on `device`, which must
// be current; taken once per device and kept.
int noalloc_scratch(int device, void** out);

// Refreshes bank->router_wp from bank->router_w on the context stream (a
// no-op when the hidden size has no residue-major copy).
int permute_router(k3x_hip_bank* bank);

// Bank-side helpers for other weight holders (official.hip), on the context
// stream: retile a bf16 matrix [rows][cols] (src on the device, or NULL for
// the seeded N(0, sigma) generator under `key`) into the tile layout as
// matrix `which` of S interleaved ones; seeded normal and constant fp32 fills.
int retile_bf16_matrix(k3x_hip_ctx* ctx, const uint16_t* src, uint64_t key, float sigma,
                       uint32_t rows, uint32_t cols, uint32_t S, uint32_t which, uint4* dst);
int fill_normal_f32_dev(k3x_hip_ctx* ctx, uint64_t key, size_t n, float sigma, float* out);
int fill_const_f32_dev(k3x_hip_ctx* ctx, size_t n, float v, float* out);

// Launchers shared with the official layer (official.hip), all on the
// context stream unless a stream is given: RMSNorm (bf16 in/out, fp32 gamma),
// router logits (fp32 W [E][H], fp64 canonical order), natural Top-K with
// renormalisation, and dense bf16 projections in the bank's tile layout
// (gate/up pair [I/16][H/128][2][4][64] -> GLU -> bf16 act [T][I]; one
// matrix [N/16][K/128][4][64] -> fp32 [T][N]).
int launch_rmsnorm(k3x_hip_ctx* ctx, const uint16_t* x, const float* gamma, uint32_t T,
                   uint32_t H, float eps, uint16_t* xn);
// Router logits; with the residue-major router copy Wp (router_wp_floats)
// and router_uses_mfma(H, T), on the matrix cores through xp, a scratch of
// router_xp_bytes(T) that receives the residue-major copy of xn.
int launch_router_logits(k3x_hip_ctx* ctx, const float* W, const float* Wp, const uint16_t* xn,
                         uint16_t* xp, uint32_t E, uint32_t H, uint32_t T, float* logits);
// The residue-major copy Wp (router_wp_floats(E) floats) of a router [E][H].
int permute_router_matrix(k3x_hip_ctx* ctx, const float* W, uint32_t E, uint32_t H, float* Wp);
bool router_uses_mfma(uint32_t H, uint32_t T);
size_t router_xp_bytes(uint32_t T);
int launch_topk(k3x_hip_ctx* ctx, const float* logits, const float* bias, uint32_t E, uint32_t K,
                uint32_t T, float routed_scale, uint32_t renorm, uint32_t* ids, float* weights);
// split: activations stored as rows [hi | lo] of 2 I (dense_gate_up) and read
// as such (dense_down, K = the activation width I), the down projection
// running over both halves: an fp32 activation into the bf16 MFMA.
int dense_gate_up(k3x_hip_ctx* ctx, const uint4* tiles, uint32_t I, uint32_t H, const uint16_t* x,
                  uint32_t T, const k3x_dev::GluParams& glu, uint16_t* act, hipStream_t stream,
                  bool split = false);
// Up to kDenseDirectTokens rows the projections run as a split-K GEMV on
// any stream, and dense_down can round its output to bf16 itself (y_bf16;
// y is then unused); above, y_bf16 must be null, and the projections run on
// the wide GEMM (any stream) where its shape rules allow, else on the narrow
// GEMM (the context stream only).
constexpr uint32_t kDenseDirectTokens = 16;
// True when both projections of a dense GLU MLP (gate/up I x H, down H x I)
// may be enqueued on a stream other than the context's for T rows.
bool dense_mlp_any_stream(uint32_t I, uint32_t H, uint32_t T);
// True when dense_down of an N x K projection over T rows may be enqueued on
// a stream other than the context's.
bool dense_down_any_stream(uint32_t N, uint32_t K, uint32_t T);
int dense_down(k3x_hip_ctx* ctx, const uint4* tiles, uint32_t N, uint32_t K, const uint16_t* a,
               uint32_t T, float* y, hipStream_t stream, uint16_t* y_bf16 = nullptr,
               bool split = false);
// Up to kDenseDirectTokens rows on the context stream: y = tiles . a with the
// official layer's output in the epilogue: routed = y (fp32) and out =
// bf16(bf16(prefix) + bf16(bf16(y) + bf16(shared))) (shared may be null).
int dense_down_output(k3x_hip_ctx* ctx, const uint4* tiles, uint32_t N, uint32_t K,
                      const uint16_t* a, uint32_t T, const float* prefix, const float* shared,
                      float* routed, uint16_t* out);
// The same output from the raw rows x: RMSNorm(x, gamma, eps) (bit for bit
// as launch_rmsnorm) formed by every workgroup in LDS, then the projection,
// in one launch.  x and gamma 16-byte aligned; shapes per
// dense_norm_output_ok.
bool dense_norm_output_ok(uint32_t N, uint32_t K, uint32_t T);
int dense_norm_output(k3x_hip_ctx* ctx, const uint4* tiles, uint32_t N, uint32_t K,
                      const uint16_t* x, const float* gamma, float eps, uint32_t T,
                      const float* prefix, const float* shared, float* routed, uint16_t* out);

// CRC32C of device bytes (storage.hip); *crc the standard value.
int crc32c_device(k3x_hip_ctx* ctx, const void* data, size_t bytes, uint32_t* crc);
// Whether any of `bytes` device bytes is 0xFF (MXFP4 scale validity).
int any_ff_device(k3x_hip_ctx* ctx, const void* data, size_t bytes, bool* found);
void free_crc(k3x_hip_ctx* ctx);
int retile_expert_device(k3x_hip_bank* b, uint32_t e, const uint8_t* const src[6]);
// Marks slot e admitted (1) or not (0) on the host and, in stream order, on
// the device.
int set_expert_ready(k3x_hip_bank* b, uint32_t e, bool ready);

// Whether a bank of this hidden size keeps the residue-major router copy,
// and that copy's size in floats (experts padded to 16).
bool router_mfma_eligible(uint32_t hidden);
size_t router_wp_floats(uint32_t experts);

// Brackets the launches made between begin and end with an event pair when
// profiling is on.  begin_stage returns the index of the open mark or -1.
int begin_stage(k3x_hip_ctx* ctx, uint32_t stage);
void end_stage(k3x_hip_ctx* ctx, int mark);
// Reads back every pending mark into the per-stage totals (synchronises).
int drain_stage_marks(k3x_hip_ctx* ctx);

}  // namespace k3x_hip
