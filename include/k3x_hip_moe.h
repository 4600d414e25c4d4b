/*
 * k3x_hip_moe.h -- C ABI of the MI355X (gfx950) routed-expert MoE layer.
 *
 * Plain C: opaque handles, plain pointers and sizes, int status codes.  No
 * exception crosses this boundary and no torch type appears in it.  Every
 * entry point validates its arguments before it touches device state
 * (fail-closed), and returns one of the k3x_status values, which are the
 * numeric values of k3x::ErrorCode (runtime/include/k3x/status.hpp:9-31).
 *
 * Pointer conventions: parameters documented "host" are CPU memory, "device"
 * are HIP device memory of the context's device.  All device work is
 * enqueued on the context's stream; entry points return after enqueueing
 * unless documented otherwise.  Errors detected by kernels (non-finite input,
 * invalid router scores) are latched in a per-context status word that
 * k3x_hip_ctx_synchronize() returns and clears; a latched error makes every
 * later kernel of the context skip its work until it is read.
 *
 * Each declaration names the reference interface it replaces (file:line in
 * the rsb1813/project-k3x tree).
 */
#ifndef K3X_HIP_MOE_H
#define K3X_HIP_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define K3X_HIP_ABI_VERSION 1

/* k3x::ErrorCode values (runtime/include/k3x/status.hpp:9-31). */
enum k3x_status {
    K3X_OK = 0,
    K3X_ERR_IO = 1,
    K3X_ERR_BAD_MAGIC = 2,
    K3X_ERR_UNSUPPORTED_VERSION = 3,
    K3X_ERR_UNSUPPORTED_REQUIRED_FEATURE = 4,
    K3X_ERR_SUPERBLOCK_CRC_MISMATCH = 6,
    K3X_ERR_TRUNCATED_FILE = 7,
    K3X_ERR_INVALID_DIRECTORY = 8,
    K3X_ERR_INVALID_EXTENT = 9,
    K3X_ERR_DATA_CRC_MISMATCH = 10,
    K3X_ERR_AUXILIARY_CRC_MISMATCH = 11,
    K3X_ERR_DIRECTORY_SHA256_MISMATCH = 12,
    K3X_ERR_ROOT_SHA256_MISMATCH = 13,
    K3X_ERR_TENSOR_NOT_FOUND = 14,
    K3X_ERR_INVALID_MXFP4 = 15,
    K3X_ERR_INVALID_STATE = 16,
    K3X_ERR_BACKEND_UNAVAILABLE = 17,
};

/* GLU activation policy.  SiTU: runtime/src/ops.cpp:20-30.
 * SwiGLU: silu(g) * u with silu from runtime/src/model.cpp:60-61. */
enum k3x_glu { K3X_GLU_SWIGLU = 0, K3X_GLU_SITU = 1 };

/* Renormalisation of the selected router scores.
 * FLOAT:  runtime/src/routing_policy.cpp:146-157 (synthetic/resident path).
 * DOUBLE: runtime/src/official_moe.cpp:235-242 (official path). */
enum k3x_renorm { K3X_RENORM_FLOAT = 0, K3X_RENORM_DOUBLE = 1 };

/* Matrices of one expert, as addressed by the debug/read-back entry points. */
enum k3x_matrix { K3X_MATRIX_GATE = 0, K3X_MATRIX_UP = 1, K3X_MATRIX_DOWN = 2 };

/* Streams of the portable synthetic generator (k3x_hip_bank_fill_synthetic):
 * stream id = (kind << 32) | expert index. */
enum k3x_synth_stream {
    K3X_STREAM_GATE_CODES = 1,
    K3X_STREAM_GATE_SCALES = 2,
    K3X_STREAM_UP_CODES = 3,
    K3X_STREAM_UP_SCALES = 4,
    K3X_STREAM_DOWN_CODES = 5,
    K3X_STREAM_DOWN_SCALES = 6,
    K3X_STREAM_ROUTER = 7,
    K3X_STREAM_BIAS = 8,
    K3X_STREAM_SHARED_GATE = 9,
    K3X_STREAM_SHARED_UP = 10,
    K3X_STREAM_SHARED_DOWN = 11,
    K3X_STREAM_INPUT = 12,
};

typedef struct k3x_hip_ctx k3x_hip_ctx;
typedef struct k3x_hip_bank k3x_hip_bank;

/* Shape of one MoE layer.  hidden and inter must be multiples of 128,
 * group_size must be 32 (the CUDA backend's contract,
 * runtime/cuda/backend_cuda.cu:1865-1867), shared_inter is 0 (no shared
 * expert) or a multiple of 128. */
typedef struct k3x_hip_layer_desc {
    uint32_t hidden;
    uint32_t inter;
    uint32_t experts;
    uint32_t group_size;
    uint32_t shared_inter;
} k3x_hip_layer_desc;

/* Per-call parameters of the layer.  Mirrors the scalar arguments of
 * ComputeBackend::resident_mxfp4_moe_layer (runtime/include/k3x/
 * backend.hpp:369-375) plus the router controls that runtime/src/
 * model.cpp:917-1010 applies on the host. */
typedef struct k3x_hip_moe_params {
    uint32_t tokens;          /* T, rows of x */
    uint32_t top_k;           /* natural Top-K, 1..64 and <= experts */
    float routed_scale;       /* multiplies renormalised weights */
    float rms_epsilon;        /* > 0 */
    uint32_t glu;             /* enum k3x_glu */
    float situ_beta;          /* > 0, SiTU only */
    uint32_t has_situ_linear; /* SiTU only */
    float situ_linear_beta;   /* > 0 when has_situ_linear */
    uint32_t renorm;          /* enum k3x_renorm */
    uint32_t flags;           /* K3X_FLAG_* */
} k3x_hip_moe_params;

/* k3x_hip_moe_params.flags */
enum k3x_flags {
    /* Use the general multi-launch path even where the decode path
     * (tokens <= 4) applies; both compute the same layer. */
    K3X_FLAG_GENERAL_PATH = 1u,
    /* Round each expert output to bf16 before the slot-ordered mix, as the
     * official layer does (runtime/src/official_moe.cpp:99-101, :318-326);
     * runs the general path. */
    K3X_FLAG_ROUND_EXPERT_OUT = 2u,
    /* Keep the routed GLU activation at fp32 precision into the down
     * projection (stored as a bf16 hi + lo pair per element, the down
     * projection run over both halves), as the official layer does
     * (runtime/src/official_moe.cpp:82-101); runs the general path. */
    K3X_FLAG_SPLIT_ACT = 4u,
    /* k3x_hip_moe_forward_routed only: the input rows are fp32 values held
     * as bf16 hi + lo halves, [T][2 H] (hi = bf16(v), lo = bf16(v - hi)),
     * and the gate/up projections run over both halves; the latent layer's
     * fp32 experts (runtime/src/backend_cpu.cpp:317-318).  Runs the
     * general path's narrow GEMMs. */
    K3X_FLAG_SPLIT_INPUT = 8u,
    /* Multiply the routed experts of the wide GEMM (prefill chunks, many
     * rows per expert) on the scaled FP4 MFMA: the bf16 activation rows are
     * re-encoded as two FP8 E4M3 terms with one power-of-two scale per 32
     * values each (exact for bf16 values down to 2^-13 of their block's
     * largest, within 2^-21 of it below), the MXFP4 weights go in as they
     * are stored.  Ignored with K3X_FLAG_SPLIT_ACT and on the decode and
     * narrow paths. */
    K3X_FLAG_SCALED_FP4 = 16u,
};

/* Optional device buffers that receive intermediates of k3x_hip_moe_forward;
 * any member may be NULL.  Shapes use T = tokens, K = top_k, E = experts,
 * H = hidden, I = inter, S = shared_inter. */
typedef struct k3x_hip_moe_taps {
    uint16_t* normed_x;          /* [T][H] bf16 bits, RMSNorm output */
    float* logits;               /* [T][E] */
    uint32_t* ids;               /* [T][K] router order */
    float* weights;              /* [T][K] contributions */
    uint32_t* counts;            /* [E] pairs per expert */
    uint32_t* offsets;           /* [E+1] expert-major CSR offsets */
    uint32_t* pair_token;        /* [T*K] CSR rows -> token */
    uint32_t* pair_slot;         /* [T*K] CSR rows -> router slot */
    uint32_t* first_use;         /* [E] min(token*K+slot), 0xffffffff unused */
    uint32_t* n_active;          /* [1] experts with at least one pair */
    uint32_t* active_first_use;  /* [E] active experts in first-use order */
    uint16_t* act;               /* [T*K][I] bf16 bits, CSR row order */
    float* expert_out;           /* [T][K][H] per-pair down projections */
    float* shared_out;           /* [T][H] shared expert output */
    float* out_f32;              /* [T][H] output before the bf16 cast */
    uint16_t* shared_act;        /* [T][S] bf16 bits, shared-expert GLU output */
} k3x_hip_moe_taps;

/* Descriptor of the seeded synthetic bank (no reference counterpart: the
 * reference's benches read converted checkpoints).  Codes are uniform over
 * the 16 E2M1 codes, scale bytes uniform over [scale_lo, scale_hi], normal
 * tensors are Irwin-Hall(12) approximations of N(0, sigma^2). */
typedef struct k3x_hip_synth_desc {
    uint64_t seed;
    uint32_t scale_lo;
    uint32_t scale_hi;
    float router_sigma;
    float bias_sigma;
    float shared_sigma;
    float gamma_value;
} k3x_hip_synth_desc;

/* Stages of k3x_hip_moe_forward timed by k3x_hip_ctx_set_profiling. */
enum k3x_stage {
    K3X_STAGE_ROUTE = 0,        /* RMSNorm, router logits, Top-K */
    K3X_STAGE_GROUP = 1,        /* expert-major grouping */
    K3X_STAGE_GATE_UP = 2,      /* routed MXFP4 gate/up + GLU */
    K3X_STAGE_SHARED_GATE_UP = 3,
    K3X_STAGE_DOWN = 4,         /* routed MXFP4 down projection */
    K3X_STAGE_SHARED_DOWN = 5,
    K3X_STAGE_COMBINE = 6,      /* slot-ordered mix + shared add + bf16 cast */
    /* Decode path (T <= 4); its combine is part of K3X_STAGE_DECODE_DOWN. */
    K3X_STAGE_DECODE_FRONT = 7,   /* RMSNorm, router logits, shared gate/up */
    K3X_STAGE_DECODE_SELECT = 8,  /* Top-K, grouping, shared down */
    K3X_STAGE_DECODE_GATE_UP = 9, /* routed gate/up + GLU */
    K3X_STAGE_DECODE_DOWN = 10,   /* routed down, then the slot-ordered mix */
    K3X_STAGE_COUNT = 11,
};

/* Counters, after BackendRuntimeStats (runtime/include/k3x/backend.hpp:50-129). */
typedef struct k3x_hip_stats {
    uint64_t forward_calls;
    uint64_t kernel_launches;
    uint64_t scratch_bytes;
    uint64_t resident_weight_bytes;
    uint64_t weight_h2d_bytes;
    uint64_t experts_resident;
} k3x_hip_stats;

/* ---- context ------------------------------------------------------------ */

/* Replaces make_cuda_backend (runtime/include/k3x/backend.hpp:465-466;
 * runtime/cuda/backend_cuda.cu:5264-5367): one device, one stream. */
int k3x_hip_ctx_create(int device, k3x_hip_ctx** out);
/* Fails with K3X_ERR_INVALID_STATE while banks created on the context are
 * alive: destroy them first. */
int k3x_hip_ctx_destroy(k3x_hip_ctx* ctx);
/* Enqueue on a caller-owned hipStream_t (NULL = the device's null stream). */
int k3x_hip_ctx_set_stream(k3x_hip_ctx* ctx, void* hip_stream);
/* Back to the context's own non-blocking stream (the default). */
int k3x_hip_ctx_use_own_stream(k3x_hip_ctx* ctx);
void* k3x_hip_ctx_stream(k3x_hip_ctx* ctx);
/* Waits for the stream, returns and clears the latched kernel status.
 * Replaces the cudaStreamSynchronize at the end of each backend call
 * (e.g. runtime/cuda/backend_cuda.cu:2421). */
int k3x_hip_ctx_synchronize(k3x_hip_ctx* ctx);
/* Replaces ComputeBackend::runtime_stats (backend.hpp:331). */
int k3x_hip_ctx_stats(k3x_hip_ctx* ctx, k3x_hip_stats* out);
const char* k3x_hip_status_name(int status); /* error_code_name, status.hpp:33-56 */
/* Per-stage device timing: when enabled, every stage that a forward call
 * enqueues is bracketed by a hipEvent pair on the context stream (the
 * reference brackets each launch with cudaEvent pairs and records
 * ProfileEvent::device_nanoseconds, runtime/cuda/backend_cuda.cu:2251-2298,
 * runtime/include/k3x/profile.hpp:32-42). */
int k3x_hip_ctx_set_profiling(k3x_hip_ctx* ctx, int enabled);
/* Waits for the stream, then adds the elapsed milliseconds and the number of
 * timed launches of each stage since the last reset into ms[K3X_STAGE_COUNT]
 * and launches[K3X_STAGE_COUNT] (host arrays, overwritten); reset != 0
 * clears the totals afterwards. */
int k3x_hip_ctx_stage_times(k3x_hip_ctx* ctx, double* ms, uint64_t* launches,
                            int reset);

/* ---- resident expert bank ------------------------------------------------ */

/* Replaces ResidentWeightTable (runtime/cuda/resident_weights.cuh:19-25,
 * resident_weights.cu:107-166): the whole layer's bank is allocated once in
 * HBM in the gfx950 tile layout and admitted expert by expert. */
int k3x_hip_bank_create(k3x_hip_ctx* ctx, const k3x_hip_layer_desc* desc,
                        k3x_hip_bank** out);
int k3x_hip_bank_destroy(k3x_hip_bank* bank);
/* Admits one expert from host memory in the K3X reference layout (packed
 * [rows][cols/2], low nibble = even column; scales [rows][cols/32] E8M0),
 * gate/up [inter x hidden], down [hidden x inter].  tensor_ids are the
 * residency identities (non-zero, unique within the bank), as in
 * Mxfp4WeightView::tensor_id (backend.hpp:150-157).  Scale byte 0xFF is
 * rejected with K3X_ERR_INVALID_MXFP4 (runtime/src/ops.cpp:46-49).
 * Synchronous. */
int k3x_hip_bank_upload_expert(k3x_hip_bank* bank, uint32_t expert,
                               const uint64_t tensor_ids[3],
                               const uint8_t* gate_packed,
                               const uint8_t* gate_scales,
                               const uint8_t* up_packed,
                               const uint8_t* up_scales,
                               const uint8_t* down_packed,
                               const uint8_t* down_scales);
/* Finds the expert/matrix admitted under tensor_id (host). */
int k3x_hip_bank_find(k3x_hip_bank* bank, uint64_t tensor_id,
                      uint32_t* expert, uint32_t* matrix);
/* Shared expert, host bf16 bits: gate/up [shared_inter x hidden],
 * down [hidden x shared_inter] (Bf16MlpView, backend.hpp:165-169). */
int k3x_hip_bank_upload_shared(k3x_hip_bank* bank, const uint16_t* gate,
                               const uint16_t* up, const uint16_t* down);
/* Router weight fp32 [experts x hidden], correction bias fp32 [experts],
 * RMSNorm weight fp32 [hidden]; host memory (router_weight /
 * correction_bias of runtime/src/model.cpp:918-922). */
int k3x_hip_bank_upload_router(k3x_hip_bank* bank, const float* weight,
                               const float* bias, const float* gamma);
/* Same, from device memory (no host round trip). */
int k3x_hip_bank_set_router_device(k3x_hip_bank* bank, const float* weight,
                                   const float* bias, const float* gamma);
/* Fills every expert, the router, the bias, gamma and the shared expert
 * from the seeded generator on the device (identical to the oracle's
 * generator, so the CPU checker can regenerate any expert). */
int k3x_hip_bank_fill_synthetic(k3x_hip_bank* bank,
                                const k3x_hip_synth_desc* desc);
/* Fills a device bf16 tensor of n elements with the seeded normal generator
 * (stream K3X_STREAM_INPUT). */
int k3x_hip_synth_normal_bf16(k3x_hip_ctx* ctx, uint64_t seed,
                              uint64_t stream, float sigma, size_t n,
                              uint16_t* out);
/* Debug read-back: rows [row0, row0+nrows) of one matrix, dequantised to
 * fp32 by the same conversion the GEMM kernels use, into device memory
 * out [nrows][cols].  Replaces decode_mxfp4 (runtime/src/ops.cpp:32-55)
 * for the bit-exact weight check. */
int k3x_hip_bank_dequant_rows(k3x_hip_bank* bank, uint32_t expert,
                              uint32_t matrix, uint32_t row0, uint32_t nrows,
                              float* out);
uint64_t k3x_hip_bank_bytes(const k3x_hip_bank* bank);

/* ---- the layer ----------------------------------------------------------- */

/* One routed-expert MoE layer over T tokens with device routing:
 *   xn  = bf16(RMSNorm(x) * gamma)                        (ops.cpp:10-18)
 *   ids, w = natural Top-K of sigmoid(W_r xn) + bias,
 *            renormalised, * routed_scale    (model.cpp:917-1009,
 *            routing_policy.cpp:31-160 / official_moe.cpp:211-245)
 *   expert-major grouping                          (expert_major.cpp:10-54)
 *   y[t][k] = down(bf16(GLU(gate xn, up xn)))   (backend_cpu.cpp:124-154)
 *   out = bf16(sum_k w[t][k] y[t][k] + shared(xn))  (backend_cpu.cpp:295-301,
 *                                                    model.cpp:1145)
 * x: device bf16 [T][hidden]; out: device bf16 [T][hidden]; taps optional.
 * Replaces ComputeBackend::resident_mxfp4_moe_layer (backend.hpp:369-375,
 * runtime/cuda/backend_cuda.cu:1789-2545) for a latent-free layer with
 * routing on the device.  Asynchronous. */
int k3x_hip_moe_forward(k3x_hip_ctx* ctx, k3x_hip_bank* bank,
                        const k3x_hip_moe_params* params, const uint16_t* x,
                        uint16_t* out, const k3x_hip_moe_taps* taps);

/* Bytes of the fixed device scratch behind k3x_hip_moe_forward_noalloc. */
#define K3X_HIP_NOALLOC_SCRATCH_BYTES (32u << 20)

/* k3x_hip_moe_forward that allocates nothing: no reference counterpart.  It
 * is for callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  The
 * per-call buffers (normalised input, logits, routes, grouping, activations,
 * per-pair outputs, shared expert) come from a fixed device array of
 * K3X_HIP_NOALLOC_SCRATCH_BYTES per device (32 MiB, held until the process
 * ends) instead of the context's grow-only scratch; a call whose buffers do
 * not fit in it less its last 16 KiB returns K3X_ERR_INVALID_EXTENT before
 * anything is enqueued (the config-3 decode layer needs about 1.1 MiB, T=16
 * of it about 9 MiB).  The array is shared by every call on the device,
 * whatever the context or stream: calls that overlap on one GPU race, so a
 * caller serialises them (one stream, or events).  Its last 16 KiB hold the
 * decode path's combine counters, zero when the process loads the library
 * and left zero by every call that completes; nothing else in it needs to
 * start at zero (every other buffer a call reads was written earlier in the
 * same call).  Stage timing
 * (k3x_hip_ctx_set_profiling) is not recorded for these calls.  Results are
 * bit-identical to k3x_hip_moe_forward's.  Asynchronous. */
int k3x_hip_moe_forward_noalloc(k3x_hip_ctx* ctx, k3x_hip_bank* bank,
                                const k3x_hip_moe_params* params, const uint16_t* x,
                                uint16_t* out, const k3x_hip_moe_taps* taps);

/* The same layer with host-decided routes (the reference's own contract:
 * routing on the host, model.cpp:917-1010): xn is the already-normalised
 * bf16 input [T][hidden], ids/weights device [T][K] in router order.  Routes
 * must not repeat an expert within a token and weights must be finite
 * (checked on the host copy passed in host_ids/host_weights, which may be
 * NULL to skip the host check).  Only the routed slots must hold admitted
 * experts: with host_ids the call returns K3X_ERR_INVALID_STATE otherwise;
 * without, the grouping latches K3X_ERR_INVALID_STATE for a route to an
 * empty slot, an expert id out of range or an expert repeated within a
 * token.  Replaces ComputeBackend::mxfp4_situ_moe
 * (backend.hpp:364-368) batched over tokens.  Asynchronous. */
int k3x_hip_moe_forward_routed(k3x_hip_ctx* ctx, k3x_hip_bank* bank,
                               const k3x_hip_moe_params* params,
                               const uint16_t* xn, const uint32_t* ids,
                               const float* weights, const uint32_t* host_ids,
                               const float* host_weights, uint16_t* out,
                               const k3x_hip_moe_taps* taps);

/* Expert-major grouping of device ids [T][K] into the CSR taps (counts,
 * offsets, pair_token, pair_slot, first_use, n_active, active_first_use must
 * be non-NULL).  Replaces build_expert_major_plan
 * (runtime/include/k3x/expert_major.hpp:33-34, expert_major.cpp:10-54).
 * Asynchronous. */
int k3x_hip_expert_major_plan(k3x_hip_ctx* ctx, const uint32_t* ids,
                              uint32_t tokens, uint32_t top_k,
                              uint32_t experts, const k3x_hip_moe_taps* taps);

/* ---- official K3 MoE FFN (Stable LatentMoE) ------------------------------ */

/* The official layer wraps a bank of experts that run at the latent width L
 * (the bank's hidden): routed_down [L][H] bf16 -> experts -> slot-ordered
 * mix -> routed_norm RMSNorm -> routed_up [H][L] bf16, plus a bf16 shared
 * FFN at H (shared_inter Is, the reference's two shared experts side by
 * side) and the prefix add (runtime/src/official_moe.cpp:271-344;
 * OfficialMoeFfnView, runtime/include/k3x/backend.hpp:171-176). */
typedef struct k3x_hip_official k3x_hip_official;

typedef struct k3x_hip_official_desc {
    uint32_t hidden;          /* H, multiple of 128 */
    uint32_t shared_inter;    /* Is, 0 (none) or a multiple of 128 */
    uint32_t router_experts;  /* rows of the router: 0 (the bank's experts) with
                                 a bank; without one (a route-only object:
                                 uploads of the route and prepare only;
                                 shared_inter 0), the router's row count */
} k3x_hip_official_desc;

/* Optional device buffers for intermediates of k3x_hip_official_ffn (any may
 * be NULL).  T tokens, K top_k, E experts, L latent, H hidden. */
typedef struct k3x_hip_official_taps {
    float* logits;         /* [T][E] (device routing only) */
    uint32_t* ids;         /* [T][K] route order */
    float* contributions;  /* [T][K] */
    uint16_t* latent;      /* [T][L] bf16 bits, routed_down output */
    float* expert_out;     /* [T][K][L] expert outputs before their bf16 rounding */
    uint16_t* mixed;       /* [T][L] bf16 bits, slot-ordered mix */
    float* routed;         /* [T][H] routed_up output before rounding */
    float* shared;         /* [T][H] shared FFN output before rounding */
} k3x_hip_official_taps;

/* experts: a bank of hidden L (its own shared expert unused); the official
 * layer keeps a reference to it and must be destroyed first.  experts NULL
 * makes a route-only object (desc->router_experts rows): upload_route,
 * fill_synthetic and prepare work on it, upload_ffn and ffn return
 * K3X_ERR_INVALID_STATE -- route preparation needs no experts, as
 * prepare_official_moe_route (backend.hpp:384-389) takes none. */
int k3x_hip_official_create(k3x_hip_ctx* ctx, k3x_hip_bank* experts,
                            const k3x_hip_official_desc* desc,
                            k3x_hip_official** out);
int k3x_hip_official_destroy(k3x_hip_official* official);

/* Host bf16 words: routed_down [L][H], routed_norm [L], routed_up [H][L];
 * shared gate, up [Is][H] and down [H][Is] (NULL when Is = 0).
 * OfficialMoeFfnView (backend.hpp:171-176).  Synchronous. */
int k3x_hip_official_upload_ffn(k3x_hip_official* official, const uint16_t* routed_down,
                                const uint16_t* routed_norm, const uint16_t* routed_up,
                                const uint16_t* shared_gate, const uint16_t* shared_up,
                                const uint16_t* shared_down);

/* Host: bf16 words residual_norm [H], residual_proj [H], post_norm [H],
 * router [E][H]; fp32 correction [E].  OfficialMoeRoutePrepareView
 * (backend.hpp:184-189) plus the router correction.  Synchronous. */
int k3x_hip_official_upload_route(k3x_hip_official* official, const uint16_t* residual_norm,
                                  const uint16_t* residual_proj, const uint16_t* post_norm,
                                  const uint16_t* router, const float* correction);

/* Seeded synthetic weights for both uploads (no reference counterpart):
 * dense matrices and the router ~ N(0, sigma^2) in bf16, the three norm
 * vectors 1, residual_proj ~ N(0, proj_sigma^2), correction ~
 * N(0, correction_sigma^2).  Synchronous. */
int k3x_hip_official_fill_synthetic(k3x_hip_official* official, uint64_t seed, float sigma,
                                    float router_sigma, float proj_sigma,
                                    float correction_sigma);

/* Route preparation for T tokens: the two-source attention-residual mix and
 * post-norm (official_moe.cpp:156-209) -> hidden bf16 [T][H], and, when
 * logits is non-NULL, the router logits [T][E] over it (official_moe.cpp:
 * 247-269).  prefix and block_residual device fp32 [T][H].  Replaces
 * ComputeBackend::prepare_official_moe_route (backend.hpp:384-389) with the
 * hidden kept on the device.  Asynchronous. */
int k3x_hip_official_prepare(k3x_hip_ctx* ctx, k3x_hip_official* official, uint32_t tokens,
                             float rms_epsilon, const float* prefix,
                             const float* block_residual, uint16_t* hidden, float* logits);

/* The FFN for T tokens: hidden bf16 [T][H] (prepared), prefix fp32 [T][H];
 * the route as device ids [T][K] + contributions [T][K], or ids ==
 * contributions == NULL to route on the device (router logits over hidden,
 * sigmoid + correction, natural Top-K, contributions s / sum s in double:
 * official_moe.cpp:211-245; every slot of the bank must then hold an
 * admitted expert, while a given route needs only its own slots).  out bf16 [T][H] = bf16(bf16(prefix) +
 * bf16(routed + shared)).  params: tokens, top_k, rms_epsilon and the GLU
 * (SiTU for the reference's layer); routed_scale, renorm and flags are not
 * used.  Replaces ComputeBackend::official_mxfp4_moe_ffn
 * (backend.hpp:376-383) batched over tokens.  Asynchronous. */
int k3x_hip_official_ffn(k3x_hip_ctx* ctx, k3x_hip_official* official,
                         const k3x_hip_moe_params* params, const uint16_t* hidden,
                         const float* prefix, const uint32_t* ids,
                         const float* contributions, uint16_t* out,
                         const k3x_hip_official_taps* taps);

/* ---- fp32 products and the resident latent layer ------------------------ */

/* The fp32 operations of ComputeBackend: each product is formed exactly in
 * double and summed in double, one rounding to fp32 at the end (the
 * reference sums sequentially; only the order differs).  All pointers are
 * device memory; every call is asynchronous on the context stream.  Inputs
 * x are [tokens][cols] fp32, outputs [tokens][rows] fp32. */

/* y = W x, W fp32 [rows][cols] row-major.  Replaces
 * ComputeBackend::dense_matvec (runtime/include/k3x/backend.hpp:333-335;
 * runtime/src/backend_cpu.cpp:22-45). */
int k3x_hip_dense_f32_matvec(k3x_hip_ctx* ctx, const float* W, uint32_t rows, uint32_t cols,
                             const float* x, uint32_t tokens, float* y);

/* y = W x for an MXFP4 matrix in the K3X layout: packed [rows][cols / 2]
 * (low nibble = even column, 16-byte aligned), E8M0 scales
 * [rows][cols / 32], group size 32.  Replaces ComputeBackend::mxfp4_matvec
 * (backend.hpp:336-338; backend_cpu.cpp:47-59, runtime/src/ops.cpp:57-76);
 * scale bytes must be checked for 0xFF by the caller (the reference's
 * decode_mxfp4 rejects them). */
int k3x_hip_mxfp4_matvec(k3x_hip_ctx* ctx, const uint8_t* packed, const uint8_t* scales,
                         uint32_t rows, uint32_t cols, const float* x, uint32_t tokens, float* y);

/* The fp32 SiTU MLP: act [tokens][inter] = situ_glu(gate x, up x) (gate and
 * up [inter][hidden]), y [tokens][out_rows] = down act (down
 * [out_rows][inter]).  Replaces ComputeBackend::dense_situ_mlp
 * (backend.hpp:345-348; backend_cpu.cpp:108-122). */
int k3x_hip_dense_situ_mlp(k3x_hip_ctx* ctx, const float* gate, const float* up,
                           const float* down, uint32_t hidden, uint32_t inter, uint32_t out_rows,
                           float situ_beta, int has_situ_linear, float situ_linear_beta,
                           const float* x, uint32_t tokens, float* act, float* y);

/* fp32 dense weights of the resident latent MoE layer, device row-major
 * (ResidentMoeLayerView, backend.hpp:302-307). */
typedef struct k3x_hip_latent_weights {
    const float* routed_down;  /* [latent][hidden] */
    const float* routed_norm;  /* [latent] */
    const float* routed_up;    /* [hidden][latent] */
    const float* shared_gate;  /* [shared_inter][hidden] */
    const float* shared_up;    /* [shared_inter][hidden] */
    const float* shared_down;  /* [hidden][shared_inter] */
    uint32_t hidden, latent, shared_inter;
    /* The width routed_norm's RMSNorm divides the sum of squares by: 0 means
     * latent.  A caller that pads the latent to the bank's width with zeros
     * (zero routed_down rows, zero expert codes in the padded rows and
     * columns, zero routed_norm entries and routed_up columns) passes the
     * unpadded width, so the padded layer computes the unpadded one. */
    uint32_t latent_norm;
} k3x_hip_latent_weights;

/* The resident latent MoE layer for T tokens: latent = routed_down x; the
 * routed experts of `bank` (hidden = latent, no shared expert) on the fp32
 * latent, slots ids [T][K] (device) mixed in slot order with contributions
 * [T][K] in fp32; normalized = RMSNorm(mixed, routed_norm); out [T][hidden]
 * = routed_up normalized + the fp32 SiTU MLP of x.  x, out device fp32;
 * mixed_out (optional) receives the mix [T][latent].  params: tokens,
 * top_k, rms_epsilon, glu = SiTU and its betas; flags must be 0 (the call
 * sets its own).  host_ids / host_contributions as
 * k3x_hip_moe_forward_routed.  Replaces
 * ComputeBackend::resident_mxfp4_moe_layer (backend.hpp:369-375;
 * runtime/src/backend_cpu.cpp:305-339, runtime/cuda/backend_cuda.cu:
 * 1789-2545). */
int k3x_hip_resident_moe_layer(k3x_hip_ctx* ctx, k3x_hip_bank* bank,
                               const k3x_hip_latent_weights* weights,
                               const k3x_hip_moe_params* params, const float* x,
                               const uint32_t* ids, const float* contributions,
                               const uint32_t* host_ids, const float* host_contributions,
                               float* out, float* mixed_out);

/* ---- Measurement --------------------------------------------------------- */

/* Streams `bytes` device bytes at `data` (16-byte aligned, a multiple of 16)
 * through the vector memory path once, on the context stream, and XORs
 * every 32-bit word of them into *fold (device memory, left as is
 * otherwise): the device's plain streaming-read rate, the practical ceiling
 * that a streaming kernel's HBM rate is read against beside the nominal
 * 8 TB/s.  No counterpart in the reference (measurement only).
 * Asynchronous. */
int k3x_hip_stream_read(k3x_hip_ctx* ctx, const void* data, size_t bytes, uint32_t* fold);

/* ---- K3X storage records -------------------------------------------------- */

/* CRC32C (Castagnoli, reflected, preset and final inversion 0xFFFFFFFF) of
 * `bytes` device bytes at `data` (16-byte aligned), computed on the device:
 * the value runtime/src/crc32c.cpp:22-28 computes on the host, for data
 * already in HBM.  Synchronous (the context stream is drained). */
int k3x_hip_crc32c(k3x_hip_ctx* ctx, const void* data, size_t bytes, uint32_t* crc);

/* Uploads expert `expert` of the bank from six device extents in the K3X
 * storage order -- gate codes, gate scales, up codes, up scales, down codes,
 * down scales (runtime/src/storage_slice.cpp:56-73), each 16-byte aligned
 * and of the bank's sizes -- after checking each against its CRC32C
 * (crc32c[6] as the tensor records hold them, runtime/src/reader.cpp:98-99;
 * NULL skips the check): K3X_ERR_DATA_CRC_MISMATCH or
 * K3X_ERR_AUXILIARY_CRC_MISMATCH, slot untouched, on a mismatch; a scale
 * byte 0xFF is K3X_ERR_INVALID_MXFP4.  Identities as
 * k3x_hip_bank_upload_expert.  Synchronous. */
int k3x_hip_bank_upload_expert_device(k3x_hip_bank* bank, uint32_t expert,
                                      const uint64_t tensor_ids[3],
                                      const uint8_t* const extents[6],
                                      const uint32_t crc32c[6]);

/* A K3X checkpoint opened for expert loads (K3X_FORMAT.md).  Opening reads
 * and checks the superblock and the directories as Reader::open does
 * (runtime/src/reader.cpp:414-560): magic, version, superblock CRC32C,
 * required features, reserved bytes, finalized state and length, directory
 * ranges and headers, model-config invariants, tensor record fields,
 * distinct tensor ids; every tensor extent in range, 4 KiB aligned and
 * disjoint from the others.  Status codes are the reader's (K3X_ERR_IO ..
 * K3X_ERR_INVALID_EXTENT).  Host work only. */
typedef struct k3x_hip_storage k3x_hip_storage;
int k3x_hip_storage_open(const char* path, k3x_hip_storage** out);
int k3x_hip_storage_close(k3x_hip_storage* storage);
/* The checks Reader::open adds with VerifyMode::checksums
 * (runtime/src/reader.cpp:672-721), in its order: every tensor's data and
 * auxiliary CRC32C (K3X_ERR_DATA_CRC_MISMATCH, K3X_ERR_AUXILIARY_CRC_MISMATCH),
 * the SHA-256 of the tensor, layer and expert directories and the model
 * config concatenated against superblock bytes 168..199
 * (K3X_ERR_DIRECTORY_SHA256_MISMATCH), the SHA-256 of the whole file with
 * bytes 200..231 and 4092..4095 read as zeros against bytes 200..231
 * (K3X_ERR_ROOT_SHA256_MISMATCH).  Host work only (SHA-256 is sequential). */
int k3x_hip_storage_verify(k3x_hip_storage* storage);

/* load_storage_expert (runtime/src/storage_slice.cpp:42-92) into bank slot
 * `expert`: the tensors model.layers.<layer>.feed_forward.experts.<id>.
 * {gate,up,down}, found by the FNV-1a 64 hash of their names, must be
 * native MXFP4 matrices of the bank's shape (gate/up [inter][hidden], down
 * [hidden][inter]; K3X_ERR_INVALID_MXFP4) of that layer and expert; the
 * artifact must carry the STORAGE_FIXTURE optional feature
 * (K3X_ERR_INVALID_EXTENT otherwise).  The six extents are read in one batch
 * into pinned host memory, copied to the device once, checked against their
 * records' CRC32C on the device and uploaded with
 * k3x_hip_bank_upload_expert_device; the slot's tensor ids are the records'.
 * *bytes_read (may be NULL): the six extents' total.  ordered_sha256 (may be
 * NULL; 32 bytes): the SHA-256 of the six extents in their order (gate data,
 * gate scales, up data, up scales, down data, down scales), the digest
 * load_storage_expert returns (storage_slice.cpp:80-90), formed on the host
 * from the bytes read.  Synchronous. */
int k3x_hip_storage_upload_expert(k3x_hip_storage* storage, k3x_hip_bank* bank, uint32_t expert,
                                  uint32_t layer_id, uint32_t expert_id, uint64_t* bytes_read,
                                  uint8_t* ordered_sha256);

#ifdef __cplusplus
}
#endif
#endif
