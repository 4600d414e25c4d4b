/*
 * k3x_oracle.h -- CPU restatement of the K3X routed-expert MoE-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (project-k3x_amd/) links,
 * loads or calls this code.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the rsb1813/project-k3x tree).  Functions marked
 * "canonical order" fix a floating-point summation order that the HIP kernels
 * reproduce exactly; tests compare them against the reference-order variant.
 */
#ifndef K3X_ORACLE_H
#define K3X_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Numeric values of k3x::ErrorCode (runtime/include/k3x/status.hpp:9-31). */
enum {
    K3XO_OK = 0,
    K3XO_INVALID_EXTENT = 9,
    K3XO_INVALID_MXFP4 = 15,
    K3XO_INVALID_STATE = 16,
};

/* GLU policies.  SiTU: runtime/src/ops.cpp:20-30.  SwiGLU: silu(g)*u with
 * silu from runtime/src/model.cpp:60-61. */
enum { K3XO_GLU_SWIGLU = 0, K3XO_GLU_SITU = 1 };

/* Renormalisation conventions of the selected router scores.
 * FLOAT:  runtime/src/routing_policy.cpp:146-157 (float sum, float divide)
 * DOUBLE: runtime/src/official_moe.cpp:235-242 (double sum, double divide). */
enum { K3XO_RENORM_FLOAT = 0, K3XO_RENORM_DOUBLE = 1 };

/* Sigmoid flavours for the router.  REF uses the C library expf exactly as
 * runtime/src/model.cpp:60 and official_moe.cpp:221 do; CR uses the
 * correctly-rounded exp below, which the HIP router kernel also uses. */
enum { K3XO_SIGMOID_REF = 0, K3XO_SIGMOID_CR = 1 };

/* Logit summation orders.  SEQ: sequential double (backend_cpu.cpp:33-41,
 * official_moe.cpp:255-266).  CANON: the 256-way strided partials + pairwise
 * tree that the HIP kernels use. */
enum { K3XO_ORDER_SEQ = 0, K3XO_ORDER_CANON = 1 };

/* ---- bf16 ---------------------------------------------------------------- */
float k3xo_round_bf16(float value);          /* official_moe.cpp:18-26 */
uint16_t k3xo_bf16_bits(float value);        /* bits of k3xo_round_bf16 */
float k3xo_bf16_to_f32(uint16_t word);       /* official_moe.cpp:135-137 */

/* ---- MXFP4 --------------------------------------------------------------- */
int k3xo_decode_mxfp4(const uint8_t* packed, size_t packed_len,
                      const uint8_t* scales, size_t scales_len, size_t rows,
                      size_t cols, size_t group_size, float* out);
int k3xo_mxfp4_matvec(const float* input, size_t input_len,
                      const uint8_t* packed, size_t packed_len,
                      const uint8_t* scales, size_t scales_len, size_t rows,
                      size_t cols, size_t group_size, float* out);

/* ---- element-wise / norms ------------------------------------------------ */
void k3xo_rms_norm(float* out, const float* in, const float* weight, size_t n,
                   float epsilon);
void k3xo_rms_norm_canon(float* out, const float* in, const float* weight,
                         size_t n, float epsilon);
void k3xo_glu(float* out, const float* gate, const float* up, size_t n,
              int kind, float beta, int has_linear, float linear_beta);
float k3xo_expf_cr(float x);
float k3xo_sigmoid(float x, int mode);

/* ---- router ---------------------------------------------------------------*/
double k3xo_canon_dot(const float* a, const float* b, size_t n);
void k3xo_router_logits(const float* weight, const float* x, size_t experts,
                        size_t hidden, int order, float* logits);
int k3xo_select(const float* scores, const float* bias, size_t experts,
                size_t top_k, int renorm, float routed_scale, uint32_t* ids,
                float* weights);
int k3xo_route(const float* logits, const float* bias, size_t experts,
               size_t top_k, int renorm, float routed_scale, int sigmoid_mode,
               uint32_t* ids, float* weights, float* scores);

/* ---- expert-major grouping ------------------------------------------------*/
int k3xo_expert_major_plan(const uint32_t* ids, const float* contributions,
                           size_t tokens, size_t top_k, size_t* n_groups,
                           uint32_t* group_expert, uint32_t* group_start,
                           uint32_t* assign_token, uint32_t* assign_slot,
                           float* assign_contribution);
int k3xo_expert_major_csr(const uint32_t* ids, size_t tokens, size_t top_k,
                          size_t experts, uint32_t* counts, uint32_t* offsets,
                          uint32_t* pair_token, uint32_t* pair_slot,
                          uint32_t* first_use, uint32_t* n_active,
                          uint32_t* active_ascending,
                          uint32_t* active_first_use);

/* ---- expert FFN and the layer --------------------------------------------*/
int k3xo_expert_ffn(const float* x, size_t hidden, size_t inter,
                    const uint8_t* gate_packed, const uint8_t* gate_scales,
                    const uint8_t* up_packed, const uint8_t* up_scales,
                    const uint8_t* down_packed, const uint8_t* down_scales,
                    int glu, float beta, int has_linear, float linear_beta,
                    int round_act, float* act_out, float* out);
void k3xo_bf16_matvec(const float* x, const uint16_t* weight, size_t rows,
                      size_t cols, float* out);
void k3xo_shared_ffn(const float* x, size_t hidden, size_t inter,
                     const uint16_t* gate, const uint16_t* up,
                     const uint16_t* down, int glu, float beta, int has_linear,
                     float linear_beta, int round_act, float* out);
void k3xo_ordered_mix(const float* expert_out, const float* weights,
                      size_t top_k, size_t width, float* mixed);

/* ---- official K3 MoE FFN (Stable LatentMoE) -----------------------------*/
void k3xo_bf16_matvec_rounded(const float* x, const uint16_t* weight,
                              size_t rows, size_t cols, float* out);
void k3xo_official_norm(const float* in, const uint16_t* weight, size_t n,
                        float epsilon, float* out);
int k3xo_official_prepare(const float* prefix, const float* block_residual,
                          size_t width, const uint16_t* residual_norm,
                          const uint16_t* residual_proj,
                          const uint16_t* post_norm, float epsilon,
                          float* hidden);
void k3xo_official_shared(const float* x, size_t hidden, size_t inter,
                          const uint16_t* gate, const uint16_t* up,
                          const uint16_t* down, int glu, float beta,
                          int has_linear, float linear_beta, float* out);
/* experts: per routed slot, six pointers (gate packed, gate scales, up
 * packed, up scales, down packed, down scales) of an expert of hidden L.
 * Intermediate outputs may be NULL. */
int k3xo_official_ffn(const float* hidden, const float* prefix, size_t width,
                      size_t latent, size_t inter, size_t shared_inter,
                      const uint16_t* routed_down, const uint16_t* routed_norm,
                      const uint16_t* routed_up, const uint16_t* shared_gate,
                      const uint16_t* shared_up, const uint16_t* shared_down,
                      const uint8_t* const* experts, const float* contributions,
                      size_t top_k, float epsilon, int glu, float beta,
                      int has_linear, float linear_beta, float* latent_out,
                      float* expert_out, float* mixed_out, float* routed_out,
                      float* shared_out, float* out);

/* ---- fp32 backend operations and the resident latent layer --------------*/
/* y = W x, W fp32 [rows][cols], sequential double sum per row. */
void k3xo_dense_matvec(const float* x, const float* weight, size_t rows,
                       size_t cols, float* out);
/* act = situ_glu(gate x, up x) [inter], out = down act [out_rows]; act may
 * be NULL. */
void k3xo_dense_situ_mlp(const float* x, size_t hidden, size_t inter,
                         size_t out_rows, const float* gate, const float* up,
                         const float* down, float beta, int has_linear,
                         float linear_beta, float* act, float* out);
/* The executed path of the resident latent MoE layer for one token.
 * experts: per slot, the six pointers of k3xo_official_ffn (an expert of
 * hidden `latent`, down rows `latent`).  mixed_out [latent] may be NULL. */
int k3xo_resident_layer(const float* input, size_t hidden, size_t latent,
                        size_t inter, size_t shared_inter,
                        const float* routed_down, const float* routed_norm,
                        const float* routed_up, const float* shared_gate,
                        const float* shared_up, const float* shared_down,
                        const uint8_t* const* experts, const float* contributions,
                        size_t n_experts, float epsilon, float beta,
                        int has_linear, float linear_beta, float* mixed_out,
                        float* out);

/* ---- the whole layer, threaded (CPU baseline) ---------------------------*/
/* expert_bytes: [experts][6] pointers (gate packed, gate scales, up packed,
 * up scales, down packed, down scales); experts no route reaches may be
 * NULL.  x: [tokens][hidden] input; shared_*: bf16 words (shared_inter 0:
 * none). */
typedef struct k3xo_layer_args {
    const float* x;
    const float* gamma;
    float epsilon;
    const float* router;
    const float* bias;
    size_t tokens, hidden, inter, experts, top_k, shared_inter;
    float routed_scale;
    int renorm;
    const uint8_t* const* expert_bytes;
    const uint16_t* shared_gate;
    const uint16_t* shared_up;
    const uint16_t* shared_down;
    int glu;
    float beta;
    int has_linear;
    float linear_beta;
    int round_act;
} k3xo_layer_args;
/* ids_out, weights_out [tokens][top_k]; out [tokens][hidden]. */
int k3xo_moe_layer(const k3xo_layer_args* a, int nthreads, uint32_t* ids_out,
                   float* weights_out, float* out);

/* ---- portable synthetic inputs (no reference counterpart) ---------------*/
uint64_t k3xo_mix64(uint64_t z);
uint64_t k3xo_stream_key(uint64_t seed, uint64_t stream);
void k3xo_synth_codes(uint64_t key, size_t nbytes, uint8_t* out);
void k3xo_synth_scales(uint64_t key, size_t n, uint32_t lo, uint32_t hi,
                       uint8_t* out);
void k3xo_synth_normal(uint64_t key, size_t n, float sigma, float* out);
void k3xo_synth_normal_bf16(uint64_t key, size_t n, float sigma,
                            uint16_t* out);

/* ---- K3X storage records --------------------------------------------------*/
/* CRC32C (Castagnoli, reflected polynomial 0x82F63B78, register preset and
 * final inversion 0xFFFFFFFF), bit at a time: runtime/src/crc32c.cpp:6-28. */
uint32_t k3xo_crc32c(const uint8_t* data, size_t n);
/* The same value with the byte table of runtime/src/crc32c.cpp:7-28. */
uint32_t k3xo_crc32c_table(const uint8_t* data, size_t n);
/* FNV-1a 64 of a NUL-terminated name: runtime/src/reader.cpp:405-412. */
uint64_t k3xo_fnv1a64(const char* name);

#ifdef __cplusplus
}
#endif
#endif
