/*
 * k3x_oracle.c -- CPU restatement of the K3X routed-expert MoE-layer path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels.  The product
 * never links or calls it.  Compiled with -ffp-contract=off so every float
 * and double operation below rounds exactly where it is written.
 *
 * Reference citations are file:line in the rsb1813/project-k3x tree.
 */
#include "k3x_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bf16                                                                     */
/* ------------------------------------------------------------------------ */

/* Round-to-nearest-even to bf16, kept in a float; NaN stays quiet NaN.
 * Restates runtime/src/official_moe.cpp:18-26. */
float k3xo_round_bf16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if ((bits & 0x7f800000u) == 0x7f800000u) {
        if (bits & 0x007fffffu) bits |= 0x00400000u;
        bits &= 0xffff0000u;
    } else {
        bits += 0x7fffu + ((bits >> 16) & 1u);
        bits &= 0xffff0000u;
    }
    memcpy(&value, &bits, 4);
    return value;
}

uint16_t k3xo_bf16_bits(float value) {
    const float rounded = k3xo_round_bf16(value);
    uint32_t bits;
    memcpy(&bits, &rounded, 4);
    return (uint16_t)(bits >> 16);
}

/* runtime/src/official_moe.cpp:135-137 */
float k3xo_bf16_to_f32(uint16_t word) {
    const uint32_t bits = (uint32_t)word << 16;
    float value;
    memcpy(&value, &bits, 4);
    return value;
}

/* ------------------------------------------------------------------------ */
/* MXFP4                                                                    */
/* ------------------------------------------------------------------------ */

/* E2M1 code -> value, low nibble = even column.  runtime/src/ops.cpp:40-43 */
static const float k_e2m1[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

static int mxfp4_contract_ok(size_t packed_len, size_t scales_len,
                             size_t rows, size_t cols, size_t group) {
    /* runtime/src/ops.cpp:36-39 */
    if (!rows || !cols || !group || cols % group || cols % 2) return 0;
    if (rows > ((size_t)-1) / cols) return 0;
    if (packed_len != rows * cols / 2) return 0;
    if (scales_len != rows * cols / group) return 0;
    return 1;
}

static int scales_ok(const uint8_t* scales, size_t n) {
    /* runtime/src/ops.cpp:46-49: 0xFF (E8M0 NaN) is rejected. */
    for (size_t i = 0; i < n; ++i)
        if (scales[i] == 0xffu) return 0;
    return 1;
}

static void decode_row(const uint8_t* packed, const uint8_t* scales,
                       size_t row, size_t cols, size_t group, float* out) {
    const size_t base = row * cols;
    for (size_t c = 0; c < cols; ++c) {
        const size_t index = base + c;
        const uint8_t pair = packed[index / 2];
        const uint8_t code = (index % 2) ? (uint8_t)(pair >> 4)
                                         : (uint8_t)(pair & 0x0fu);
        const int exponent = (int)scales[index / group] - 127;
        out[c] = ldexpf(k_e2m1[code], exponent);
    }
}

/* runtime/src/ops.cpp:32-55 */
int k3xo_decode_mxfp4(const uint8_t* packed, size_t packed_len,
                      const uint8_t* scales, size_t scales_len, size_t rows,
                      size_t cols, size_t group_size, float* out) {
    if (!mxfp4_contract_ok(packed_len, scales_len, rows, cols, group_size) ||
        !scales_ok(scales, scales_len))
        return K3XO_INVALID_MXFP4;
    for (size_t r = 0; r < rows; ++r)
        decode_row(packed, scales, r, cols, group_size, out + r * cols);
    return K3XO_OK;
}

/* y[r] = float(sum_c double(x[c]) * W[r][c]), sequential in c.
 * runtime/src/ops.cpp:57-76 (decoded row by row instead of materialising
 * the whole matrix; same values, same order, same result). */
int k3xo_mxfp4_matvec(const float* input, size_t input_len,
                      const uint8_t* packed, size_t packed_len,
                      const uint8_t* scales, size_t scales_len, size_t rows,
                      size_t cols, size_t group_size, float* out) {
    if (input_len != cols) return K3XO_INVALID_MXFP4;
    if (!mxfp4_contract_ok(packed_len, scales_len, rows, cols, group_size) ||
        !scales_ok(scales, scales_len))
        return K3XO_INVALID_MXFP4;
    float* row_values = (float*)malloc(cols * sizeof(float));
    if (!row_values) return K3XO_INVALID_MXFP4;
    for (size_t r = 0; r < rows; ++r) {
        decode_row(packed, scales, r, cols, group_size, row_values);
        double sum = 0.0;
        for (size_t c = 0; c < cols; ++c)
            sum += (double)input[c] * (double)row_values[c];
        out[r] = (float)sum;
    }
    free(row_values);
    return K3XO_OK;
}

/* ------------------------------------------------------------------------ */
/* Canonical double reduction shared with the HIP kernels                   */
/* ------------------------------------------------------------------------ */

#define K3XO_CANON_LANES 256

/* Pairwise tree: tree(p, n) = tree(p, n/2) + tree(p + n/2, n/2).  This is
 * what an xor-butterfly over 64 lanes followed by (w0+w1)+(w2+w3) across
 * four waves produces. */
static double tree_sum(const double* p, size_t n) {
    if (n == 1) return p[0];
    return tree_sum(p, n / 2) + tree_sum(p + n / 2, n / 2);
}

/* 256 strided partials (lane i sums elements i, i+256, ... sequentially),
 * then the pairwise tree.  Canonical order; no reference counterpart. */
double k3xo_canon_dot(const float* a, const float* b, size_t n) {
    double partial[K3XO_CANON_LANES];
    for (size_t lane = 0; lane < K3XO_CANON_LANES; ++lane) {
        double sum = 0.0;
        for (size_t k = lane; k < n; k += K3XO_CANON_LANES)
            sum += (double)a[k] * (double)b[k];
        partial[lane] = sum;
    }
    return tree_sum(partial, K3XO_CANON_LANES);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm and GLU                                                          */
/* ------------------------------------------------------------------------ */

static void rms_scale(float* out, const float* in, const float* weight,
                      size_t n, float epsilon, double squares) {
    /* runtime/src/ops.cpp:14-17 */
    const float inverse =
        1.0f / sqrtf((float)(squares / (double)n) + epsilon);
    for (size_t i = 0; i < n; ++i) out[i] = in[i] * inverse * weight[i];
}

/* runtime/src/ops.cpp:10-18 (sequential double sum of squares). */
void k3xo_rms_norm(float* out, const float* in, const float* weight, size_t n,
                   float epsilon) {
    double squares = 0.0;
    for (size_t i = 0; i < n; ++i) squares += (double)in[i] * in[i];
    rms_scale(out, in, weight, n, epsilon, squares);
}

/* Same as k3xo_rms_norm with the canonical order for the sum of squares. */
void k3xo_rms_norm_canon(float* out, const float* in, const float* weight,
                         size_t n, float epsilon) {
    rms_scale(out, in, weight, n, epsilon, k3xo_canon_dot(in, in, n));
}

/* SiTU-GLU: runtime/src/ops.cpp:20-30.
 * SwiGLU:   silu(g)*u, silu(v) = v * sigmoid(v): runtime/src/model.cpp:60-61. */
void k3xo_glu(float* out, const float* gate, const float* up, size_t n,
              int kind, float beta, int has_linear, float linear_beta) {
    for (size_t i = 0; i < n; ++i) {
        const float g = gate[i];
        const float sigmoid = 1.0f / (1.0f + expf(-g));
        if (kind == K3XO_GLU_SITU) {
            const float bounded_gate = beta * tanhf(g / beta) * sigmoid;
            const float bounded_up =
                has_linear ? linear_beta * tanhf(up[i] / linear_beta) : up[i];
            out[i] = bounded_gate * bounded_up;
        } else {
            out[i] = (g * sigmoid) * up[i];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Router                                                                   */
/* ------------------------------------------------------------------------ */

/* Correctly rounded expf evaluated in double: x = k*ln2 + r, Taylor series
 * of degree 13 on |r| <= ln2/2 (truncation < 5e-18), one rounding to float.
 * The HIP router evaluates the identical operation sequence. */
float k3xo_expf_cr(float x) {
    if (x != x) return x;
    if (x > 100.0f) return INFINITY;
    if (x < -110.0f) return 0.0f;
    const double xd = (double)x;
    const double k = rint(xd * 1.4426950408889634);
    double r = fma(-k, 6.93147180369123816490e-01, xd);
    r = fma(-k, 1.90821492927058770002e-10, r);
    double p = 1.6059043836821614599e-10;          /* 1/13! */
    p = fma(p, r, 2.0876756987868098979e-09);       /* 1/12! */
    p = fma(p, r, 2.5052108385441718775e-08);       /* 1/11! */
    p = fma(p, r, 2.7557319223985890653e-07);       /* 1/10! */
    p = fma(p, r, 2.7557319223985890653e-06);       /* 1/9!  */
    p = fma(p, r, 2.4801587301587301587e-05);       /* 1/8!  */
    p = fma(p, r, 1.9841269841269841270e-04);       /* 1/7!  */
    p = fma(p, r, 1.3888888888888888889e-03);       /* 1/6!  */
    p = fma(p, r, 8.3333333333333333333e-03);       /* 1/5!  */
    p = fma(p, r, 4.1666666666666666667e-02);       /* 1/4!  */
    p = fma(p, r, 1.6666666666666666667e-01);       /* 1/3!  */
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    return (float)ldexp(p, (int)k);
}

/* sigmoid(v) = 1 / (1 + exp(-v)) in float.  runtime/src/model.cpp:60,
 * runtime/src/official_moe.cpp:221. */
float k3xo_sigmoid(float x, int mode) {
    const float e = mode == K3XO_SIGMOID_CR ? k3xo_expf_cr(-x) : expf(-x);
    return 1.0f / (1.0f + e);
}

/* logits[e] = float(sum_h double(W[e][h]) * x[h]).
 * SEQ:   runtime/src/backend_cpu.cpp:33-41 (dense_matvec, fp32 router W,
 *        called from runtime/src/model.cpp:919-921).
 * CANON: the order of the HIP router kernel. */
void k3xo_router_logits(const float* weight, const float* x, size_t experts,
                        size_t hidden, int order, float* logits) {
    for (size_t e = 0; e < experts; ++e) {
        const float* row = weight + e * hidden;
        double sum;
        if (order == K3XO_ORDER_CANON) {
            sum = k3xo_canon_dot(row, x, hidden);
        } else {
            sum = 0.0;
            for (size_t h = 0; h < hidden; ++h)
                sum += (double)row[h] * (double)x[h];
        }
        logits[e] = (float)sum;
    }
}

static int finitef(float v) { return isfinite(v) != 0; }

/* Bias-adjusted natural Top-K over given scores (ties -> lower expert
 * index), renormalised contributions times routed_scale.
 * Selection: runtime/src/routing_policy.cpp:76-87 (stable_sort descending),
 *            runtime/src/official_moe.cpp:224-233 (explicit tie comparator).
 * FLOAT renorm + validation: runtime/src/routing_policy.cpp:40-50,76-80,
 *            89-95,146-157; routed_scale: runtime/src/model.cpp:1004-1009.
 * DOUBLE renorm: runtime/src/official_moe.cpp:234-242 (its finiteness
 *            checks on logits and bias are made by k3xo_route). */
int k3xo_select(const float* scores, const float* bias, size_t experts,
                size_t top_k, int renorm, float routed_scale, uint32_t* ids,
                float* weights) {
    const int dims_error =
        renorm == K3XO_RENORM_DOUBLE ? K3XO_INVALID_EXTENT : K3XO_INVALID_STATE;
    if (!experts || !top_k || top_k > experts) return dims_error;
    float* adjusted = (float*)malloc(experts * sizeof(float));
    unsigned char* taken = (unsigned char*)calloc(experts, 1);
    int status = K3XO_OK;
    if (!adjusted || !taken) {
        status = dims_error;
        goto done;
    }
    for (size_t e = 0; e < experts; ++e) {
        if (renorm == K3XO_RENORM_FLOAT &&
            (!finitef(scores[e]) || scores[e] < 0.0f || scores[e] > 1.0f ||
             !finitef(bias[e]))) {
            status = K3XO_INVALID_STATE;
            goto done;
        }
    }
    for (size_t e = 0; e < experts; ++e) {
        adjusted[e] = scores[e] + bias[e];
        if (renorm == K3XO_RENORM_FLOAT && !finitef(adjusted[e])) {
            status = K3XO_INVALID_STATE;
            goto done;
        }
    }
    /* Repeated arg-max with strict '>' keeps the lowest index among equal
     * adjusted scores, which is the order a stable descending sort gives. */
    for (size_t slot = 0; slot < top_k; ++slot) {
        size_t best = experts;
        for (size_t e = 0; e < experts; ++e) {
            if (taken[e]) continue;
            if (best == experts || adjusted[e] > adjusted[best]) best = e;
        }
        taken[best] = 1;
        ids[slot] = (uint32_t)best;
    }
    if (renorm == K3XO_RENORM_DOUBLE) {
        double total = 0.0;
        for (size_t slot = 0; slot < top_k; ++slot) total += scores[ids[slot]];
        if (!isfinite(total) || total <= 0.0) {
            status = K3XO_INVALID_EXTENT;
            goto done;
        }
        for (size_t slot = 0; slot < top_k; ++slot)
            weights[slot] =
                (float)((double)scores[ids[slot]] / total) * routed_scale;
    } else {
        float denominator = 0.0f;
        for (size_t slot = 0; slot < top_k; ++slot)
            denominator += scores[ids[slot]];
        if (!finitef(denominator) || denominator <= 0.0f) {
            status = K3XO_INVALID_STATE;
            goto done;
        }
        for (size_t slot = 0; slot < top_k; ++slot)
            weights[slot] = (scores[ids[slot]] / denominator) * routed_scale;
    }
done:
    free(adjusted);
    free(taken);
    return status;
}

/* Sigmoid scores of the logits, then k3xo_select.  Scores:
 * runtime/src/model.cpp:923-925 (FLOAT convention, the synthetic path) and
 * runtime/src/official_moe.cpp:214-223 (DOUBLE convention, which first
 * rejects non-finite logits or bias with invalid_extent). */
int k3xo_route(const float* logits, const float* bias, size_t experts,
               size_t top_k, int renorm, float routed_scale, int sigmoid_mode,
               uint32_t* ids, float* weights, float* scores) {
    if (renorm == K3XO_RENORM_DOUBLE) {
        if (!experts || !top_k || top_k > experts) return K3XO_INVALID_EXTENT;
        for (size_t e = 0; e < experts; ++e)
            if (!finitef(logits[e]) || !finitef(bias[e])) return K3XO_INVALID_EXTENT;
    }
    for (size_t e = 0; e < experts; ++e)
        scores[e] = k3xo_sigmoid(logits[e], sigmoid_mode);
    return k3xo_select(scores, bias, experts, top_k, renorm, routed_scale, ids,
                       weights);
}

/* ------------------------------------------------------------------------ */
/* Expert-major grouping                                                    */
/* ------------------------------------------------------------------------ */

/* Groups in first-use order (scan tokens, then router slots); assignments
 * inside a group in (token, slot) order.  runtime/src/expert_major.cpp:10-54.
 * Routes have a fixed length top_k here (natural Top-K). */
int k3xo_expert_major_plan(const uint32_t* ids, const float* contributions,
                           size_t tokens, size_t top_k, size_t* n_groups,
                           uint32_t* group_expert, uint32_t* group_start,
                           uint32_t* assign_token, uint32_t* assign_slot,
                           float* assign_contribution) {
    if (!tokens || !top_k) return K3XO_INVALID_EXTENT;
    const size_t pairs = tokens * top_k;
    for (size_t t = 0; t < tokens; ++t) {
        for (size_t s = 0; s < top_k; ++s) {
            if (!finitef(contributions[t * top_k + s])) return K3XO_INVALID_STATE;
            for (size_t q = 0; q < s; ++q)
                if (ids[t * top_k + q] == ids[t * top_k + s])
                    return K3XO_INVALID_STATE;
        }
    }
    /* First-use group order. */
    size_t groups = 0;
    uint32_t* group_of_pair = (uint32_t*)malloc(pairs * sizeof(uint32_t));
    uint32_t* sizes = (uint32_t*)calloc(pairs, sizeof(uint32_t));
    if (!group_of_pair || !sizes) {
        free(group_of_pair);
        free(sizes);
        return K3XO_INVALID_EXTENT;
    }
    for (size_t p = 0; p < pairs; ++p) {
        size_t g = 0;
        while (g < groups && group_expert[g] != ids[p]) ++g;
        if (g == groups) group_expert[groups++] = ids[p];
        group_of_pair[p] = (uint32_t)g;
        ++sizes[g];
    }
    group_start[0] = 0;
    for (size_t g = 0; g < groups; ++g) group_start[g + 1] = group_start[g] + sizes[g];
    memset(sizes, 0, pairs * sizeof(uint32_t));
    for (size_t p = 0; p < pairs; ++p) {
        const uint32_t g = group_of_pair[p];
        const uint32_t at = group_start[g] + sizes[g]++;
        assign_token[at] = (uint32_t)(p / top_k);
        assign_slot[at] = (uint32_t)(p % top_k);
        assign_contribution[at] = contributions[p];
    }
    *n_groups = groups;
    free(group_of_pair);
    free(sizes);
    return K3XO_OK;
}

/* The ascending-expert CSR form of the same grouping, plus each expert's
 * first-use key min(token*top_k + slot); sorting active experts by that key
 * reproduces the group order of k3xo_expert_major_plan.  Rejects what the
 * plan rejects about ids: out of range, or one expert twice in one token
 * (runtime/src/expert_major.cpp:30-35). */
int k3xo_expert_major_csr(const uint32_t* ids, size_t tokens, size_t top_k,
                          size_t experts, uint32_t* counts, uint32_t* offsets,
                          uint32_t* pair_token, uint32_t* pair_slot,
                          uint32_t* first_use, uint32_t* n_active,
                          uint32_t* active_ascending,
                          uint32_t* active_first_use) {
    if (!tokens || !top_k || !experts) return K3XO_INVALID_EXTENT;
    const size_t pairs = tokens * top_k;
    memset(counts, 0, experts * sizeof(uint32_t));
    for (size_t e = 0; e < experts; ++e) first_use[e] = 0xffffffffu;
    for (size_t p = 0; p < pairs; ++p) {
        if (ids[p] >= experts) return K3XO_INVALID_STATE;
        for (size_t q = p - p % top_k; q < p; ++q)
            if (ids[q] == ids[p]) return K3XO_INVALID_STATE;
    }
    for (size_t p = 0; p < pairs; ++p) {
        ++counts[ids[p]];
        if (first_use[ids[p]] == 0xffffffffu) first_use[ids[p]] = (uint32_t)p;
    }
    offsets[0] = 0;
    uint32_t active = 0;
    for (size_t e = 0; e < experts; ++e) {
        offsets[e + 1] = offsets[e] + counts[e];
        if (counts[e]) active_ascending[active++] = (uint32_t)e;
    }
    uint32_t* fill = (uint32_t*)calloc(experts, sizeof(uint32_t));
    if (!fill) return K3XO_INVALID_EXTENT;
    for (size_t p = 0; p < pairs; ++p) {
        const uint32_t e = ids[p];
        const uint32_t at = offsets[e] + fill[e]++;
        pair_token[at] = (uint32_t)(p / top_k);
        pair_slot[at] = (uint32_t)(p % top_k);
    }
    free(fill);
    /* Insertion sort of the active experts by first-use key. */
    for (uint32_t i = 0; i < active; ++i) active_first_use[i] = active_ascending[i];
    for (uint32_t i = 1; i < active; ++i) {
        const uint32_t v = active_first_use[i];
        uint32_t j = i;
        while (j > 0 && first_use[active_first_use[j - 1]] > first_use[v]) {
            active_first_use[j] = active_first_use[j - 1];
            --j;
        }
        active_first_use[j] = v;
    }
    *n_active = active;
    return K3XO_OK;
}

/* ------------------------------------------------------------------------ */
/* Expert FFN, shared expert, ordered mix                                   */
/* ------------------------------------------------------------------------ */

/* gate/up GEMV -> GLU -> (optional bf16 rounding of the activation) -> down.
 * runtime/src/backend_cpu.cpp:124-154 (mxfp4_situ_mlp_group, one expert);
 * runtime/src/official_moe.cpp:82-103 for the same composition.  act_out,
 * when non-NULL, receives the activation fed to the down projection. */
int k3xo_expert_ffn(const float* x, size_t hidden, size_t inter,
                    const uint8_t* gate_packed, const uint8_t* gate_scales,
                    const uint8_t* up_packed, const uint8_t* up_scales,
                    const uint8_t* down_packed, const uint8_t* down_scales,
                    int glu, float beta, int has_linear, float linear_beta,
                    int round_act, float* act_out, float* out) {
    const size_t gate_len = inter * hidden / 2, gate_scale_len = inter * hidden / 32;
    float* gate = (float*)malloc(inter * sizeof(float));
    float* up = (float*)malloc(inter * sizeof(float));
    float* act = (float*)malloc(inter * sizeof(float));
    int status = K3XO_INVALID_MXFP4;
    if (!gate || !up || !act) goto done;
    status = k3xo_mxfp4_matvec(x, hidden, gate_packed, gate_len, gate_scales,
                               gate_scale_len, inter, hidden, 32, gate);
    if (status) goto done;
    status = k3xo_mxfp4_matvec(x, hidden, up_packed, gate_len, up_scales,
                               gate_scale_len, inter, hidden, 32, up);
    if (status) goto done;
    k3xo_glu(act, gate, up, inter, glu, beta, has_linear, linear_beta);
    if (round_act)
        for (size_t i = 0; i < inter; ++i) act[i] = k3xo_round_bf16(act[i]);
    if (act_out) memcpy(act_out, act, inter * sizeof(float));
    status = k3xo_mxfp4_matvec(act, inter, down_packed, hidden * inter / 2,
                               down_scales, hidden * inter / 32, hidden, inter,
                               32, out);
done:
    free(gate);
    free(up);
    free(act);
    return status;
}

/* Double-accumulated bf16-weight GEMV without output rounding.
 * runtime/src/official_moe.cpp:39-59 minus the final round_bf16 (the
 * layer here keeps the shared projections in fp32). */
void k3xo_bf16_matvec(const float* x, const uint16_t* weight, size_t rows,
                      size_t cols, float* out) {
    for (size_t r = 0; r < rows; ++r) {
        double sum = 0.0;
        const uint16_t* row = weight + r * cols;
        for (size_t c = 0; c < cols; ++c)
            sum += (double)k3xo_bf16_to_f32(row[c]) * (double)x[c];
        out[r] = (float)sum;
    }
}

/* Shared expert: runtime/src/official_moe.cpp:105-117 (bf16 weights) with
 * the activation optionally rounded to bf16 before the down projection. */
void k3xo_shared_ffn(const float* x, size_t hidden, size_t inter,
                     const uint16_t* gate, const uint16_t* up,
                     const uint16_t* down, int glu, float beta, int has_linear,
                     float linear_beta, int round_act, float* out) {
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* a = (float*)malloc(inter * sizeof(float));
    if (!g || !u || !a) goto done;
    k3xo_bf16_matvec(x, gate, inter, hidden, g);
    k3xo_bf16_matvec(x, up, inter, hidden, u);
    k3xo_glu(a, g, u, inter, glu, beta, has_linear, linear_beta);
    if (round_act)
        for (size_t i = 0; i < inter; ++i) a[i] = k3xo_round_bf16(a[i]);
    k3xo_bf16_matvec(a, down, hidden, inter, out);
done:
    free(g);
    free(u);
    free(a);
}

/* mixed[h] = sum over slots in router order of w[slot] * y[slot][h], float,
 * starting from 0.  runtime/src/backend_cpu.cpp:295-301, model.cpp:1127-1138. */
void k3xo_ordered_mix(const float* expert_out, const float* weights,
                      size_t top_k, size_t width, float* mixed) {
    for (size_t h = 0; h < width; ++h) mixed[h] = 0.0f;
    for (size_t slot = 0; slot < top_k; ++slot)
        for (size_t h = 0; h < width; ++h)
            mixed[h] += weights[slot] * expert_out[slot * width + h];
}

/* ------------------------------------------------------------------------ */
/* fp32 backend operations and the resident latent layer:                   */
/* runtime/src/backend_cpu.cpp                                              */
/* ------------------------------------------------------------------------ */

/* backend_cpu.cpp:22-45 (dense_matvec): double sum in column order of
 * double(weight) * input, one rounding to float. */
void k3xo_dense_matvec(const float* x, const float* weight, size_t rows,
                       size_t cols, float* out) {
    for (size_t r = 0; r < rows; ++r) {
        double sum = 0.0;
        const float* row = weight + r * cols;
        for (size_t c = 0; c < cols; ++c) sum += (double)row[c] * x[c];
        out[r] = (float)sum;
    }
}

/* backend_cpu.cpp:108-122 (dense_situ_mlp): gate and up dense_matvec, SiTU
 * (runtime/src/ops.cpp:20-30), down dense_matvec. */
void k3xo_dense_situ_mlp(const float* x, size_t hidden, size_t inter,
                         size_t out_rows, const float* gate, const float* up,
                         const float* down, float beta, int has_linear,
                         float linear_beta, float* act, float* out) {
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* a = (float*)malloc(inter * sizeof(float));
    if (g && u && a) {
        k3xo_dense_matvec(x, gate, inter, hidden, g);
        k3xo_dense_matvec(x, up, inter, hidden, u);
        k3xo_glu(a, g, u, inter, K3XO_GLU_SITU, beta, has_linear, linear_beta);
        if (act) memcpy(act, a, inter * sizeof(float));
        k3xo_dense_matvec(a, down, out_rows, inter, out);
    }
    free(g);
    free(u);
    free(a);
}

/* backend_cpu.cpp:305-339 (resident_mxfp4_moe_layer, executed path):
 * latent = routed_down . input; each expert on the latent
 * (mxfp4_situ_mlp_group, :124-154); mixed[row] += contribution * output in
 * slot order from 0; rms_norm (runtime/src/ops.cpp:10-18) with routed_norm;
 * routed = routed_up . normalized; out = routed + dense_situ_mlp(input). */
int k3xo_resident_layer(const float* input, size_t hidden, size_t latent,
                        size_t inter, size_t shared_inter,
                        const float* routed_down, const float* routed_norm,
                        const float* routed_up, const float* shared_gate,
                        const float* shared_up, const float* shared_down,
                        const uint8_t* const* experts, const float* contributions,
                        size_t n_experts, float epsilon, float beta,
                        int has_linear, float linear_beta, float* mixed_out,
                        float* out) {
    int status = K3XO_INVALID_MXFP4;
    float* lat = (float*)malloc(latent * sizeof(float));
    float* y = (float*)malloc(n_experts * latent * sizeof(float));
    float* mixed = (float*)malloc(latent * sizeof(float));
    float* normed = (float*)malloc(latent * sizeof(float));
    float* routed = (float*)malloc(hidden * sizeof(float));
    float* shared = (float*)malloc(hidden * sizeof(float));
    if (!lat || !y || !mixed || !normed || !routed || !shared) goto done;
    k3xo_dense_matvec(input, routed_down, latent, hidden, lat);
    for (size_t k = 0; k < n_experts; ++k) {
        const uint8_t* const* e = experts + 6 * k;
        status = k3xo_expert_ffn(lat, latent, inter, e[0], e[1], e[2], e[3], e[4], e[5],
                                 K3XO_GLU_SITU, beta, has_linear, linear_beta, 0, NULL,
                                 y + k * latent);
        if (status) goto done;
    }
    k3xo_ordered_mix(y, contributions, n_experts, latent, mixed);
    if (mixed_out) memcpy(mixed_out, mixed, latent * sizeof(float));
    k3xo_rms_norm(normed, mixed, routed_norm, latent, epsilon);
    k3xo_dense_matvec(normed, routed_up, hidden, latent, routed);
    k3xo_dense_situ_mlp(input, hidden, shared_inter, hidden, shared_gate, shared_up,
                        shared_down, beta, has_linear, linear_beta, NULL, shared);
    for (size_t h = 0; h < hidden; ++h) out[h] = routed[h] + shared[h];
    status = K3XO_OK;
done:
    free(lat);
    free(y);
    free(mixed);
    free(normed);
    free(routed);
    free(shared);
    return status;
}

/* ------------------------------------------------------------------------ */
/* Official K3 MoE FFN (Stable LatentMoE): runtime/src/official_moe.cpp     */
/* ------------------------------------------------------------------------ */

/* bf16 GEMV, double accumulation in column order, bf16-rounded output.
 * runtime/src/official_moe.cpp:39-59. */
void k3xo_bf16_matvec_rounded(const float* x, const uint16_t* weight,
                              size_t rows, size_t cols, float* out) {
    k3xo_bf16_matvec(x, weight, rows, cols, out);
    for (size_t r = 0; r < rows; ++r) out[r] = k3xo_round_bf16(out[r]);
}

/* RMSNorm with a bf16 weight and bf16-rounded output, sequential double
 * sum of squares.  runtime/src/official_moe.cpp:61-80. */
void k3xo_official_norm(const float* in, const uint16_t* weight, size_t n,
                        float epsilon, float* out) {
    double squares = 0.0;
    for (size_t i = 0; i < n; ++i) squares += (double)in[i] * in[i];
    const float inverse = 1.0f / sqrtf((float)(squares / (double)n) + epsilon);
    for (size_t i = 0; i < n; ++i)
        out[i] = k3xo_round_bf16(in[i] * inverse * k3xo_bf16_to_f32(weight[i]));
}

/* Two-source attention-residual mix and post-norm feeding the router:
 * sources (block residual, prefix sum) rounded to bf16, one softmax score
 * each (normalised source . residual_norm . residual_proj, double), the
 * bf16-rounded mix, then the post-norm.  runtime/src/official_moe.cpp:156-209. */
int k3xo_official_prepare(const float* prefix, const float* block_residual,
                          size_t width, const uint16_t* residual_norm,
                          const uint16_t* residual_proj,
                          const uint16_t* post_norm, float epsilon,
                          float* hidden) {
    if (!width || !(epsilon > 0.0f)) return K3XO_INVALID_EXTENT;
    float* v0 = (float*)malloc(width * sizeof(float));
    float* v1 = (float*)malloc(width * sizeof(float));
    float* mix = (float*)malloc(width * sizeof(float));
    int status = K3XO_INVALID_EXTENT;
    if (!v0 || !v1 || !mix) goto done;
    for (size_t i = 0; i < width; ++i) {
        v0[i] = k3xo_round_bf16(block_residual[i]);
        v1[i] = k3xo_round_bf16(prefix[i]);
    }
    float score[2];
    for (int row = 0; row < 2; ++row) {
        const float* v = row ? v1 : v0;
        double squares = 0.0;
        for (size_t i = 0; i < width; ++i) squares += (double)v[i] * v[i];
        const float inverse =
            1.0f / sqrtf((float)(squares / (double)width) + epsilon);
        double sc = 0.0;
        for (size_t i = 0; i < width; ++i)
            sc += (double)(v[i] * inverse) * (double)k3xo_bf16_to_f32(residual_norm[i]) *
                  (double)k3xo_bf16_to_f32(residual_proj[i]);
        score[row] = (float)sc;
    }
    const float maximum = score[0] > score[1] ? score[0] : score[1];
    float p0 = expf(score[0] - maximum), p1 = expf(score[1] - maximum);
    const float denominator = p0 + p1;
    p0 /= denominator;
    p1 /= denominator;
    for (size_t i = 0; i < width; ++i) mix[i] = k3xo_round_bf16(p0 * v0[i] + p1 * v1[i]);
    k3xo_official_norm(mix, post_norm, width, epsilon, hidden);
    status = K3XO_OK;
done:
    free(v0);
    free(v1);
    free(mix);
    return status;
}

/* Shared FFN with bf16-rounded gate, up and down outputs.
 * runtime/src/official_moe.cpp:105-117. */
void k3xo_official_shared(const float* x, size_t hidden, size_t inter,
                          const uint16_t* gate, const uint16_t* up,
                          const uint16_t* down, int glu, float beta,
                          int has_linear, float linear_beta, float* out) {
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* a = (float*)malloc(inter * sizeof(float));
    if (g && u && a) {
        k3xo_bf16_matvec_rounded(x, gate, inter, hidden, g);
        k3xo_bf16_matvec_rounded(x, up, inter, hidden, u);
        k3xo_glu(a, g, u, inter, glu, beta, has_linear, linear_beta);
        k3xo_bf16_matvec_rounded(a, down, hidden, inter, out);
    }
    free(g);
    free(u);
    free(a);
}

/* One token of the official FFN around experts of hidden `latent`:
 * latent = bf16(routed_down . hidden); expert outputs bf16-rounded; mixed =
 * bf16(sum over slots in route order of c * y); routed = bf16(routed_up .
 * norm(mixed)); out = bf16(bf16(prefix) + bf16(routed + shared)).
 * runtime/src/official_moe.cpp:271-344 (official_moe_cpu) with :82-103
 * (expert_ffn). */
int k3xo_official_ffn(const float* hidden, const float* prefix, size_t width,
                      size_t latent, size_t inter, size_t shared_inter,
                      const uint16_t* routed_down, const uint16_t* routed_norm,
                      const uint16_t* routed_up, const uint16_t* shared_gate,
                      const uint16_t* shared_up, const uint16_t* shared_down,
                      const uint8_t* const* experts, const float* contributions,
                      size_t top_k, float epsilon, int glu, float beta,
                      int has_linear, float linear_beta, float* latent_out,
                      float* expert_out, float* mixed_out, float* routed_out,
                      float* shared_out, float* out) {
    float* lat = (float*)malloc(latent * sizeof(float));
    float* y = (float*)malloc(top_k * latent * sizeof(float));
    float* mixed = (float*)malloc(latent * sizeof(float));
    float* normed = (float*)malloc(latent * sizeof(float));
    float* routed = (float*)malloc(width * sizeof(float));
    float* shared = (float*)calloc(width, sizeof(float));
    int status = K3XO_INVALID_MXFP4;
    if (!lat || !y || !mixed || !normed || !routed || !shared) goto done;
    k3xo_bf16_matvec_rounded(hidden, routed_down, latent, width, lat);
    if (shared_inter)
        k3xo_official_shared(hidden, width, shared_inter, shared_gate, shared_up,
                             shared_down, glu, beta, has_linear, linear_beta, shared);
    for (size_t slot = 0; slot < top_k; ++slot) {
        const uint8_t* const* e = experts + 6 * slot;
        status = k3xo_expert_ffn(lat, latent, inter, e[0], e[1], e[2], e[3], e[4],
                                 e[5], glu, beta, has_linear, linear_beta, 0, NULL,
                                 y + slot * latent);
        if (status) goto done;
        for (size_t i = 0; i < latent; ++i)
            y[slot * latent + i] = k3xo_round_bf16(y[slot * latent + i]);
    }
    k3xo_ordered_mix(y, contributions, top_k, latent, mixed);
    for (size_t i = 0; i < latent; ++i) mixed[i] = k3xo_round_bf16(mixed[i]);
    k3xo_official_norm(mixed, routed_norm, latent, epsilon, normed);
    k3xo_bf16_matvec_rounded(normed, routed_up, width, latent, routed);
    for (size_t i = 0; i < width; ++i) {
        const float combined = k3xo_round_bf16(routed[i] + shared[i]);
        out[i] = k3xo_round_bf16(k3xo_round_bf16(prefix[i]) + combined);
    }
    if (latent_out) memcpy(latent_out, lat, latent * sizeof(float));
    if (expert_out) memcpy(expert_out, y, top_k * latent * sizeof(float));
    if (mixed_out) memcpy(mixed_out, mixed, latent * sizeof(float));
    if (routed_out) memcpy(routed_out, routed, width * sizeof(float));
    if (shared_out) memcpy(shared_out, shared, width * sizeof(float));
    status = K3XO_OK;
done:
    free(lat);
    free(y);
    free(mixed);
    free(normed);
    free(routed);
    free(shared);
    return status;
}

/* ------------------------------------------------------------------------ */
/* Portable synthetic inputs (no reference counterpart)                     */
/* ------------------------------------------------------------------------ */

/* SplitMix64 output function (Steele, Lea & Flood, OOPSLA 2014). */
uint64_t k3xo_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

#define K3XO_GAMMA 0x9e3779b97f4a7c15ull

uint64_t k3xo_stream_key(uint64_t seed, uint64_t stream) {
    return k3xo_mix64(seed + K3XO_GAMMA * (stream + 1));
}

static uint64_t word_at(uint64_t key, uint64_t index) {
    return k3xo_mix64(key + K3XO_GAMMA * (index + 1));
}

/* Packed E2M1 bytes: byte p is byte (p % 8) of word p / 8, so both nibbles
 * are uniform over the 16 codes. */
void k3xo_synth_codes(uint64_t key, size_t nbytes, uint8_t* out) {
    for (size_t p = 0; p < nbytes; p += 8) {
        const uint64_t w = word_at(key, p >> 3);  /* byte p + b is byte b of word p / 8 */
        for (size_t b = 0; b < 8 && p + b < nbytes; ++b) out[p + b] = (uint8_t)(w >> (8 * b));
    }
}

/* E8M0 scale bytes uniform over [lo, hi]. */
void k3xo_synth_scales(uint64_t key, size_t n, uint32_t lo, uint32_t hi,
                       uint8_t* out) {
    const uint64_t span = (uint64_t)(hi - lo + 1);
    for (size_t i = 0; i < n; ++i)
        out[i] = (uint8_t)(lo + (uint32_t)(word_at(key, i) % span));
}

/* Irwin-Hall(12) approximation of N(0, sigma^2): twelve 16-bit uniforms from
 * three words, summed as integers; every float step is exact except the
 * final multiply by sigma. */
static float normal_at(uint64_t key, size_t i, float sigma) {
    int32_t sum = 0;
    for (int j = 0; j < 3; ++j) {
        const uint64_t w = word_at(key, 3 * (uint64_t)i + (uint64_t)j);
        for (int q = 0; q < 4; ++q) sum += (int32_t)((w >> (16 * q)) & 0xffffu);
    }
    return ((float)(sum - 393216) * 0x1p-16f) * sigma;
}

void k3xo_synth_normal(uint64_t key, size_t n, float sigma, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = normal_at(key, i, sigma);
}

void k3xo_synth_normal_bf16(uint64_t key, size_t n, float sigma,
                            uint16_t* out) {
    for (size_t i = 0; i < n; ++i) out[i] = k3xo_bf16_bits(normal_at(key, i, sigma));
}

/* ---- K3X storage records ------------------------------------------------- */
/* runtime/src/crc32c.cpp:6-28 computes a byte table from the reflected
 * Castagnoli polynomial and folds each byte; this restatement shifts one bit
 * at a time (the definition the table tabulates). */
uint32_t k3xo_crc32c(const uint8_t* data, size_t n) {
    uint32_t crc = 0xffffffffu;
    for (size_t i = 0; i < n; ++i) {
        crc ^= data[i];
        for (int b = 0; b < 8; ++b) crc = (crc >> 1) ^ (0x82f63b78u & (0u - (crc & 1u)));
    }
    return ~crc;
}

/* The same value by the reference's own method, one 256-entry byte table
 * built from the reflected polynomial and one lookup per byte
 * (runtime/src/crc32c.cpp:7-28); the bench times it as the CPU baseline of
 * the device CRC32C. */
uint32_t k3xo_crc32c_table(const uint8_t* data, size_t n) {
    static uint32_t table[256];
    static int ready;
    if (!ready) {
        for (uint32_t v = 0; v < 256; ++v) {
            uint32_t c = v;
            for (int b = 0; b < 8; ++b) c = (c >> 1) ^ (0x82f63b78u & (0u - (c & 1u)));
            table[v] = c;
        }
        ready = 1;
    }
    uint32_t crc = 0xffffffffu;
    for (size_t i = 0; i < n; ++i) crc = table[(crc ^ data[i]) & 0xffu] ^ (crc >> 8);
    return ~crc;
}

/* runtime/src/reader.cpp:405-412. */
uint64_t k3xo_fnv1a64(const char* name) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (; *name; ++name) {
        h ^= (unsigned char)*name;
        h *= 0x100000001b3ull;
    }
    return h;
}

/* ---- the whole layer, threaded (the CPU baseline of the benchmark) ------- */
/* One layer over T tokens as the reference CPU backend composes it, token by
 * token: rms_norm (runtime/src/ops.cpp:10-18), the router's double-sum
 * logits and libm sigmoid + bias Top-K (runtime/src/model.cpp:917-1010,
 * runtime/src/routing_policy.cpp:31-160), one expert FFN per (token, slot)
 * pair (decode to fp32, double GEMVs, GLU: runtime/src/backend_cpu.cpp:
 * 124-189, runtime/src/ops.cpp:57-76), the slot-ordered mix
 * (backend_cpu.cpp:295-301) and the shared expert (bf16 weights, double
 * sums).  The reference runs this on one thread; here the tokens and the
 * pairs are spread over `nthreads` POSIX threads that take work items from a
 * shared counter, so every item computes exactly what the one-thread run
 * computes. */
#include <pthread.h>
#include <stdatomic.h>

typedef struct {
    const k3xo_layer_args* a;
    int phase;                 /* 0 route, 1 pairs, 2 mix + shared */
    atomic_size_t next;
    atomic_int status;
    float* xn;                 /* [T][H] */
    uint32_t* ids;             /* [T][K] */
    float* w;                  /* [T][K] */
    float* y;                  /* [T][K][H] */
    float* out;                /* [T][H] */
} layer_job;

static void layer_item(layer_job* j, size_t i) {
    const k3xo_layer_args* a = j->a;
    const size_t H = a->hidden, K = a->top_k, E = a->experts;
    int st = K3XO_OK;
    if (j->phase == 0) {
        float* xn = j->xn + i * H;
        float* logits = (float*)malloc(E * sizeof(float));
        float* scores = (float*)malloc(E * sizeof(float));
        if (!logits || !scores) {
            st = K3XO_INVALID_STATE;
        } else {
            k3xo_rms_norm(xn, a->x + i * H, a->gamma, H, a->epsilon);
            k3xo_router_logits(a->router, xn, E, H, K3XO_ORDER_SEQ, logits);
            st = k3xo_route(logits, a->bias, E, K, a->renorm, a->routed_scale, K3XO_SIGMOID_REF,
                            j->ids + i * K, j->w + i * K, scores);
        }
        free(logits);
        free(scores);
    } else if (j->phase == 1) {
        const size_t t = i / K;
        const uint32_t e = j->ids[i];
        const uint8_t* const* ex = a->expert_bytes + (size_t)e * 6;
        if (e >= E || !ex[0])
            st = K3XO_INVALID_STATE;
        else
            st = k3xo_expert_ffn(j->xn + t * H, H, a->inter, ex[0], ex[1], ex[2], ex[3], ex[4],
                                 ex[5], a->glu, a->beta, a->has_linear, a->linear_beta,
                                 a->round_act, NULL, j->y + i * H);
    } else {
        float* o = j->out + i * H;
        k3xo_ordered_mix(j->y + i * K * H, j->w + i * K, K, H, o);
        if (a->shared_inter) {
            float* s = (float*)malloc(H * sizeof(float));
            if (!s) {
                st = K3XO_INVALID_STATE;
            } else {
                k3xo_shared_ffn(j->xn + i * H, H, a->shared_inter, a->shared_gate, a->shared_up,
                                a->shared_down, a->glu, a->beta, a->has_linear, a->linear_beta,
                                a->round_act, s);
                for (size_t h = 0; h < H; ++h) o[h] += s[h];
                free(s);
            }
        }
    }
    if (st) {
        int zero = 0;
        atomic_compare_exchange_strong(&j->status, &zero, st);
    }
}

static void* layer_worker(void* p) {
    layer_job* j = (layer_job*)p;
    const size_t n = j->phase == 1 ? j->a->tokens * j->a->top_k : j->a->tokens;
    for (;;) {
        const size_t i = atomic_fetch_add(&j->next, 1);
        if (i >= n || atomic_load(&j->status)) break;
        layer_item(j, i);
    }
    return NULL;
}

int k3xo_moe_layer(const k3xo_layer_args* a, int nthreads, uint32_t* ids_out,
                   float* weights_out, float* out) {
    const size_t T = a->tokens, K = a->top_k, H = a->hidden;
    if (!T || !K || K > a->experts || nthreads < 1) return K3XO_INVALID_EXTENT;
    layer_job j;
    memset(&j, 0, sizeof j);
    j.a = a;
    j.xn = (float*)malloc(T * H * sizeof(float));
    j.ids = ids_out;
    j.w = weights_out;
    j.y = (float*)malloc(T * K * H * sizeof(float));
    j.out = out;
    atomic_init(&j.status, 0);
    if (!j.xn || !j.y) {
        free(j.xn);
        free(j.y);
        return K3XO_INVALID_STATE;
    }
    pthread_t* th = (pthread_t*)malloc((size_t)nthreads * sizeof(pthread_t));
    int st = th ? K3XO_OK : K3XO_INVALID_STATE;
    for (int phase = 0; phase < 3 && !st; ++phase) {
        j.phase = phase;
        atomic_init(&j.next, 0);
        int started = 0;
        for (; started < nthreads - 1; ++started)
            if (pthread_create(&th[started], NULL, layer_worker, &j)) break;
        layer_worker(&j);
        for (int q = 0; q < started; ++q) pthread_join(th[q], NULL);
        st = atomic_load(&j.status);
    }
    free(th);
    free(j.xn);
    free(j.y);
    return st;
}
