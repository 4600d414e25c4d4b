// k3x_device.hpp -- gfx950 device helpers shared by the MoE-layer kernels.
//
// Data layout of the resident bank (both MXFP4 and bf16 matrices) is built
// around one MFMA: v_mfma_f32_16x16x32_bf16.  A weight "tile" covers 16
// output rows x 128 K.  Lane l of a wave owns row n = l % 16 and the 32-wide
// K block g = l / 16 of the tile; for the j-th of the four MFMAs of a tile the
// lane supplies K = 32g + 8j .. 32g + 8j + 7.  Activations are fed with the
// same K mapping, so the dot product is unchanged while every lane reads
// contiguous memory (an MXFP4 lane reads its whole 32-code block -- one E8M0
// scale -- with a single 16-byte load and a wave reads 1 KiB contiguous).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/k3x_hip_moe.h"

namespace k3x_dev {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
// Native 4 x 32-bit vector.  Register arrays that are carried around a loop
// must use it rather than HIP's uint4 (a struct of unions), which the
// compiler then keeps in scratch memory.
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

constexpr int kWave = 64;
constexpr int kTileRows = 16;
constexpr int kTileK = 128;

__device__ inline float bf16_to_f32(uint16_t w) { return __uint_as_float((uint32_t)w << 16); }

// Round-to-nearest-even to bf16 bits; NaN stays a quiet NaN.  Same rule as
// round_bf16 in runtime/src/official_moe.cpp:18-26.
__device__ inline uint16_t f32_to_bf16(float v) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7f800000u) == 0x7f800000u) {
        if (b & 0x007fffffu) b |= 0x00400000u;
        return (uint16_t)(b >> 16);
    }
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

// Two floats -> packed bf16 bits {lo, hi}, the rule of f32_to_bf16: the
// conversion instruction (v_cvt_pk_bf16_f32, round to nearest even) for
// numbers and infinities, f32_to_bf16 itself for NaN (quiet bit set, low
// payload bits dropped).
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
    if (__builtin_isnan(lo) || __builtin_isnan(hi))
        return (uint32_t)f32_to_bf16(lo) | (uint32_t)f32_to_bf16(hi) << 16;
    const bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// E8M0 byte -> 2^(s-127) as an fp32 (s = 0 gives the subnormal 2^-127).
__device__ inline float e8m0_to_f32(uint32_t s) {
    return __uint_as_float(s ? (s << 23) : 0x00400000u);
}

// Eight E2M1 codes (one dword, low nibble first) -> eight bf16 values scaled
// by 2^(s-127).  v_cvt_scalef32_pk_bf16_fp4 converts the two codes of one
// byte; the results are exact (two significant bits times a power of two).
__device__ inline bf16x8 dequant8(uint32_t codes, float scale) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale, 0);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale, 1);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale, 2);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale, 3);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ inline bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ inline bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ inline f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef __attribute__((ext_vector_type(8))) int i32x8;

// 32 E4M3 codes of one lane (two 16-byte pieces, element i in byte i) as the
// A operand of the scaled MFMA.
__device__ inline i32x8 q8_operand(u32x4 p0, u32x4 p1) {
    return i32x8{(int)p0[0], (int)p0[1], (int)p0[2], (int)p0[3],
                 (int)p1[0], (int)p1[1], (int)p1[2], (int)p1[3]};
}

// C += (A * 2^(sa-127)) (B * 2^(sb-127)) over K = 128: A = E4M3 codes
// (lane (n, g): row n, K 32 g .. 32 g + 31), B = the lane's 32 E2M1 codes
// of the bank tile (one 16-byte word, low nibble first); sa = E8M0 byte in
// bits 0..7.  Output in the 16x16 accumulator layout of mfma16x16x32.
// sb's byte OPB is the weights' scale (op_sel of the scale operand).
template <int OPB>
__device__ inline f32x4 mfma_q8_fp4(i32x8 a, u32x4 b, f32x4 c, uint32_t sa, uint32_t sb) {
    const i32x8 b8 = {(int)b[0], (int)b[1], (int)b[2], (int)b[3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b8, c, 0, 4, 0, (int)sa, OPB,
                                                            (int)sb);
}

// The same with the byte chosen by opb = 0..3, a constant once unrolled.
__device__ inline f32x4 mfma_q8_fp4_sel(int opb, i32x8 a, u32x4 b, f32x4 c, uint32_t sa,
                                        uint32_t sb) {
    switch (opb) {
        case 0: return mfma_q8_fp4<0>(a, b, c, sa, sb);
        case 1: return mfma_q8_fp4<1>(a, b, c, sa, sb);
        case 2: return mfma_q8_fp4<2>(a, b, c, sa, sb);
        default: return mfma_q8_fp4<3>(a, b, c, sa, sb);
    }
}

// Correctly rounded expf evaluated in double (x = k ln2 + r, degree-13
// Taylor polynomial on |r| <= ln2/2, one final rounding).  The operation
// sequence is fixed with explicit fma so the CPU checker reproduces it bit
// for bit.
__device__ inline float expf_cr(float x) {
    if (x != x) return x;
    if (x > 100.0f) return __builtin_inff();
    if (x < -110.0f) return 0.0f;
    const double xd = (double)x;
    const double k = __builtin_rint(xd * 1.4426950408889634);
    double r = __builtin_fma(-k, 6.93147180369123816490e-01, xd);
    r = __builtin_fma(-k, 1.90821492927058770002e-10, r);
    double p = 1.6059043836821614599e-10;
    p = __builtin_fma(p, r, 2.0876756987868098979e-09);
    p = __builtin_fma(p, r, 2.5052108385441718775e-08);
    p = __builtin_fma(p, r, 2.7557319223985890653e-07);
    p = __builtin_fma(p, r, 2.7557319223985890653e-06);
    p = __builtin_fma(p, r, 2.4801587301587301587e-05);
    p = __builtin_fma(p, r, 1.9841269841269841270e-04);
    p = __builtin_fma(p, r, 1.3888888888888888889e-03);
    p = __builtin_fma(p, r, 8.3333333333333333333e-03);
    p = __builtin_fma(p, r, 4.1666666666666666667e-02);
    p = __builtin_fma(p, r, 1.6666666666666666667e-01);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return (float)__builtin_ldexp(p, (int)k);
}

// Router sigmoid 1 / (1 + exp(-v)) with a correctly rounded exp, a float add
// and a correctly rounded float divide.
__device__ inline float sigmoid_cr(float v) {
    const float t = __fadd_rn(1.0f, expf_cr(-v));
    return __fdiv_rn(1.0f, t);
}

// Sort key: larger adjusted score first, then lower expert index
// (runtime/src/official_moe.cpp:226-232).  -0 folds into +0; 0 = no entry.
__device__ inline uint64_t topk_key(float adj, uint32_t e) {
    const float a = adj == 0.0f ? 0.0f : adj;
    const uint32_t u = __float_as_uint(a);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - e);
}

// Maximum of v over the 64 lanes with DPP moves (quad permutes, row
// rotates, row broadcasts): VALU latency instead of LDS-crossbar shuffles.
// Rows not selected by a row_bcast keep their own value (max(v, v) = v).
template <int Ctrl, int RowMask>
__device__ inline uint32_t dpp_max_step(uint32_t x) {
    const uint32_t y =
        (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, Ctrl, RowMask, 0xf, false);
    return x > y ? x : y;
}

__device__ inline uint32_t wave_max_u32(uint32_t v) {
    v = dpp_max_step<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_max_step<0x124, 0xf>(v);  // row_ror:4
    v = dpp_max_step<0x128, 0xf>(v);  // row_ror:8
    v = dpp_max_step<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    v = dpp_max_step<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Top-K of one token by one wave, KPL keys per lane (lane + 64 i: expert
// E + ... absent), given the token's logits lgv and the bias bv of those
// experts.  Scores, validation and renormalisation as
// runtime/src/routing_policy.cpp:40-95,146-157 (renorm_double false) or
// runtime/src/official_moe.cpp:214-242 (true), then * routed_scale
// (runtime/src/model.cpp:1004-1009).  Each lane sorts its keys; each slot
// takes the largest head by a DPP wave maximum of the score half of the key
// (ties on it resolved by a second maximum of the expert half), and the
// winning lane pops its head.  Returns 0 or the error code (the same on
// every lane); lane s < K then holds slot s's expert and weight.
template <int KPL>
__device__ inline uint32_t topk_wave(const float (&lgv)[KPL], const float (&bv)[KPL], uint32_t E,
                                     uint32_t K, bool renorm_double, float routed_scale,
                                     uint32_t* selid_out, float* weight_out) {
    constexpr uint32_t kErrExtent = K3X_ERR_INVALID_EXTENT, kErrState = K3X_ERR_INVALID_STATE;
    const int lane = threadIdx.x & 63;
    uint64_t key[KPL];
    float score[KPL];
    uint32_t bad = 0;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
        const uint32_t e = lane + 64u * i;
        key[i] = 0;
        score[i] = 0.0f;
        if (e < E) {
            const float lg = lgv[i];
            const float b = bv[i];
            if (renorm_double && (!__builtin_isfinite(lg) || !__builtin_isfinite(b)))
                bad = kErrExtent;
            const float s = sigmoid_cr(lg);
            const float adj = __fadd_rn(s, b);
            if (!renorm_double &&
                (!__builtin_isfinite(s) || s < 0.0f || s > 1.0f || !__builtin_isfinite(b) ||
                 !__builtin_isfinite(adj)))
                bad = kErrState;
            score[i] = s;
            key[i] = topk_key(adj, e);
        }
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) bad = max(bad, (uint32_t)__shfl_xor((int)bad, d));
    if (bad) return bad;
    // Local selection sort, descending: the lane's head is key[0].
#pragma unroll
    for (int i = 0; i < KPL; ++i)
#pragma unroll
        for (int j = i + 1; j < KPL; ++j)
            if (key[j] > key[i]) {
                const uint64_t tk = key[i];
                key[i] = key[j];
                key[j] = tk;
                const float ts = score[i];
                score[i] = score[j];
                score[j] = ts;
            }
    float selsc = 0.0f;  // lane s < K keeps the score of slot s
    uint32_t selid = 0;
    for (uint32_t s = 0; s < K; ++s) {
        // Largest head: first the score half of the key, then, among lanes
        // whose heads tie on it, the expert half (a larger value there is a
        // lower expert index).
        const uint32_t hi = (uint32_t)(key[0] >> 32);
        const uint32_t mhi = wave_max_u32(hi);
        uint64_t tie = __ballot(hi == mhi);
        if (__popcll(tie) > 1) {
            const uint32_t lo = hi == mhi ? (uint32_t)key[0] : 0u;
            const uint32_t mlo = wave_max_u32(lo);
            tie = __ballot(hi == mhi && lo == mlo);
        }
        const int wlane = __ffsll((unsigned long long)tie) - 1;
        const uint32_t win =
            0xffffffffu - (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key[0], wlane);
        const float wsc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(score[0]), wlane));
        if ((uint32_t)lane == s) {
            selsc = wsc;
            selid = win;
        }
        if (lane == wlane) {
#pragma unroll
            for (int i = 0; i < KPL - 1; ++i) {
                key[i] = key[i + 1];
                score[i] = score[i + 1];
            }
            key[KPL - 1] = 0;
        }
    }
    // Renormalise in slot order (sequential sums as the reference).
    float den_f = 0.0f;
    double den_d = 0.0;
    for (uint32_t s = 0; s < K; ++s) {
        const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(selsc), s));
        den_f = __fadd_rn(den_f, v);
        den_d = __dadd_rn(den_d, (double)v);
    }
    if (renorm_double) {
        if (!__builtin_isfinite(den_d) || !(den_d > 0.0)) return kErrExtent;
    } else if (!__builtin_isfinite(den_f) || !(den_f > 0.0f)) {
        return kErrState;
    }
    *selid_out = selid;
    *weight_out = renorm_double ? __fmul_rn((float)__ddiv_rn((double)selsc, den_d), routed_scale)
                                : __fmul_rn(__fdiv_rn(selsc, den_f), routed_scale);
    return 0;
}

struct GluParams {
    int kind;        // 0 SwiGLU, 1 SiTU
    float beta;
    int has_linear;
    float linear_beta;
    int round_in;    // 1: gate and up rounded to bf16 first (a bf16 projection's output)
};

// SiTU-GLU (runtime/src/ops.cpp:20-30) or SwiGLU (silu(g) * u).  The gate
// sigmoid 1 / (1 + exp(-g)) runs on the hardware exp2 and reciprocal (about
// one ulp each, far inside the bf16 rounding that follows): it is evaluated
// for every element of a GEMM epilogue, where the library expf and IEEE
// divide made the epilogue a sizeable share of the kernel.  g -> -inf gives
// exp2 = inf and a sigmoid of 0; NaN propagates.
__device__ inline float glu(float g, float u, const GluParams& p) {
    if (p.round_in) {
        g = __uint_as_float((uint32_t)f32_to_bf16(g) << 16);
        u = __uint_as_float((uint32_t)f32_to_bf16(u) << 16);
    }
    const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504f));
    if (p.kind == 1) {
        const float bg = p.beta * tanhf(g / p.beta) * sig;
        const float bu = p.has_linear ? p.linear_beta * tanhf(u / p.linear_beta) : u;
        return bg * bu;
    }
    return (g * sig) * u;
}

// A GLU activation v as two bf16 words, hi = bf16(v) and lo = bf16(v - hi):
// hi + lo carries v to about 2^-17 relative, so a bf16 MFMA over both
// halves (the activation as a row [hi | lo] against the weights repeated
// along K) multiplies by an fp32 activation.
__device__ inline uint16_t act_lo_bf16(float v, uint16_t hi) {
    return f32_to_bf16(__fsub_rn(v, __uint_as_float((uint32_t)hi << 16)));
}

// ---------------------------------------------------------------------------
// Two-term FP8 activation blocks ("q8 rows") for the scaled FP4 MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4: OCP E4M3 activations x E2M1 weights,
// one E8M0 scale per 32-element block of each operand).
//
// A block of 32 values x is stored as hi + lo with
//   s_hi = 2^(floor(log2 max|x|) - 7)       (max|x| / s_hi in [128, 256))
//   hi   = E4M3(x / s_hi)                   (round to nearest even)
//   r    = x - hi * s_hi                    (exact in fp32)
//   s_lo = 2^(floor(log2 max|r|) - 7),  lo = E4M3(r / s_lo).
// For bf16 x the residual r of every element within 2^-13 of max|x| has at
// most four significant bits, so lo holds it exactly; smaller elements are
// off by at most 2^-21 max|x|.  hi * s_hi + lo * s_lo is thus the bf16 value
// (to that bound), and two scaled MFMAs (hi, lo) reproduce the bf16 product.
//
// Row layout, per 128-element K tile: 128 hi codes then 128 lo codes (256
// bytes, as many as the bf16 row); scales [row][tile] = {hi, lo} dwords, byte
// b = 32-element block b of the tile.
// ---------------------------------------------------------------------------

// Biased E8M0 exponent e with m / 2^(e-127) in [128, 256) for m = max|x| (at
// least 1: the scale stays a normal fp32).
__device__ inline uint32_t q8_exponent(float m) {
    const int e = (int)((__float_as_uint(m) >> 23) & 0xffu) - 7;
    return (uint32_t)(e < 1 ? 1 : e);
}

// Four values -> four E4M3 codes (byte i = v[i] * inv), rounded to nearest
// even; inv is an exact power of two, so the scaling adds no rounding.
__device__ inline uint32_t q8_pack4(float a, float b, float c, float d, float inv) {
    typedef __attribute__((ext_vector_type(2))) short i16x2;
    i16x2 o = {0, 0};
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, a * inv, b * inv, 1.0f, false);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, c * inv, d * inv, 1.0f, true);
    return __builtin_bit_cast(uint32_t, o);
}

// Four E4M3 codes -> their values times s.
__device__ inline void q8_unpack4(uint32_t q, float s, float* out) {
    typedef __attribute__((ext_vector_type(2))) float f32x2;
    const f32x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)q, 1.0f, false);
    const f32x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)q, 1.0f, true);
    out[0] = lo[0] * s;
    out[1] = lo[1] * s;
    out[2] = hi[0] * s;
    out[3] = hi[1] * s;
}

// One 32-element block: hi and lo codes (eight dwords each, element i in
// byte i % 4 of dword i / 4) and the two E8M0 exponents.
__device__ inline void q8_block(const float (&x)[32], uint32_t (&hi)[8], uint32_t (&lo)[8],
                                uint32_t& ehi, uint32_t& elo) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(x[i]));
    ehi = q8_exponent(m);
    const float inv_hi = __uint_as_float((254u - ehi) << 23), s_hi = __uint_as_float(ehi << 23);
    float r[32];
    float rm = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        hi[i] = q8_pack4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3], inv_hi);
        float b[4];
        q8_unpack4(hi[i], s_hi, b);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r[4 * i + j] = __fsub_rn(x[4 * i + j], b[j]);
            rm = fmaxf(rm, fabsf(r[4 * i + j]));
        }
    }
    elo = q8_exponent(rm);
    const float inv_lo = __uint_as_float((254u - elo) << 23);
#pragma unroll
    for (int i = 0; i < 8; ++i)
        lo[i] = q8_pack4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3], inv_lo);
}

// SplitMix64 output function (Steele, Lea & Flood, OOPSLA 2014) and the
// counter-based streams of the synthetic generator.
__device__ __host__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
constexpr uint64_t kGamma = 0x9e3779b97f4a7c15ull;
__device__ __host__ inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(seed + kGamma * (stream + 1));
}
__device__ __host__ inline uint64_t word_at(uint64_t key, uint64_t i) {
    return mix64(key + kGamma * (i + 1));
}
// Irwin-Hall(12) normal: integer sum of twelve 16-bit uniforms; only the
// final multiply by sigma rounds.
__device__ inline float normal_at(uint64_t key, uint64_t i, float sigma) {
    int32_t sum = 0;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const uint64_t w = word_at(key, 3 * i + (uint64_t)j);
#pragma unroll
        for (int q = 0; q < 4; ++q) sum += (int32_t)((w >> (16 * q)) & 0xffffu);
    }
    return __fmul_rn((float)(sum - 393216) * 0x1p-16f, sigma);
}

}  // namespace k3x_dev
