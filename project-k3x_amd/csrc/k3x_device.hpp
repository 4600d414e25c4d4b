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

struct GluParams {
    int kind;        // 0 SwiGLU, 1 SiTU
    float beta;
    int has_linear;
    float linear_beta;
};

// SiTU-GLU (runtime/src/ops.cpp:20-30) or SwiGLU (silu(g) * u).  The gate
// sigmoid 1 / (1 + exp(-g)) runs on the hardware exp2 and reciprocal (about
// one ulp each, far inside the bf16 rounding that follows): it is evaluated
// for every element of a GEMM epilogue, where the library expf and IEEE
// divide made the epilogue a sizeable share of the kernel.  g -> -inf gives
// exp2 = inf and a sigmoid of 0; NaN propagates.
__device__ inline float glu(float g, float u, const GluParams& p) {
    const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504f));
    if (p.kind == 1) {
        const float bg = p.beta * tanhf(g / p.beta) * sig;
        const float bu = p.has_linear ? p.linear_beta * tanhf(u / p.linear_beta) : u;
        return bg * bu;
    }
    return (g * sig) * u;
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
