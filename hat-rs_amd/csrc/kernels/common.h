// Shared device helpers for the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>

#include "../kargs.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define HAT_LOG2E 1.4426950408889634f

// v_mfma_f32_16x16x4_f32: A 16x4 (lane l: row l%16, k l/16), B 4x16 (lane l:
// k l/16, col l%16), D 16x16 (lane l, reg r: row 4*(l/16)+r, col l%16).
__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x2_f32: A 32x2 (lane l: row l%32, k l/32), B 2x32 (lane l:
// k l/32, col l%32), D 32x32 (lane l, reg r: row 8*(r/4)+4*(l/32)+r%4, col l%32).
__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// erf by Abramowitz & Stegun 7.1.26 (max abs error 1.5e-7), the same published
// method the reference CPU path uses for nn.GELU's exact-erf form.
__device__ __forceinline__ float erf_as(float x)
{
    float sign = x < 0.0f ? -1.0f : 1.0f;
    x = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * x);
    float poly = ((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t
                 + 0.254829592f;
    float e = fast_exp2(-x * x * HAT_LOG2E);
    return sign * (1.0f - poly * t * e);
}

// GELU(v) = v/2 (1 + erf(v/sqrt2)) = v/2 + |v|/2 erf(|v|/sqrt2), with the same
// A&S 7.1.26 erf on a = |v|/sqrt2 >= 0 (no sign select), the reciprocal by
// v_rcp_f32 (1 ulp) rather than the IEEE division sequence: 13 VALU + 2
// transcendental ops. It stays within 2e-7 of erf_as's GELU.
__device__ __forceinline__ float gelu(float v)
{
    const float a = fabsf(v) * 0.70710677f;
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, a, 1.0f));
    float poly = __builtin_fmaf(1.061405429f, t, -1.453152027f);
    poly = __builtin_fmaf(poly, t, 1.421413741f);
    poly = __builtin_fmaf(poly, t, -0.284496736f);
    poly = __builtin_fmaf(poly, t, 0.254829592f);
    poly *= t;
    const float e = fast_exp2((a * -HAT_LOG2E) * a);
    const float erf_a = __builtin_fmaf(-poly, e, 1.0f);  // erf(a), a >= 0
    return __builtin_fmaf(0.5f * fabsf(v), erf_a, 0.5f * v);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
