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

// A compile-time int carried by a value, for generic lambdas: decltype(x)::value.
template <int V> struct CInt {
    static constexpr int value = V;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// GELU(v) = v Phi(v) = max(v, 0) - |v|/2 erfc(a), a = |v|/sqrt2, with erfc(a) =
// t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-a^2), t = 1/(1 + p a): the same
// published method (Abramowitz & Stegun 7.1.26, |erf error| <= 1.5e-7) as the
// reference CPU path's erf, arranged for few instructions: the 1/2 folded into
// the coefficients, p/sqrt2 into the reciprocal's argument, exp(-a^2) taken as
// exp2(v^2 * (-log2(e)/2)), the reciprocal by v_rcp_f32 (1 ulp). 11 VALU + 2
// transcendental ops; within 3.4e-7 of the exact GELU over [-12, 12] in fp32.
__device__ __forceinline__ float gelu(float v)
{
    const float av = fabsf(v);
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f * 0.70710678f, av, 1.0f));
    float q = __builtin_fmaf(0.5f * 1.061405429f, t, 0.5f * -1.453152027f);
    q = __builtin_fmaf(q, t, 0.5f * 1.421413741f);
    q = __builtin_fmaf(q, t, 0.5f * -0.284496736f);
    q = __builtin_fmaf(q, t, 0.5f * 0.254829592f);
    const float e = fast_exp2((v * v) * (-0.5f * HAT_LOG2E));
    return __builtin_fmaf(-av, (q * t) * e, fmaxf(v, 0.0f));
}

// 1 KB of zeros in global memory, never written (and not const, so the
// compiler cannot fold loads from it). Loads that fall outside an operand -
// rows past M, padding channels, taps outside the plane, padding slots of the
// weight chunks - read here. The alternatives cost more: a branch around the
// load makes the number of loads in flight path-dependent, so the compiler's
// later waits drain every load; zeroing the value after the load makes it wait
// for that load at once.
__device__ __attribute__((aligned(16))) float hat_zero_row[256] = {};

// A float4 from p, or zeros (from hat_zero_row) where ok is false.
__device__ __forceinline__ f32x4 load_or_zero(const float* p, bool ok)
{
    return *(const f32x4*)(ok ? p : hat_zero_row);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
