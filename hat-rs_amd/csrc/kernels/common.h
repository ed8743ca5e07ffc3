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

// ---- split-bf16 arithmetic (the BF16 MFMA path at fp32 accuracy): an fp32
// operand as three bf16 parts, a product as the six terms of order <= 2
// (attnx.hip states the accuracy).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// (a, b) rounded to nearest bf16, packed: a in the low half (element 0).
__device__ __forceinline__ unsigned pk_bf16(float a, float b)
{
    return __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// The three-way split of a pair: (a, b) = p0 + p1 + p2 (+ below 2^-27 of
// each), every part a packed pair of bf16, each the round-to-nearest of what
// the earlier parts leave (x - its rounding is exact in fp32).
__device__ __forceinline__ void split3_pk(float a, float b, unsigned& p0, unsigned& p1, unsigned& p2)
{
    p0 = pk_bf16(a, b);
    a -= __uint_as_float(p0 << 16);
    b -= __uint_as_float(p0 & 0xffff0000u);
    p1 = pk_bf16(a, b);
    a -= __uint_as_float(p1 << 16);
    b -= __uint_as_float(p1 & 0xffff0000u);
    p2 = pk_bf16(a, b);
}

// Part pl (0, 1, 2) of x's three-way split, as bf16 bits.
__device__ __forceinline__ unsigned short split3_part(float x, int pl)
{
    unsigned p0, p1, p2;
    split3_pk(x, 0.0f, p0, p1, p2);
    return (unsigned short)((pl == 0 ? p0 : pl == 1 ? p1 : p2) & 0xffffu);
}

// Eight consecutive fp32 values as three 8-wide bf16 parts.
__device__ __forceinline__ void split3_x8(const float (&v)[8], u32x4 (&out)[3])
{
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        unsigned p0, p1, p2;
        split3_pk(v[2 * j], v[2 * j + 1], p0, p1, p2);
        out[0][j] = p0;
        out[1][j] = p1;
        out[2][j] = p2;
    }
}

// v_mfma_f32_16x16x32_bf16: A 16x32 (lane l: row l%16, k 8*(l/16) .. +7), B
// 32x16 (lane l: k 8*(l/16) .. +7, col l%16), D as mfma16's.
__device__ __forceinline__ f32x4 mfma16_bf16(u32x4 a, u32x4 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16x6(const u32x4 (&a)[3], const u32x4 (&b)[3], f32x4 c)
{
    c = mfma16_bf16(a[2], b[0], c);
    c = mfma16_bf16(a[1], b[1], c);
    c = mfma16_bf16(a[0], b[2], c);
    c = mfma16_bf16(a[1], b[0], c);
    c = mfma16_bf16(a[0], b[1], c);
    return mfma16_bf16(a[0], b[0], c);
}

// The packed last k-step of a K = 144 linear (the host's split_half_step):
// the lane's four activations v (k = 128 + 4 lg + j) as the operand pairs
// (b0 | b1), (b0 | b2), (b1 | b0), the weights' planes holding (a0 | a0),
// (a1 | a0), (a1 | a2): three MFMAs give the six products of order <= 2 that
// six give for a whole step, and the split covers four values, not eight.
__device__ __forceinline__ void half_operands(const f32x4& v, u32x4 (&b)[3])
{
    unsigned p0a, p1a, p2a, p0b, p1b, p2b;
    split3_pk(v[0], v[1], p0a, p1a, p2a);
    split3_pk(v[2], v[3], p0b, p1b, p2b);
    b[0] = (u32x4){p0a, p0b, p1a, p1b};
    b[1] = (u32x4){p0a, p0b, p2a, p2b};
    b[2] = (u32x4){p1a, p1b, p0a, p0b};
}

__device__ __forceinline__ f32x4 mfma16x3(const u32x4 (&a)[3], const u32x4 (&b)[3], f32x4 c)
{
    c = mfma16_bf16(a[2], b[2], c);  // a1 b1 + a2 b0
    c = mfma16_bf16(a[1], b[1], c);  // a1 b0 + a0 b2
    return mfma16_bf16(a[0], b[0], c);  // a0 b0 + a0 b1
}

// The same on v_mfma_f32_32x32x16_bf16 (lane l: row / column l % 32, k 8 (l / 32)
// .. +7; D: column l % 32, rows 8 (i / 4) + 4 (l / 32) + i % 4).
__device__ __forceinline__ f32x16 mfma_bf16(u32x4 a, u32x4 b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma6(const u32x4 (&a)[3], const u32x4 (&b)[3], f32x16 c)
{
    c = mfma_bf16(a[2], b[0], c);
    c = mfma_bf16(a[1], b[1], c);
    c = mfma_bf16(a[0], b[2], c);
    c = mfma_bf16(a[1], b[0], c);
    c = mfma_bf16(a[0], b[1], c);
    return mfma_bf16(a[0], b[0], c);
}

// ---- weight chunks for the split-bf16 linears: one 32-k step of up to 192
// rows as three bf16 planes [rows][32] with swizzled k-groups (ws_mma), packed
// on the host WC_CHUNK elements apart. A block copies chunk c + 1 into one of
// two LDS buffers while its waves multiply chunk c out of the other.

// The NL loads (1 KB each) of one chunk into an LDS buffer, NL / WAVES from
// every wave: wave w issues loads w, w + WAVES, ...; lane l of a load writes
// 16 bytes at the load's LDS base + 16 l. Straight-line code: as a loop, the
// per-load scalar bookkeeping (M0, the address, the counter and the branch)
// cost the tails 1-4% (same-box timings). The compiler's waits stay where
// they were: the callers wait for the copies explicitly before reading a
// buffer.
template <int NL, int WAVES>
__device__ __forceinline__ void wc_issue(unsigned short* dst, const unsigned short* src, int wave, int lane)
{
    static_assert(NL % WAVES == 0 && NL * 512 <= WC_CHUNK, "whole loads per wave, within a chunk");
    const unsigned loff = (unsigned)lane * 16;  // the lane's bytes within a load: one VGPR for every load
#pragma unroll
    for (int j = 0; j < NL / WAVES; ++j) {
        const int i = wave + j * WAVES;  // wave-uniform: the load's base goes in scalar registers
        const char* base = (const char*)src + (size_t)i * 1024;
        __builtin_amdgcn_global_load_lds((const void*)(base + loff),
                                         (__attribute__((address_space(3))) void*)(dst + i * 512), 16, 0, 0);
    }
}

// acc[mt][nt] += W[rows 16 nt .. +15] . xb[mt] for one chunk in the swizzled
// layout of the weight-stationary kernels:
// three planes [ROWS][32] (plane stride ROWS * 32), row r's four 16-byte
// k-groups g stored at slot ws_slot(r, g), so that the fragment reads down the
// rows at one k-group are free of bank conflicts without padding (a 192-row
// chunk fits TX_BUF). HALF: the packed last step of a K = 144 linear (xb from
// half_operands, three MFMAs per tile).
template <int NT, int ROWS, bool HALF = false>
__device__ __forceinline__ void ws_mma(const unsigned short* Ws, int lr, int lg, const u32x4 (&xb)[2][3],
                                       f32x4 (&acc)[2][NT])
{
    const unsigned short* wr = Ws + lr * 32 + (hatk::ws_slot(lr, lg) * 8);
    u32x4 wa[2][3];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) wa[0][pl] = *(const u32x4*)(wr + pl * ROWS * 32);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        __builtin_amdgcn_sched_barrier(0);
        if (nt + 1 < NT) {
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
                wa[(nt + 1) & 1][pl] = *(const u32x4*)(wr + (nt + 1) * 16 * 32 + pl * ROWS * 32);
        }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
            acc[mt][nt] = HALF ? mfma16x3(wa[nt & 1], xb[mt], acc[mt][nt]) : mfma16x6(wa[nt & 1], xb[mt], acc[mt][nt]);
    }
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

// A 1 then zeros: the activation of a bias column (see WcRows::load_b).
__device__ __attribute__((aligned(16))) float hat_one_row[4] = {1.0f, 0.0f, 0.0f, 0.0f};

// Where stores of rows past the end of an output go, so that a wave issues
// the same number of stores whatever the row count (never read).
__device__ __attribute__((aligned(16))) float hat_sink_row[64];

// s_waitcnt for "at most n vector memory operations of this wave still
// outstanding, and every LDS operation done" (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4 left at its maximum, lgkmcnt 11:8 = 0). Vector
// memory operations complete in issue order for this count (the compiler's
// own waits rely on it), so waiting for an operation means waiting until no
// more than the number issued after it are outstanding.
constexpr int wc_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x70; }

// A workgroup barrier for LDS data only: this wave's LDS accesses complete,
// then the barrier. __syncthreads() adds a release fence, which on gfx950 waits
// for every outstanding vector memory operation as well - global loads issued
// ahead for later use included. The memory clobber keeps the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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

// The wave's sum in registers alone (DPP, no LDS round trips), wave-uniform:
// pairs, quads, 8 (half-row mirror), 16 (row mirror), then row 0 into row 1
// and row 2 into row 3 (row_bcast:15), rows 0-1 into row 3 (row_bcast:31);
// lane 63 ends with the total. A fixed order, so the result does not depend on
// timing.
__device__ __forceinline__ float wave_sum_dpp(float v)
{
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
