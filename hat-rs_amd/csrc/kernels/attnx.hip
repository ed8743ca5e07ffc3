// Shifted-window attention on BF16 MFMA with fp32 accuracy: QK^T + relative-
// position bias + shift mask + softmax + PV for one (window, head) per block.
//
// The same operator as attn.hip (cpu.rs:772-844; hat.cu:246-316) on gfx950's
// BF16 matrix path, whose peak is 16x the FP32 MFMA rate. VALU and MFMA work
// share a SIMD's issue time (measured: they do not overlap, from one wave or
// from two), so the splits and exponentials below cost their full time. Every fp32
// operand x enters as three bf16 parts, x = x0 + x1 + x2 + e with |e| <=
// 2^-27 |x| (each part the round-to-nearest of what the earlier ones leave),
// and a product as the six terms a_i b_j with i + j <= 2, accumulated in fp32
// by v_mfma_f32_32x32x16_bf16; the terms dropped (i + j >= 3) are below
// 2^-26 |ab|. Measured at K = 144 against a double reference: worst error
// 1.25e-7 of sum|ab| against 1.42e-7 for FP32 MFMA.
//
// Layout (all per item, in LDS): K as three bf16 planes [256 keys][KS] and V^T
// as three planes [D + 1][VS] whose key order is permuted within each 16 so
// that a lane's eight keys of one MFMA step are contiguous; row D of V^T is
// ones in the high plane and zeros in the others, so row D of O^T is the
// softmax denominator. The bias table of the head is kept in log2 units. Wave
// w owns queries [32w, 32w+32). Scores are computed transposed, S^T = K Q^T
// (A = a 32-key tile of K, B = the wave's q, split in registers): lane l holds
// 16 scores of query l%32, which after the softmax are split and used directly
// as the B operand of O^T += V^T P^T. Bias, mask, online softmax in base 2 and
// the output are those of attn.hip.
#include "common.h"

using namespace hatk;

template <int D>
struct AttnXShape {
    static constexpr int NK = 256;
    // K row stride in bf16: 24 (48 B) and 40 (80 B) put the 16 rows a ds_read_b128
    // phase touches on distinct banks.
    static constexpr int KS = D == 24 ? 24 : 40;
    static constexpr int VS = NK + 8;  // V^T row stride (528 B: rows 4 banks apart)
    static constexpr int KPL = NK * KS, VPL = (D + 1) * VS;  // elements per plane
    static constexpr int TROWS = 961;
    static constexpr int LDS_BYTES = 2 * 3 * (KPL + VPL) + 4 * TROWS;
};

// Position of key k in the V^T planes: within each 16 keys, bits 2 and 3
// swap, so that lane half h's eight keys of an MFMA step (16s + 8a + 4h + t,
// a, t the slot's high bit and low two bits) are positions 16s + 8h .. +7.
__device__ __forceinline__ int vpos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

// Item staging: this thread's K and V units (attn_fetch's registers), split
// into the LDS planes; row D of V^T: ones (high plane), zeros; K dims D .. 31
// of D = 30 zeroed (the q operand is zero there; LDS that was never written
// could hold a NaN).
template <int D>
__device__ __forceinline__ void attnx_stash(unsigned short* Kp, unsigned short* Vp,
                                            const typename AttnShape<D, false>::vec (&ks)[AttnShape<D, false>::NE],
                                            const typename AttnShape<D, false>::vec (&vs)[AttnShape<D, false>::NE])
{
    using S = AttnShape<D, false>;
    using X = AttnXShape<D>;
    constexpr int PER_KEY = D / S::U;
#pragma unroll
    for (int i = 0; i < S::NE; ++i) {
        const int e = threadIdx.x + i * 512;
        if (e < S::NK * PER_KEY) {
            const int k = e / PER_KEY, d = (e - k * PER_KEY) * S::U;
            float kv[4], vv[4];
            if constexpr (S::U == 4) {
                kv[0] = ks[i].x, kv[1] = ks[i].y, kv[2] = ks[i].z, kv[3] = ks[i].w;
                vv[0] = vs[i].x, vv[1] = vs[i].y, vv[2] = vs[i].z, vv[3] = vs[i].w;
            } else {
                kv[0] = ks[i].x, kv[1] = ks[i].y, kv[2] = kv[3] = 0.f;
                vv[0] = vs[i].x, vv[1] = vs[i].y, vv[2] = vv[3] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < S::U; j += 2) {
                unsigned k0, k1, k2, v0, v1, v2;
                split3_pk(kv[j], kv[j + 1], k0, k1, k2);
                *(unsigned*)(Kp + 0 * X::KPL + k * X::KS + d + j) = k0;
                *(unsigned*)(Kp + 1 * X::KPL + k * X::KS + d + j) = k1;
                *(unsigned*)(Kp + 2 * X::KPL + k * X::KS + d + j) = k2;
                split3_pk(vv[j], vv[j + 1], v0, v1, v2);
                const int pos = vpos(k);
                Vp[0 * X::VPL + (d + j) * X::VS + pos] = (unsigned short)v0;
                Vp[0 * X::VPL + (d + j + 1) * X::VS + pos] = (unsigned short)(v0 >> 16);
                Vp[1 * X::VPL + (d + j) * X::VS + pos] = (unsigned short)v1;
                Vp[1 * X::VPL + (d + j + 1) * X::VS + pos] = (unsigned short)(v1 >> 16);
                Vp[2 * X::VPL + (d + j) * X::VS + pos] = (unsigned short)v2;
                Vp[2 * X::VPL + (d + j + 1) * X::VS + pos] = (unsigned short)(v2 >> 16);
            }
        }
    }
    for (int e = threadIdx.x; e < 3 * (S::NK / 2); e += 512) {
        const int pl = e / (S::NK / 2), k2 = e - pl * (S::NK / 2);
        *(unsigned*)(Vp + pl * X::VPL + D * X::VS + 2 * k2) = pl == 0 ? 0x3f803f80u : 0u;  // bf16 1.0 pairs
    }
    if (D == 30) {
        for (int e = threadIdx.x; e < 3 * S::NK; e += 512) {
            const int pl = e / S::NK, k = e - pl * S::NK;
            *(unsigned*)(Kp + pl * X::KPL + k * X::KS + 30) = 0u;
        }
    }
}

// The lane's q, pre-scaled and split: qb[s][part] = dims 16s + 8h .. 16s + 8h
// + 7 of its query (zeros past D). For D = 24 the second step is packed (see
// AttnxKRows): qb[1][0] = dims 16..23 of part h ? 0 : 2, qb[1][1] = of part
// h ? 0 : 1.
template <int D>
__device__ __forceinline__ int attnx_query(const AttnArgs& p, int wi, int head, u32x4 (&qb)[2][3])
{
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in a scalar register
    const int ql = lane & 31, h = lane >> 5;
    const int q = wave * 32 + ql, qy = q >> 4, qx = q & 15;
    const int wy = wi / p.nx, wx = wi - (wi / p.nx) * p.nx;
    int y = wy * 16 + qy + p.shift, x = wx * 16 + qx + p.shift;
    if (y >= p.hp) y -= p.hp;
    if (x >= p.wp) x -= p.wp;
    const int qpix = y * p.wp + x;
    const float* Qg = p.qkv + (size_t)head * p.T * D + (size_t)qpix * D;
    float qv[2][8];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if constexpr (D == 24) {
            // both halves of the packed second step hold dims 16..23
            const int d0 = s == 0 ? 8 * h : 16;
            const f32x4 a = *(const f32x4*)(Qg + d0), b = *(const f32x4*)(Qg + d0 + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) qv[s][j] = a[j], qv[s][4 + j] = b[j];
        } else {
            const int d0 = 16 * s + 8 * h;
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const bool live = d0 + j + 2 <= D;
                const float2 v = *(const float2*)(live ? Qg + d0 + j : hat_zero_row);
                qv[s][j] = v.x;
                qv[s][j + 1] = v.y;
            }
        }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int j = 0; j < 8; ++j) qv[s][j] *= p.qscale;
        split3_x8(qv[s], qb[s]);
    }
    if constexpr (D == 24) {
        const u32x4 q0 = qb[1][0], q1 = qb[1][1], q2 = qb[1][2];
        qb[1][0] = h ? q0 : q2;
        qb[1][1] = h ? q0 : q1;
    }
    return qpix;
}

// The lane's K rows for S^T = K Q^T over 32-key tiles of three planes [keys][KS]
// (A = 32 keys x 16 dims: lane l gives key l % 32, dims 8h .. 8h + 7 of the step).
// Step 0 (dims 0..15) is the six products of mfma6. For D = 24, step 1 has only
// dims 16..23, so each MFMA carries two of the six products, one per lane half:
// [k1 | k2] . [q1 | q0], [k0 | k1] . [q2 | q0], [k0 | k0] . [q1 | q0] (half 0 |
// half 1): the same terms in three MFMAs instead of six. For D = 30 step 1 is
// dims 16..31 (30, 31 zero) as step 0.
template <int D, int KS, int KPL>
struct AttnxKRows {
    const unsigned short *r0, *r12, *r3;
    __device__ __forceinline__ void init(const unsigned short* Kp, int ql, int h)
    {
        r0 = Kp + ql * KS + 8 * h;
        r12 = Kp + ql * KS + 16 + h * KPL;  // plane h (+1)
        r3 = Kp + ql * KS + 16;             // plane 0
    }
    // s += K Q^T for the tile whose first key row is koff elements in
    __device__ __forceinline__ f32x16 qk(int koff, const u32x4 (&qb)[2][3], f32x16 s) const
    {
        u32x4 ka[3];
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) ka[pl] = *(const u32x4*)(r0 + pl * KPL + koff);
        s = mfma6(ka, qb[0], s);
        if constexpr (D == 24) {
            const u32x4 a12 = *(const u32x4*)(r12 + KPL + koff), a01 = *(const u32x4*)(r12 + koff),
                        a00 = *(const u32x4*)(r3 + koff);
            s = mfma_bf16(a12, qb[1][1], s);
            s = mfma_bf16(a01, qb[1][0], s);
            return mfma_bf16(a00, qb[1][1], s);
        } else {
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) ka[pl] = *(const u32x4*)(r0 + pl * KPL + koff + 16);
            return mfma6(ka, qb[1], s);
        }
    }
};

// O^T (with the softmax denominator in row D) of the lane's query over the
// item's 256 keys. SAFE: the online softmax (the running base raised when a
// score exceeds it by more than 8, in log2 units), as the reference subtracts
// the row maximum (cpu.rs:801-812). Otherwise the base is 0: P = exp2(s)
// straight from the scores, no maximum, no subtraction, no rescaling (16 VALU
// a tile fewer); the caller checks the result and runs the SAFE form instead
// when a sum could have overflowed or lost its range (see attnx_item_done).
// Either way o / o[row D] is the softmax-weighted sum, the same quantity.
template <int D, bool MASKED, bool SAFE>
__device__ __forceinline__ f32x16 attnx_tiles(const AttnArgs& p, const unsigned char* lds, int wi,
                                              const u32x4 (&qb)[2][3])
{
    using X = AttnXShape<D>;
    constexpr int NKT = X::NK / 32;
    const unsigned short* Kp = (const unsigned short*)lds;
    const unsigned short* Vp = Kp + 3 * X::KPL;
    const float* Tb = (const float*)(Vp + 3 * X::VPL);

    const int wy = wi / p.nx, wx = wi - (wi / p.nx) * p.nx;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in a scalar register
    const int ql = lane & 31, h = lane >> 5;
    const int q = wave * 32 + ql;
    const int qy = q >> 4, qx = q & 15;
    const int sw_rbase = 960 - ((qy + 15) * 31 + qx + 15 - 4 * h);
    const float NEG = -100.0f * HAT_LOG2E;
    const bool mrow = MASKED && wy == p.ny - 1;
    const bool mcol = MASKED && wx == p.nx - 1;
    const bool r_lo = mrow && (qy & 8), r_hi = mrow && !(qy & 8);
    const bool c_lo = mcol && (qx & 8), c_hi = mcol && !(qx & 8);
    const float madd[2][2] = {{(r_lo || c_lo) ? NEG : 0.0f, (r_lo || c_hi) ? NEG : 0.0f},
                              {(r_hi || c_lo) ? NEG : 0.0f, (r_hi || c_hi) ? NEG : 0.0f}};
    static_assert(D < 32, "a spare V^T row is needed");

    // The lane's V^T row (dims past D read row D: their outputs are not used)
    // and K rows.
    const unsigned short* vrow = Vp + (ql < D ? ql : D) * X::VS + 8 * h;
    AttnxKRows<D, X::KS, X::KPL> kr;
    kr.init(Kp, ql, h);

    f32x16 o;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = 0.0f;
    float mrun = SAFE ? -INFINITY : 0.0f;

// unrolled: the K, V and bias addresses of every tile are immediate offsets
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
        // S^T = bias (+ mask) + K Q^T
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int key0 = kt * 32 + (i >> 2) * 8 + (i & 3);
            const int ky = key0 >> 4, kx = key0 & 15;
            float b = Tb[sw_rbase + (ky * 31 + kx)];
            if (MASKED) b += madd[(ky >> 3) & 1][(kx >> 3) & 1];
            s[i] = b;
        }
        s = kr.qk(kt * 32 * X::KS, qb, s);
        if constexpr (SAFE) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
            if (kt == 0 || __any(mx > mrun + 8.0f)) {  // wave-uniform
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float mnew = fmaxf(mrun, mx);
                const float corr = fast_exp2(mrun - mnew);
#pragma unroll
                for (int i = 0; i < 16; ++i) o[i] *= corr;
                mrun = mnew;
            }
        }
        // O^T += V^T P^T, P = exp2(S - base): the B operand of step st is
        // registers 8st .. 8st+7, split.
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            float pv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) pv[j] = fast_exp2(SAFE ? s[8 * st + j] - mrun : s[8 * st + j]);
            u32x4 pb[3], va[3];
            split3_x8(pv, pb);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) va[pl] = *(const u32x4*)(vrow + pl * X::VPL + kt * 32 + 16 * st);
            o = mfma6(va, pb, o);
        }
    }
    return o;
}

// Whether an item's base-0 pass (attnx_tiles with SAFE false) may stand, for
// every query of the wave: the denominator within [2^-60, 2^100] (no
// overflow, and far from the range where P's split parts would underflow;
// with the row maximum subtracted it lies in [1, 256 * 2^8]) and every
// accumulator finite. Wave-uniform.
template <int D>
__device__ __forceinline__ bool attnx_item_done(const f32x16& o)
{
    constexpr int RH = (D % 8) / 4, RR = (D / 8) * 4 + D % 4;
    const int ql = threadIdx.x & 31;
    const float ltot = __shfl(o[RR], ql + 32 * RH, 64);
    bool ok = ltot >= 0x1p-60f && ltot <= 0x1p100f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ok = ok && __builtin_isfinite(o[i]);
    return __all(ok);
}

// out[query][head * D + d] = O^T[d] / O^T[D] for the lane's query.
template <int D>
__device__ __forceinline__ void attnx_store(const AttnArgs& p, int head, int qpix, const f32x16& o)
{
    constexpr int RH = (D % 8) / 4, RR = (D / 8) * 4 + D % 4;
    const int lane = threadIdx.x & 63;
    const int ql = lane & 31, h = lane >> 5;
    const float ltot = __shfl(o[RR], ql + 32 * RH, 64);
    const float inv = 1.0f / ltot;
    float* orow = p.out + (size_t)qpix * p.C + head * D;
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
        const int d0 = 8 * i4 + 4 * h;
        if (D % 4 == 0) {
            if (d0 + 3 < D)
                *(float4*)(orow + d0) = make_float4(o[i4 * 4] * inv, o[i4 * 4 + 1] * inv,
                                                    o[i4 * 4 + 2] * inv, o[i4 * 4 + 3] * inv);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (d0 + j < D) orow[d0 + j] = o[i4 * 4 + j] * inv;
        }
    }
}

template <int D, bool MASKED>
__device__ __forceinline__ void attnx_compute(const AttnArgs& p, const unsigned char* lds, int wi, int head,
                                              const u32x4 (&qb)[2][3], int qpix)
{
    f32x16 o = attnx_tiles<D, MASKED, false>(p, lds, wi, qb);
    if (!attnx_item_done<D>(o)) {  // wave-uniform
        // the same LDS through an offset the compiler cannot see is zero, so
        // that it does not keep the first pass's loaded values for this one
        int z = 0;
        asm volatile("" : "+s"(z));
        o = attnx_tiles<D, MASKED, true>(p, lds + z, wi, qb);
    }
    attnx_store<D>(p, head, qpix, o);
}

template <int D>
__device__ __forceinline__ void attnx_item_kernel(const AttnArgs& p, unsigned char* lds)
{
    using S = AttnShape<D, false>;
    using X = AttnXShape<D>;
    const int wi = blockIdx.x, head = blockIdx.y;
    if (p.with_gate && wi == 0 && head == 0) {  // block-uniform
        static_assert(4 * CAB_GATE_LDS <= X::LDS_BYTES, "the gate's scratch fits the item LDS");
        cab_gate_body<8>(p.gate, (float*)lds);
        __syncthreads();
    }
    if (p.with_se && wi == 0 && head == 0) {  // block-uniform
        static_assert(4 * SE_GATE_LDS <= X::LDS_BYTES, "the gate's scratch fits the item LDS");
        se_gate_body<8>(p.se, (float*)lds);
        __syncthreads();
    }
    unsigned short* Kp = (unsigned short*)lds;
    unsigned short* Vp = Kp + 3 * X::KPL;
    float* Tb = (float*)(Vp + 3 * X::VPL);
    u32x4 qb[2][3];
    int qpix;
    {
        typename S::vec ks[S::NE], vs[S::NE];
        attn_fetch<D, false>(p, wi, head, ks, vs);
        AttnTableRegs<D, false> tr;
        attn_table_load<D, false>(p, head, tr);
        qpix = attnx_query<D>(p, wi, head, qb);
        attnx_stash<D>(Kp, Vp, ks, vs);
        attn_table_store<D, false>(Tb, tr);
    }
    __syncthreads();
    if (p.shift > 0 && (wi / p.nx == p.ny - 1 || wi % p.nx == p.nx - 1))
        attnx_compute<D, true>(p, lds, wi, head, qb, qpix);
    else
        attnx_compute<D, false>(p, lds, wi, head, qb, qpix);
}

// ---------------------------------------------------------------------------
// OCA (overlapping cross-attention: 576 keys of the 24x24 unfold with padding
// 4, zero outside the plane, biased and unmasked; hat_arch.py:373-427,
// cpu.rs:852-900), one (window, head) item per block. The three-plane K and
// V^T of 576 keys would need 177 KB of LDS, so an item runs as parts of NK
// keys (D = 24: three of 192, key rows 0-7, 8-15, 16-23; D = 30: six of 96)
// that share the online softmax; each part is split into LDS between two
// barriers and computed, and the next part's fetch into registers is issued
// before the computing, so that its latency runs under this part's tiles. At
// most 80 KB of LDS and 128 VGPRs, so that two blocks share a CU and one's
// staging overlaps the other's MFMAs.

// SW: the same part-wise staging for shifted-window attention (256 keys of the
// rolled window, the shift mask on the last window row and column, the 961-row
// table), which head_dim 30 needs for two blocks per CU: its whole item, K and
// V^T in three planes, takes 114 KB of LDS, two parts of 128 keys 60 KB.
template <int D, int NK, bool SW = false>
struct AttnXOcaShape {
    static constexpr int NKEYS = SW ? 256 : 576;
    static_assert(NKEYS % NK == 0 && NK % 32 == 0, "whole 32-key tiles, whole parts");
    static constexpr int NPART = NKEYS / NK;
    static constexpr int KS = D == 24 ? 24 : 40;
    static constexpr int VS = NK + 8;                 // V^T row stride: 16 rows of a phase on distinct banks
    static constexpr int KPL = NK * KS, VPL = (D + 1) * VS;
    static constexpr int TROWS = SW ? 961 : 1521;
    static constexpr int LDS_BYTES = 2 * 3 * (KPL + VPL) + 4 * TROWS;
    static constexpr int U = D % 4 == 0 ? 4 : 2;       // floats per staging unit
    static constexpr int NE = (NK * D / U + 511) / 512;
    using vec = typename pick_t<U == 4, float4, float2>::type;
};

// This thread's share of part `part` of item (wi, head): K and V units.
template <int D, int NK, bool SW = false>
__device__ __forceinline__ void attnx_oca_fetch(const AttnArgs& p, int wi, int head, int part,
                                                typename AttnXOcaShape<D, NK, SW>::vec (&ks)[AttnXOcaShape<D, NK, SW>::NE],
                                                typename AttnXOcaShape<D, NK, SW>::vec (&vs)[AttnXOcaShape<D, NK, SW>::NE])
{
    using X = AttnXOcaShape<D, NK, SW>;
    using vec = typename X::vec;
    constexpr int PER_KEY = D / X::U;
    const float* Kg = p.qkv + (size_t)(p.heads + head) * p.T * D;
    const float* Vg = p.qkv + (size_t)(2 * p.heads + head) * p.T * D;
#pragma unroll
    for (int i = 0; i < X::NE; ++i) {
        const int e = threadIdx.x + i * 512;
        vec kv{}, vv{};
        if (e < NK * PER_KEY) {
            const int kl = e / PER_KEY, d = (e - kl * PER_KEY) * X::U;
            const int pix = attn_key_pixel<!SW>(p, wi, part * NK + kl);
            if (pix >= 0) {
                kv = *(const vec*)(Kg + (size_t)pix * D + d);
                vv = *(const vec*)(Vg + (size_t)pix * D + d);
            }
        }
        ks[i] = kv;
        vs[i] = vv;
    }
}

template <int D, int NK, bool SW = false>
__device__ __forceinline__ void attnx_oca_stash(unsigned short* Kp, unsigned short* Vp,
                                                const typename AttnXOcaShape<D, NK, SW>::vec (&ks)[AttnXOcaShape<D, NK, SW>::NE],
                                                const typename AttnXOcaShape<D, NK, SW>::vec (&vs)[AttnXOcaShape<D, NK, SW>::NE])
{
    using X = AttnXOcaShape<D, NK, SW>;
    constexpr int PER_KEY = D / X::U;
#pragma unroll
    for (int i = 0; i < X::NE; ++i) {
        const int e = threadIdx.x + i * 512;
        if (e < NK * PER_KEY) {
            const int k = e / PER_KEY, d = (e - k * PER_KEY) * X::U;
            float kv[4], vv[4];
            if constexpr (X::U == 4) {
                kv[0] = ks[i].x, kv[1] = ks[i].y, kv[2] = ks[i].z, kv[3] = ks[i].w;
                vv[0] = vs[i].x, vv[1] = vs[i].y, vv[2] = vs[i].z, vv[3] = vs[i].w;
            } else {
                kv[0] = ks[i].x, kv[1] = ks[i].y, kv[2] = kv[3] = 0.f;
                vv[0] = vs[i].x, vv[1] = vs[i].y, vv[2] = vv[3] = 0.f;
            }
            const int pos = vpos(k);
#pragma unroll
            for (int j = 0; j < X::U; j += 2) {
                unsigned k0, k1, k2, v0, v1, v2;
                split3_pk(kv[j], kv[j + 1], k0, k1, k2);
                *(unsigned*)(Kp + 0 * X::KPL + k * X::KS + d + j) = k0;
                *(unsigned*)(Kp + 1 * X::KPL + k * X::KS + d + j) = k1;
                *(unsigned*)(Kp + 2 * X::KPL + k * X::KS + d + j) = k2;
                split3_pk(vv[j], vv[j + 1], v0, v1, v2);
                Vp[0 * X::VPL + (d + j) * X::VS + pos] = (unsigned short)v0;
                Vp[0 * X::VPL + (d + j + 1) * X::VS + pos] = (unsigned short)(v0 >> 16);
                Vp[1 * X::VPL + (d + j) * X::VS + pos] = (unsigned short)v1;
                Vp[1 * X::VPL + (d + j + 1) * X::VS + pos] = (unsigned short)(v1 >> 16);
                Vp[2 * X::VPL + (d + j) * X::VS + pos] = (unsigned short)v2;
                Vp[2 * X::VPL + (d + j + 1) * X::VS + pos] = (unsigned short)(v2 >> 16);
            }
        }
    }
}

// One part's key tiles onto the running (o, mrun) of the item; SAFE as in
// attnx_tiles (without it the base stays 0 and mrun is not used).
template <int D, int NK, bool SAFE>
__device__ __forceinline__ void attnx_oca_compute(const unsigned char* lds, int part, const u32x4 (&qb)[2][3],
                                                  f32x16& o, float& mrun)
{
    using X = AttnXOcaShape<D, NK>;
    constexpr int NKT = NK / 32;
    const unsigned short* Kp = (const unsigned short*)lds;
    const unsigned short* Vp = Kp + 3 * X::KPL;
    const float* Tb = (const float*)(Vp + 3 * X::VPL);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in a scalar register
    const int ql = lane & 31, h = lane >> 5;
    const int q = wave * 32 + ql;
    const int qy = q >> 4, qx = q & 15;
    // idx = (ky*39 + kx) - (qy*39 + qx) + 600 on the rotated table (attn.hip)
    const int oca_base = 600 - (qy * 39 + qx);
    const unsigned short* vrow = Vp + (ql < D ? ql : D) * X::VS + 8 * h;
    AttnxKRows<D, X::KS, X::KPL> kr;
    kr.init(Kp, ql, h);
#pragma unroll 1
    for (int kt = 0; kt < NKT; ++kt) {
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int key = part * NK + kt * 32 + (i >> 2) * 8 + (i & 3) + 4 * h;
            const int ky = (int)((unsigned)key / 24u);
            s[i] = Tb[oca_base + key + 15 * ky];
        }
        s = kr.qk(kt * 32 * X::KS, qb, s);
        if constexpr (SAFE) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
            if ((part == 0 && kt == 0) || __any(mx > mrun + 8.0f)) {  // wave-uniform
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float mnew = fmaxf(mrun, mx);
                const float corr = fast_exp2(mrun - mnew);
#pragma unroll
                for (int i = 0; i < 16; ++i) o[i] *= corr;
                mrun = mnew;
            }
        }
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            float pv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) pv[j] = fast_exp2(SAFE ? s[8 * st + j] - mrun : s[8 * st + j]);
            u32x4 pb[3], va[3];
            split3_x8(pv, pb);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) va[pl] = *(const u32x4*)(vrow + pl * X::VPL + kt * 32 + 16 * st);
            o = mfma6(va, pb, o);
        }
    }
}

// One part of a shifted-window item (the SW form of attnx_oca_compute): the
// keys part * NK .. + NK - 1 of the rolled window, bias and mask as attnx_tiles.
template <int D, int NK, bool SAFE, bool MASKED>
__device__ __forceinline__ void attnx_swp_compute(const AttnArgs& p, const unsigned char* lds, int wi, int part,
                                                  const u32x4 (&qb)[2][3], f32x16& o, float& mrun)
{
    using X = AttnXOcaShape<D, NK, true>;
    constexpr int NKT = NK / 32;
    static_assert(NK % 16 == 0, "parts of whole window rows");
    const unsigned short* Kp = (const unsigned short*)lds;
    const unsigned short* Vp = Kp + 3 * X::KPL;
    const float* Tb = (const float*)(Vp + 3 * X::VPL);
    const int wy = wi / p.nx, wx = wi - (wi / p.nx) * p.nx;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in a scalar register
    const int ql = lane & 31, h = lane >> 5;
    const int q = wave * 32 + ql;
    const int qy = q >> 4, qx = q & 15;
    // the part's first key row: NK / 16 rows of 31 table entries each
    const float* Tr = Tb + 960 - ((qy + 15) * 31 + qx + 15 - 4 * h) + part * (NK / 16) * 31;
    const float NEG = -100.0f * HAT_LOG2E;
    const bool mrow = MASKED && wy == p.ny - 1;
    const bool mcol = MASKED && wx == p.nx - 1;
    const bool r_lo = mrow && (qy & 8), r_hi = mrow && !(qy & 8);
    const bool c_lo = mcol && (qx & 8), c_hi = mcol && !(qx & 8);
    const float madd[2][2] = {{(r_lo || c_lo) ? NEG : 0.0f, (r_lo || c_hi) ? NEG : 0.0f},
                              {(r_hi || c_lo) ? NEG : 0.0f, (r_hi || c_hi) ? NEG : 0.0f}};
    const unsigned short* vrow = Vp + (ql < D ? ql : D) * X::VS + 8 * h;
    AttnxKRows<D, X::KS, X::KPL> kr;
    kr.init(Kp, ql, h);
#pragma unroll 1
    for (int kt = 0; kt < NKT; ++kt) {
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kl = kt * 32 + (i >> 2) * 8 + (i & 3);  // key within the part (lane half 0)
            const int ky = kl >> 4, kx = kl & 15;
            float b = Tr[ky * 31 + kx];
            // the mask's row band: the key row within the window, part * NK / 16 + ky
            if (MASKED) b += madd[((part * (NK / 16) + ky) >> 3) & 1][(kx >> 3) & 1];
            s[i] = b;
        }
        s = kr.qk(kt * 32 * X::KS, qb, s);
        if constexpr (SAFE) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
            if ((part == 0 && kt == 0) || __any(mx > mrun + 8.0f)) {  // wave-uniform
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float mnew = fmaxf(mrun, mx);
                const float corr = fast_exp2(mrun - mnew);
#pragma unroll
                for (int i = 0; i < 16; ++i) o[i] *= corr;
                mrun = mnew;
            }
        }
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            float pv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) pv[j] = fast_exp2(SAFE ? s[8 * st + j] - mrun : s[8 * st + j]);
            u32x4 pb[3], va[3];
            split3_x8(pv, pb);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) va[pl] = *(const u32x4*)(vrow + pl * X::VPL + kt * 32 + 16 * st);
            o = mfma6(va, pb, o);
        }
    }
}

template <int D, int NK, bool SW = false>
__device__ __forceinline__ void attnx_oca_kernel(const AttnArgs& p, unsigned char* lds)
{
    using X = AttnXOcaShape<D, NK, SW>;
    const int wi = blockIdx.x, head = blockIdx.y;
    // SW: the windows of the last row and column of a shifted grid carry the mask
    const bool masked = SW && p.shift > 0 && (wi / p.nx == p.ny - 1 || wi % p.nx == p.nx - 1);  // block-uniform
    if constexpr (SW) {
        // the CAB's gates ride on the SW launch, in its first block, as in
        // attnx_item_kernel
        if (p.with_gate && wi == 0 && head == 0) {  // block-uniform
            static_assert(4 * CAB_GATE_LDS <= X::LDS_BYTES, "the gate's scratch fits the item LDS");
            cab_gate_body<8>(p.gate, (float*)lds);
            __syncthreads();
        }
        if (p.with_se && wi == 0 && head == 0) {  // block-uniform
            static_assert(4 * SE_GATE_LDS <= X::LDS_BYTES, "the gate's scratch fits the item LDS");
            se_gate_body<8>(p.se, (float*)lds);
            __syncthreads();
        }
    }
    unsigned short* Kp = (unsigned short*)lds;
    unsigned short* Vp = Kp + 3 * X::KPL;
    float* Tb = (float*)(Vp + 3 * X::VPL);
    // Written once (no part's staging touches them): row D of V^T (ones in the
    // high plane), K dims 30, 31 (D = 30).
    for (int e = threadIdx.x; e < 3 * (NK / 2); e += 512) {
        const int pl = e / (NK / 2), k2 = e - pl * (NK / 2);
        *(unsigned*)(Vp + pl * X::VPL + D * X::VS + 2 * k2) = pl == 0 ? 0x3f803f80u : 0u;
    }
    if (D == 30) {
        for (int e = threadIdx.x; e < 3 * NK; e += 512) {
            const int pl = e / NK, k = e - pl * NK;
            *(unsigned*)(Kp + pl * X::KPL + k * X::KS + 30) = 0u;
        }
    }
    const int lane = threadIdx.x & 63;
    const int ql = lane & 31, h = lane >> 5;
    constexpr int RH = (D % 8) / 4, RR = (D / 8) * 4 + D % 4;
    typename X::vec ks[X::NE], vs[X::NE];
    u32x4 qb[2][3];
    int qpix;
    {
        attnx_oca_fetch<D, NK, SW>(p, wi, head, 0, ks, vs);
        AttnTableRegs<D, !SW> tr;
        attn_table_load<D, !SW>(p, head, tr);
        qpix = attnx_query<D>(p, wi, head, qb);
        attn_table_store<D, !SW>(Tb, tr);
    }
    f32x16 o;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = 0.0f;
    float mrun = 0.0f;
    // the base-0 pass (see attnx_tiles)
#pragma unroll 1
    for (int part = 0; part < X::NPART; ++part) {
        if (part > 0) __syncthreads();  // every read of the previous part's K and V is done
        attnx_oca_stash<D, NK, SW>(Kp, Vp, ks, vs);
        __syncthreads();
        // the next part's K and V in flight while this part's tiles run (the
        // registers are free once stashed; same-box: head_dim 30 SW 356 ->
        // 344 us, OCA 677 -> 661, head_dim 24 OCA 589 -> 585)
        if (part + 1 < X::NPART) attnx_oca_fetch<D, NK, SW>(p, wi, head, part + 1, ks, vs);
        if constexpr (SW) {
            if (masked) attnx_swp_compute<D, NK, false, true>(p, lds, wi, part, qb, o, mrun);
            else attnx_swp_compute<D, NK, false, false>(p, lds, wi, part, qb, o, mrun);
        } else {
            attnx_oca_compute<D, NK, false>(lds, part, qb, o, mrun);
        }

    }
    // The parts are staged by the whole block, so the block redoes the item
    // with the max-subtracted softmax if any of its waves needs it.
    __shared__ int item_ok[8];
    const bool ok = attnx_item_done<D>(o);
    if (lane == 0) item_ok[threadIdx.x >> 6] = ok;
    __syncthreads();  // also: every read of the last part's K and V is done
    bool all_ok = true;
#pragma unroll
    for (int w = 0; w < 8; ++w) all_ok = all_ok && item_ok[w];
    if (!all_ok) {  // block-uniform
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] = 0.0f;
        mrun = -INFINITY;
#pragma unroll 1
        for (int part = 0; part < X::NPART; ++part) {
            attnx_oca_fetch<D, NK, SW>(p, wi, head, part, ks, vs);
            if (part > 0) __syncthreads();  // every read of the previous part's K and V is done
            attnx_oca_stash<D, NK, SW>(Kp, Vp, ks, vs);
            __syncthreads();
            if constexpr (SW) {
                if (masked) attnx_swp_compute<D, NK, true, true>(p, lds, wi, part, qb, o, mrun);
                else attnx_swp_compute<D, NK, true, false>(p, lds, wi, part, qb, o, mrun);
            } else {
                attnx_oca_compute<D, NK, true>(lds, part, qb, o, mrun);
            }
        }
    }
    const float ltot = __shfl(o[RR], ql + 32 * RH, 64);
    const float inv = 1.0f / ltot;
    float* orow = p.out + (size_t)qpix * p.C + head * D;
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
        const int d0 = 8 * i4 + 4 * h;
        if (D % 4 == 0) {
            if (d0 + 3 < D)
                *(float4*)(orow + d0) = make_float4(o[i4 * 4] * inv, o[i4 * 4 + 1] * inv,
                                                    o[i4 * 4 + 2] * inv, o[i4 * 4 + 3] * inv);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (d0 + j < D) orow[d0 + j] = o[i4 * 4 + j] * inv;
        }
    }
}

#define ATTNX_OCA_INST(NAME, D, NK)                                                                 \
    extern "C" __global__ __launch_bounds__(512, 4) void NAME(AttnArgs p)                           \
    {                                                                                               \
        static_assert(AttnXOcaShape<D, NK>::LDS_BYTES <= 80 * 1024, "two blocks per CU");           \
        __shared__ __attribute__((aligned(16))) unsigned char lds[AttnXOcaShape<D, NK>::LDS_BYTES]; \
        attnx_oca_kernel<D, NK>(p, lds);                                                            \
    }

ATTNX_OCA_INST(hat_attnx_oca_d24, 24, 192)
ATTNX_OCA_INST(hat_attnx_oca_d30, 30, 96)

// Shifted-window attention for head_dim 30 in two parts of 128 keys (60 KB of
// LDS: two blocks per CU), the masked form for the windows of the last row
// and column of a shifted grid.
#define ATTNX_SWP_INST(NAME, D, NK)                                                                      \
    extern "C" __global__ __launch_bounds__(512, 4) void NAME(AttnArgs p)                                \
    {                                                                                                    \
        static_assert(AttnXOcaShape<D, NK, true>::LDS_BYTES <= 80 * 1024, "two blocks per CU");          \
        __shared__ __attribute__((aligned(16))) unsigned char lds[AttnXOcaShape<D, NK, true>::LDS_BYTES]; \
        attnx_oca_kernel<D, NK, true>(p, lds);                                                           \
    }

ATTNX_SWP_INST(hat_attnx_swp_d30, 30, 64)

#define ATTNX_INST(NAME, D, OCC)                                                             \
    extern "C" __global__ __launch_bounds__(512, OCC) void NAME(AttnArgs p)                  \
    {                                                                                        \
        __shared__ __attribute__((aligned(16))) unsigned char lds[AttnXShape<D>::LDS_BYTES]; \
        attnx_item_kernel<D>(p, lds);                                                        \
    }

ATTNX_INST(hat_attnx_sw_d24, 24, 4)
ATTNX_INST(hat_attnx_sw_d30, 30, 2)
