// Fused window attention on FP32 MFMA: QK^T + relative-position bias + shift
// mask + softmax + PV for one (window, head) per block.
//
// Replaces hat_attention_d24/_d30 (cuda/hat.cu:246-316) and, by folding them
// into its load/store addressing, the launches around it in the reference
// graph: lg_window_gather/lg_window_scatter with the cyclic roll (cuda.rs:
// 298-319, plan.rs:129-151), hat_bias_gather (hat.cu:98-112), hat_mask_build
// (hat.cu:137-152) and hat_unfold_kv (hat.cu:170-198). The arithmetic it
// reproduces is src/cpu.rs:772-844 (window_attention) and :852-900
// (overlap_attention):  s = (q.k)*scale + bias (+ mask), softmax, P.V.
//
// Two key sources:
//  * SW (OCA = false): the 256 tokens of a 16x16 window taken at a cyclic shift
//    (plan.rs:129-151); when shifted, the SW-MSA mask of the reference's
//    calculate_mask (hat_arch.py:921-940) is applied as -100 between tokens of
//    different regions. Only the last window row/column straddles regions, and
//    there the region of a token is its (y >= 8, x >= 8) half, so the mask is
//    two bit compares per score.
//  * OCA (OCA = true): the 24x24 nn.Unfold(24, stride 16, padding 4) window of
//    keys (hat_arch.py:373-410); keys outside the plane are zero and keep their
//    bias (they are not masked: hat_arch.py:419-427, cpu.rs:866-875).
//
// Work split: 512 threads = 8 waves, wave w owns queries [32w, 32w+32). The
// scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x2_f32: the
// A operand is a 32-key tile of K from LDS, the B operand the wave's 32 queries
// held in registers. Lane l owns query l%32 and, per 32-key tile, 16 of its
// scores: exactly the B operand of the next product O^T += V^T P^T, so the
// probabilities never leave registers. V^T is staged in LDS so that a lane's
// four consecutive keys are one float4 read. The dot-product dimension is
// split between the two lane halves: half h reduces dims [h*D/2, (h+1)*D/2),
// so D = 24 and D = 30 both need no padding in QK^T.
//
// Softmax is computed in base 2 (q pre-scaled by scale*log2(e), the bias table
// by log2(e)) over key chunks with a running base that is raised only when a
// score exceeds it by more than 2^8; after the division by the sum this equals
// the reference's row max subtraction up to rounding.
#include "common.h"

using namespace hatk;

template <bool B, class T, class F>
struct pick_t {
    using type = T;
};
template <class T, class F>
struct pick_t<false, T, F> {
    using type = F;
};

template <int D, bool OCA>
struct AttnShape {
    static constexpr int HALF = D / 2;                 // dims per lane half
    static constexpr int HP = (HALF + 3) / 4 * 4;      // LDS offset of the second half
    static constexpr int RSK = 2 * HP + 4;             // K row stride in LDS (floats)
    static constexpr int NK = OCA ? 576 : 256;         // keys per window
    static constexpr int RSV = NK + 4;                 // V^T row stride in LDS
    static constexpr int TROWS = OCA ? 1521 : 961;     // bias table rows
    static constexpr int LDS = NK * RSK + 32 * RSV + TROWS;  // floats
    // K and V move global -> registers -> LDS in units of U floats (float4 for
    // D = 24, float2 for D = 30), NE units of each per thread.
    static constexpr int U = D % 4 == 0 ? 4 : 2;
    static constexpr int NE = (NK * D / U + 511) / 512;
    using vec = typename pick_t<U == 4, float4, float2>::type;
};

// Pixel of key k of window wi (SW: the window at the cyclic shift, plan.rs:
// 129-151; OCA: the 24x24 unfold with padding 4, -1 outside the plane).
template <bool OCA>
__device__ __forceinline__ int attn_key_pixel(const AttnArgs& p, int wi, int k)
{
    const int wy = wi / p.nx, wx = wi - (wi / p.nx) * p.nx;
    if (OCA) {
        const int ky = k / 24, kx = k - (k / 24) * 24;
        const int y = wy * 16 - 4 + ky, x = wx * 16 - 4 + kx;
        return (y >= 0 && y < p.hp && x >= 0 && x < p.wp) ? y * p.wp + x : -1;
    }
    int y = wy * 16 + (k >> 4) + p.shift, x = wx * 16 + (k & 15) + p.shift;
    if (y >= p.hp) y -= p.hp;
    if (x >= p.wp) x -= p.wp;
    return y * p.wp + x;
}

// This thread's share of item (wi, head)'s K and V, into registers.
template <int D, bool OCA>
__device__ __forceinline__ void attn_fetch(const AttnArgs& p, int wi, int head,
                                           typename AttnShape<D, OCA>::vec (&ks)[AttnShape<D, OCA>::NE],
                                           typename AttnShape<D, OCA>::vec (&vs)[AttnShape<D, OCA>::NE])
{
    using S = AttnShape<D, OCA>;
    using vec = typename S::vec;
    constexpr int PER_KEY = D / S::U;
    const float* Kg = p.qkv + (size_t)(p.heads + head) * p.T * D;
    const float* Vg = p.qkv + (size_t)(2 * p.heads + head) * p.T * D;
#pragma unroll
    for (int i = 0; i < S::NE; ++i) {
        const int e = threadIdx.x + i * 512;
        vec kv{}, vv{};
        if (e < S::NK * PER_KEY) {
            const int k = e / PER_KEY, d = (e - k * PER_KEY) * S::U;
            const int pix = attn_key_pixel<OCA>(p, wi, k);
            if (pix >= 0) {
                if (OCA) {
                    kv = *(const vec*)(Kg + (size_t)pix * D + d);
                    vv = *(const vec*)(Vg + (size_t)pix * D + d);
                } else if constexpr (S::U == 4) {
                    // SW: this item is the only reader of these keys and values;
                    // non-temporal loads leave the last-level cache to the
                    // attention output and residual the next kernel reads
                    const f32x4 a = __builtin_nontemporal_load((const f32x4*)(Kg + (size_t)pix * D + d));
                    const f32x4 b = __builtin_nontemporal_load((const f32x4*)(Vg + (size_t)pix * D + d));
                    kv = make_float4(a[0], a[1], a[2], a[3]);
                    vv = make_float4(b[0], b[1], b[2], b[3]);
                } else {
                    kv = *(const vec*)(Kg + (size_t)pix * D + d);
                    vv = *(const vec*)(Vg + (size_t)pix * D + d);
                }
            }
        }
        ks[i] = kv;
        vs[i] = vv;
    }
}

// The registers of attn_fetch into LDS: K row-major with the head_dim halves
// at 0 and HP, V transposed.
template <int D, bool OCA>
__device__ __forceinline__ void attn_stash(float* Kl, float* Vt,
                                           const typename AttnShape<D, OCA>::vec (&ks)[AttnShape<D, OCA>::NE],
                                           const typename AttnShape<D, OCA>::vec (&vs)[AttnShape<D, OCA>::NE])
{
    using S = AttnShape<D, OCA>;
    constexpr int PER_KEY = D / S::U;
#pragma unroll
    for (int i = 0; i < S::NE; ++i) {
        const int e = threadIdx.x + i * 512;
        if (e < S::NK * PER_KEY) {
            const int k = e / PER_KEY, d = (e - k * PER_KEY) * S::U;
            if constexpr (S::U == 4) {
                static_assert(S::HP == S::HALF, "float4 rows need no gap between the halves");
                *(float4*)(Kl + k * S::RSK + d) = ks[i];
                Vt[(d + 0) * S::RSV + k] = vs[i].x;
                Vt[(d + 1) * S::RSV + k] = vs[i].y;
                Vt[(d + 2) * S::RSV + k] = vs[i].z;
                Vt[(d + 3) * S::RSV + k] = vs[i].w;
            } else {
                Kl[k * S::RSK + (d < S::HALF ? d : S::HP + d - S::HALF)] = ks[i].x;
                Kl[k * S::RSK + (d + 1 < S::HALF ? d + 1 : S::HP + d + 1 - S::HALF)] = ks[i].y;
                Vt[(d + 0) * S::RSV + k] = vs[i].x;
                Vt[(d + 1) * S::RSV + k] = vs[i].y;
            }
        }
    }
}

// Bias table of a head, in log2 units. For OCA the table is stored rotated so
// that the reference's negative-index wrap (plan.rs:397-416) becomes a plain
// offset: Tb[j] = table[(j - 880) mod 1521]. For SW it is stored reversed,
// Tb[j] = table[960 - j], so that consecutive keys of a row read ascending
// consecutive entries (straight into consecutive accumulator registers).
template <int D, bool OCA>
__device__ __forceinline__ void attn_table(const AttnArgs& p, float* Tb, int head)
{
    for (int i = threadIdx.x; i < AttnShape<D, OCA>::TROWS; i += 512) {
        int row = 960 - i;
        if (OCA) {
            row = i - 880;
            if (row < 0) row += 1521;
        }
        Tb[i] = p.table[(size_t)row * p.heads + head] * HAT_LOG2E;
    }
}

// attn_table in two steps, so that its loads can be in flight together with
// the item's other loads: this thread's entries into registers, then into LDS.
template <int D, bool OCA>
struct AttnTableRegs {
    static constexpr int N = (AttnShape<D, OCA>::TROWS + 511) / 512;
    float v[N];
};
template <int D, bool OCA>
__device__ __forceinline__ void attn_table_load(const AttnArgs& p, int head, AttnTableRegs<D, OCA>& t)
{
#pragma unroll
    for (int j = 0; j < AttnTableRegs<D, OCA>::N; ++j) {
        const int i = threadIdx.x + 512 * j;
        int row = 960 - i;
        if (OCA) {
            row = i - 880;
            if (row < 0) row += 1521;
        }
        const bool ok = i < AttnShape<D, OCA>::TROWS;
        t.v[j] = p.table[(size_t)(ok ? row : 0) * p.heads + head];
    }
}
template <int D, bool OCA>
__device__ __forceinline__ void attn_table_store(float* Tb, const AttnTableRegs<D, OCA>& t)
{
#pragma unroll
    for (int j = 0; j < AttnTableRegs<D, OCA>::N; ++j) {
        const int i = threadIdx.x + 512 * j;
        if (i < AttnShape<D, OCA>::TROWS) Tb[i] = t.v[j] * HAT_LOG2E;
    }
}

// This lane's query of item (wi, head): its pixel and its half of q, as
// stored (the caller scales it by head_dim^-0.5 * log2(e) where it is used:
// scaling here would make the persistent kernel wait for the loads, and with
// them for the next item's K and V, before the current item's work).
template <int D>
__device__ __forceinline__ int attn_query(const AttnArgs& p, int wi, int head, float (&qv)[D / 2], bool oca)
{
    constexpr int HALF = D / 2;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ql = lane & 31, h = lane >> 5;
    const int q = wave * 32 + ql, qy = q >> 4, qx = q & 15;
    const int wy = wi / p.nx, wx = wi - (wi / p.nx) * p.nx;
    const int shift = oca ? 0 : p.shift;
    int y = wy * 16 + qy + shift, x = wx * 16 + qx + shift;
    if (y >= p.hp) y -= p.hp;
    if (x >= p.wp) x -= p.wp;
    const int qpix = y * p.wp + x;
    const float* Qg = p.qkv + (size_t)head * p.T * D + (size_t)qpix * D + h * HALF;
    if constexpr (HALF % 4 == 0) {
#pragma unroll
        for (int s4 = 0; s4 < HALF; s4 += 4) {
            const float4 v = *(const float4*)(Qg + s4);
            qv[s4] = v.x;
            qv[s4 + 1] = v.y;
            qv[s4 + 2] = v.z;
            qv[s4 + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < HALF; ++s) qv[s] = Qg[s];
    }
    return qpix;
}

// The attention of one staged item. MASKED: the window is in the last row or
// column of a shifted SW grid, so its scores get the region mask; every other
// window runs the loop without it.
template <int D, bool OCA, bool MASKED>
__device__ __forceinline__ void attn_compute(const AttnArgs& p, const float* lds, int wi, int head,
                                             const float (&qv)[D / 2], int qpix)
{
    using S = AttnShape<D, OCA>;
    constexpr int HALF = S::HALF, HP = S::HP, RSK = S::RSK, NK = S::NK, RSV = S::RSV;
    constexpr int NKT = NK / 32;                // 32-key tiles
    constexpr int CHT = OCA ? 3 : 1;            // tiles per softmax chunk
    constexpr int NCH = NKT / CHT;
    static_assert(NKT % CHT == 0, "chunking");

    const float* Kl = lds;                      // [NK][RSK]
    const float* Vt = Kl + NK * RSK;            // [32][RSV]: V^T, then row D ones, rows D+1.. zeros
    const float* Tb = Vt + 32 * RSV;            // [TROWS]

    const int wy = wi / p.nx, wx = wi - (wi / p.nx) * p.nx;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ql = lane & 31, h = lane >> 5;
    const int q = wave * 32 + ql;
    const int qy = q >> 4, qx = q & 15;

    // Bias addressing. SW: idx = (qy-ky+15)*31 + (qx-kx+15) = sw_base - (ky*31+kx),
    // entry 960 - idx = sw_rbase + (ky*31+kx) of the reversed table.
    // OCA: idx = (ky*39+kx) - (qy*39+qx) + 600 on the rotated table.
    const int sw_rbase = 960 - ((qy + 15) * 31 + qx + 15 - 4 * h);
    const int oca_base = 600 - (qy * 39 + qx);
    // Mask addends (SW, shifted): a key differs in region from the query when
    // its half (bit 3 of y or x) differs, in the last window row / column.
    const float NEG = -100.0f * HAT_LOG2E;
    const bool mrow = MASKED && wy == p.ny - 1;
    const bool mcol = MASKED && wx == p.nx - 1;
    const bool r_lo = mrow && (qy & 8), r_hi = mrow && !(qy & 8);
    const bool c_lo = mcol && (qx & 8), c_hi = mcol && !(qx & 8);
    const float madd[2][2] = {{(r_lo || c_lo) ? NEG : 0.0f, (r_lo || c_hi) ? NEG : 0.0f},
                              {(r_hi || c_lo) ? NEG : 0.0f, (r_hi || c_hi) ? NEG : 0.0f}};

    // Row D of the 32-row V^T tile is padding; it holds ones, so row D of
    // O^T accumulates the softmax denominator sum_k P[k][q] - rescaled along
    // with the rest of O - inside the PV products. In the MFMA output layout
    // it is register RR of lane half RH.
    static_assert(D < 32, "a spare V^T row is needed");
    constexpr int RH = (D % 8) / 4, RR = (D / 8) * 4 + D % 4;

    f32x16 o;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = 0.0f;
    float mrun = -INFINITY;

    // The chunk loop stays rolled: unrolled, the compiler hoists the K operand
    // reads of every key tile ahead of the MFMAs and spills.
#pragma unroll 1
    for (int ch = 0; ch < NCH; ++ch) {
        f32x16 s[CHT];
#pragma unroll
        for (int t = 0; t < CHT; ++t) {
            const int kt = ch * CHT + t;
            const float* kp = Kl + (kt * 32 + ql) * RSK + h * HP;
            // The scores accumulate onto their bias (+ mask): S = bias + K Q^T.
            f32x16 a;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key0 = kt * 32 + (i >> 2) * 8 + (i & 3);  // key for h = 0
                float b;
                if (OCA) {
                    // (ky*39 + kx) = key + 15*ky for a 24-wide key grid
                    const int key = key0 + 4 * h;
                    const int ky = (int)((unsigned)key / 24u);
                    b = Tb[oca_base + key + 15 * ky];
                } else {
                    const int ky = key0 >> 4, kx = key0 & 15;
                    b = Tb[sw_rbase + (ky * 31 + kx)];
                    if (MASKED) b += madd[(ky >> 3) & 1][(kx >> 3) & 1];
                }
                a[i] = b;
            }
#pragma unroll
            for (int st = 0; st < HALF; ++st) a = mfma32(kp[st], qv[st], a);
            s[t] = a;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < CHT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[t][i]);
        // Lazy rescaling: the exponent base mrun (shared by the two lane halves
        // of a query) is raised only in the first chunk or when a score of the
        // wave exceeds it by more than 8 (log2 units: probabilities stay below
        // 2^8, sums below 2^16); the final division by the accumulated sum
        // makes the result independent of the base.
        if (ch == 0 || __any(mx > mrun + 8.0f)) {  // wave-uniform
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(mrun, mx);
            const float corr = fast_exp2(mrun - mnew);
#pragma unroll
            for (int i = 0; i < 16; ++i) o[i] *= corr;
            mrun = mnew;
        }
#pragma unroll
        for (int t = 0; t < CHT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[t][i] = fast_exp2(s[t][i] - mrun);
        // O^T += V^T P^T
#pragma unroll
        for (int t = 0; t < CHT; ++t) {
            const int kt = ch * CHT + t;
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                // The padding rows come from LDS for OCA; for SW (more blocks per
                // CU, LDS-bound in this phase) the idle lanes skip the read.
                f32x4 vv;
                if (OCA || ql < D) vv = *(const f32x4*)(Vt + ql * RSV + kt * 32 + i4 * 8 + h * 4);
                else vv = ql == D ? (f32x4){1.f, 1.f, 1.f, 1.f} : (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) o = mfma32(vv[j], s[t][i4 * 4 + j], o);
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

// One (window, head) per block (grid nw x heads). SW runs 4 waves per SIMD (2
// blocks per CU, <= 128 VGPRs), so one block's K/V staging overlaps the
// other's MFMA work; its V^T padding rows are not read (the idle lanes
// substitute them). OCA with head_dim 30 also runs this way (its staging
// registers do not fit the persistent form).
template <int D, bool OCA>
__device__ __forceinline__ void attn_item_kernel(const AttnArgs& p, float* lds)
{
    using S = AttnShape<D, OCA>;
    float* Vt = lds + S::NK * S::RSK;
    const int wi = blockIdx.x, head = blockIdx.y;
    if (!OCA && p.with_gate && wi == 0 && head == 0) {  // block-uniform
        // The CAB gate rides in this launch's first block: one block of work
        // that would otherwise hold the whole GPU for a launch of its own.
        static_assert(CAB_GATE_LDS <= S::LDS, "the gate's scratch fits the item LDS");
        cab_gate_body<8>(p.gate, lds);
        __syncthreads();  // the LDS is the item's next
    }
    if (!OCA && p.with_se && wi == 0 && head == 0) {  // block-uniform; the unfolded CAB's gate
        static_assert(SE_GATE_LDS <= S::LDS, "the gate's scratch fits the item LDS");
        se_gate_body<8>(p.se, lds);
        __syncthreads();
    }
    // Every load of the item (K, V, the bias table, q) is issued before any
    // of them is waited for.
    float qv[D / 2];
    int qpix;
    {
        typename S::vec ks[S::NE], vs[S::NE];
        attn_fetch<D, OCA>(p, wi, head, ks, vs);
        AttnTableRegs<D, OCA> tr;
        attn_table_load<D, OCA>(p, head, tr);
        qpix = attn_query<D>(p, wi, head, qv, OCA);
        attn_stash<D, OCA>(lds, Vt, ks, vs);
        attn_table_store<D, OCA>(Vt + 32 * S::RSV, tr);
    }
    if (OCA) {
        // V^T rows past D: row D all ones (it sums the probabilities), the rest zero.
        for (int e = threadIdx.x; e < (32 - D) * S::NK; e += 512) {
            const int r = D + e / S::NK, k = e - (e / S::NK) * S::NK;
            Vt[r * S::RSV + k] = r == D ? 1.0f : 0.0f;
        }
    }
#pragma unroll
    for (int s = 0; s < D / 2; ++s) qv[s] *= p.qscale;
    __syncthreads();
    if (!OCA && p.shift > 0 && (wi / p.nx == p.ny - 1 || wi % p.nx == p.nx - 1))
        attn_compute<D, OCA, true>(p, lds, wi, head, qv, qpix);
    else
        attn_compute<D, OCA, false>(p, lds, wi, head, qv, qpix);
}

// OCA, head_dim 24: the LDS holds one block per CU, so the kernel is
// persistent (grid: one block per CU at most) over the (window, head) items, head-major (a block's consecutive items mostly share
// the bias table): the next item's K, V and q travel through registers while
// this item computes, and go to LDS between two barriers.
template <int D, bool OCA>
__device__ __forceinline__ void attn_persistent_kernel(const AttnArgs& p, float* lds)
{
    using S = AttnShape<D, OCA>;
    float* Kl = lds;
    float* Vt = Kl + S::NK * S::RSK;
    float* Tb = Vt + 32 * S::RSV;
    const int nw = p.nx * p.ny, nitems = nw * p.heads;
    int item = blockIdx.x;
    if (item >= nitems) return;  // whole block, before any barrier
    if (OCA) {
        // V^T rows past D: row D all ones (it sums the probabilities), the rest zero.
        for (int e = threadIdx.x; e < (32 - D) * S::NK; e += 512) {
            const int r = D + e / S::NK, k = e - (e / S::NK) * S::NK;
            Vt[r * S::RSV + k] = r == D ? 1.0f : 0.0f;
        }
    }
    typename S::vec ks[S::NE], vs[S::NE];
    float qn[D / 2];
    int head = item / nw, wi = item - head * nw;
    attn_fetch<D, OCA>(p, wi, head, ks, vs);
    int qpix_n = attn_query<D>(p, wi, head, qn, OCA);
    int table_head = -1;
    while (true) {
        __syncthreads();  // every read of the previous item's LDS is done
        attn_stash<D, OCA>(Kl, Vt, ks, vs);
        if (head != table_head) {  // block-uniform
            attn_table<D, OCA>(p, Tb, head);
            table_head = head;
        }
        float qv[D / 2];
#pragma unroll
        for (int s = 0; s < D / 2; ++s) qv[s] = qn[s] * p.qscale;
        const int qpix = qpix_n;
        __syncthreads();
        const int next = item + gridDim.x;
        const int nhead = next / nw, nwi = next - nhead * nw;
        if (next < nitems) {
            attn_fetch<D, OCA>(p, nwi, nhead, ks, vs);
            qpix_n = attn_query<D>(p, nwi, nhead, qn, OCA);
        }
        if (!OCA && p.shift > 0 && (wi / p.nx == p.ny - 1 || wi % p.nx == p.nx - 1))
            attn_compute<D, OCA, true>(p, lds, wi, head, qv, qpix);
        else
            attn_compute<D, OCA, false>(p, lds, wi, head, qv, qpix);
        if (next >= nitems) break;
        item = next;
        head = nhead;
        wi = nwi;
    }
}

#define ATTN_INST(NAME, D, OCA)                                                              \
    extern "C" __global__ __launch_bounds__(512, OCA ? 2 : 4) void NAME(AttnArgs p)          \
    {                                                                                        \
        __shared__ __attribute__((aligned(16))) float lds[AttnShape<D, OCA>::LDS];           \
        if (attn_persistent(D, OCA))                                                         \
            attn_persistent_kernel<D, OCA>(p, lds);                                          \
        else                                                                                 \
            attn_item_kernel<D, OCA>(p, lds);                                                \
    }

ATTN_INST(hat_attn_sw_d24, 24, false)
ATTN_INST(hat_attn_sw_d30, 30, false)
ATTN_INST(hat_attn_oca_d24, 24, true)
ATTN_INST(hat_attn_oca_d30, 30, true)
