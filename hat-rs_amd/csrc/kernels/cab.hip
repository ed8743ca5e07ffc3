// The channel-attention block (CAB) of the compress-to-6 family (HAT-S):
//   CAB(x) = gate * conv2(gelu(conv1(x))),  gate = sigmoid(Wb relu(Wa mean_p conv2(..) + ba) + bb)
// (hat_arch.py CAB / ChannelAttention; cpu.rs cab, 1090-1120; the reference's
// GPU path runs it as lg_conv3x3 x2, a column mean and the squeeze-excite,
// src/cuda.rs:171-183, 201-214).
//
// conv2 is linear, so two of its three uses need no conv2 output at all:
//   * its pixel mean is b2 + (1/HW) sum_{tap,ci} w2[c][ci][tap] * S[tap][ci],
//     S[tap][ci] = sum of t1[.][ci] over the plane shifted by the tap (zero
//     padding): the whole-plane sum minus the row / column the shift pushes out,
//     plus the corner counted twice. hat_cab_conv1 leaves per-tile sums of t1
//     over the tile and over its pixels on the four border lines;
//   * gate[c] * conv2(t1)[p][c] * cscale is a GEMM of the 3x3 neighbourhood of
//     t1 at p (9 taps x 6 channels, k = tap*6 + ci) with weights cscale *
//     gate[c] * w2 - hat_cab_gate folds them, and the attention projection GEMM
//     (hat_gemmws_cab_ln) runs them as 56 more K.
// So conv2's T x 144 output is never written or read back.
#include "common.h"

using namespace hatk;

// ---------------------------------------------------------------------------
// conv1 (144 -> 6, 3x3, zero padding) + GELU on split-bf16 MFMA, one 16-wide,
// TY-tall output tile at a time: persistent over the tiles, one block of four
// waves per CU.
//
// Per-tap products: for each pixel q of the tile's 18 x (TY+2) halo,
// P[q][tap*6+co] = sum_ci xn[q][ci] * w[co][ci][tap] is a 144-deep product with
// 54 outputs (padded to 64): v_mfma_f32_32x32x16_bf16 with the 64 weight rows as
// A (two tiles of 32) and 32 halo pixels as B, nine 16-channel steps, every fp32
// operand as three bf16 parts and every product as the six terms of order <= 2
// (the arithmetic of the split-bf16 attention, as accurate as FP32 MFMA). The
// conv output at p is then the sum over the 9 taps of P[p + d(tap)][tap*6 + co],
// read from LDS in fp32. The split weights (216 registers a lane) stay in
// registers for the whole kernel, which takes the register file of one wave per
// SIMD. Each wave streams its 32-pixel halo tiles (TY = 32: 612 pixels in 20
// tiles, five a wave; TY = 16: 324 in 11), loading the next tile's 144 channels
// step by step while this one's MFMAs run, across the output tiles too: the
// barriers here wait for LDS only, so those loads stay in flight through them.
#define CX_WAVES 4
#define CX_HS 18  // halo width
#define CX_PS 60  // LDS row stride of P (56 written, 54 used): a b128 phase's 16 rows on distinct banks

template <int TY>
struct Cx1Shape {
    static constexpr int HY = TY + 2;
    static constexpr int HP = CX_HS * HY;      // halo pixels
    static constexpr int PT = (HP + 31) / 32;  // 32-pixel halo tiles
    static constexpr int NPW = (PT + CX_WAVES - 1) / CX_WAVES;  // per wave (past PT: zeros, not stored)
    static constexpr int NPX = TY / 16;        // output pixels per thread
    static_assert(16 * TY == CX_WAVES * 64 * NPX, "whole pixels per thread");
};

template <int TY>
__device__ __forceinline__ void cab_conv1_body(const CabConvArgs& p)
{
    using S = Cx1Shape<TY>;
    __shared__ __attribute__((aligned(16))) float Ps[S::HP * CX_PS];
    __shared__ float red[CX_WAVES][CAB_NSUM * CAB_CC];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int pl = lane & 31, h = lane >> 5;
    const int H = p.H, W = p.W;
    const int ntx = W / 16;
    const int ntiles = ntx * (H / TY);

    // The split weights go through LDS (the P region, free until the first
    // halo tile's stores) once per block, then into every wave's registers.
    constexpr int NWU = CX_WPACK / 8, WIT = (NWU + CX_WAVES * 64 - 1) / (CX_WAVES * 64);  // 16-byte units
    static_assert(NWU * 16 <= S::HP * CX_PS * 4, "the weights fit the P region");
    u32x4 stage[WIT];
#pragma unroll
    for (int i = 0; i < WIT; ++i) {
        const int e = min(tid + i * CX_WAVES * 64, NWU - 1);  // the last units again past the end
        stage[i] = ((const u32x4*)p.w)[e];
    }
    float bias[CAB_CC];
#pragma unroll
    for (int co = 0; co < CAB_CC; ++co) bias[co] = p.bias[co];

    // The lane's input row (channels 8h.. of each 16-channel step) for halo
    // tile i of output tile tl; hat_zero_row outside the plane, past the halo
    // and past the last tile, so that the loads are issued on every path.
    auto src_of = [&](int tl, int i) -> const float* {
        const int ty = tl / ntx, tx = tl - ty * ntx;
        const int hi = (wave + CX_WAVES * i) * 32 + pl;
        const int hy = hi / CX_HS, hx = hi - hy * CX_HS;
        const int gy = ty * TY - 1 + hy, gx = tx * 16 - 1 + hx;
        const bool valid = tl < ntiles && hi < S::HP && gy >= 0 && gy < H && gx >= 0 && gx < W;
        return valid ? p.xn + (size_t)(gy * W + gx) * CAB_C + 8 * h : hat_zero_row;
    };
    f32x4 xr[9][2];
    {
        const float* first = src_of(blockIdx.x, 0);
#pragma unroll
        for (int ks = 0; ks < 9; ++ks) {
            xr[ks][0] = *(const f32x4*)(first + ks * 16);
            xr[ks][1] = *(const f32x4*)(first + ks * 16 + 4);
        }
    }
#pragma unroll
    for (int i = 0; i < WIT; ++i) ((u32x4*)Ps)[min(tid + i * CX_WAVES * 64, NWU - 1)] = stage[i];
    lds_barrier();
    u32x4 wr[9][2][3];
#pragma unroll
    for (int ks = 0; ks < 9; ++ks)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int part = 0; part < 3; ++part)
                wr[ks][nt][part] = ((const u32x4*)Ps)[((ks * 2 + nt) * 3 + part) * 64 + lane];
    lds_barrier();  // every wave has its weights before P is written

    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int ty = tile / ntx, tx = tile - ty * ntx;
        const int y0 = ty * TY, x0 = tx * 16;
        // unrolled: with no back-edge here, the compiler's waits for the rows
        // read ahead are exact
#pragma unroll
        for (int i = 0; i < S::NPW; ++i) {
            const float* nxt = i + 1 < S::NPW ? src_of(tile, i + 1) : src_of(tile + gridDim.x, 0);
            f32x16 acc[2];
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[0][j] = acc[1][j] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 9; ++ks) {
                const float f[8] = {xr[ks][0][0], xr[ks][0][1], xr[ks][0][2], xr[ks][0][3],
                                    xr[ks][1][0], xr[ks][1][1], xr[ks][1][2], xr[ks][1][3]};
                u32x4 xb[3];
                split3_x8(f, xb);
                xr[ks][0] = *(const f32x4*)(nxt + ks * 16);  // step ks of the next halo tile
                xr[ks][1] = *(const f32x4*)(nxt + ks * 16 + 4);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) acc[nt] = mfma6(wr[ks][nt], xb, acc[nt]);
                __builtin_amdgcn_sched_barrier(0);  // the loads stay in their step
            }
            // lane (pl, h) holds P[hi][32 nt + 8 g + 4 h .. +3] in acc[nt][4g .. 4g+3];
            // columns 56.. (nt = 1, g = 3) are not stored
            const int hi = (wave + CX_WAVES * i) * 32 + pl;
            if (hi < S::HP) {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int g = 0; g < (nt == 0 ? 4 : 3); ++g)
                        *(f32x4*)(Ps + hi * CX_PS + 32 * nt + 8 * g + 4 * h) =
                            (f32x4){acc[nt][4 * g], acc[nt][4 * g + 1], acc[nt][4 * g + 2], acc[nt][4 * g + 3]};
            }
        }
        lds_barrier();  // P complete

        // The 9 taps from the halo products, NPX output pixels per thread
        // (rows oy, oy + 16).
        const int ox = tid & 15;
        float v[S::NPX][CAB_CC];
#pragma unroll
        for (int r = 0; r < S::NPX; ++r) {
            const int oy = (tid >> 4) + 16 * r;
#pragma unroll
            for (int co = 0; co < CAB_CC; ++co) v[r][co] = bias[co];
#pragma unroll
            for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) {
                    const float* q = Ps + ((oy + ky) * CX_HS + ox + kx) * CX_PS + (ky * 3 + kx) * CAB_CC;
#pragma unroll
                    for (int j = 0; j < CAB_CC / 2; ++j) {
                        const float2 t = *(const float2*)(q + 2 * j);
                        v[r][2 * j] += t.x;
                        v[r][2 * j + 1] += t.y;
                    }
                }
#pragma unroll
            for (int co = 0; co < CAB_CC; ++co) v[r][co] = gelu(v[r][co]);
            float* dst = p.t1 + ((size_t)(y0 + oy) * W + x0 + ox) * CAB_CS;
            *(float4*)dst = make_float4(v[r][0], v[r][1], v[r][2], v[r][3]);
            *(float4*)(dst + 4) = make_float4(v[r][4], v[r][5], 0.f, 0.f);
        }

        // Per-tile sums: the tile, and its pixels on row 0, row H-1, col 0,
        // col W-1 - only tiles on the plane's border have any of the latter.
        // A thread adds its pixels in row order, then the wave tree.
        const bool border = y0 == 0 || y0 + TY == H || x0 == 0 || x0 + 16 == W;  // tile-uniform
#pragma unroll
        for (int l = 0; l < CAB_NSUM; ++l) {
            if (l > 0 && !border) break;
#pragma unroll
            for (int co = 0; co < CAB_CC; ++co) {
                float s = 0.0f;
#pragma unroll
                for (int r = 0; r < S::NPX; ++r) {
                    const int gy = y0 + (tid >> 4) + 16 * r, gx = x0 + ox;
                    const bool on = l == 0 || (l == 1 && gy == 0) || (l == 2 && gy == H - 1) ||
                                    (l == 3 && gx == 0) || (l == 4 && gx == W - 1);
                    s += on ? v[r][co] : 0.0f;
                }
                s = wave_sum_dpp(s);
                if (lane == 0) red[wave][l * CAB_CC + co] = s;
            }
        }
        lds_barrier();
        if (tid < CAB_NSUM * CAB_CS) {
            const int l = tid / CAB_CS, co = tid - l * CAB_CS;
            float s = 0.0f;
            if (co < CAB_CC && (l == 0 || border)) {
                const int k = l * CAB_CC + co;
#pragma unroll
                for (int w = 0; w < CX_WAVES; ++w) s += red[w][k];  // waves in order
            }
            p.partial[(size_t)tid * ntiles + tile] = s;  // value-major: [40][tiles]
        }
        // The next tile's P stores come after this barrier; every read of Ps
        // and red above precedes it.
        lds_barrier();
    }
}

extern "C" __global__ __launch_bounds__(CX_WAVES * 64, 1) void hat_cab_conv1(CabConvArgs p)
{
    cab_conv1_body<16>(p);
}
extern "C" __global__ __launch_bounds__(CX_WAVES * 64, 1) void hat_cab_conv1_t32(CabConvArgs p)
{
    cab_conv1_body<32>(p);
}

// ---------------------------------------------------------------------------
// The gate, and conv2 folded with it: one block of 16 waves. Every reduction
// is a fixed-order per-lane sum followed by a fixed shuffle tree, so the
// result does not depend on timing.
#define CG_WAVES 16

// The gate computation for a block of WAVES waves; lds: CAB_GATE_LDS floats.
#define CAB_GATE_LDS (CAB_NSUM * CAB_CS + 9 * CAB_CC + CAB_C + 64 + CAB_C)
template <int WAVES>
__device__ __forceinline__ void cab_gate_body(const CabGateArgs& p, float* lds)
{
    constexpr int NV = CAB_NSUM * CAB_CS;  // 40 sums per tile
    float* s_sum = lds;
    float* s_S = s_sum + NV;
    float* s_mean = s_S + 9 * CAB_CC;
    float* s_z = s_mean + CAB_C;
    float* s_gate = s_z + 64;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;

    // Tile sums: partial is value-major, so a wave reads 64 tiles per load.
    for (int v = wave; v < NV; v += WAVES) {
        const float* src = p.partial + (size_t)v * p.tiles;
        float acc = 0.0f;
#pragma unroll 8
        for (int t = lane; t < p.tiles; t += 64) acc += src[t];
        acc = wave_sum(acc);
        if (lane == 0) s_sum[v] = acc;
    }
    __syncthreads();
    const int H = p.H, W = p.W;
    if (tid < 9 * CAB_CC) {
        const int tap = tid / CAB_CC, ci = tid - tap * CAB_CC;
        const int dy = tap / 3 - 1, dx = tap % 3 - 1;
        float s = s_sum[0 * CAB_CS + ci];
        if (dy == 1) s -= s_sum[1 * CAB_CS + ci];   // source rows 1 .. H-1: row 0 is out
        if (dy == -1) s -= s_sum[2 * CAB_CS + ci];  // rows 0 .. H-2: row H-1 is out
        if (dx == 1) s -= s_sum[3 * CAB_CS + ci];
        if (dx == -1) s -= s_sum[4 * CAB_CS + ci];
        if (dy != 0 && dx != 0)  // the corner both lines removed
            s += p.t1[((size_t)(dy == 1 ? 0 : H - 1) * W + (dx == 1 ? 0 : W - 1)) * CAB_CS + ci];
        s_S[tid] = s;
    }
    __syncthreads();
    const float inv = 1.0f / ((float)H * (float)W);
    for (int c = tid; c < CAB_C; c += WAVES * 64) {
        float acc = 0.0f;
#pragma unroll
        for (int ci = 0; ci < CAB_CC; ++ci)
#pragma unroll
            for (int tap = 0; tap < 9; ++tap) acc += p.w2[(c * CAB_CC + ci) * 9 + tap] * s_S[tap * CAB_CC + ci];
        s_mean[c] = p.b2[c] + acc * inv;
    }
    __syncthreads();
    for (int j = wave; j < p.sq; j += WAVES) {
        float acc = 0.0f;
        for (int c = lane; c < CAB_C; c += 64) acc += s_mean[c] * p.wa[j * CAB_C + c];
        acc = wave_sum(acc) + p.ba[j];
        if (lane == 0) s_z[j] = acc < 0.0f ? 0.0f : acc;
    }
    __syncthreads();
    for (int c = tid; c < CAB_C; c += WAVES * 64) {
        float acc = p.bb[c];
        for (int j = 0; j < p.sq; ++j) acc += s_z[j] * p.wb[c * p.sq + j];
        const float g = 1.0f / (1.0f + __expf(-acc));
        s_gate[c] = g;
        p.gate[c] = g;
        p.bias2[c] = p.bproj[c] + (p.cscale * g) * p.b2[c];
    }
    __syncthreads();
    for (int i = tid; i < CAB_C * CAB_K2; i += WAVES * 64) {
        const int c = i / CAB_K2, k = i - c * CAB_K2;
        const int tap = k / CAB_CC, ci = k - tap * CAB_CC;
        float v = 0.0f;
        if (tap < 9) v = (p.cscale * s_gate[c]) * p.w2[(c * CAB_CC + ci) * 9 + tap];
        p.w2g[i] = v;
    }
    // the same weights as hat_projx_cab's two weight chunks: [s][plane][c][32],
    // row c's k-group g at slot ws_slot(c, g), k = 32 s + j, zeros elsewhere
    if (p.w2gx) {
        constexpr int PLANE = CAB_C * 32;
        for (int i = tid; i < 2 * WC_CHUNK; i += WAVES * 64) {
            const int s = i / WC_CHUNK, r = i - s * WC_CHUNK;
            unsigned short h = 0;
            if (r < 3 * PLANE) {
                const int pl = r / PLANE, c = (r - pl * PLANE) / 32, pos = r - pl * PLANE - c * 32;
                const int j = (ws_slot(c, pos >> 3) << 3) | (pos & 7);
                const int k = 32 * s + j, tap = k / CAB_CC, ci = k - tap * CAB_CC;
                const float v = tap < 9 ? (p.cscale * s_gate[c]) * p.w2[(c * CAB_CC + ci) * 9 + tap] : 0.0f;
                h = split3_part(v, pl);
            }
            p.w2gx[i] = h;
        }
    }
}

// The unfolded CAB's gate (the C = 180 family; hat_arch.py:40-55, cpu.rs:
// 940-955) for a block of WAVES waves, straight from the conv2 partial column
// sums: wave w adds rows w, w + WAVES, ... (its lanes over the columns), the
// waves' sums are added in wave order through LDS, then mean, squeeze + ReLU,
// excite + sigmoid. lds: SE_GATE_LDS floats.
#define SE_GATE_LDS (8 * 192 + 192 + 64)
template <int WAVES>
__device__ __forceinline__ void se_gate_body(const SeArgs& p, float* lds)
{
    static_assert(WAVES <= 8, "the LDS holds eight waves' sums");
    float* s_part = lds;              // [WAVES][192]
    float* s_mean = s_part + 8 * 192;  // [192]
    float* s_sq = s_mean + 192;        // [64]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int c0 = 0; c0 < p.C; c0 += 64) {
        const int c = c0 + lane;
        float a0 = 0.0f, a1 = 0.0f;
        if (c < p.C) {
            int b = wave;
            for (; b + WAVES < p.nblk; b += 2 * WAVES) {
                a0 += p.partial[(size_t)b * p.co_stride + c];
                a1 += p.partial[(size_t)(b + WAVES) * p.co_stride + c];
            }
            if (b < p.nblk) a0 += p.partial[(size_t)b * p.co_stride + c];
            s_part[wave * 192 + c] = a0 + a1;
        }
    }
    __syncthreads();
    for (int c = tid; c < p.C; c += WAVES * 64) {
        float acc = 0.0f;
        for (int w = 0; w < WAVES; ++w) acc += s_part[w * 192 + c];
        s_mean[c] = acc / p.count;
    }
    __syncthreads();
    for (int j = tid; j < p.sq; j += WAVES * 64) {
        float acc = p.b1[j];
        for (int c = 0; c < p.C; ++c) acc += s_mean[c] * p.w1[(size_t)j * p.C + c];
        s_sq[j] = acc < 0.0f ? 0.0f : acc;
    }
    __syncthreads();
    for (int c = tid; c < p.C; c += WAVES * 64) {
        float acc = p.b2[c];
        for (int j = 0; j < p.sq; ++j) acc += s_sq[j] * p.w2[(size_t)c * p.sq + j];
        p.gate[c] = 1.0f / (1.0f + __expf(-acc));
    }
}

extern "C" __global__ __launch_bounds__(CG_WAVES * 64) void hat_cab_gate(CabGateArgs p)
{
    __shared__ float lds[CAB_GATE_LDS];
    cab_gate_body<CG_WAVES>(p, lds);
}
