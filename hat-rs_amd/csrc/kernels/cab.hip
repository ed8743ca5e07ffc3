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
// conv1 (144 -> 6, 3x3, zero padding) + GELU, one 16-wide, TY-tall output tile
// at a time.
//
// Per-tap products: for each pixel q of the tile's 18 x (TY+2) halo,
// P[q][tap*6+co] = sum_ci xn[q][ci] * w[co][ci][tap] is a 144-deep product with
// 54 (padded to 64) outputs - one MFMA row tile of 16 halo pixels x 4 column
// tiles. The conv output at p is then sum over the 9 taps of
// P[p + d(tap)][tap*6 + co], read from LDS. The weights (64 x 144) stay in
// registers for the whole kernel, so a block streams its tiles with no weight
// traffic.
//   TY = 16: 4 waves, two blocks per CU (73 KB of LDS each); the halo is 21 row
//            tiles (one wave has six, the others five).
//   TY = 32: 8 waves, one block per CU (137 KB); the halo is 39 row tiles (five
//            per wave, one wave four) for twice the pixels: fewer halo pixels
//            per output pixel and a better balance across the waves.
#define CC1_HS 18   // halo width
#define CC1_PS 56   // LDS row stride of P (54 used)

template <int TY>
struct Cc1Shape {
    static constexpr int WAVES = TY == 32 ? 8 : 4;
    static constexpr int THREADS = WAVES * 64;
    static constexpr int HY = TY + 2;            // halo height
    static constexpr int HP = CC1_HS * HY;       // halo pixels
    static constexpr int RT = (HP + 15) / 16;    // row tiles of 16 pixels
    static_assert(16 * TY == THREADS, "one output pixel per thread");
};

template <int TY>
__device__ __forceinline__ void cab_conv1_body(const CabConvArgs& p)
{
    using S = Cc1Shape<TY>;
    constexpr int WAVES = S::WAVES;
    __shared__ float Ps[S::HP * CC1_PS];
    __shared__ float red[WAVES][CAB_NSUM * CAB_CC];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int H = p.H, W = p.W;
    const int ntx = W / 16;
    const int ntiles = ntx * (H / TY);

    f32x4 wreg[4][CAB_C / 16];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int kc = 0; kc < CAB_C / 16; ++kc)
            wreg[nt][kc] = *(const f32x4*)(p.w + (nt * 16 + lr) * CAB_C + kc * 16 + lg * 4);
    float bias[CAB_CC];
#pragma unroll
    for (int co = 0; co < CAB_CC; ++co) bias[co] = p.bias[co];

    // This wave's halo row tiles rt = wave, wave + WAVES, ... of the block's
    // tiles are walked as one stream of 16-channel chunks (9 per row tile), the
    // input rows held in nine register slots: chunk kc of the next row tile (of
    // this tile, or the first of the block's next tile) is loaded as soon as
    // chunk kc of this one has gone to its MFMAs, a whole row tile (144 MFMAs)
    // ahead.
    const int nrt = (S::RT - wave + WAVES - 1) / WAVES;
    auto src_of = [&](int tl, int i) -> const float* {  // lane's input row of row tile i of tile tl, or null
        if (tl >= ntiles) return nullptr;
        const int ty = tl / ntx, tx = tl - ty * ntx;
        const int hi = (wave + WAVES * i) * 16 + lr;
        const int hy = hi / CC1_HS, hx = hi - hy * CC1_HS;
        const int gy = ty * TY - 1 + hy, gx = tx * 16 - 1 + hx;
        const bool valid = hi < S::HP && gy >= 0 && gy < H && gx >= 0 && gx < W;
        return valid ? p.xn + (size_t)(gy * W + gx) * CAB_C + lg * 4 : nullptr;
    };
    f32x4 xa[CAB_C / 16];
    auto load = [&](int slot, const float* src, int kc) {
        f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
        if (src) v = *(const f32x4*)(src + kc * 16);
        xa[slot] = v;
    };
    {
        const float* first = src_of(blockIdx.x, 0);
#pragma unroll
        for (int s = 0; s < CAB_C / 16; ++s) load(s, first, s);
    }

    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int ty = tile / ntx, tx = tile - ty * ntx;
        const int y0 = ty * TY, x0 = tx * 16;
#pragma unroll 1
        for (int i = 0; i < nrt; ++i) {
            const float* nxt = i + 1 < nrt ? src_of(tile, i + 1) : src_of(tile + gridDim.x, 0);
            f32x4 acc[4];
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) acc[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < CAB_C / 16; ++kc) {
                const f32x4 a = xa[kc];
                load(kc, nxt, kc);  // chunk kc of the next row tile
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt) acc[nt] = mfma16(wreg[nt][kc][s], a[s], acc[nt]);
            }
            // lane (lr, lg) holds P[hi][16nt + 4lg .. +3]; columns 56.. are not stored
            const int hi = (wave + WAVES * i) * 16 + lr;
            if (hi < S::HP) {
#pragma unroll
                for (int nt = 0; nt < 4; ++nt)
                    if (nt * 16 + lg * 4 < CC1_PS) *(f32x4*)(Ps + hi * CC1_PS + nt * 16 + lg * 4) = acc[nt];
            }
        }
        __syncthreads();

        // One output pixel per thread: the 9 taps from the halo products.
        const int oy = tid >> 4, ox = tid & 15;
        float v[CAB_CC];
#pragma unroll
        for (int co = 0; co < CAB_CC; ++co) v[co] = bias[co];
#pragma unroll
        for (int ky = 0; ky < 3; ++ky)
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                const float* q = Ps + ((oy + ky) * CC1_HS + ox + kx) * CC1_PS + (ky * 3 + kx) * CAB_CC;
#pragma unroll
                for (int j = 0; j < CAB_CC / 2; ++j) {
                    const float2 t = *(const float2*)(q + 2 * j);
                    v[2 * j] += t.x;
                    v[2 * j + 1] += t.y;
                }
            }
#pragma unroll
        for (int co = 0; co < CAB_CC; ++co) v[co] = gelu(v[co]);
        const int gy = y0 + oy, gx = x0 + ox;
        float* dst = p.t1 + ((size_t)gy * W + gx) * CAB_CS;
        *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
        *(float4*)(dst + 4) = make_float4(v[4], v[5], 0.f, 0.f);

        // Per-tile sums: the tile, and its pixels on row 0, row H-1, col 0,
        // col W-1 - only tiles on the plane's border have any of the latter.
        const bool border = y0 == 0 || y0 + TY == H || x0 == 0 || x0 + 16 == W;  // tile-uniform
        const bool line[CAB_NSUM] = {true, gy == 0, gy == H - 1, gx == 0, gx == W - 1};
#pragma unroll
        for (int l = 0; l < CAB_NSUM; ++l) {
            if (l > 0 && !border) break;
#pragma unroll
            for (int co = 0; co < CAB_CC; ++co) {
                const float s = wave_sum(line[l] ? v[co] : 0.0f);
                if (lane == 0) red[wave][l * CAB_CC + co] = s;
            }
        }
        __syncthreads();
        if (tid < CAB_NSUM * CAB_CS) {
            const int l = tid / CAB_CS, co = tid - l * CAB_CS;
            float s = 0.0f;
            if (co < CAB_CC && (l == 0 || border)) {
                const int i = l * CAB_CC + co;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) s += red[w][i];  // waves in order
            }
            p.partial[(size_t)tid * ntiles + tile] = s;  // value-major: [40][tiles]
        }
        // The next tile's P stores come after this barrier; every read of Ps
        // and red above precedes it.
        __syncthreads();
    }
}

extern "C" __global__ __launch_bounds__(256, 2) void hat_cab_conv1(CabConvArgs p)
{
    cab_conv1_body<16>(p);
}
extern "C" __global__ __launch_bounds__(512, 1) void hat_cab_conv1_t32(CabConvArgs p)
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
    // the same weights as hat_projx_cab's two weight chunks: [s][plane][c][WC_KS],
    // k = 32 s + j (j < 32), zeros elsewhere
    if (p.w2gx) {
        constexpr int PLANE = CAB_C * WC_KS;
        for (int i = tid; i < 2 * WC_CHUNK; i += WAVES * 64) {
            const int s = i / WC_CHUNK, r = i - s * WC_CHUNK;
            unsigned short h = 0;
            if (r < 3 * PLANE) {
                const int pl = r / PLANE, c = (r - pl * PLANE) / WC_KS, j = r - pl * PLANE - c * WC_KS;
                const int k = 32 * s + j, tap = k / CAB_CC, ci = k - tap * CAB_CC;
                const float v = j < 32 && tap < 9 ? (p.cscale * s_gate[c]) * p.w2[(c * CAB_CC + ci) * 9 + tap] : 0.0f;
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
