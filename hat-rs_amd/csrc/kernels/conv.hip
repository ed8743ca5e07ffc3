// 3x3 convolution (stride 1, zero padding 1) as an implicit GEMM on FP32 MFMA,
// NHWC in and out.
//
// Replaces lg_conv3x3_winograd (src/cuda.rs:88-106) at every call site of the
// reference graph (CAB convs gpu.rs:426,429; RHAG conv :605; conv_first :722;
// conv_after_body :742; head :636,643,650), and folds into the epilogue what
// the reference runs as separate passes: GELU / LeakyReLU, the residual add,
// the PixelShuffle (lg_pixel_shuffle, cuda.rs:516-522), the per-channel sums
// of the channel-attention pool (lg_channel_mean, cuda.rs:259-272) and the
// final crop + denormalisation (backend.rs:94-109).
//
// Tiling: 256 threads = 4 waves; a block owns an 8x16 pixel tile and 16*NT
// output channels. Wave w owns pixel rows 2w and 2w+1 of the tile, one 16-pixel
// MFMA tile each, so lane l%16 is the pixel's x. Input channels are walked in
// chunks of 16: the (8+2)x(16+2) halo patch and the 9-tap weight slice of the
// chunk are staged in LDS and every tap reads the same patch at an offset.
// MFMA operands: weights (A, rows = output channels) and patch pixels (B,
// columns = pixels); lane group g (= lane/16) reduces channels 4g..4g+3 of the
// chunk, one float4 read each.
#include "common.h"

using namespace hatk;

#define CV_TY 8
#define CV_TX 16
#define CV_PY (CV_TY + 2)
#define CV_PX (CV_TX + 2)
#define CV_CS 20  // 16 channels + 4 pad

template <int NT, int EPI>
__device__ __forceinline__ void conv_body(const ConvArgs& p)
{
    constexpr int BN = 16 * NT;
    __shared__ float Ps[CV_PY * CV_PX * CV_CS];
    __shared__ float Ws[9 * BN * CV_CS];
    __shared__ float s_col[EPI == CEPI_COLSUM ? 4 * BN : 1];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int tiles_x = (p.W + CV_TX - 1) / CV_TX;
    const int ty0 = (blockIdx.x / tiles_x) * CV_TY;
    const int tx0 = (blockIdx.x % tiles_x) * CV_TX;
    const int co0 = blockIdx.y * BN;
    const int H = p.H, W = p.W;

    f32x4 acc[2][NT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const int nchunks = p.CIp / 16;
    for (int cc = 0; cc < nchunks; ++cc) {
        const int ci0 = cc * 16;
        __syncthreads();
        // Halo patch: 180 pixels x 4 float4.
        for (int idx = tid; idx < CV_PY * CV_PX * 4; idx += 256) {
            const int pix = idx >> 2, c4 = (idx & 3) * 4;
            const int py = pix / CV_PX, px = pix - py * CV_PX;
            const int y = ty0 + py - 1, x = tx0 + px - 1;
            const int ci = ci0 + c4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (y >= 0 && y < H && x >= 0 && x < W && ci < p.CI) {
                const float* src = p.in + ((size_t)y * W + x) * p.cin_stride + ci;
                if (ci + 3 < p.CI) {
                    v = *(const float4*)src;
                } else {
                    // channels past CI are padding and read as zero
                    v.x = src[0];
                    if (ci + 1 < p.CI) v.y = src[1];
                    if (ci + 2 < p.CI) v.z = src[2];
                }
            }
            *(float4*)(Ps + pix * CV_CS + c4) = v;
        }
        // Weights: packed [chunk][tap][COp][16].
        const float* wc = p.w + (size_t)cc * 9 * p.COp * 16;
        for (int idx = tid; idx < 9 * BN * 4; idx += 256) {
            const int row = idx >> 2, c4 = (idx & 3) * 4;
            const int tap = row / BN, co = row - tap * BN;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (co0 + co < p.COp) v = *(const float4*)(wc + ((size_t)tap * p.COp + co0 + co) * 16 + c4);
            *(float4*)(Ws + row * CV_CS + c4) = v;
        }
        __syncthreads();
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int dy = tap / 3, dx = tap - dy * 3;
            f32x4 xv[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
                xv[mt] = *(const f32x4*)(Ps + ((wave * 2 + mt + dy) * CV_PX + lr + dx) * CV_CS + lg * 4);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f32x4 wv = *(const f32x4*)(Ws + (tap * BN + nt * 16 + lr) * CV_CS + lg * 4);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) acc[mt][nt] = mfma16(wv[s], xv[mt][s], acc[mt][nt]);
            }
        }
    }

    // Epilogue: lane holds output channels co .. co+3 of pixel (y, x).
    float colsum[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int j = 0; j < 4; ++j) colsum[nt][j] = 0.0f;

#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int y = ty0 + wave * 2 + mt;
        const int x = tx0 + lr;
        const bool live = y < H && x < W;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int co = co0 + nt * 16 + lg * 4;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = acc[mt][nt][j] + (co + j < p.COp ? p.bias[co + j] : 0.0f);
                if (p.act == 1) v[j] = gelu(v[j]);
                else if (p.act == 2) v[j] = v[j] < 0.0f ? v[j] * 0.01f : v[j];
            }
            if (!live || co >= p.CO) continue;
            if (EPI == CEPI_STORE || EPI == CEPI_RESID || EPI == CEPI_COLSUM) {
                float* o = p.out + ((size_t)y * W + x) * p.co_stride + co;
                if (EPI == CEPI_RESID) {
                    const float* r = p.res + ((size_t)y * W + x) * p.co_stride + co;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (co + j < p.CO) v[j] = v[j] + r[j];
                }
                if (EPI == CEPI_COLSUM) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (co + j < p.CO) colsum[nt][j] += v[j];
                }
                if (co + 3 < p.CO && (p.co_stride & 3) == 0) {
                    *(float4*)o = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (co + j < p.CO) o[j] = v[j];
                }
            } else if (EPI == CEPI_SHUFFLE) {
                // Channels were permuted at upload to o' = (i*r + j)*Cf + c.
                const int r = p.r, Cf = p.CO / (r * r);
                const int sub = co / Cf, c = co - sub * Cf;
                const int i = sub / r, jj = sub - i * r;
                float* o = p.out + ((size_t)(y * r + i) * (W * r) + x * r + jj) * p.co_stride + c;
                *(float4*)o = make_float4(v[0], v[1], v[2], v[3]);
            } else if (EPI == CEPI_FINAL) {
                if (y < p.crop_h && x < p.crop_w) {
                    const float mean[3] = {p.mean0, p.mean1, p.mean2};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int ch = co + j;
                        if (ch < 3)
                            p.out[((size_t)ch * p.crop_h + y) * p.crop_w + x] = v[j] / p.img_range + mean[ch];
                    }
                }
            }
        }
    }

    if (EPI == CEPI_COLSUM) {
        // Reduce over the 16 pixels of each row tile (lanes with equal lg), then
        // over the 4 waves through LDS; one partial row per block.
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float s = colsum[nt][j];
                s += __shfl_xor(s, 1, 64);
                s += __shfl_xor(s, 2, 64);
                s += __shfl_xor(s, 4, 64);
                s += __shfl_xor(s, 8, 64);
                colsum[nt][j] = s;
            }
        if (lr == 0) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int j = 0; j < 4; ++j) s_col[wave * BN + nt * 16 + lg * 4 + j] = colsum[nt][j];
        }
        __syncthreads();
        const int blk = blockIdx.x;
        for (int c = tid; c < BN; c += 256) {
            const int co = co0 + c;
            if (co < p.CO) {
                float s = s_col[c] + s_col[BN + c] + s_col[2 * BN + c] + s_col[3 * BN + c];
                p.partial[(size_t)blk * p.co_stride + co] = s;
            }
        }
    }
}

#define CONV_INST(NAME, NT, EPI)                                                             \
    extern "C" __global__ __launch_bounds__(256) void NAME(ConvArgs p) { conv_body<NT, EPI>(p); }

CONV_INST(hat_conv_n1_store, 1, CEPI_STORE)
CONV_INST(hat_conv_n3_store, 3, CEPI_STORE)
CONV_INST(hat_conv_n4_store, 4, CEPI_STORE)
CONV_INST(hat_conv_n3_resid, 3, CEPI_RESID)
CONV_INST(hat_conv_n3_colsum, 3, CEPI_COLSUM)
CONV_INST(hat_conv_n4_shuffle, 4, CEPI_SHUFFLE)
CONV_INST(hat_conv_n1_final, 1, CEPI_FINAL)

// ---------------------------------------------------------------------------
// conv_last (64 -> 3, 3x3, zero padding) + crop + denormalise (gpu.rs:648-653,
// backend.rs:92-109), by per-tap products: for each pixel q of a 16 x 32 output
// tile's 18 x 34 halo, P[q][tap*3 + co] = sum_ci h[q][ci] * w[co][ci][tap] is a
// 64-deep product with 27 (of 32) outputs on MFMA, and the conv output at p is
// sum over the 9 taps of P[p + d(tap)][tap*3 + co], read from LDS. Against a
// GEMM with the 3 output channels padded to 16 columns this executes 2.4x less
// MFMA work. The products run on split-bf16 MFMA (v_mfma_f32_16x16x32_bf16,
// every fp32 operand as three bf16 parts and every product as the six terms of
// order <= 2, as accurate as FP32 MFMA; common.h split3_x8 / mfma16x6): per
// 16-pixel row tile two 32-channel steps of 2 x 6 MFMAs, against 32 FP32
// 16x16x4 MFMAs of twice the issue time each. The weights (32 x 64) are split
// once per block and stay in registers; each wave streams its halo row tiles,
// reading each one's channels two row tiles ahead.
// Requires CI = CIp = 64, CO = 3 (the repacked [4][9][COp][16] weights).
#define CL_TH 16
#define CL_TW 32
#define CL_HH (CL_TH + 2)
#define CL_HW (CL_TW + 2)
#define CL_HP (CL_HH * CL_HW)               // 612 halo pixels
#define CL_RT ((CL_HP + 15) / 16)           // 39 row tiles of 16 pixels
#define CL_PS 28                            // LDS row stride of P (27 used)
#define CL_WAVES 8

extern "C" __global__ __launch_bounds__(CL_WAVES * 64) void hat_conv_last3(ConvArgs p)
{
    __shared__ __attribute__((aligned(16))) float Ps[CL_HP * CL_PS];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int H = p.H, W = p.W;
    const int ntx = (W + CL_TW - 1) / CL_TW;
    // Tiles are taken bottom row first: the conv before this one wrote its
    // bottom rows last, so those are the ones still in the last-level cache.
    // tile0: the first tile of a band of tile rows (0 for the whole plane)
    const int bt = p.tile0 + (int)gridDim.x - 1 - (int)blockIdx.x;
    const int ty = bt / ntx, tx = bt - ty * ntx;
    const int y0 = ty * CL_TH, x0 = tx * CL_TW;

    // A operand: row n = tap*3 + co of the per-tap products (rows 27.. zero),
    // k-step ks: channels 32 ks + 8 lg .. +7 (in the repacked layout, 16-channel
    // chunk 2 ks + lg / 2 at 8 (lg & 1)), split.
    u32x4 wb[2][2][3];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int n = nt * 16 + lr, tap = n / 3, co = n - tap * 3;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            f32x4 v0 = (f32x4){0.f, 0.f, 0.f, 0.f}, v1 = v0;
            if (n < 27) {
                const float* w = p.w + ((size_t)((2 * ks + (lg >> 1)) * 9 + tap) * p.COp + co) * 16 + 8 * (lg & 1);
                v0 = *(const f32x4*)w;
                v1 = *(const f32x4*)(w + 4);
            }
            const float f[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            split3_x8(f, wb[nt][ks]);
        }
    }
    // Every wave walks NPW row tiles (the last one past the 39 for wave 7:
    // zeros, not stored). The lane's input row of row tile i: hat_zero_row
    // outside the plane and past the halo, so that the loads are issued on every
    // path, and the loop is unrolled, so that the compiler's waits for the rows
    // read ahead are exact (a loop back-edge would make them vmcnt(0)).
    constexpr int NPW = (CL_RT + CL_WAVES - 1) / CL_WAVES;
    auto src_of = [&](int i) -> const float* {
        const int hi = (wave + CL_WAVES * i) * 16 + lr;
        const int hy = hi / CL_HW, hx = hi - hy * CL_HW;
        const int gy = y0 - 1 + hy, gx = x0 - 1 + hx;
        const bool valid = i < NPW && hi < CL_HP && gy >= 0 && gy < H && gx >= 0 && gx < W;
        return valid ? p.in + ((size_t)gy * W + gx) * p.cin_stride + lg * 8 : hat_zero_row;
    };
    // the lane's channels 32 ks + 8 lg .. +7 of its pixel, as two float4s, for
    // two row tiles: row tile i in slot i % 2, read two row tiles ahead
    f32x4 xa[2][2][2];
    auto load = [&](int slot, int ks, const float* src) {
        xa[slot][ks][0] = *(const f32x4*)(src + ks * 32);
        xa[slot][ks][1] = *(const f32x4*)(src + ks * 32 + 4);
    };
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float* first = src_of(i);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) load(i, ks, first);
    }
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
        const float* nxt = src_of(i + 2);
        f32x4 acc[2] = {(f32x4){0.f, 0.f, 0.f, 0.f}, (f32x4){0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const f32x4(&x)[2] = xa[i % 2][ks];
            const float f[8] = {x[0][0], x[0][1], x[0][2], x[0][3], x[1][0], x[1][1], x[1][2], x[1][3]};
            u32x4 xb[3];
            split3_x8(f, xb);
            load(i % 2, ks, nxt);  // step ks of row tile i + 2
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) acc[nt] = mfma16x6(wb[nt][ks], xb, acc[nt]);
            __builtin_amdgcn_sched_barrier(0);  // the loads stay in their step
        }
        // lane (lr, lg) holds P[hi][16nt + 4lg .. +3]; columns 28.. are not stored
        const int hi = (wave + CL_WAVES * i) * 16 + lr;
        if (hi < CL_HP) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                if (nt * 16 + lg * 4 < CL_PS) *(f32x4*)(Ps + hi * CL_PS + nt * 16 + lg * 4) = acc[nt];
        }
    }
    __syncthreads();

    // One output pixel per thread: the 9 taps, then crop and denormalise into
    // the planar [3][crop_h][crop_w] image.
    const int oy = tid / CL_TW, ox = tid - oy * CL_TW;
    const int y = y0 + oy, x = x0 + ox;
    if (y >= p.crop_h || x >= p.crop_w) return;
    float v[3] = {p.bias[0], p.bias[1], p.bias[2]};
#pragma unroll
    for (int ky = 0; ky < 3; ++ky)
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
            const float* q = Ps + ((oy + ky) * CL_HW + ox + kx) * CL_PS + (ky * 3 + kx) * 3;
            v[0] += q[0];
            v[1] += q[1];
            v[2] += q[2];
        }
    const size_t plane = (size_t)p.crop_h * p.crop_w, o = (size_t)y * p.crop_w + x;
    p.out[o] = v[0] / p.img_range + p.mean0;
    p.out[plane + o] = v[1] / p.img_range + p.mean1;
    p.out[2 * plane + o] = v[2] / p.img_range + p.mean2;
}
