// The qkv linear of the C = 144 family on split-bf16 MFMA: out = A . Wqkv^T +
// b scattered head-major into q, k, v ([3][heads][T][24]), as hat_gemmws_qkv
// (lg_linear + lg_extract_rows of the reference, cuda.rs:428-453).
//
// Arithmetic: every fp32 operand as three bf16 parts and each product as the
// six terms of order <= 2 (attnx.hip explains the split and its accuracy), on
// v_mfma_f32_16x16x32_bf16 with the weight rows as the A operand and the
// token rows as B: a lane's four accumulators are four consecutive output
// columns of one token, the layout of the FP32 kernels, so the epilogue is
// theirs. K = 144 runs as five 32-k steps; in the last one the activation
// at k = 144 is 1 and the weights there hold the bias (split like the rest,
// so it is added exactly), k 145..159 are zeros against zeros.
//
// Data flow: a block of 4 waves takes one 128-token row tile through one of
// the three 144-column slices (q, k or v): its waves hold their 32 token rows
// in registers for the whole block (all five k-steps, read once) and the
// slice's five weight chunks (one 32-k step each, pre-split on the host, 40
// KB) stream through two LDS buffers, chunk c + 1 in flight while chunk c's
// MFMAs run (common.h). The two buffers are two LDS objects, so that the
// compiler sees that reading one need not wait for the copy into the other.
// Two blocks share a CU, so one block's reads overlap the other's MFMAs, and
// the results leave once, at the block's end. The three blocks of a tile are
// placed on one XCD (blocks are dealt to the 8 XCDs in turn), so that two of
// the three reads of the tile's rows hit its L2.
//
// The host launches it for heads = 6, head_dim = 24 (the slices are q, k, v),
// on ceil(tiles / 8) * 24 blocks.

#define GX_WAVES 4
#define GX_ROWS (GX_WAVES * 32)  // tokens per tile

// This wave's 32 token rows of a [M][144] plane, 8 values at k = 32 ks + 8 lg
// per token, for the B operand (zeros past M and past k = 144).
struct WcRows {
    const float* rows[2];
    bool alive[2];
    __device__ __forceinline__ void init(const float* base, int mbase, int M, int lr)
    {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int m = mbase + mt * 16 + lr;
            alive[mt] = m < M;
            rows[mt] = base + (size_t)(alive[mt] ? m : 0) * 144;
        }
    }
    __device__ __forceinline__ void load(int ks, int lg, f32x4 (&dst)[2][2]) const
    {
        const int k0 = ks * 32 + lg * 8;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const bool kin = alive[mt] && k0 < 144;
            dst[mt][0] = load_or_zero(rows[mt] + k0, kin);
            dst[mt][1] = load_or_zero(rows[mt] + k0 + 4, kin);
        }
    }
    // load, with the 1 at k = 144 that multiplies the bias column (read from
    // memory like the rest, so that nothing waits for the loads here)
    __device__ __forceinline__ void load_b(int ks, int lg, f32x4 (&dst)[2][2]) const
    {
        const int k0 = ks * 32 + lg * 8;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const bool kin = alive[mt] && k0 < 144;
            dst[mt][0] = *(const f32x4*)(kin ? rows[mt] + k0 : (k0 == 144 ? hat_one_row : hat_zero_row));
            dst[mt][1] = load_or_zero(rows[mt] + k0 + 4, kin);
        }
    }
};

__device__ __forceinline__ void split_pre(const f32x4 (&pre)[2][2], u32x4 (&xb)[2][3])
{
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const float f[8] = {pre[mt][0][0], pre[mt][0][1], pre[mt][0][2], pre[mt][0][3],
                            pre[mt][1][0], pre[mt][1][1], pre[mt][1][2], pre[mt][1][3]};
        split3_x8(f, xb[mt]);
    }
}

extern "C" __global__ __launch_bounds__(GX_WAVES * 64, 2) void hat_gemmx_qkv(GemmArgs p)
{
    constexpr int NT = 9, QS_S = 52, NL = 36;  // a 144-row chunk as 9 loads from each wave
    __shared__ __attribute__((aligned(16))) unsigned short Ws0[36 * 512];  // also the results' staging
    __shared__ __attribute__((aligned(16))) unsigned short Ws1[36 * 512];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    // block -> (tile, slice): blocks b, b + 8, b + 16 (one XCD) take the three
    // slices of one tile
    const int xcd = blockIdx.x & 7, i = blockIdx.x >> 3;
    const int tile = (i / 3) * 8 + xcd, sl = i - (i / 3) * 3;
    if (tile * GX_ROWS >= M) return;  // whole block, before any barrier
    const unsigned short* wx = (const unsigned short*)p.w + (size_t)sl * 5 * WC_CHUNK;  // this slice's chunks
    wc_issue<NL, GX_WAVES>(Ws0, wx, wave, lane);
    const int mbase = tile * GX_ROWS + wave * 32;
    WcRows xr;
    xr.init(p.a, mbase, M, lr);
    f32x4 y[5][2][2];
#pragma unroll
    for (int ks = 0; ks < 5; ++ks) xr.load_b(ks, lg, y[ks]);
    f32x4 acc[2][NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[0][nt] = acc[1][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 5; ++c) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of chunk c (and its rows) have landed
        __syncthreads();                // everyone's have, and everyone is done with chunk c - 1
        if (c + 1 < 5) wc_issue<NL, GX_WAVES>(c & 1 ? Ws0 : Ws1, wx + (size_t)(c + 1) * WC_CHUNK, wave, lane);
        u32x4 xb[2][3];
        split_pre(y[c], xb);
        wc_mma<NT, 144 * WC_KS>(c & 1 ? Ws1 : Ws0, lr, lg, xb, acc);
    }
    __syncthreads();  // every wave is done with the weights
    // Two heads at a time go through the wave's LDS region and leave as 16
    // consecutive rows of each head (1536 contiguous bytes), non-temporal.
    float* Q = (float*)Ws0 + wave * 16 * QS_S;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int mb = mbase + mt * 16;
        const int mrows = M - mb;
#pragma unroll
        for (int ph = 0; ph < 3; ++ph) {
#pragma unroll
            for (int t = 0; t < 3; ++t) *(f32x4*)(Q + lr * QS_S + t * 16 + lg * 4) = acc[mt][3 * ph + t];
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
#pragma unroll
            for (int i2 = 0; i2 < 3; ++i2) {
                const int f = lane + 64 * i2, hh = f / 96, r = (f - hh * 96) / 6, d4 = f - hh * 96 - r * 6;
                const f32x4 v = *(const f32x4*)(Q + r * QS_S + hh * 24 + d4 * 4);
                if (r < mrows) {
                    const int head = 2 * ph + hh;
                    __builtin_nontemporal_store(
                        v, (f32x4*)(p.out + ((size_t)(sl * p.heads + head) * M + mb + r) * 24 + d4 * 4));
                }
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next phase's writes
        }
    }
}
