// The qkv linear of the C = 144 family on split-bf16 MFMA: out = A . Wqkv^T +
// b scattered head-major into q, k, v ([3][heads][T][24]), as hat_gemmws_qkv
// (lg_linear + lg_extract_rows of the reference, cuda.rs:428-453).
//
// Arithmetic: every fp32 operand as three bf16 parts and each product as the
// six terms of order <= 2 (attnx.hip explains the split and its accuracy), on
// v_mfma_f32_16x16x32_bf16 with the weight rows as the A operand and the
// token rows as B: a lane's four accumulators are four consecutive output
// columns of one token, the layout of the FP32 kernels, so the epilogue is
// theirs. K = 144 runs as five 32-k steps; in the last one lane groups 2 and
// 3 (k 144..159) hold zero activations, so whatever finite weights they meet
// contribute nothing.
//
// Data flow: with the MFMAs this fast the kernel is bound by HBM, and the
// weight-stationary FP32 kernel, whose blocks each hold one 144-column slice
// for many row tiles, reads the activations from HBM once per slice (3x).
// Here a block takes a row tile of 256 tokens through all three slices in
// turn, streaming the slices (pre-split on the host, 121.5 KB each) through
// LDS from L2; its waves read their 32 token rows again per slice, one 32-k
// step ahead of the MFMAs, and split them in registers - the second and third
// reads of a tile's 147 KB find it in the caches, so HBM sees the activations
// once. A block of 8 waves walks the row tiles.
//
// The host launches it for heads = 6, head_dim = 24 (the slices are q, k, v).
// Included after attnx.hip (the split helpers).

#define GX_WAVES 8
#define GX_ROWS (GX_WAVES * 32)     // tokens per tile
#define GX_KS 152                   // LDS row stride of a weight plane (bf16)
#define GX_BN 144                   // columns per slice
#define GX_PLANE (GX_BN * GX_KS)    // bf16 per plane
#define GX_SLICE (3 * GX_PLANE)     // bf16 per slice (3 planes)
// a slice as packed by the host: the planes, then zeros up to a whole number
// of 64-lane x 16-byte loads (the zeros also serve the last row's k 152..159)
#define GX_SLICE_PAD ((GX_SLICE / 8 + 63) / 64 * 64 * 8)

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

extern "C" __global__ __launch_bounds__(GX_WAVES * 64, 2) void hat_gemmx_qkv(GemmArgs p)
{
    constexpr int NT = GX_BN / 16, KSTEPS = 5, MT = 2;
    constexpr int QS_S = 52;
    // the three planes of one slice with the zero tail, the bias, the q/k/v staging
    __shared__ __attribute__((aligned(16))) unsigned short Ws[GX_SLICE_PAD];
    __shared__ __attribute__((aligned(16))) float Cs[GX_BN];
    __shared__ __attribute__((aligned(16))) float Qs[GX_WAVES * 16 * QS_S];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M, N = p.N;
    const int nslices = N / GX_BN;
    const int ntiles = (M + GX_ROWS - 1) / GX_ROWS;
    if ((int)blockIdx.x >= ntiles) return;  // whole block, before any barrier
    const unsigned short* wx = (const unsigned short*)p.w;  // [slices][GX_SLICE_PAD], pre-split

    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int mbase = tile * GX_ROWS + wave * 32;
        // This wave's 32 token rows: lane (lr, lg) reads k = 32 ks + 8 lg .. +7 of
        // token mbase + 16 mt + lr, one step ahead of its MFMAs, and splits it
        // there. Every slice reads the rows again: the first read brings them
        // from HBM, the others find them in the caches.
        const float* rows[MT];
        bool alive[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = mbase + mt * 16 + lr;
            alive[mt] = m < M;
            rows[mt] = p.a + (size_t)(alive[mt] ? m : 0) * p.lda;
        }
        auto load_step = [&](int ks, f32x4 (&dst)[MT][2]) {
            const int k0 = ks * 32 + lg * 8;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const bool kin = alive[mt] && k0 < 144;
                dst[mt][0] = load_or_zero(rows[mt] + k0, kin);
                dst[mt][1] = load_or_zero(rows[mt] + k0 + 4, kin);
            }
        };
        for (int sl = 0; sl < nslices; ++sl) {
            const int n0 = sl * GX_BN;
            __syncthreads();  // every wave is done with the previous slice
            // the slice straight into LDS, every load in flight at once (lane l
            // of a load writes 16 bytes at the load's LDS base + 16 l)
            for (int c = wave; c < GX_SLICE_PAD / 512; c += GX_WAVES) {
                const unsigned short* src = wx + (size_t)sl * GX_SLICE_PAD + (size_t)(c * 64 + lane) * 8;
                __builtin_amdgcn_global_load_lds((const void*)src,
                                                 (__attribute__((address_space(3))) void*)(Ws + c * 512), 16, 0, 0);
            }
            for (int i = tid; i < GX_BN; i += GX_WAVES * 64) Cs[i] = p.bias[n0 + i];
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            f32x4 acc[MT][NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f32x4 b4 = *(const f32x4*)(Cs + nt * 16 + lg * 4);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = b4;
            }
            f32x4 pre[MT][2];
            load_step(0, pre);
#pragma unroll 1
            for (int ks = 0; ks < KSTEPS; ++ks) {
                u32x4 xb[MT][3];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const float f[8] = {pre[mt][0][0], pre[mt][0][1], pre[mt][0][2], pre[mt][0][3],
                                        pre[mt][1][0], pre[mt][1][1], pre[mt][1][2], pre[mt][1][3]};
                    split3_x8(f, xb[mt]);
                }
                if (ks + 1 < KSTEPS) load_step(ks + 1, pre);
                // the weight planes of tile nt + 1 are read while tile nt's 12
                // MFMAs run (the barriers keep the scheduler from hoisting every
                // tile's reads, which costs more registers than there are)
                const unsigned short* wr = Ws + lr * GX_KS + ks * 32 + lg * 8;
                u32x4 wa[2][3];
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) wa[0][pl] = *(const u32x4*)(wr + pl * GX_PLANE);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (nt + 1 < NT) {
#pragma unroll
                        for (int pl = 0; pl < 3; ++pl)
                            wa[(nt + 1) & 1][pl] = *(const u32x4*)(wr + (nt + 1) * 16 * GX_KS + pl * GX_PLANE);
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma16x6(wa[nt & 1], xb[mt], acc[mt][nt]);
                }
            }
            // The slice is one of q, k, v (6 heads x 24): two heads at a time go
            // through the wave's LDS region and leave as 16 consecutive rows of
            // each head (1536 contiguous bytes), non-temporal.
            float* Q = Qs + wave * 16 * QS_S;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int mb = mbase + mt * 16;
                const int mrows = M - mb;
#pragma unroll
                for (int ph = 0; ph < 3; ++ph) {
#pragma unroll
                    for (int t = 0; t < 3; ++t) *(f32x4*)(Q + lr * QS_S + t * 16 + lg * 4) = acc[mt][3 * ph + t];
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
#pragma unroll
                    for (int i = 0; i < 3; ++i) {
                        const int f = lane + 64 * i, hh = f / 96, r = (f - hh * 96) / 6, d4 = f - hh * 96 - r * 6;
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
    }
}
