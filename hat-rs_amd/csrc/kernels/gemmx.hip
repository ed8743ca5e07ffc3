// The qkv linear on split-bf16 MFMA: out = A . Wqkv^T + b scattered head-major
// into q, k, v ([3][heads][T][head_dim]), as hat_gemmws_qkv (lg_linear +
// lg_extract_rows of the reference, cuda.rs:428-453), for the C = 144 family
// (head_dim 24) and the C = 180 family (head_dim 30).
//
// Arithmetic: every fp32 operand as three bf16 parts and each product as the
// six terms of order <= 2 (attnx.hip explains the split and its accuracy), on
// v_mfma_f32_16x16x32_bf16 with the weight rows as the A operand and the
// token rows as B: a lane's four accumulators are four consecutive output
// columns of one token, the layout of the FP32 kernels. K runs as 32-k steps
// (144: five, 180: six); in the last one the activation at k = K is 1 and the
// weights there hold the bias (split like the rest, so it is added exactly),
// the k past it are zeros against zeros.
//
// Data flow: weight-stationary. A block of 8 waves holds one column slice in
// LDS for the whole launch, loaded once (C = 144: 144 columns, one of q, k,
// v, 135 KB; C = 180: 96 columns holding three heads of 30, 108 KB, two
// slices per q, k and v); after that its waves share nothing and meet at no
// barrier. Each wave walks subtiles of 16 MT tokens on its own (C = 144: 32,
// C = 180: 48, the faster in same-box timings): a k-step's rows are split in
// registers, the next k-step's rows (at the last step the next subtile's
// first) are read, and 6 MT MFMAs run per 16-column tile while the weight
// fragments of the tile two ahead are read from LDS (a ring of three: 1.5%
// faster than one ahead, same-box; three ahead no better). Rows read one k-step ahead take
// 8 MT registers a lane (a whole subtile ahead took 80 at C = 144).
// The NS slices' blocks of a group sit on one XCD (blocks are dealt to the
// 8 XCDs in turn) and walk the same subtiles in the same order, so that all
// but one of a subtile's NS reads find its rows in that XCD's L2. Results
// leave through a wave-private LDS stage as runs of one head (16 rows:
// 1.5 KB for head_dim 24, 1.9 KB for 30).
//
// The host launches NS * gemmx_qkv_groups(CUs, NS) blocks.

#define GX_WAVES 8

// This wave's 16 MT token rows of a [M][K] plane, 8 values at k = 32 ks + 8 lg
// per token, for the B operand: zeros past M and past k = K, with load_b the
// 1 at k = K that multiplies the bias column (read from hat_one_row like the
// rest, so that nothing waits for the loads here).
template <int K, int MT = 2>
struct WcRows {
    static_assert(K % 4 == 0, "float4 units");
    const float* rows[MT];
    bool alive[MT];
    __device__ __forceinline__ void init(const float* base, int mbase, int M, int lr)
    {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = mbase + mt * 16 + lr;
            alive[mt] = m < M;
            rows[mt] = base + (size_t)(alive[mt] ? m : 0) * K;
        }
    }
    // zeros from k = K on (for a bias added elsewhere)
    __device__ __forceinline__ void load(int ks, int lg, f32x4 (&dst)[MT][2]) const
    {
        const int k0 = ks * 32 + lg * 8;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < 2; ++j) dst[mt][j] = load_or_zero(rows[mt] + k0 + 4 * j, alive[mt] && k0 + 4 * j < K);
    }
    // the packed last step of K = 144: channels 128 + 4 lg .. +3 (dst[mt][1] unused)
    __device__ __forceinline__ void load_half(int lg, f32x4 (&dst)[MT][2]) const
    {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) dst[mt][0] = load_or_zero(rows[mt] + 128 + 4 * lg, alive[mt]);
    }
    __device__ __forceinline__ void load_b(int ks, int lg, f32x4 (&dst)[MT][2]) const
    {
        const int k0 = ks * 32 + lg * 8;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int kq = k0 + 4 * j;
                dst[mt][j] = *(const f32x4*)(alive[mt] && kq < K ? rows[mt] + kq : (kq == K ? hat_one_row : hat_zero_row));
            }
    }
};

template <int MT>
__device__ __forceinline__ void split_pre(const f32x4 (&pre)[MT][2], u32x4 (&xb)[MT][3])
{
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const float f[8] = {pre[mt][0][0], pre[mt][0][1], pre[mt][0][2], pre[mt][0][3],
                            pre[mt][1][0], pre[mt][1][1], pre[mt][1][2], pre[mt][1][3]};
        split3_x8(f, xb[mt]);
    }
}

// The epilogue's staging rows (floats): 48 at head_dim 24 (two heads of a
// 16-row tile at a time), 100 at 30 (all 96 columns, padded).
constexpr int gx_stage_stride(int hd) { return hd == 24 ? 48 : 100; }

// K: input width; NT: 16-column tiles per slice; NS: slices; HD: head_dim;
// NH: heads per slice (HD * NH <= 16 NT columns are real, the rest zero); MT:
// 16-token tiles per subtile (each weight fragment read from LDS feeds MT
// tiles, so MT sets the LDS bytes per MFMA).
// K = 144 (HALF): the last step packed (half_operands, mfma16x3: k = 128 ..
// 143, no bias column), the bias the accumulators' start value (Bs, the
// slice's 144 columns in LDS); K = 180: the bias as column k = K.
template <int K, int NT, int NS, int HD, int NH, int MT>
__device__ __forceinline__ void gemmx_qkv_body(const GemmArgs& p, unsigned short* Wsl, float* Qs, float* Bs)
{
    constexpr bool HALF = K == 144;
    constexpr int KS = (K + 32) / 32;             // 32-k steps (the bias column or the packed step included)
    constexpr int ROWS = 16 * NT;                 // slice rows in LDS
    constexpr int CHUNK = 3 * ROWS * 32;          // one k-step: three bf16 planes [ROWS][32]
    constexpr int NLOAD = KS * CHUNK / 512;       // 1 KB loads
    constexpr int QS_S = gx_stage_stride(HD);     // staging row stride (floats)
    constexpr int TOK = 16 * MT;                  // tokens per subtile
    static_assert(KS * CHUNK % 512 == 0, "whole loads");
    static_assert(HD * NH <= ROWS, "the heads fit the slice");

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    // block -> (group, slice): with a multiple of 8 groups, blocks b, b + 8,
    // ..., b + 8 (NS - 1) (one XCD) are one group's slices
    const int G = gridDim.x / NS;
    int grp, sl;
    if (G % 8 == 0) {
        const int i = blockIdx.x >> 3;
        sl = i % NS;
        grp = (i / NS) * 8 + (blockIdx.x & 7);
    } else {
        sl = blockIdx.x / G;
        grp = blockIdx.x - sl * G;
    }
    {
        const unsigned short* src = (const unsigned short*)p.w + (size_t)sl * KS * CHUNK;
        const unsigned loff = (unsigned)lane * 16;
#pragma unroll 1
        for (int i = wave; i < NLOAD; i += GX_WAVES)
            __builtin_amdgcn_global_load_lds((const void*)((const char*)src + (size_t)i * 1024 + loff),
                                             (__attribute__((address_space(3))) void*)(Wsl + i * 512), 16, 0, 0);
        if (HALF)
            for (int i = tid; i < 16 * NT; i += GX_WAVES * 64) Bs[i] = p.bias[sl * 16 * NT + i];
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // the slice is in LDS; no barrier after this one
    }
    // this lane's A-operand offset: row lr of a 16-row tile, k-group lg swizzled
    const unsigned short* wl = Wsl + lr * 32 + (hatk::ws_slot(lr, lg) * 8);
    float* out = p.out + (size_t)sl * NH * M * HD;  // the slice's first head
    float* Q = Qs + wave * 16 * QS_S;
    const int nsub = (M + TOK - 1) / TOK;
    const int stride = G * GX_WAVES;
    int sub = grp * GX_WAVES + wave;
    if (sub >= nsub) return;
    WcRows<K, MT> xr;
    xr.init(p.a, sub * TOK, M, lr);
    f32x4 y[MT][2];  // the rows of the next k-step
    xr.load_b(0, lg, y);
#pragma unroll 1
    for (; sub < nsub; sub += stride) {
        f32x4 acc[MT][NT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                acc[mt][nt] = HALF ? *(const f32x4*)(Bs + 16 * nt + 4 * lg) : (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const bool half = HALF && ks == KS - 1;  // compile-time: the loop is unrolled
            u32x4 xb[MT][3];
            if (half) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) half_operands(y[mt][0], xb[mt]);
            } else {
                split_pre(y, xb);
            }
            if (ks + 1 < KS) {
                if (HALF && ks + 1 == KS - 1) xr.load_half(lg, y);
                else xr.load_b(ks + 1, lg, y);
            } else {
                // the next subtile's first k-step, or (past the last) this
                // one's again: the loads are issued either way, so that their
                // count never depends on the path and the compiler's waits
                // stay exact
                xr.init(p.a, (sub + stride < nsub ? sub + stride : sub) * TOK, M, lr);
                xr.load_b(0, lg, y);
            }
            // weight fragments of tile nt + 2 read while tile nt's 6 MT MFMAs run
            const unsigned short* wr = wl + ks * CHUNK;
            u32x4 wa[3][3];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) wa[t][pl] = *(const u32x4*)(wr + t * 16 * 32 + pl * ROWS * 32);
            // The k-step's MFMAs at raised wave priority, so that the SIMD's
            // arbiter takes them ahead of the other wave's splits and epilogue
            // when both can issue: same-box 169.3 -> 166.5 us (C = 180: 321.0
            // -> 318.0). The same in the tails, the attention and the Winograd
            // convs measured 1-2.4% slower.
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                __builtin_amdgcn_sched_barrier(0);
                if (nt + 2 < NT) {
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl)
                        wa[(nt + 2) % 3][pl] = *(const u32x4*)(wr + (nt + 2) * 16 * 32 + pl * ROWS * 32);
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt][nt] = half ? mfma16x3(wa[nt % 3], xb[mt], acc[mt][nt]) : mfma16x6(wa[nt % 3], xb[mt], acc[mt][nt]);
            }
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int mb = sub * TOK + mt * 16;
            const int mrows = M - mb;
            if constexpr (HD == 24) {
                // Two heads at a time go through the wave's LDS region and leave
                // as 16 consecutive rows of each head (1536 contiguous bytes),
                // non-temporal. Row r's twelve float4 slots are rotated by
                // r >> 1, so that the writes (8 lanes: rows r0 .. r0 + 7 at one
                // slot) meet no bank conflicts in the 48-float rows.
                auto slot = [](int r, int s) {
                    const int v = s + (r >> 1);
                    return (v >= 12 ? v - 12 : v) * 4;
                };
#pragma unroll
                for (int ph = 0; ph < 3; ++ph) {
#pragma unroll
                    for (int t = 0; t < 3; ++t) *(f32x4*)(Q + lr * QS_S + slot(lr, t * 4 + lg)) = acc[mt][3 * ph + t];
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
#pragma unroll
                    for (int i2 = 0; i2 < 3; ++i2) {
                        const int f = lane + 64 * i2, hh = f / 96, r = (f - hh * 96) / 6, d4 = f - hh * 96 - r * 6;
                        const f32x4 v = *(const f32x4*)(Q + r * QS_S + slot(r, hh * 6 + d4));
                        // rows past M go to the sink (a store is issued either way)
                        float* dst = r < mrows ? out + ((size_t)(2 * ph + hh) * M + mb + r) * 24 + d4 * 4
                                               : hat_sink_row + d4 * 4;
                        __builtin_nontemporal_store(v, (f32x4*)dst);
                    }
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next phase's writes
                }
            } else {
                // All NH heads at once: 16 rows x 16 NT columns into the stage
                // (rows 100 floats apart, so that the writes, 8 lanes at rows
                // r0 .. r0 + 7, meet no bank conflicts), then 16 consecutive
                // rows of each head (30 floats, 1920 contiguous bytes) leave as
                // float2 pairs (a pair never straddles a row: head_dim is
                // even), non-temporal.
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) *(f32x4*)(Q + lr * QS_S + nt * 16 + lg * 4) = acc[mt][nt];
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
                // lane l < 4 PR: pair l % PR of row l / PR in each group of four
                // rows; group i2 is rows 4 (i2 % 4) .. +3 of head i2 / 4
                constexpr int PR = HD / 2;
                static_assert(4 * PR <= 64, "four rows of pairs per wave");
                const int rq = lane / PR, d2 = lane - rq * PR;
#pragma unroll
                for (int i2 = 0; i2 < 4 * NH; ++i2) {
                    const int hh = i2 / 4, r = 4 * (i2 % 4) + rq;
                    const f32x2 v = *(const f32x2*)(Q + (lane < 4 * PR ? r * QS_S + hh * HD + d2 * 2 : 0));
                    // lanes past the pairs and rows past M go to the sink
                    float* dst = lane < 4 * PR && r < mrows ? out + ((size_t)hh * M + mb + r) * HD + d2 * 2
                                                            : hat_sink_row + (lane & 31) * 2;
                    __builtin_nontemporal_store(v, (f32x2*)dst);
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next tile's writes
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(GX_WAVES * 64, 1) void hat_gemmx_qkv(GemmArgs p)
{
    __shared__ __attribute__((aligned(16))) unsigned short Wsl[5 * WS_CHUNK];  // the slice
    __shared__ __attribute__((aligned(16))) float Qs[GX_WAVES * 16 * gx_stage_stride(24)];  // per-wave staging
    __shared__ __attribute__((aligned(16))) float Bs[144];  // the slice's bias
    gemmx_qkv_body<144, 9, 3, 24, 6, 2>(p, Wsl, Qs, Bs);
}

extern "C" __global__ __launch_bounds__(GX_WAVES * 64, 1) void hat_gemmx_qkv180(GemmArgs p)
{
    __shared__ __attribute__((aligned(16))) unsigned short Wsl[6 * WS_CHUNK180];  // the slice
    __shared__ __attribute__((aligned(16))) float Qs[GX_WAVES * 16 * gx_stage_stride(30)];  // per-wave staging
    gemmx_qkv_body<180, 6, 6, 30, 3, 3>(p, Wsl, Qs, nullptr);
}
