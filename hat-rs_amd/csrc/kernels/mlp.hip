// Fused MLP on FP32 MFMA:
//   out = res + fc2(gelu(fc1(a)))   and, for EPI_RESID_LN, xn = LayerNorm(out).
//
// Replaces the reference's two lg_linear launches of the MLP (src/cuda.rs:
// 162-169; cpu.rs mlp, 1148-1160) with the GELU between them (cuda.rs:195-199)
// and the residual add / next LayerNorm after them (cuda.rs:227-248, 185-191).
// The hidden activation (T x 2C) never reaches HBM.
//
// A block of 8 waves walks 128-row tiles (persistent over gridDim.x); wave w
// owns rows [16w, 16w+16) and keeps their C inputs in registers for the whole
// tile. The hidden dimension is walked in chunks of 48: the chunk's fc1 rows
// (48 x KP) and fc2 columns (NO x 48) are double-buffered in LDS, the next
// chunk's slices copied global -> LDS by the loads that write LDS directly
// (global_load_lds_dwordx4, lane l of a wave's load filling 16 bytes at the
// load's LDS base + 16 l) while this chunk computes, one barrier per chunk. The
// slices sit unpadded in LDS with each row's float4 XOR-swizzled so the MFMA
// operand reads of 16 consecutive rows hit 16 distinct bank groups: the lanes
// choose which global float4 lands in their slot. Both GEMMs use v_mfma_f32_16x16x4_f32 with weights as the A
// operand, so fc1's accumulators - lane (r, g) holds hidden units 4g..4g+3 of
// each 16-unit tile for row r - are exactly the B operand fc2 needs for k =
// 4g..4g+3: after bias + GELU they feed fc2 with no data movement. The fc2
// accumulators then have the layout of the GEMM kernels' epilogue, which is
// reused (bias, residual, LayerNorm of whole rows).
//
// Shapes: C = 144 (KP = 144, hidden 288, NO = 144) and C = 180 (K 180 in
// KP = 192, hidden 360 in NH = 384, NO = 192). Padding is zero: weights past
// the real rows / columns are not read, and GELU(0 + 0) = 0 feeds fc2 nothing.
//
// Included after gemm.hip (gemm_epilogue) in the one translation unit.

#define MLP_HC 48  // hidden units per chunk
#define MLP_THREADS (MLP_WAVES * 64)

// The LDS slots that lie past the real weights (the padded C = 180 shape) load
// from hat_zero_row, since a direct-to-LDS load always writes its slot.

// Swizzle of float4 column c4 in LDS row `row` of a slice whose rows are R
// float4 long: rows r..r+15 read at one c4 land in 16 distinct groups of four
// banks (R = 36 or 12: rows 4 apart share a bank offset, the XOR separates
// them; R = 48: all rows share one, the XOR spreads them over 16).
template <int R>
__device__ __forceinline__ int mlp_swz(int row)
{
    static_assert(R % 16 == 0 || R % 16 == 4 || R % 16 == 12, "slice row length");
    return R % 16 == 0 ? (row & 15) : ((row >> 2) & 3);
}

// PAD: the real K, hidden and output widths are below KP, NH, NO (C = 180);
// without it they are exactly KP, NH, NO and nothing is masked.
template <int EPI, int KP, int NH, int NO, bool PAD>
__device__ __forceinline__ void mlp_body(const MlpArgs& p)
{
    constexpr int NCH = NH / MLP_HC;             // hidden chunks
    constexpr int R1 = KP / 4;                   // float4 per fc1 slice row [48][R1]
    constexpr int R2 = MLP_HC / 4;               // float4 per fc2 slice row [NO][R2]
    constexpr int W1F4 = MLP_HC * R1;            // float4 per fc1 slice
    constexpr int F4 = W1F4 + NO * R2;           // + the fc2 slice
    constexpr int BUF = F4 * 4;
    constexpr int PER = (F4 + MLP_THREADS - 1) / MLP_THREADS;
    static_assert(NCH % 2 == 0, "chunk parity must repeat across tiles");
    static_assert(KP % 16 == 0 && NO % 16 == 0 && NH % MLP_HC == 0, "tile multiples");
    static_assert(W1F4 % 64 == 0 && F4 % 64 == 0, "a wave's load lies in one slice");
    // The two chunk buffers are separate objects and every access names one at
    // compile time (chunk c uses buffer c & 1): the compiler then knows that a
    // read of one does not depend on the DMA filling the other, and does not
    // wait for it.
    __shared__ __attribute__((aligned(16))) float Wb0[BUF];
    __shared__ __attribute__((aligned(16))) float Wb1[BUF];
    // The per-column constants, read in every chunk and every epilogue, from
    // LDS rather than through the cache hierarchy: b1, then b2, nw, nb.
    __shared__ __attribute__((aligned(16))) float Cs[NH + 3 * NO];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int M = p.M;
    const int K = PAD ? p.K : KP, H = PAD ? p.H : NH, N = PAD ? p.N : NO;
    const int ntiles = (M + MLP_ROWS - 1) / MLP_ROWS;
    int tile = blockIdx.x;
    if (tile >= ntiles) return;  // whole block: no barrier has been passed yet

    // This thread's LDS slots of a chunk, float4 idx = tid + 512 i: fc1 slice
    // slots (row = the hidden unit within the chunk) then fc2 slice slots (row =
    // output column); the lane fetches the global float4 whose swizzled column
    // is the slot's. Without padding the global offsets (relative to the
    // chunk's bases) are kept in registers; with it they are recomputed and
    // slots past the real weights read hat_zero_row.
    unsigned goff[PAD ? 1 : PER];
    if constexpr (!PAD) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = tid + i * MLP_THREADS;
            if (idx < W1F4) {
                const int r = idx / R1, c4 = (idx - r * R1) ^ mlp_swz<R1>(r);
                goff[i] = r * p.ldw1 + c4 * 4;  // + chunk * 48 fc1 rows
            } else {
                const int j = idx - W1F4;
                const int r = j / R2, c4 = (j - r * R2) ^ mlp_swz<R2>(r);
                goff[i] = r * p.ldw2 + c4 * 4;  // + chunk * 48 fc2 columns
            }
        }
    }
    // Chunk c's slices into LDS buffer buf. The LDS side of each load is the
    // wave's 64 consecutive slots; the writes land asynchronously, so a
    // vmcnt(0) wait precedes the barrier that publishes them.
    auto fetch = [&](int c, auto bufc) {
        const int h0 = c * MLP_HC;
        const float* w1c = p.w1 + (size_t)h0 * p.ldw1;  // uniform chunk bases
        const float* w2c = p.w2 + h0;
        float* B = decltype(bufc)::value ? Wb1 : Wb0;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int base = i * MLP_THREADS + wave * 64;  // wave-uniform
            if (base >= F4) break;
            int idx = base + lane;
            // (with padding) an index the compiler cannot see through, so the
            // per-slot addresses are recomputed here instead of hoisted out of
            // the loops and kept, 64 bits each
            if constexpr (PAD) asm volatile("" : "+v"(idx));
            const float* src;
            if constexpr (!PAD) {
                src = (base < W1F4 ? w1c : w2c) + goff[i];
            } else if (base < W1F4) {
                const int r = idx / R1, c4 = (idx - r * R1) ^ mlp_swz<R1>(r);
                src = h0 + r < H ? p.w1 + (size_t)(h0 + r) * p.ldw1 + c4 * 4 : hat_zero_row;
            } else {
                const int j = idx - W1F4;
                const int r = j / R2, c4 = (j - r * R2) ^ mlp_swz<R2>(r);
                src = r < N && h0 + c4 * 4 < H ? p.w2 + (size_t)r * p.ldw2 + h0 + c4 * 4 : hat_zero_row;
            }
            __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(B + base * 4),
                                             16, 0, 0);
        }
    };
    // The residual is loaded a chunk ahead of the epilogue where the registers
    // allow it (the 144-wide shape).
    constexpr bool PRE = NO <= 144;
    constexpr int RN = PRE ? NO / 16 : 1;

    f32x4 xa[KP / 16];
    auto load_a = [&](int t) {
        const int m = t * MLP_ROWS + wave * 16 + lr;
        const float* arow = m < M ? p.a + (size_t)m * K + lg * 4 : hat_zero_row;  // + kc*16 stays in it
#pragma unroll
        for (int kc = 0; kc < KP / 16; ++kc) {
            // k beyond K (180 in 192) reads as zero: past it lies the next row
            xa[kc] = load_or_zero(arow + kc * 16, !PAD || kc * 16 + lg * 4 < K);
        }
    };

    for (int i = tid; i < NH + 3 * NO; i += MLP_THREADS) {
        float v = 0.0f;
        if (i < NH) {
            if (i < H) v = p.b1[i];
        } else {
            const int j = (i - NH) % NO, which = (i - NH) / NO;
            if (j < N) {
                if (which == 0) v = p.b2[j];
                else if (EPI == EPI_RESID_LN) v = which == 1 ? p.nw[j] : p.nb[j];
            }
        }
        Cs[i] = v;
    }
    GemmArgs g{};
    g.out = p.out;
    g.res = p.res;
    g.xn = p.xn;
    const EpiConsts kc{Cs + NH, Cs + NH + NO, Cs + NH + 2 * NO};
    g.M = M;
    g.N = N;
    g.ldo = N;
    g.eps = p.eps;

    // The lane's swizzled float4 column in the operand reads: rows nt*16 + lr
    // and n2*16 + lr give (row >> 2) & 3 == (lr >> 2) & 3 and row & 15 == lr.
    static_assert(R2 % 16 != 0, "the fc2 slice's swizzle is the 2-bit one");
    const int sg = lg ^ mlp_swz<R1>(lr), sg2 = lg ^ mlp_swz<R2>(lr);
    fetch(0, CInt<0>{});
    load_a(tile);
    __builtin_amdgcn_s_waitcnt(0);  // the LDS writes of fetch have landed
    __syncthreads();

    for (; tile < ntiles; tile += gridDim.x) {
        const bool last_tile = tile + (int)gridDim.x >= ntiles;
        f32x4 acc2[1][NO / 16];
        f32x4 rres[1][RN];
#pragma unroll
        for (int j = 0; j < NO / 16; ++j) acc2[0][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
        auto chunk = [&](int c, auto bufc) {
            constexpr int Q = decltype(bufc)::value;  // c & 1
            const float* B = Q ? Wb1 : Wb0;
            const bool more = c + 1 < NCH || !last_tile;  // block-uniform
            // the other buffer was last read in the previous chunk, before its barrier
            if (more) fetch(c + 1 < NCH ? c + 1 : 0, CInt<Q ^ 1>{});
            // The residual rows for the epilogue, one chunk ahead of it.
            if constexpr (PRE) {
                if (c == NCH - 1) {
                    const int m = tile * MLP_ROWS + wave * 16 + lr;
                    const float* rrow = m < M ? p.res + (size_t)m * N + lg * 4 : hat_zero_row;
#pragma unroll
                    for (int n2 = 0; n2 < RN; ++n2) {
                        rres[0][n2] = load_or_zero(rrow + n2 * 16, n2 * 16 + lg * 4 < N);
                    }
                }
            }

            // fc1 for this chunk: h[16 rows][48] = b1 + a . w1[chunk]^T, the
            // accumulators starting from the bias (cpu.rs linear's order)
            f32x4 h[MLP_HC / 16];
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt) h[nt] = *(const f32x4*)(Cs + c * MLP_HC + nt * 16 + lg * 4);
            // per 16-k step: the three weight reads, then their 12 MFMAs
#pragma unroll
            for (int kc = 0; kc < KP / 16; ++kc) {
                __builtin_amdgcn_sched_barrier(0);
                // physical column: (kc*4 + lg) ^ swizzle, which for R1 % 16 != 0
                // (a 2-bit swizzle) is kc*4 + (lg ^ swizzle)
                const int pc = R1 % 16 == 0 ? ((kc * 4 + lg) ^ lr) : kc * 4 + sg;
                f32x4 wv[MLP_HC / 16];
#pragma unroll
                for (int nt = 0; nt < MLP_HC / 16; ++nt) wv[nt] = *(const f32x4*)(B + (nt * 16 + lr) * KP + pc * 4);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int nt = 0; nt < MLP_HC / 16; ++nt) h[nt] = mfma16(wv[nt][s], xa[kc][s], h[nt]);
            }
            // The inputs are dead after the last chunk's fc1: fetch the next
            // tile's rows now, under this chunk's fc2 and the epilogue.
            if (c == NCH - 1 && !last_tile) load_a(tile + gridDim.x);
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt)
#pragma unroll
                for (int j = 0; j < 4; ++j) h[nt][j] = gelu(h[nt][j]);
            // fc2 partial sums: out[16 rows][NO] += h . w2[:, chunk]^T, three
            // output column tiles at a time: their reads, then 12 MFMAs
            static_assert((NO / 16) % 3 == 0, "output column tiles go in threes");
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt)
#pragma unroll
                for (int g3 = 0; g3 < NO / 16; g3 += 3) {
                    __builtin_amdgcn_sched_barrier(0);
                    f32x4 wv[3];
#pragma unroll
                    for (int j = 0; j < 3; ++j)
                        wv[j] = *(const f32x4*)(B + W1F4 * 4 + ((g3 + j) * 16 + lr) * MLP_HC + nt * 16 + sg2 * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int j = 0; j < 3; ++j) acc2[0][g3 + j] = mfma16(wv[j][s], h[nt][s], acc2[0][g3 + j]);
                }
            __builtin_amdgcn_s_waitcnt(0);  // the next chunk's LDS writes have landed
            __syncthreads();
        };
#pragma unroll 1
        for (int c = 0; c < NCH; c += 2) {
            chunk(c, CInt<0>{});
            chunk(c + 1, CInt<1>{});
        }
        if constexpr (PRE)
            gemm_epilogue<1, NO / 16, EPI>(g, kc, acc2, tile * MLP_ROWS + wave * 16, 0, lr, lg, nullptr, rres);
        else
            gemm_epilogue<1, NO / 16, EPI>(g, kc, acc2, tile * MLP_ROWS + wave * 16, 0, lr, lg, nullptr);
    }
}

#define MLP_INST(NAME, EPI, KP, NH, NO, PAD)                                                 \
    extern "C" __global__ __launch_bounds__(MLP_THREADS) void NAME(MlpArgs p)                \
    {                                                                                        \
        mlp_body<EPI, KP, NH, NO, PAD>(p);                                                   \
    }

MLP_INST(hat_mlp_resid, EPI_RESID, 144, 288, 144, false)
MLP_INST(hat_mlp_resid_ln, EPI_RESID_LN, 144, 288, 144, false)
MLP_INST(hat_mlp12_resid, EPI_RESID, 192, 384, 192, true)
MLP_INST(hat_mlp12_resid_ln, EPI_RESID_LN, 192, 384, 192, true)
