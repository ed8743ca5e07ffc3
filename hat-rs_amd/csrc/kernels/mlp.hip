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
// (48 x KP) and fc2 columns (NO x 48) are double-buffered in LDS, with the next
// chunk's slices fetched into registers while this chunk computes (one barrier
// per chunk). Both GEMMs use v_mfma_f32_16x16x4_f32 with weights as the A
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

// PAD: the real K, hidden and output widths are below KP, NH, NO (C = 180);
// without it they are exactly KP, NH, NO and nothing is masked.
template <int EPI, int KP, int NH, int NO, bool PAD>
__device__ __forceinline__ void mlp_body(const MlpArgs& p)
{
    constexpr int NCH = NH / MLP_HC;             // hidden chunks
    constexpr int S1 = KP + 4;                   // LDS row stride of the fc1 slice [48][S1]
    constexpr int S2 = MLP_HC + 4;               // LDS row stride of the fc2 slice [NO][S2]
    constexpr int W1F4 = MLP_HC * KP / 4;        // float4 per fc1 slice
    constexpr int F4 = W1F4 + NO * MLP_HC / 4;   // + the fc2 slice
    constexpr int BUF = MLP_HC * S1 + NO * S2;
    constexpr int PER = (F4 + MLP_THREADS - 1) / MLP_THREADS;
    static_assert(NCH % 2 == 0, "chunk parity must repeat across tiles");
    static_assert(KP % 16 == 0 && NO % 16 == 0 && NH % MLP_HC == 0, "tile multiples");
    __shared__ float Wb[2 * BUF];
    // The per-column constants, read in every chunk and every epilogue, from
    // LDS rather than through the cache hierarchy: b1, then b2, nw, nb.
    __shared__ __attribute__((aligned(16))) float Cs[NH + 3 * NO];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int M = p.M;
    const int K = PAD ? p.K : KP, H = PAD ? p.H : NH, N = PAD ? p.N : NO;
    const int ntiles = (M + MLP_ROWS - 1) / MLP_ROWS;
    int tile = blockIdx.x;
    if (tile >= ntiles) return;  // whole block: no barrier has been passed yet

    // This thread's share of a chunk, float4 i: fc1 slice entries (row = the
    // hidden unit within the chunk, column k) then fc2 slice entries (row =
    // output column, column = hidden unit within the chunk). A float4 outside
    // the real weights (hidden >= H, fc2 column >= N) is zero.
    // Without padding the per-thread offsets are kept in registers (relative
    // to the chunk's uniform bases); with it they are recomputed, which leaves
    // the registers to the wider tiles.
    unsigned goff[PAD ? 1 : PER];
    int loff[PAD ? 1 : PER];
    if constexpr (!PAD) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = tid + i * MLP_THREADS;
            if (idx < W1F4) {
                const int r = idx / (KP / 4), c4 = idx - r * (KP / 4);
                goff[i] = r * p.ldw1 + c4 * 4;  // + chunk * 48 fc1 rows
                loff[i] = r * S1 + c4 * 4;
            } else {
                const int j = idx - W1F4;
                const int r = j / (MLP_HC / 4), c4 = j - r * (MLP_HC / 4);
                goff[i] = r * p.ldw2 + c4 * 4;  // + chunk * 48 fc2 columns
                loff[i] = MLP_HC * S1 + r * S2 + c4 * 4;
            }
        }
    }
    float4 stg[PER];
    auto fetch = [&](int c) {
        const int h0 = c * MLP_HC;
        const float* w1c = p.w1 + (size_t)h0 * p.ldw1;  // uniform chunk bases
        const float* w2c = p.w2 + h0;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = tid + i * MLP_THREADS;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (!PAD) {
                if (idx < W1F4) v = *(const float4*)(w1c + goff[i]);
                else if (idx < F4) v = *(const float4*)(w2c + goff[i]);
            } else if (idx < W1F4) {
                const int r = idx / (KP / 4), c4 = idx - r * (KP / 4);
                if (h0 + r < H) v = *(const float4*)(p.w1 + (size_t)(h0 + r) * p.ldw1 + c4 * 4);
            } else if (idx < F4) {
                const int j = idx - W1F4;
                const int r = j / (MLP_HC / 4), c4 = j - r * (MLP_HC / 4);
                if (r < N && h0 + c4 * 4 < H) v = *(const float4*)(p.w2 + (size_t)r * p.ldw2 + h0 + c4 * 4);
            }
            stg[i] = v;
        }
    };
    auto stash = [&](int buf) {
        float* B = Wb + buf * BUF;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = tid + i * MLP_THREADS;
            if constexpr (!PAD) {
                if (idx < F4) *(float4*)(B + loff[i]) = stg[i];
            } else if (idx < W1F4) {
                const int r = idx / (KP / 4), c4 = idx - r * (KP / 4);
                *(float4*)(B + r * S1 + c4 * 4) = stg[i];
            } else if (idx < F4) {
                const int j = idx - W1F4;
                const int r = j / (MLP_HC / 4), c4 = j - r * (MLP_HC / 4);
                *(float4*)(B + MLP_HC * S1 + r * S2 + c4 * 4) = stg[i];
            }
        }
    };
    // The residual is loaded a chunk ahead of the epilogue where the registers
    // allow it (the 144-wide shape).
    constexpr bool PRE = NO <= 144;
    constexpr int RN = PRE ? NO / 16 : 1;

    f32x4 xa[KP / 16];
    auto load_a = [&](int t) {
        const int m = t * MLP_ROWS + wave * 16 + lr;
        const float* arow = p.a + (size_t)(m < M ? m : 0) * K + lg * 4;
#pragma unroll
        for (int kc = 0; kc < KP / 16; ++kc) {
            f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
            // k beyond K (180 in 192) reads as zero: past it lies the next row
            if (m < M && (!PAD || kc * 16 + lg * 4 < K)) v = *(const f32x4*)(arow + kc * 16);
            xa[kc] = v;
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

    fetch(0);
    stash(0);
    load_a(tile);
    __syncthreads();

    for (; tile < ntiles; tile += gridDim.x) {
        const bool last_tile = tile + (int)gridDim.x >= ntiles;
        f32x4 acc2[1][NO / 16];
        f32x4 rres[1][RN];
#pragma unroll
        for (int j = 0; j < NO / 16; ++j) acc2[0][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
        for (int c = 0; c < NCH; ++c) {
            const float* B = Wb + (c & 1) * BUF;
            const bool more = c + 1 < NCH || !last_tile;  // block-uniform
            if (more) fetch(c + 1 < NCH ? c + 1 : 0);
            // The residual rows for the epilogue, one chunk ahead of it.
            if constexpr (PRE) {
                if (c == NCH - 1) {
                    const int m = tile * MLP_ROWS + wave * 16 + lr;
                    const float* rrow = p.res + (size_t)(m < M ? m : 0) * N + lg * 4;
#pragma unroll
                    for (int n2 = 0; n2 < RN; ++n2) {
                        f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
                        if (m < M && n2 * 16 + lg * 4 < N) v = *(const f32x4*)(rrow + n2 * 16);
                        rres[0][n2] = v;
                    }
                }
            }

            // fc1 for this chunk: h[16 rows][48] = a . w1[chunk]^T
            f32x4 h[MLP_HC / 16];
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt) h[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < KP / 16; ++kc)
#pragma unroll
                for (int nt = 0; nt < MLP_HC / 16; ++nt) {
                    const f32x4 wv = *(const f32x4*)(B + (nt * 16 + lr) * S1 + kc * 16 + lg * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s) h[nt] = mfma16(wv[s], xa[kc][s], h[nt]);
                }
            // The inputs are dead after the last chunk's fc1: fetch the next
            // tile's rows now, under this chunk's fc2 and the epilogue.
            if (c == NCH - 1 && !last_tile) load_a(tile + gridDim.x);
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt) {
                const float4 b4 = *(const float4*)(Cs + c * MLP_HC + nt * 16 + lg * 4);
                h[nt][0] = gelu(h[nt][0] + b4.x);
                h[nt][1] = gelu(h[nt][1] + b4.y);
                h[nt][2] = gelu(h[nt][2] + b4.z);
                h[nt][3] = gelu(h[nt][3] + b4.w);
            }
            // fc2 partial sums: out[16 rows][NO] += h . w2[:, chunk]^T
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt)
#pragma unroll
                for (int n2 = 0; n2 < NO / 16; ++n2) {
                    const f32x4 wv = *(const f32x4*)(B + MLP_HC * S1 + (n2 * 16 + lr) * S2 + nt * 16 + lg * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s) acc2[0][n2] = mfma16(wv[s], h[nt][s], acc2[0][n2]);
                }
            if (more) stash((c + 1) & 1);
            __syncthreads();
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
