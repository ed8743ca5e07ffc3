// Fused MLP of the C = 144 family on FP32 MFMA:
//   out = res + fc2(gelu(fc1(a)))   and, for EPI_RESID_LN, xn = LayerNorm(out).
//
// Replaces the reference's two lg_linear launches of the MLP (src/cuda.rs:
// 162-169; cpu.rs mlp, 1148-1160) with the GELU between them (cuda.rs:195-199)
// and the residual add / next LayerNorm after them (cuda.rs:227-248, 185-191).
// The hidden activation (T x 288) never reaches HBM.
//
// A block of 8 waves walks 128-row tiles (persistent over gridDim.x); wave w
// owns rows [16w, 16w+16) and keeps their 144 inputs in registers for the whole
// tile. The hidden dimension is walked in 6 chunks of 48: the chunk's fc1 rows
// (48 x 144) and fc2 columns (144 x 48) are double-buffered in LDS, with the
// next chunk's slices fetched into registers while this chunk computes (one
// barrier per chunk). Both GEMMs use v_mfma_f32_16x16x4_f32 with weights as the
// A operand, so fc1's accumulators - lane (r, g) holds hidden units 4g..4g+3 of
// each 16-unit tile for row r - are exactly the B operand fc2 needs for k =
// 4g..4g+3: after bias + GELU they feed fc2 with no data movement. The fc2
// accumulators then have the layout of the GEMM kernels' epilogue, which is
// reused (bias, residual, LayerNorm of whole rows).
//
// Included after gemm.hip (gemm_epilogue) in the one translation unit.

#define MLP_HC 48                           // hidden units per chunk
#define MLP_NCH (MLP_H / MLP_HC)            // 6
#define MLP_S1 (MLP_C + 4)                  // LDS row stride of the fc1 slice [48][148]
#define MLP_S2 (MLP_HC + 4)                 // LDS row stride of the fc2 slice [144][52]
#define MLP_W1F4 (MLP_HC * MLP_C / 4)       // 1728 float4 per fc1 slice
#define MLP_F4 (2 * MLP_W1F4)               // fc2 slice has as many
#define MLP_BUF (MLP_HC * MLP_S1 + MLP_C * MLP_S2)
#define MLP_THREADS (MLP_WAVES * 64)
#define MLP_PER ((MLP_F4 + MLP_THREADS - 1) / MLP_THREADS)  // 7

template <int EPI>
__device__ __forceinline__ void mlp_body(const MlpArgs& p)
{
    static_assert(MLP_NCH % 2 == 0, "chunk parity must repeat across tiles");
    __shared__ float Wb[2 * MLP_BUF];
    // The per-column constants, read in every chunk and every epilogue, from
    // LDS rather than through the cache hierarchy: b1, then b2, nw, nb.
    __shared__ __attribute__((aligned(16))) float Cs[MLP_H + 3 * MLP_C];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int M = p.M;
    const int ntiles = (M + MLP_ROWS - 1) / MLP_ROWS;
    int tile = blockIdx.x;
    if (tile >= ntiles) return;  // whole block: no barrier has been passed yet

    // This thread's share of a chunk: global offset (relative to the chunk) and
    // LDS offset of each of its float4, for the fc1 rows then the fc2 columns.
    unsigned goff[MLP_PER];
    int loff[MLP_PER];
#pragma unroll
    for (int i = 0; i < MLP_PER; ++i) {
        const int idx = tid + i * MLP_THREADS;
        if (idx < MLP_W1F4) {
            const int r = idx / (MLP_C / 4), c4 = idx - r * (MLP_C / 4);
            goff[i] = r * MLP_C + c4 * 4;  // + chunk * 48 * 144 (w1 rows)
            loff[i] = r * MLP_S1 + c4 * 4;
        } else {
            const int j = idx - MLP_W1F4;
            const int r = j / (MLP_HC / 4), c4 = j - r * (MLP_HC / 4);
            goff[i] = r * MLP_H + c4 * 4;  // + chunk * 48 (w2 columns)
            loff[i] = MLP_HC * MLP_S1 + r * MLP_S2 + c4 * 4;
        }
    }
    float4 stg[MLP_PER];
    auto fetch = [&](int c) {
        // uniform chunk bases + 32-bit per-thread offsets
        const float* w1c = p.w1 + c * MLP_HC * MLP_C;
        const float* w2c = p.w2 + c * MLP_HC;
#pragma unroll
        for (int i = 0; i < MLP_PER; ++i) {
            const int idx = tid + i * MLP_THREADS;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (idx < MLP_W1F4)
                v = *(const float4*)(w1c + goff[i]);
            else if (idx < MLP_F4)
                v = *(const float4*)(w2c + goff[i]);
            stg[i] = v;
        }
    };
    auto stash = [&](int buf) {
        float* B = Wb + buf * MLP_BUF;
#pragma unroll
        for (int i = 0; i < MLP_PER; ++i)
            if (tid + i * MLP_THREADS < MLP_F4) *(float4*)(B + loff[i]) = stg[i];
    };

    f32x4 xa[MLP_C / 16];
    auto load_a = [&](int t) {
        const int m = t * MLP_ROWS + wave * 16 + lr;
        const float* arow = p.a + (size_t)(m < M ? m : 0) * MLP_C + lg * 4;
#pragma unroll
        for (int kc = 0; kc < MLP_C / 16; ++kc) {
            f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
            if (m < M) v = *(const f32x4*)(arow + kc * 16);
            xa[kc] = v;
        }
    };

    for (int i = tid; i < MLP_H + 3 * MLP_C; i += MLP_THREADS) {
        float v;
        if (i < MLP_H) v = p.b1[i];
        else if (i < MLP_H + MLP_C) v = p.b2[i - MLP_H];
        else if (EPI != EPI_RESID_LN) v = 0.0f;
        else if (i < MLP_H + 2 * MLP_C) v = p.nw[i - MLP_H - MLP_C];
        else v = p.nb[i - MLP_H - 2 * MLP_C];
        Cs[i] = v;
    }
    GemmArgs g{};
    g.out = p.out;
    g.res = p.res;
    g.xn = p.xn;
    const EpiConsts kc{Cs + MLP_H, Cs + MLP_H + MLP_C, Cs + MLP_H + 2 * MLP_C};
    g.M = M;
    g.N = MLP_C;
    g.ldo = MLP_C;
    g.eps = p.eps;

    fetch(0);
    stash(0);
    load_a(tile);
    __syncthreads();

    for (; tile < ntiles; tile += gridDim.x) {
        const bool last_tile = tile + (int)gridDim.x >= ntiles;
        f32x4 acc2[1][MLP_C / 16];
        f32x4 rres[1][MLP_C / 16];
#pragma unroll
        for (int j = 0; j < MLP_C / 16; ++j) acc2[0][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
        for (int c = 0; c < MLP_NCH; ++c) {
            const float* B = Wb + (c & 1) * MLP_BUF;
            const bool more = c + 1 < MLP_NCH || !last_tile;  // block-uniform
            if (more) fetch(c + 1 < MLP_NCH ? c + 1 : 0);
            // The residual rows for the epilogue, one chunk ahead of it.
            if (c == MLP_NCH - 1) {
                const int m = tile * MLP_ROWS + wave * 16 + lr;
                const float* rrow = p.res + (size_t)(m < M ? m : 0) * MLP_C + lg * 4;
#pragma unroll
                for (int n2 = 0; n2 < MLP_C / 16; ++n2) {
                    f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
                    if (m < M) v = *(const f32x4*)(rrow + n2 * 16);
                    rres[0][n2] = v;
                }
            }

            // fc1 for this chunk: h[16 rows][48] = a . w1[chunk]^T
            f32x4 h[MLP_HC / 16];
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt) h[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < MLP_C / 16; ++kc)
#pragma unroll
                for (int nt = 0; nt < MLP_HC / 16; ++nt) {
                    const f32x4 wv = *(const f32x4*)(B + (nt * 16 + lr) * MLP_S1 + kc * 16 + lg * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s) h[nt] = mfma16(wv[s], xa[kc][s], h[nt]);
                }
            // The inputs are dead after the last chunk's fc1: fetch the next
            // tile's rows now, under this chunk's fc2 and the epilogue.
            if (c == MLP_NCH - 1 && !last_tile) load_a(tile + gridDim.x);
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt) {
                const float4 b4 = *(const float4*)(Cs + c * MLP_HC + nt * 16 + lg * 4);
                h[nt][0] = gelu(h[nt][0] + b4.x);
                h[nt][1] = gelu(h[nt][1] + b4.y);
                h[nt][2] = gelu(h[nt][2] + b4.z);
                h[nt][3] = gelu(h[nt][3] + b4.w);
            }
            // fc2 partial sums: out[16 rows][144] += h . w2[:, chunk]^T
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt)
#pragma unroll
                for (int n2 = 0; n2 < MLP_C / 16; ++n2) {
                    const f32x4 wv =
                        *(const f32x4*)(B + MLP_HC * MLP_S1 + (n2 * 16 + lr) * MLP_S2 + nt * 16 + lg * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s) acc2[0][n2] = mfma16(wv[s], h[nt][s], acc2[0][n2]);
                }
            if (more) stash((c + 1) & 1);
            __syncthreads();
        }
        gemm_epilogue<1, MLP_C / 16, EPI>(g, kc, acc2, tile * MLP_ROWS + wave * 16, 0, lr, lg, nullptr, rres);
    }
}

extern "C" __global__ __launch_bounds__(MLP_THREADS) void hat_mlp_resid(MlpArgs p) { mlp_body<EPI_RESID>(p); }
extern "C" __global__ __launch_bounds__(MLP_THREADS) void hat_mlp_resid_ln(MlpArgs p)
{
    mlp_body<EPI_RESID_LN>(p);
}
