// 3x3 convolution (stride 1, zero padding 1) over NHWC with all BN = 16*NT
// output channels of a column block in one block, so that for BN = C the
// GEMM epilogues apply: bias + residual and the LayerNorm of whole rows.
//
// Used for the C -> C convs of the trunk: conv_first (+ patch_embed.norm), the
// RHAG conv (+ stage input, + the next stage's norm1 or the final norm) and
// conv_after_body (+ the conv_first skip) - lg_conv3x3_winograd at gpu.rs:605,
// 722, 742 with the lg_add and lg_channel_layer_norm passes that follow them
// (cuda.rs:227-248, 185-191).
//
// A block owns a 16x16 pixel tile; 8 waves owning two tile rows each; a tile
// row is one 16-pixel MFMA tile, lane l%16 the pixel's x. Input channels are
// walked in chunks of 16: the chunk's 18x18 halo patch and its [9 taps][BN][16]
// weight slice are staged in LDS (with BN = 144: 20.7 KB + 83 KB), the next
// chunk's data travelling through registers while this chunk's MFMAs run, and
// every tap reads the patch at an offset. The input is read once per column
// block (the C -> C convs have one), the weights once per 256 pixels.
//
// Included after gemm.hip (gemm_epilogue) in the one translation unit.

#define CW_T 16                        // output tile side
#define CW_P (CW_T + 2)                // halo side
#define CW_PX (CW_P * CW_P)            // 324 halo pixels

// HEAD selects a direct epilogue instead of a GEMM one: CEPI_SHUFFLE (store
// into the PixelShuffle'd plane, channels pre-permuted at upload), CEPI_STORE
// (bias + activation) or CEPI_COLSUM (bias, store, per-tile column sums);
// -1 = none (EPI applies).
template <int NT, int EPI, int HEAD, int WAVES>
__device__ __forceinline__ void convw_body(const ConvArgs& p)
{
    constexpr int MT = CW_T / WAVES;               // tile rows per wave
    constexpr int CW_THREADS = WAVES * 64;
    static_assert(MT * WAVES == CW_T, "waves must split the tile rows");
    constexpr int BN = 16 * NT;
    constexpr int PF4 = CW_PX * 4;                 // patch float4 per chunk
    constexpr int WF4 = 9 * BN * 4;                // weight float4 per chunk
    constexpr int PPER = (PF4 + CW_THREADS - 1) / CW_THREADS;
    constexpr int WPER = (WF4 + CW_THREADS - 1) / CW_THREADS;
    __shared__ __attribute__((aligned(16))) float Ps[CW_PX * 16];
    __shared__ __attribute__((aligned(16))) float Ws[9 * BN * 16];
    __shared__ __attribute__((aligned(16))) float Cs[3 * BN];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int H = p.H, W = p.W;
    const int tiles_x = W / CW_T;
    const int ty0 = (blockIdx.x / tiles_x) * CW_T;
    const int tx0 = (blockIdx.x % tiles_x) * CW_T;
    const int co0 = blockIdx.y * BN;
    constexpr bool LNOUT = EPI == EPI_RESID_LN || EPI == EPI_STORE_LN;

    // Column constants (bias, LayerNorm weight and bias) of the block.
    for (int i = tid; i < (LNOUT ? 3 : 1) * BN; i += CW_THREADS) {
        const int j = i % BN, co = co0 + j;
        const float* src = i < BN ? p.bias : (i < 2 * BN ? p.nw : p.nb);
        Cs[i] = co < p.CO ? src[co] : 0.0f;
    }

    float4 pst[PPER], wst[WPER];
    auto fetch = [&](int cc) {
        const int ci0 = cc * 16;
#pragma unroll
        for (int i = 0; i < PPER; ++i) {
            const int idx = tid + i * CW_THREADS;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (idx < PF4) {
                const int pix = idx >> 2, c4 = (idx & 3) * 4;
                const int py = pix / CW_P, px = pix - py * CW_P;
                const int y = ty0 + py - 1, x = tx0 + px - 1;
                const int ci = ci0 + c4;
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
            }
            pst[i] = v;
        }
        // packed weights [chunk][tap][COp][16]: this block's BN rows of each tap
        const float* wc = p.w + (size_t)cc * 9 * p.COp * 16;
#pragma unroll
        for (int i = 0; i < WPER; ++i) {
            const int idx = tid + i * CW_THREADS;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (idx < WF4) {
                const int row = idx >> 2, c4 = (idx & 3) * 4;
                const int tap = row / BN, co = row - tap * BN;
                if (co0 + co < p.COp) v = *(const float4*)(wc + ((size_t)tap * p.COp + co0 + co) * 16 + c4);
            }
            wst[i] = v;
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < PPER; ++i) {
            const int idx = tid + i * CW_THREADS;
            if (idx < PF4) *(float4*)(Ps + idx * 4) = pst[i];
        }
#pragma unroll
        for (int i = 0; i < WPER; ++i) {
            const int idx = tid + i * CW_THREADS;
            if (idx < WF4) *(float4*)(Ws + idx * 4) = wst[i];
        }
    };

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // The residual of the GEMM epilogues, loaded under the last chunk's MFMAs
    // (loaded in the epilogue, each row's loads would wait in turn).
    constexpr bool PRE = HEAD < 0 && (EPI == EPI_RESID || EPI == EPI_RESID_LN);
    f32x4 rres[PRE ? MT : 1][NT];
    auto load_res = [&]() {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const size_t m = (size_t)(ty0 + wave * MT + mt) * W + tx0 + lr;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int co = co0 + nt * 16 + lg * 4;
                rres[mt][nt] = load_or_zero(p.res + m * p.co_stride + co, co < p.CO);
            }
        }
    };

    auto chunk_mfma = [&]() {
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int dy = tap / 3, dx = tap - dy * 3;
            f32x4 xv[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                xv[mt] = *(const f32x4*)(Ps + ((wave * MT + mt + dy) * CW_P + lr + dx) * 16 + lg * 4);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f32x4 wv = *(const f32x4*)(Ws + (tap * BN + nt * 16 + lr) * 16 + lg * 4);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma16(wv[s], xv[mt][s], acc[mt][nt]);
            }
        }
    };

    const int nchunks = p.CIp / 16;
    fetch(0);
    if constexpr (PRE) {
        // The last chunk is peeled: it loads the residual where the others
        // load the next chunk (in the loop, the residual's registers would be
        // held across it, beside the staging registers).
#pragma unroll 1
        for (int cc = 0; cc + 1 < nchunks; ++cc) {
            __syncthreads();  // every read of the previous chunk is done
            stash();
            __syncthreads();
            fetch(cc + 1);
            chunk_mfma();
        }
        __syncthreads();
        stash();
        __syncthreads();
        load_res();
        chunk_mfma();
    } else {
        // (the MFMAs written out here rather than through chunk_mfma: through
        // the lambda the compiler copies accumulators around in this loop)
#pragma unroll 1
        for (int cc = 0; cc < nchunks; ++cc) {
            __syncthreads();  // every read of the previous chunk is done
            stash();
            __syncthreads();
            if (cc + 1 < nchunks) fetch(cc + 1);
#pragma unroll
            for (int tap = 0; tap < 9; ++tap) {
                const int dy = tap / 3, dx = tap - dy * 3;
                f32x4 xv[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    xv[mt] = *(const f32x4*)(Ps + ((wave * MT + mt + dy) * CW_P + lr + dx) * 16 + lg * 4);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const f32x4 wv = *(const f32x4*)(Ws + (tap * BN + nt * 16 + lr) * 16 + lg * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma16(wv[s], xv[mt][s], acc[mt][nt]);
                }
            }
        }
    }

    if (HEAD == CEPI_SHUFFLE || HEAD == CEPI_STORE || HEAD == CEPI_COLSUM) {
        // Lane (lr, lg) holds channels co .. co+3 of pixel (y, x), x = tx0 + lr.
        f32x4 colsum[HEAD == CEPI_COLSUM ? NT : 1];
#pragma unroll
        for (int nt = 0; nt < (HEAD == CEPI_COLSUM ? NT : 1); ++nt) colsum[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int y = ty0 + wave * MT + mt, x = tx0 + lr;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int j0 = nt * 16 + lg * 4, co = co0 + j0;
                if (co >= p.CO) continue;
                const float4 b4 = *(const float4*)(Cs + j0);
                f32x4 v = acc[mt][nt] + (f32x4){b4.x, b4.y, b4.z, b4.w};
                if (HEAD == CEPI_COLSUM) {
                    colsum[nt] += v;
                    *(float4*)(p.out + ((size_t)y * W + x) * p.co_stride + co) = make_float4(v[0], v[1], v[2], v[3]);
                } else if (HEAD == CEPI_STORE) {
                    if (p.act == 2) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) v[j] = v[j] < 0.0f ? v[j] * 0.01f : v[j];
                    } else if (p.act == 1) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) v[j] = gelu(v[j]);
                    }
                    *(float4*)(p.out + ((size_t)y * W + x) * p.co_stride + co) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
                    // o' = (i*r + jj)*Cf + c lands at pixel (y*r + i, x*r + jj), channel c
                    const int r = p.r, Cf = p.CO / (r * r);
                    const int sub = co / Cf, c = co - sub * Cf;
                    const int i = sub / r, jj = sub - i * r;
                    *(float4*)(p.out + ((size_t)(y * r + i) * (W * r) + x * r + jj) * p.co_stride + c) =
                        make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        }
        if (HEAD == CEPI_COLSUM) {
            // Column sums of the block's 256 pixels (lg_channel_mean's first
            // stage, cuda.rs:259-272): over the 16 pixels of a tile row (the
            // lanes with equal lg), then over the waves through LDS (the patch
            // buffer, free once every wave is past its last chunk), in a fixed
            // order; one partial row per tile, [tile][co_stride].
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float v = colsum[nt][j];
                    v += __shfl_xor(v, 1, 64);
                    v += __shfl_xor(v, 2, 64);
                    v += __shfl_xor(v, 4, 64);
                    v += __shfl_xor(v, 8, 64);
                    colsum[nt][j] = v;
                }
            static_assert(WAVES * BN <= CW_PX * 16, "the column partials fit the patch buffer");
            __syncthreads();
            if (lr == 0) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) *(f32x4*)(Ps + wave * BN + nt * 16 + lg * 4) = colsum[nt];
            }
            __syncthreads();
            for (int c = tid; c < BN; c += CW_THREADS) {
                const int co = co0 + c;
                if (co < p.CO) {
                    float v = 0.0f;
                    for (int w = 0; w < WAVES; ++w) v += Ps[w * BN + c];
                    p.partial[(size_t)blockIdx.x * p.co_stride + co] = v;
                }
            }
        }
        return;
    }

    // Rows of the epilogue are pixels: m = y*W + x, 16 consecutive per tile row.
    GemmArgs g{};
    g.out = p.out;
    g.res = p.res;
    g.xn = p.xn;
    g.M = H * W;
    g.N = p.CO;
    g.ldo = p.co_stride;
    g.eps = p.eps;
    const EpiConsts kc{Cs, LNOUT ? Cs + BN : nullptr, LNOUT ? Cs + 2 * BN : nullptr};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        f32x4 a1[1][NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) a1[0][nt] = acc[mt][nt];
        const int y = ty0 + wave * MT + mt;
        // conv_first (EPI_STORE_LN): its raw output is read only by
        // conv_after_body at the end of the forward, so it goes out
        // non-temporal and leaves the last-level cache to the LayerNorm'd
        // rows, which the next kernel reads at once (that LayerNorm: 53.5 ->
        // 48.8 us)
        gemm_epilogue<1, NT, EPI, false, false, EPI == EPI_STORE_LN>(g, kc, a1, y * W + tx0, co0, lr, lg, nullptr,
                                  PRE ? (const f32x4(*)[NT]) & rres[PRE ? mt : 0] : nullptr);
    }
}

// Waves per block: CONVW_WAVES_* (kargs.h), 8 (two tile rows each) or 16 (one).
#define CONVW_INST(NAME, NT, EPI, HEAD, WAVES)                                               \
    extern "C" __global__ __launch_bounds__(WAVES * 64) void NAME(ConvArgs p)                \
    {                                                                                        \
        convw_body<NT, EPI, HEAD, WAVES>(p);                                                 \
    }

// C = 144 (NT = 9) trunk convs.
CONVW_INST(hat_convw_n9_store_ln, 9, EPI_STORE_LN, -1, CONVW_WAVES_N9_STORE_LN)
CONVW_INST(hat_convw_n9_resid_ln, 9, EPI_RESID_LN, -1, CONVW_WAVES_N9_RESID_LN)
CONVW_INST(hat_convw_n9_resid, 9, EPI_RESID, -1, CONVW_WAVES_N9_RESID)
// C = 180 (two 96-channel column blocks): the RHAG conv and conv_after_body
// with the residual (their LayerNorm, needing whole rows, runs separately).
CONVW_INST(hat_convw_n6_resid, 6, EPI_RESID, -1, CONVW_WAVES_N6_RESID)
// C = 180 CAB conv2 (60 -> 180) + per-tile column sums for the channel mean.
CONVW_INST(hat_convw_n6_colsum, 6, EPI_STORE, CEPI_COLSUM, CONVW_WAVES_N6_COLSUM)
// Head: conv_before_upsample (-> 64, LeakyReLU) and the upsample convs
// (64 -> 4*64 or 9*64 in 128-channel column blocks, + PixelShuffle).
CONVW_INST(hat_convw_n4_store, 4, EPI_STORE, CEPI_STORE, CONVW_WAVES_N4_STORE)
CONVW_INST(hat_convw_n8_shuffle, 8, EPI_STORE, CEPI_SHUFFLE, CONVW_WAVES_N8_SHUFFLE)
