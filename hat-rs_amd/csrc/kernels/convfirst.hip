// conv_first + patch_embed.norm for C = 144 and 180: out = conv3x3(x0) + b
// (3 -> C channels, zero padding 1), xn = LN(out) - lg_conv3x3 and
// lg_channel_layer_norm at gpu.rs:722-732 (cpu.rs conv3x3 and layer_norm).
//
// The conv is a GEMM with K = 27 (k = tap * 3 + ci, padded to 28): the wide
// conv kernel would stage the 3 input channels as a 16-channel chunk and run
// 5.3x the products. Weights are the A operand of v_mfma_f32_16x16x4_f32, held
// in registers for the whole block (7 k-steps x NT tiles a lane), pixels the B
// operand, gathered from x0 ([H*W][4], hat_pre's layout) with zeros outside
// the plane; a lane's four accumulators are four consecutive output channels
// of one pixel, the layout tx_row_stats (tailx.hip) reduces: the row
// statistics come from the four lanes that hold a pixel, two-pass as on the
// CPU (cpu.rs:563-581).
//
// A block of 4 waves owns a 16 x 16 pixel tile, each wave four 16-pixel rows.
// A row's 16 pixels are consecutive tokens, 16 C contiguous floats of each
// output: the wave stages them in LDS (rows C + 4 floats apart for C = 144,
// so that the staging writes, 8 lanes at a time, meet no bank conflicts) and
// stores them as whole 1 KB runs, so every cache line is written once and
// whole. out (read again only by conv_after_body at the end of the forward)
// leaves non-temporal; xn (read by the next kernel) with ordinary stores.
//
// Included after tailx.hip (tx_row_stats, tx_live).

#define CF_WAVES 4

template <int C>
__device__ __forceinline__ void conv_first_body(const ConvArgs& p)
{
    constexpr int NT = (C + 15) / 16;                 // 9 or 12 output tiles
    constexpr int KS = 7;                             // 28 k: 27 real
    constexpr int S = C % 32 == 16 ? C + 4 : C;       // staging row stride (floats)
    static_assert(C == 144 || C == 180, "conv_first widths");
    __shared__ __attribute__((aligned(16))) float St[CF_WAVES][16 * S];
    __shared__ __attribute__((aligned(16))) float Cs[3 * 16 * NT];  // bias, norm w, norm b (zero past C)

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int H = p.H, W = p.W;
    const int tiles_x = W / 16;
    const int ty0 = ((int)blockIdx.x / tiles_x) * 16, tx0 = ((int)blockIdx.x % tiles_x) * 16;

    for (int i = tid; i < 3 * 16 * NT; i += CF_WAVES * 64) {
        const int j = i % (16 * NT);
        const float* src = i < 16 * NT ? p.bias : (i < 32 * NT ? p.nw : p.nb);
        Cs[i] = j < C ? src[j] : 0.0f;
    }
    // A operand: output channel 16 nt + lr, k = 4 s + lg (tap k / 3, channel
    // k % 3) from the repacked weights [CIp/16][9][COp][16]; zeros past C and
    // at k = 27
    float wa[NT][KS];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int co = 16 * nt + lr, k = 4 * s + lg, tap = k / 3, ci = k - 3 * tap;
            wa[nt][s] = co < C && k < 27 ? p.w[((size_t)tap * p.COp + co) * 16 + ci] : 0.0f;
        }
    // B operand offsets of k-step s: this lane's tap (dy, dx) and channel
    int koff[KS], kdy[KS], kdx[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int k = 4 * s + lg, tap = k < 27 ? k / 3 : 4, ci = k < 27 ? k - 3 * (k / 3) : 0;
        kdy[s] = k < 27 ? tap / 3 - 1 : 99;  // k = 27: never in the plane
        kdx[s] = tap % 3 - 1;
        koff[s] = (kdy[s] * W + kdx[s]) * 4 + ci;
    }
    __syncthreads();  // Cs

    float* st = St[wave];
#pragma unroll 1
    for (int r = 0; r < 4; ++r) {
        const int y = ty0 + wave * 4 + r, x = tx0 + lr;
        const int m0 = y * W + tx0;  // the row's first token
        f32x4 acc[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt] = *(const f32x4*)(Cs + 16 * nt + 4 * lg);
        float xb[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int yy = y + kdy[s], xx = x + kdx[s];
            const bool ok = yy >= 0 && yy < H && xx >= 0 && xx < W;
            xb[s] = *(ok ? p.in + ((long)(y * W + x) * 4 + koff[s]) : hat_zero_row);
        }
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[nt] = mfma16(wa[nt][s], xb[s], acc[nt]);
        // the pixel lr's row: statistics over the four lanes that hold it
        const float2 stt = tx_row_stats<C>(acc, lg, p.eps);
        // out: stage, then whole runs (non-temporal)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            if (tx_live<C>(nt, lg)) *(f32x4*)(st + lr * S + 16 * nt + 4 * lg) = acc[nt];
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
        constexpr int RUN4 = 16 * C / 4;     // float4 of the 16-pixel run
#pragma unroll
        for (int i = 0; i < (RUN4 + 63) / 64; ++i) {
            const int q = lane + 64 * i;
            if (q < RUN4) {
                const int px = q / (C / 4), c4 = q - px * (C / 4);
                __builtin_nontemporal_store(*(const f32x4*)(st + px * S + 4 * c4), (f32x4*)(p.out + (size_t)m0 * C) + q);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the norm overwrites the stage
        // xn = LN(out) by (nw, nb)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f32x4 w4 = *(const f32x4*)(Cs + 16 * NT + 16 * nt + 4 * lg);
            const f32x4 b4 = *(const f32x4*)(Cs + 32 * NT + 16 * nt + 4 * lg);
            f32x4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = (acc[nt][j] - stt.x) * stt.y * w4[j] + b4[j];
            if (tx_live<C>(nt, lg)) *(f32x4*)(st + lr * S + 16 * nt + 4 * lg) = v;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
#pragma unroll
        for (int i = 0; i < (RUN4 + 63) / 64; ++i) {
            const int q = lane + 64 * i;
            if (q < RUN4) {
                const int px = q / (C / 4), c4 = q - px * (C / 4);
                *((f32x4*)(p.xn + (size_t)m0 * C) + q) = *(const f32x4*)(st + px * S + 4 * c4);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next row's writes
    }
}

extern "C" __global__ __launch_bounds__(CF_WAVES * 64) void hat_conv_first_ln144(ConvArgs p)
{
    conv_first_body<144>(p);
}

extern "C" __global__ __launch_bounds__(CF_WAVES * 64) void hat_conv_first_ln180(ConvArgs p)
{
    conv_first_body<180>(p);
}
