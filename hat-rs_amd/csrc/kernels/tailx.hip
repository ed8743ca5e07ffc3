// The second half of a HAB (and of an OCAB), C = 144 and 180, on split-bf16
// MFMA, as two kernels or one (hat_arch.py HAB.forward / OCAB.forward; cpu.rs hab
// 1090-1166, ocab 983-1055; the reference GPU graph's proj, CAB conv2 and
// channel scale, adds, norm2, fc1 + GELU + fc2 and the next norm1,
// src/gpu.rs:469-588):
//
//   hat_projx_cab / hat_projx:  x' = x + ao . Wp^T (+ nb(t1) . W2g^T) + bias
//                               out = x' (and xn = LN2(x') when asked)
//   hat_mlpx_ln / hat_mlpx:     out = x' + fc2(gelu(fc1(LN2(x')))) + b2, LN2
//                               formed from the x' rows (xn = LN_next(out))
//   hat_projx180(_hab), hat_mlpx180(_ln): the same at C = 180 (the HAB form
//                               adds the unfolded CAB's gated conv2 output)
//   hat_habx_cab_ln / hat_habx, hat_habx180_hab_ln / hat_habx180: each pair
//                               above in one kernel
//
// ao is the attention output, nb(t1) the 3x3 neighbourhood of the CAB's conv1
// output (k = tap*6 + ci, 54 values) and W2g / bias the gate-scaled conv2
// weights and combined bias written by the gate (hat_cab_gate's work); the
// OCAB form has no conv2 and its bias is the projection's. Products are the
// six-term split-bf16 ones of attnx.hip on v_mfma_f32_16x16x32_bf16, weights as
// the A operand, tokens as B; a lane's four accumulators are four consecutive
// output channels of one token.
//
// Both kernels give a block of 4 waves one 128-token row tile (32 tokens a
// wave) and stream its weights as 32-k chunks (common.h: pre-split, two LDS
// buffers, chunk c + 1 in flight while chunk c's MFMAs run); two blocks share
// a CU, so one block's reads overlap the other's MFMAs, and a block's results
// leave once, at its end. The accumulators start as the block-input rows.
// hat_projx_cab holds its waves' attention-output rows in registers (all five
// k-steps, read once); its last two chunks are conv2's (k = tap*6 + ci, 54 of
// 64 used), split by hat_cab_gate, against the t1 neighbourhood gathered one
// chunk ahead.
//
// The MLP walks the hidden layer in thirds of 96 units, so that fc1's output
// of a third (48 registers) and fc2's accumulators (72) fit a lane next to
// the operands: per third five fc1 chunks, then three fc2 chunks on those
// units; its input rows are read one chunk ahead, once per third, and normed
// as they arrive. fc1's output stays in registers and is
// fc2's B operand: fc1's rows are permuted on the host so that output tile t,
// row 4g + r (lane group g, register r) is unit 32(t/2) + 8g + 4(t%2) + r of
// the third; fc2's 32-k step s then finds units 32s + 8g .. +7 in tiles 2s
// and 2s+1 of lane group g, its weights in natural order.
//
// The forward runs the fused forms below (hat_habx*, hat_habx180*: both
// halves in one kernel, x' kept in registers); the two-kernel forms split at x'
// (written, then read back by the MLP) are the selftest's comparison and the
// fallback for the combinations the fused kernels do not take.
//
// Included after gemmx.hip (WcRows, split_pre).

#define TX_WAVES 4
#define TX_ROWS (TX_WAVES * 32)
#define TX_BUF (36 * 512)  // an LDS chunk buffer: 36 loads cover 192 rows

// Row statistics of a token over its C channels (C = 144: 36 per lane, 180:
// 45; NT = ceil(C / 16) tiles of which the last holds C % 16 real channels in
// lane group 0), the four lane groups of the token reducing with shuffles:
// two-pass mean, biased variance (cpu.rs:563-581); returns (mean, rstd).
template <int C>
__device__ __forceinline__ bool tx_live(int nt, int lg)
{
    constexpr int NT = (C + 15) / 16;
    return C % 16 == 0 || nt < NT - 1 || lg * 4 < C % 16;
}
template <int C>
__device__ __forceinline__ float2 tx_row_stats(const f32x4 (&v)[(C + 15) / 16], int lg, float eps)
{
    constexpr int NT = (C + 15) / 16;
    float s = 0.0f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int j = 0; j < 4; ++j) s += v[nt][j];  // zeros past C
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    const float mean = s / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float d = tx_live<C>(nt, lg) ? v[nt][j] - mean : 0.0f;
            q += d * d;
        }
    q += __shfl_xor(q, 16, 64);
    q += __shfl_xor(q, 32, 64);
    return make_float2(mean, 1.0f / sqrtf(q / (float)C + eps));
}

// acc = the 32 rows of res [M][C] from mbase (zeros past M and past C).
template <int C>
__device__ __forceinline__ void tx_load_res(const float* res, int mbase, int M, int lr, int lg,
                                            f32x4 (&acc)[2][(C + 15) / 16])
{
    constexpr int NT = (C + 15) / 16;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int m = mbase + mt * 16 + lr;
        const bool alive = m < M;
        const float* row = alive ? res + (size_t)m * C + lg * 4 : hat_zero_row;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] = *(const f32x4*)(alive && tx_live<C>(nt, lg) ? row + nt * 16 : hat_zero_row);
    }
}

// v = acc + bias (Cs); out = v; with xn: xn = LN(v) by (nw, nb) = (Cs + 16 NT,
// Cs + 32 NT) (Cs zero past C).
template <int C>
__device__ __forceinline__ void tx_store_rows(const f32x4 (&acc)[2][(C + 15) / 16], const float* Cs, int mbase,
                                              int M, int lr, int lg, float eps, float* out, float* xn)
{
    constexpr int NT = (C + 15) / 16;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int m = mbase + mt * 16 + lr;
        f32x4 v[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) v[nt] = acc[mt][nt] + *(const f32x4*)(Cs + nt * 16 + lg * 4);
        float2 st = make_float2(0.f, 0.f);
        if (xn) st = tx_row_stats<C>(v, lg, eps);
        if (m >= M) continue;
        float* orow = out + (size_t)m * C + lg * 4;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            if (tx_live<C>(nt, lg)) *(f32x4*)(orow + nt * 16) = v[nt];
        if (xn) {
            float* nrow = xn + (size_t)m * C + lg * 4;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f32x4 w4 = *(const f32x4*)(Cs + 16 * NT + nt * 16 + lg * 4);
                const f32x4 b4 = *(const f32x4*)(Cs + 32 * NT + nt * 16 + lg * 4);
                f32x4 y;
#pragma unroll
                for (int j = 0; j < 4; ++j) y[j] = (v[nt][j] - st.x) * st.y * w4[j] + b4[j];
                if (tx_live<C>(nt, lg)) *(f32x4*)(nrow + nt * 16) = y;
            }
        }
    }
}

// x' = x + ao . Wp^T (+ nb(t1) . W2g^T) + bias; out = x', xn = LN2(x').
template <bool CAB>
__device__ __forceinline__ void projx_body(const TailXArgs& p)
{
    constexpr int NCH = CAB ? 7 : 5, NL = 28;
    static_assert(NL * 512 >= 3 * 144 * 32, "chunk loads");
    // the two chunk buffers as two LDS objects, so that the compiler sees that
    // reads of one need not wait for the copy into the other
    __shared__ __attribute__((aligned(16))) unsigned short Ws0[TX_BUF];
    __shared__ __attribute__((aligned(16))) unsigned short Ws1[TX_BUF];
    __shared__ __attribute__((aligned(16))) float Cs[3 * 144];  // bias, norm2 w, b (the epilogue's)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    if ((int)blockIdx.x * TX_ROWS >= M) return;  // whole block, before any barrier
    auto chunk = [&](int c) { return c < 5 ? p.w + (size_t)c * WC_CHUNK : p.w2gx + (size_t)(c - 5) * WC_CHUNK; };
    wc_issue<NL, TX_WAVES>(Ws0, chunk(0), wave, lane);
    for (int i = tid; i < 3 * 144; i += TX_WAVES * 64)
        Cs[i] = i < 144 ? p.bias[i] : (!p.xn ? 0.0f : i < 288 ? p.nw[i - 144] : p.nb[i - 288]);  // norm2's when written
    const int mbase = blockIdx.x * TX_ROWS + wave * 32;
    f32x4 acc[2][9];
    tx_load_res<144>(p.res, mbase, M, lr, lg, acc);
    f32x4 y[5][2][2];
    {
        WcRows<144> ar;
        ar.init(p.a, mbase, M, lr);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) ar.load(ks, lg, y[ks]);
        ar.load_half(lg, y[4]);  // the packed step: channels 128 + 4 lg .. +3
    }
    // conv2's B operand for k-step s: the 3x3 neighbourhood of t1 at this
    // lane's tokens, k = 32 s + 8 lg + j = tap*6 + ci (pairs of channels;
    // taps outside the plane and k >= 54 read zeros)
    auto gather_t1 = [&](int s, f32x4 (&dst)[2][2]) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int m = mbase + mt * 16 + lr;
            const bool alive = m < M;
            const int yq = m / p.W, xq = m - yq * p.W;
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const int k = s * 32 + lg * 8 + j, tap = k / 6, ci = k - tap * 6;
                const int yy = yq + tap / 3 - 1, xx = xq + tap % 3 - 1;
                const bool ok = alive && tap < 9 && yy >= 0 && yy < p.H && xx >= 0 && xx < p.W;
                const float2 v = *(const float2*)(ok ? p.t1 + ((size_t)yy * p.W + xx) * CAB_CS + ci : hat_zero_row);
                dst[mt][j / 4][j % 4] = v.x;
                dst[mt][j / 4][j % 4 + 1] = v.y;
            }
        }
    };
    f32x4 t1v[2][2];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of chunk c (and its operands) have landed
        __syncthreads();                // everyone's have, and everyone is done with chunk c - 1
        if (c + 1 < NCH) wc_issue<NL, TX_WAVES>(c & 1 ? Ws0 : Ws1, chunk(c + 1), wave, lane);
        u32x4 xb[2][3];
        if (c == 4) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) half_operands(y[4][mt][0], xb[mt]);
        } else {
            split_pre(c < 5 ? y[c < 5 ? c : 0] : t1v, xb);
        }
        if (CAB && c >= 4 && c + 1 < NCH) gather_t1(c - 4, t1v);
        if (c == 4) ws_mma<9, 144, true>(Ws0, lr, lg, xb, acc);
        else ws_mma<9, 144>(c & 1 ? Ws1 : Ws0, lr, lg, xb, acc);
    }
    tx_store_rows<144>(acc, Cs, mbase, M, lr, lg, p.eps, p.out, p.xn);
}

// out = x' + fc2(gelu(fc1(y))) + b2 (+ xn = LN_next(out)); x' = p.res = p.a and
// y = LN2(x') by (p.inw, p.inb), formed from the x' rows as they are read for
// each third (so that the projection kernel need not write LN2(x') and this
// one read it three times: the row statistics come from the residual rows,
// which hold x' in the layout tx_row_stats takes, and the arithmetic is the
// projection epilogue's, so y is the same to the bit). p.w: 24 chunks (per
// third: five of fc1's 96 permuted rows, b1 as their column k = 144, then
// three of fc2 on those units).
template <bool LN>
__device__ __forceinline__ void mlpx_body(const TailXArgs& p)
{
    constexpr int NL1 = 20, NL2 = 28;
    static_assert(NL1 * 512 >= 3 * MX_HID * 32 && NL2 * 512 >= 3 * 144 * 32, "chunk loads");
    __shared__ __attribute__((aligned(16))) unsigned short Ws0[TX_BUF];
    __shared__ __attribute__((aligned(16))) unsigned short Ws1[TX_BUF];
    __shared__ __attribute__((aligned(16))) float Cs[3 * 144];  // b2, next norm w, b (the epilogue's)
    // norm2's w and b over the 160 k of fc1's input: at k = 144 w 0 and b 1
    // (the 1 that multiplies b1's column comes out as 1), past it zeros
    __shared__ __attribute__((aligned(16))) float Cn[2 * 160];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    if ((int)blockIdx.x * TX_ROWS >= M) return;  // whole block, before any barrier
    wc_issue<NL1, TX_WAVES>(Ws0, p.w, wave, lane);
    for (int i = tid; i < 3 * 144; i += TX_WAVES * 64) {
        float v;
        if (i < 144) v = p.b2[i];
        else if (i < 288) v = LN ? p.nw[i - 144] : 0.0f;
        else v = LN ? p.nb[i - 288] : 0.0f;
        Cs[i] = v;
    }
    for (int i = tid; i < 2 * 160; i += TX_WAVES * 64) {
        const int k = i < 160 ? i : i - 160;
        Cn[i] = k < 144 ? (i < 160 ? p.inw[k] : p.inb[k]) : (i >= 160 && k == 144 ? 1.0f : 0.0f);
    }
    const int mbase = blockIdx.x * TX_ROWS + wave * 32;
    f32x4 acc2[2][9];
    tx_load_res<144>(p.res, mbase, M, lr, lg, acc2);
    // norm2's statistics of the wave's tokens, from x' as the residual holds it
    float2 st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) st[mt] = tx_row_stats<144>(acc2[mt], lg, p.eps);
    // y = LN2(x') for k-step ks of the rows in pre, in place
    auto norm_pre = [&](int ks, f32x4 (&pre)[2][2]) {
        const float* wk = Cn + ks * 32 + lg * 8;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f32x4 w4 = *(const f32x4*)(wk + 4 * j), b4 = *(const f32x4*)(wk + 160 + 4 * j);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) pre[mt][j][i] = (pre[mt][j][i] - st[mt].x) * st[mt].y * w4[i] + b4[i];
        }
    };
    WcRows<144> yr;
    yr.init(p.a, mbase, M, lr);
    f32x4 pre[2][2];
    yr.load_b(0, lg, pre);
#pragma unroll 1
    for (int q = 0; q < 3; ++q) {
        const unsigned short* wq = p.w + (size_t)(8 * q) * WC_CHUNK;  // this third's eight chunks
        // fc1: the third's 96 hidden units (permuted rows), chunks 0..4 (even
        // chunks in buffer 0: eight a third keep the parities fixed)
        f32x4 h[2][6];
#pragma unroll
        for (int nt = 0; nt < 6; ++nt) h[0][nt] = h[1][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        auto fc1_step = [&](int ks, auto parv) {
            constexpr int PAR = decltype(parv)::value;  // = ks & 1
            __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the chunk (and its rows) have landed
            __syncthreads();                // everyone's have, and everyone is done with the one before
            if (ks < 4) wc_issue<NL1, TX_WAVES>(PAR ? Ws0 : Ws1, wq + (size_t)(ks + 1) * WC_CHUNK, wave, lane);
            else wc_issue<NL2, TX_WAVES>(Ws1, wq + (size_t)5 * WC_CHUNK, wave, lane);
            u32x4 xb[2][3];
            norm_pre(ks, pre);
            split_pre(pre, xb);
            // the rows of the next fc1 chunk: this third's next k-step (k =
            // 144 carries the 1 of b1's column), or k-step 0 for the next third
            if (ks < 4) yr.load_b(ks + 1, lg, pre);
            else if (q < 2) yr.load_b(0, lg, pre);
            ws_mma<6, MX_HID>(PAR ? Ws1 : Ws0, lr, lg, xb, h);
        };
#pragma unroll 1
        for (int ks = 0; ks < 4; ks += 2) {
            fc1_step(ks, CInt<0>{});
            fc1_step(ks + 1, CInt<1>{});
        }
        fc1_step(4, CInt<0>{});
        // fc2 over the third's units, from registers, chunks 5..7
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (s < 2) wc_issue<NL2, TX_WAVES>(s & 1 ? Ws1 : Ws0, wq + (size_t)(6 + s) * WC_CHUNK, wave, lane);
            else if (q < 2) wc_issue<NL1, TX_WAVES>(Ws0, wq + (size_t)8 * WC_CHUNK, wave, lane);
            if (s == 0) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 6; ++nt)
#pragma unroll
                        for (int j = 0; j < 4; ++j) h[mt][nt][j] = gelu(h[mt][nt][j]);
            }
            u32x4 xb[2][3];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const float f[8] = {h[mt][2 * s][0],     h[mt][2 * s][1],     h[mt][2 * s][2],
                                    h[mt][2 * s][3],     h[mt][2 * s + 1][0], h[mt][2 * s + 1][1],
                                    h[mt][2 * s + 1][2], h[mt][2 * s + 1][3]};
                split3_x8(f, xb[mt]);
            }
            ws_mma<9, 144>(s & 1 ? Ws0 : Ws1, lr, lg, xb, acc2);
        }
    }
    tx_store_rows<144>(acc2, Cs, mbase, M, lr, lg, p.eps, p.out, LN ? p.xn : nullptr);
}

// The C = 180 projection tail: out = x + ao . Wp^T + bias (HAB: + aux * gate *
// cscale, the unfolded CAB's gated conv2), xn = LN2(out). p.w: six chunks
// MX180_SLOT apart, k-steps of the 192-row (180 real) projection in the
// swizzled [rows][32] layout (ws_mma); ao's rows are read one k-step ahead.
template <bool HAB>
__device__ __forceinline__ void projx180_body(const TailXArgs& p)
{
    constexpr int C = 180, NT = 12, NL = 36;
    static_assert(NL * 512 == MX180_SLOT && MX180_SLOT <= TX_BUF, "chunk loads");
    __shared__ __attribute__((aligned(16))) unsigned short Ws0[TX_BUF];
    __shared__ __attribute__((aligned(16))) unsigned short Ws1[TX_BUF];
    __shared__ __attribute__((aligned(16))) float Cs[4 * 16 * NT];  // bias, norm2 w, b, gate * cscale (zero past 180)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    if ((int)blockIdx.x * TX_ROWS >= M) return;  // whole block, before any barrier
    wc_issue<NL, TX_WAVES>(Ws0, p.w, wave, lane);
    for (int i = tid; i < 4 * 16 * NT; i += TX_WAVES * 64) {
        const int part = i / (16 * NT), c = i - part * 16 * NT;
        float v = 0.0f;
        // the norm's constants only when norm2 is written here (xn given)
        if (c < C)
            v = part == 0 ? p.bias[c]
                          : part == 1 ? (p.xn ? p.nw[c] : 0.0f)
                                      : part == 2 ? (p.xn ? p.nb[c] : 0.0f) : (HAB ? p.gate[c] * p.cscale : 0.0f);
        Cs[i] = v;
    }
    const int mbase = blockIdx.x * TX_ROWS + wave * 32;
    f32x4 acc[2][NT];
    tx_load_res<C>(p.res, mbase, M, lr, lg, acc);
    WcRows<C> ar;
    ar.init(p.a, mbase, M, lr);
    f32x4 pre[2][2];
    ar.load(0, lg, pre);
#pragma unroll
    for (int c = 0; c < 6; ++c) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of chunk c (and its rows) have landed
        __syncthreads();                // everyone's have, and everyone is done with chunk c - 1
        if (c + 1 < 6) wc_issue<NL, TX_WAVES>(c & 1 ? Ws0 : Ws1, p.w + (size_t)(c + 1) * MX180_SLOT, wave, lane);
        u32x4 xb[2][3];
        split_pre(pre, xb);
        if (c + 1 < 6) ar.load(c + 1, lg, pre);
        ws_mma<NT, 16 * NT>(c & 1 ? Ws1 : Ws0, lr, lg, xb, acc);
    }
    if constexpr (HAB) {
        // + conv2's output times gate * cscale, one 16-row tile at a time
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int m = mbase + mt * 16 + lr;
            const float* arow = m < M ? p.aux + (size_t)m * C + lg * 4 : hat_zero_row;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f32x4 a4 = *(const f32x4*)(m < M && tx_live<C>(nt, lg) ? arow + nt * 16 : hat_zero_row);
                const f32x4 g4 = *(const f32x4*)(Cs + 48 * NT + nt * 16 + lg * 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[mt][nt][j] += a4[j] * g4[j];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    tx_store_rows<C>(acc, Cs, mbase, M, lr, lg, p.eps, p.out, p.xn);
}

// The C = 180 MLP: out = x' + fc2(gelu(fc1(y))) + b2 (+ xn = LN_next(out)),
// x' = p.res = p.a [M][180] and y = LN2(x') by (p.inw, p.inb), formed from the
// x' rows as hat_mlpx forms it. The hidden layer in six parts of 64 units (the
// last 40 real), so that fc2's 192 accumulator columns (96 registers), fc1's
// output of a part (32) and the operands fit a lane. p.w: 48 chunks
// MX180_SLOT apart, per part six fc1 k-steps (64 permuted rows, b1 at k = 180)
// then two fc2 k-steps (192 rows); the swizzled [rows][32] layout (ws_mma).
template <bool LN>
__device__ __forceinline__ void mlpx180_body(const TailXArgs& p)
{
    constexpr int C = 180, NT = 12, NP = 6, NL1 = 12, NL2 = 36;
    static_assert(NL1 * 512 == 3 * MX180_HID * 32 && NL2 * 512 == MX180_SLOT && MX180_SLOT <= TX_BUF, "chunk loads");
    __shared__ __attribute__((aligned(16))) unsigned short Ws0[TX_BUF];
    __shared__ __attribute__((aligned(16))) unsigned short Ws1[TX_BUF];
    __shared__ __attribute__((aligned(16))) float Cs[3 * 16 * NT];  // b2, next norm w, b (zero past 180)
    // norm2's w and b over the 192 k of fc1's input: at k = 180 w 0 and b 1
    // (the 1 that multiplies b1's column), past it zeros
    __shared__ __attribute__((aligned(16))) float Cn[2 * 192];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    if ((int)blockIdx.x * TX_ROWS >= M) return;  // whole block, before any barrier
    wc_issue<NL1, TX_WAVES>(Ws0, p.w, wave, lane);
    for (int i = tid; i < 3 * 16 * NT; i += TX_WAVES * 64) {
        const int part = i / (16 * NT), c = i - part * 16 * NT;
        float v = 0.0f;
        if (c < C) v = part == 0 ? p.b2[c] : (LN ? (part == 1 ? p.nw[c] : p.nb[c]) : 0.0f);
        Cs[i] = v;
    }
    for (int i = tid; i < 2 * 192; i += TX_WAVES * 64) {
        const int k = i < 192 ? i : i - 192;
        Cn[i] = k < C ? (i < 192 ? p.inw[k] : p.inb[k]) : (i >= 192 && k == C ? 1.0f : 0.0f);
    }
    const int mbase = blockIdx.x * TX_ROWS + wave * 32;
    f32x4 acc2[2][NT];
    tx_load_res<C>(p.res, mbase, M, lr, lg, acc2);
    // norm2's statistics of the wave's tokens, from x' as the residual holds it
    float2 st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) st[mt] = tx_row_stats<C>(acc2[mt], lg, p.eps);
    // y = LN2(x') for k-step ks of the rows in pre, in place
    auto norm_pre = [&](int ks, f32x4 (&pre)[2][2]) {
        const float* wk = Cn + ks * 32 + lg * 8;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f32x4 w4 = *(const f32x4*)(wk + 4 * j), b4 = *(const f32x4*)(wk + 192 + 4 * j);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) pre[mt][j][i] = (pre[mt][j][i] - st[mt].x) * st[mt].y * w4[i] + b4[i];
        }
    };
    WcRows<C> yr;
    yr.init(p.a, mbase, M, lr);
    f32x4 pre[2][2];
    yr.load_b(0, lg, pre);
#pragma unroll 1
    for (int q = 0; q < NP; ++q) {
        const unsigned short* wq = p.w + (size_t)(8 * q) * MX180_SLOT;  // this part's eight chunks
        // fc1: the part's 64 hidden units (permuted rows), chunks 0..5 (even
        // chunks in buffer 0: eight a part keep the parities fixed)
        f32x4 h[2][4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) h[0][nt] = h[1][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        auto fc1_step = [&](int ks, auto parv) {
            constexpr int PAR = decltype(parv)::value;  // = ks & 1
            __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the chunk (and its rows) have landed
            __syncthreads();                // everyone's have, and everyone is done with the one before
            if (ks < 5) wc_issue<NL1, TX_WAVES>(PAR ? Ws0 : Ws1, wq + (size_t)(ks + 1) * MX180_SLOT, wave, lane);
            else wc_issue<NL2, TX_WAVES>(Ws0, wq + (size_t)6 * MX180_SLOT, wave, lane);
            u32x4 xb[2][3];
            norm_pre(ks, pre);
            split_pre(pre, xb);
            // the rows of the next fc1 chunk: this part's next k-step (k =
            // 180 carries the 1 of b1's column), or k-step 0 for the next part
            if (ks < 5) yr.load_b(ks + 1, lg, pre);
            else if (q < NP - 1) yr.load_b(0, lg, pre);
            ws_mma<4, MX180_HID>(PAR ? Ws1 : Ws0, lr, lg, xb, h);
        };
#pragma unroll 1
        for (int ks = 0; ks < 6; ks += 2) {
            fc1_step(ks, CInt<0>{});
            fc1_step(ks + 1, CInt<1>{});
        }
        // fc2 over the part's units, from registers, chunks 6, 7
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (s == 0) wc_issue<NL2, TX_WAVES>(Ws1, wq + (size_t)7 * MX180_SLOT, wave, lane);
            else if (q < NP - 1) wc_issue<NL1, TX_WAVES>(Ws0, wq + (size_t)8 * MX180_SLOT, wave, lane);
            if (s == 0) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                        for (int j = 0; j < 4; ++j) h[mt][nt][j] = gelu(h[mt][nt][j]);
            }
            u32x4 xb[2][3];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const float f[8] = {h[mt][2 * s][0],     h[mt][2 * s][1],     h[mt][2 * s][2],
                                    h[mt][2 * s][3],     h[mt][2 * s + 1][0], h[mt][2 * s + 1][1],
                                    h[mt][2 * s + 1][2], h[mt][2 * s + 1][3]};
                split3_x8(f, xb[mt]);
            }
            ws_mma<NT, 16 * NT>(s == 0 ? Ws0 : Ws1, lr, lg, xb, acc2);
        }
    }
    tx_store_rows<C>(acc2, Cs, mbase, M, lr, lg, p.eps, p.out, LN ? p.xn : nullptr);
}

// The whole second half of a block in one kernel, C = 144 (HAB with the
// folded CAB, or OCAB):
//
//   x' = x + ao . Wp^T (+ nb(t1) . W2g^T) + bias
//   out = x' + fc2(gelu(fc1(LN2(x')))) + b2, xn = LN_next(out) when asked
//
// hat_projx(_cab) followed by hat_mlpx(_ln) with x' kept on the chip: the
// projection's accumulators are x' in the layout the MLP's residual takes, and
// they stay in registers for the MLP. The MLP's input for its first third of
// hidden units comes from the same registers: fc1's input columns are packed
// in the order a lane holds x' (pack_mlp_xf), so k-step ks of lane group g is
// the lane's accumulator tiles 2 ks and 2 ks + 1, i.e. channels 32 ks + 4 g +
// j and 32 ks + 16 + 4 g + j (j < 4), and the last step, channels 128 + 4 g
// + j (j < 4), is packed (half_operands, common.h: slots 4..7 carry a second
// part of the same four channels, three MFMAs instead of six); b1 (b1x) is
// added to fc1's output before the GELU. The projection's last step (channels
// 128 .. 143 of ao) is packed the same way. The first third forms
// y = norm2(x') from them and leaves y in the output rows; the other two
// thirds read y back (each lane reads exactly the addresses it wrote, so
// program order is what makes the values visible) and need no norm; those
// rows are overwritten by the result at the end.
// Against the two kernels this saves x''s round trip through HBM between them
// and lets one block's projection (memory-latency bound) overlap another's
// MLP (issue bound) on the same CU.
//
// The chunk buffers: the projection reads chunk c from buffer c & 1 and its
// last chunk (5 or 7: an odd count) from buffer 0, so the MLP's first chunk
// goes to buffer 1 during it, and the MLP runs with the buffers' roles
// swapped (its even chunks in buffer 1).

// fused input position k = 32 ks + 8 g + j -> channel of x' (-1: b1's 1, -2: zero)
__device__ __forceinline__ int habx_channel(int k)
{
    const int ks = k >> 5, g = (k >> 3) & 3, j = k & 7;
    if (ks < 4) return 32 * ks + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
    if (j < 4) return 128 + 4 * g + j;
    return g == 0 && j == 4 ? -1 : -2;
}

template <bool CAB, bool LN>
__device__ __forceinline__ void habx_body(const TailXArgs& p)
{
    constexpr int NCH = CAB ? 7 : 5, NLP = 28, NL1 = 20, NL2 = 28;
    static_assert(NCH % 2 == 1, "the projection's last chunk is in buffer 0");
    static_assert(NLP * 512 >= 3 * 144 * 32 && NL1 * 512 >= 3 * MX_HID * 32 && NL2 * 512 >= 3 * 144 * 32,
                  "chunk loads");
    __shared__ __attribute__((aligned(16))) unsigned short Ws0[TX_BUF];
    __shared__ __attribute__((aligned(16))) unsigned short Ws1[TX_BUF];
    __shared__ __attribute__((aligned(16))) float Cp[144];      // the projection's bias
    __shared__ __attribute__((aligned(16))) float Cs[3 * 144];  // b2, next norm w, b (the epilogue's)
    // norm2's w and b over fc1's 160 input positions in the fused order: at
    // b1's position w 0 and b 1, at the empty ones zeros
    __shared__ __attribute__((aligned(16))) float Cn[2 * 160];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    if ((int)blockIdx.x * TX_ROWS >= M) return;  // whole block, before any barrier
    auto pchunk = [&](int c) { return c < 5 ? p.w + (size_t)c * WC_CHUNK : p.w2gx + (size_t)(c - 5) * WC_CHUNK; };
    wc_issue<NLP, TX_WAVES>(Ws0, pchunk(0), wave, lane);
    for (int i = tid; i < 144; i += TX_WAVES * 64) Cp[i] = p.bias[i];
    for (int i = tid; i < 3 * 144; i += TX_WAVES * 64) {
        float v;
        if (i < 144) v = p.b2[i];
        else if (i < 288) v = LN ? p.nw[i - 144] : 0.0f;
        else v = LN ? p.nb[i - 288] : 0.0f;
        Cs[i] = v;
    }
    for (int i = tid; i < 2 * 160; i += TX_WAVES * 64) {
        const int k = i < 160 ? i : i - 160, c = habx_channel(k);
        Cn[i] = c >= 0 ? (i < 160 ? p.inw[c] : p.inb[c]) : (i >= 160 && c == -1 ? 1.0f : 0.0f);
    }
    const int mbase = blockIdx.x * TX_ROWS + wave * 32;
    f32x4 acc[2][9];
    tx_load_res<144>(p.res, mbase, M, lr, lg, acc);

    // ---- the projection: acc = x + ao . Wp^T (+ nb(t1) . W2g^T)
    {
        f32x4 y[5][2][2];
        {
            WcRows<144> ar;
            ar.init(p.a, mbase, M, lr);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) ar.load(ks, lg, y[ks]);
            ar.load_half(lg, y[4]);  // the packed step: channels 128 + 4 lg .. +3
        }
        auto gather_t1 = [&](int s, f32x4 (&dst)[2][2]) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const int m = mbase + mt * 16 + lr;
                const bool alive = m < M;
                const int yq = m / p.W, xq = m - yq * p.W;
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const int k = s * 32 + lg * 8 + j, tap = k / 6, ci = k - tap * 6;
                    const int yy = yq + tap / 3 - 1, xx = xq + tap % 3 - 1;
                    const bool ok = alive && tap < 9 && yy >= 0 && yy < p.H && xx >= 0 && xx < p.W;
                    const float2 v =
                        *(const float2*)(ok ? p.t1 + ((size_t)yy * p.W + xx) * CAB_CS + ci : hat_zero_row);
                    dst[mt][j / 4][j % 4] = v.x;
                    dst[mt][j / 4][j % 4 + 1] = v.y;
                }
            }
        };
        f32x4 t1v[2][2];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of chunk c (and its operands) have landed
            __syncthreads();                // everyone's have, and everyone is done with chunk c - 1
            if (c + 1 < NCH) wc_issue<NLP, TX_WAVES>(c & 1 ? Ws0 : Ws1, pchunk(c + 1), wave, lane);
            else wc_issue<NL1, TX_WAVES>(Ws1, p.wm, wave, lane);  // the MLP's first chunk
            u32x4 xb[2][3];
            if (c == 4) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) half_operands(y[4][mt][0], xb[mt]);
            } else {
                split_pre(c < 5 ? y[c < 5 ? c : 0] : t1v, xb);
            }
            if (CAB && c >= 4 && c + 1 < NCH) gather_t1(c - 4, t1v);
            if (c == 4) ws_mma<9, 144, true>(Ws0, lr, lg, xb, acc);
            else ws_mma<9, 144>(c & 1 ? Ws1 : Ws0, lr, lg, xb, acc);
        }
    }
    // x' = acc + bias, kept in acc; norm2's statistics from it
    float2 st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int nt = 0; nt < 9; ++nt) acc[mt][nt] += *(const f32x4*)(Cp + nt * 16 + lg * 4);
        st[mt] = tx_row_stats<144>(acc[mt], lg, p.eps);
    }

    // ---- the MLP on x' (acc), in thirds of 96 hidden units
    auto norm_pre = [&](int ks, f32x4 (&pre)[2][2]) {
        const float* wk = Cn + ks * 32 + lg * 8;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f32x4 w4 = *(const f32x4*)(wk + 4 * j), b4 = *(const f32x4*)(wk + 160 + 4 * j);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) pre[mt][j][i] = (pre[mt][j][i] - st[mt].x) * st[mt].y * w4[i] + b4[i];
        }
    };
    // y = LN2(x') in the fused order for k-step ks: third 0 forms it from the
    // registers and leaves it in the output rows (the lane's own channels, in
    // place of x', which stays in acc), thirds 1 and 2 read it back; the last
    // (packed) step uses only the first half
    float* yrow[2];
    bool yalive[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int m = mbase + mt * 16 + lr;
        yalive[mt] = m < M;
        yrow[mt] = p.out + (size_t)(yalive[mt] ? m : 0) * 144 + lg * 4;
    }
    auto load_y = [&](int ks, f32x4 (&dst)[2][2]) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            dst[mt][0] = *(const f32x4*)(yalive[mt] ? yrow[mt] + 32 * ks : hat_zero_row);
            dst[mt][1] = *(const f32x4*)(yalive[mt] && ks < 4 ? yrow[mt] + 32 * ks + 16 : hat_zero_row);
        }
    };
    // fc2 over a third's units from registers: chunks 5..7 of the third;
    // at_last runs in the last step, after its copies are issued (the next
    // third's first rows: read there, not in fc1's last step, so that fc2's
    // first two waits are not for them)
    auto fc2_third = [&](int q, const unsigned short* wq, f32x4 (&h)[2][6], auto&& at_last) {
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            // buffers swapped: the third's chunk 5 + s is in buffer (s & 1 ? 1 : 0)
            if (s < 2) wc_issue<NL2, TX_WAVES>(s & 1 ? Ws0 : Ws1, wq + (size_t)(6 + s) * WC_CHUNK, wave, lane);
            else if (q < 2) wc_issue<NL1, TX_WAVES>(Ws1, wq + (size_t)8 * WC_CHUNK, wave, lane);
            if (s == 2) at_last();
            if (s == 0) {
                // + b1 (the lane's four units of each tile, in the third's
                // permuted row order), then GELU
#pragma unroll
                for (int nt = 0; nt < 6; ++nt) {
                    const f32x4 b = *(const f32x4*)(p.b1x + q * MX_HID + 16 * nt + 4 * lg);
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                        for (int j = 0; j < 4; ++j) h[mt][nt][j] = gelu(h[mt][nt][j] + b[j]);
                }
            }
            u32x4 xb[2][3];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const float f[8] = {h[mt][2 * s][0],     h[mt][2 * s][1],     h[mt][2 * s][2],
                                    h[mt][2 * s][3],     h[mt][2 * s + 1][0], h[mt][2 * s + 1][1],
                                    h[mt][2 * s + 1][2], h[mt][2 * s + 1][3]};
                split3_x8(f, xb[mt]);
            }
            ws_mma<9, 144>(s & 1 ? Ws1 : Ws0, lr, lg, xb, acc);
        }
    };
    // third 0: fc1's input from the registers
    {
        const unsigned short* wq = p.wm;
        f32x4 h[2][6];
#pragma unroll
        for (int nt = 0; nt < 6; ++nt) h[0][nt] = h[1][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 5; ++ks) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (ks < 4) wc_issue<NL1, TX_WAVES>(ks & 1 ? Ws1 : Ws0, wq + (size_t)(ks + 1) * WC_CHUNK, wave, lane);
            else wc_issue<NL2, TX_WAVES>(Ws0, wq + (size_t)5 * WC_CHUNK, wave, lane);
            f32x4 pre[2][2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                pre[mt][0] = acc[mt][2 * ks < 9 ? 2 * ks : 8];
                pre[mt][1] = 2 * ks + 1 < 9 ? acc[mt][2 * ks + 1 < 9 ? 2 * ks + 1 : 8] : (f32x4){0.f, 0.f, 0.f, 0.f};
            }
            u32x4 xb[2][3];
            norm_pre(ks, pre);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                // y for thirds 1 and 2 (rows past M: the sink)
                float* yr = yalive[mt] ? yrow[mt] + 32 * ks : hat_sink_row;
                *(f32x4*)yr = pre[mt][0];
                if (ks < 4) *(f32x4*)(yr + (yalive[mt] ? 16 : 4)) = pre[mt][1];
            }
            if (ks == 4) {
                // the packed step: channels 128 + 4 g + j (pre[mt][0])
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) half_operands(pre[mt][0], xb[mt]);
                ws_mma<6, MX_HID, true>(ks & 1 ? Ws0 : Ws1, lr, lg, xb, h);
            } else {
                split_pre(pre, xb);
                ws_mma<6, MX_HID>(ks & 1 ? Ws0 : Ws1, lr, lg, xb, h);
            }
        }
        fc2_third(0, wq, h, [] {});
    }
    // thirds 1, 2: fc1's input read back from the output rows, one k-step ahead
    f32x4 pre[2][2];
    load_y(0, pre);
#pragma unroll 1
    for (int q = 1; q < 3; ++q) {
        const unsigned short* wq = p.wm + (size_t)(8 * q) * WC_CHUNK;
        f32x4 h[2][6];
#pragma unroll
        for (int nt = 0; nt < 6; ++nt) h[0][nt] = h[1][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        auto fc1_step = [&](int ks, auto parv, auto halfv) {
            constexpr int PAR = decltype(parv)::value;     // = ks & 1
            constexpr bool HALF = decltype(halfv)::value;  // ks = 4: the packed step
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (ks < 4) wc_issue<NL1, TX_WAVES>(PAR ? Ws1 : Ws0, wq + (size_t)(ks + 1) * WC_CHUNK, wave, lane);
            else wc_issue<NL2, TX_WAVES>(Ws0, wq + (size_t)5 * WC_CHUNK, wave, lane);
            u32x4 xb[2][3];
            if (HALF) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) half_operands(pre[mt][0], xb[mt]);
            } else {
                split_pre(pre, xb);
            }
            if (ks < 4) load_y(ks + 1, pre);
            ws_mma<6, MX_HID, HALF>(PAR ? Ws0 : Ws1, lr, lg, xb, h);
        };
#pragma unroll 1
        for (int ks = 0; ks < 4; ks += 2) {
            fc1_step(ks, CInt<0>{}, CInt<0>{});
            fc1_step(ks + 1, CInt<1>{}, CInt<0>{});
        }
        fc1_step(4, CInt<0>{}, CInt<1>{});
        fc2_third(q, wq, h, [&] {
            if (q < 2) load_y(0, pre);
        });
    }
    tx_store_rows<144>(acc, Cs, mbase, M, lr, lg, p.eps, p.out, LN ? p.xn : nullptr);
}

// The whole second half of a block in one kernel, C = 180 (HAB with the
// unfolded CAB's gated conv2 output p.aux, or OCAB): hat_projx180(_hab)
// followed by hat_mlpx180(_ln) with x' kept on the chip, as hat_habx* keeps it
// at C = 144. x' is the projection's accumulators (2 x 12 tiles), which stay
// in registers as the MLP's residual. fc1's input columns are packed in the
// order a lane holds x' (pack_mlp_xf180): k-step ks of lane group g is the
// lane's tiles 2 ks and 2 ks + 1, channels 32 ks + 4 g + j and 32 ks + 16 +
// 4 g + j (j < 4); positions past channel 179 (tile 11 outside lane group 0)
// are zero, and b1 (b1x) is added to fc1's output before the GELU. Part 0 of
// the hidden layer forms y = norm2(x') from the registers and leaves it in the
// output rows, each lane at its own channels; parts 1..5 read it back (each
// lane the addresses it wrote, after a full wait) and need no norm; the result
// overwrites those rows at the end.
//
// The projection's six chunks alternate buffers 0, 1, ... and end in buffer
// 1, so the MLP's first chunk goes to buffer 0 during the last one and the MLP
// keeps hat_mlpx180's parities (a part's even chunks in buffer 0).

// fused input position k = 32 ks + 8 g + j -> channel of x' (-1: an empty
// position, channel >= 180)
__device__ __forceinline__ int habx180_channel(int k)
{
    const int ks = k >> 5, g = (k >> 3) & 3, j = k & 7;
    const int c = 32 * ks + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
    return c < 180 ? c : -1;
}

template <bool HAB, bool LN>
__device__ __forceinline__ void habx180_body(const TailXArgs& p)
{
    constexpr int C = 180, NT = 12, NP = 6, NLP = 36, NL1 = 12, NL2 = 36;
    static_assert(NLP * 512 == MX180_SLOT && NL1 * 512 == 3 * MX180_HID * 32 && MX180_SLOT <= TX_BUF, "chunk loads");
    __shared__ __attribute__((aligned(16))) unsigned short Ws0[TX_BUF];
    __shared__ __attribute__((aligned(16))) unsigned short Ws1[TX_BUF];
    __shared__ __attribute__((aligned(16))) float Cp[2 * 192];  // the projection's bias, gate * cscale (zero past 180)
    __shared__ __attribute__((aligned(16))) float Cs[3 * 192];  // b2, next norm w, b (the epilogue's)
    // norm2's w and b over fc1's 192 input positions in the fused order
    // (zeros at the empty ones)
    __shared__ __attribute__((aligned(16))) float Cn[2 * 192];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    if ((int)blockIdx.x * TX_ROWS >= M) return;  // whole block, before any barrier
    wc_issue<NLP, TX_WAVES>(Ws0, p.w, wave, lane);
    for (int i = tid; i < 2 * 192; i += TX_WAVES * 64) {
        const int c = i < 192 ? i : i - 192;
        Cp[i] = c >= C ? 0.0f : i < 192 ? p.bias[c] : (HAB ? p.gate[c] * p.cscale : 0.0f);
    }
    for (int i = tid; i < 3 * 192; i += TX_WAVES * 64) {
        const int part = i / 192, c = i - part * 192;
        Cs[i] = c >= C ? 0.0f : part == 0 ? p.b2[c] : (LN ? (part == 1 ? p.nw[c] : p.nb[c]) : 0.0f);
    }
    for (int i = tid; i < 2 * 192; i += TX_WAVES * 64) {
        const int k = i < 192 ? i : i - 192, c = habx180_channel(k);
        Cn[i] = c < 0 ? 0.0f : i < 192 ? p.inw[c] : p.inb[c];
    }
    const int mbase = blockIdx.x * TX_ROWS + wave * 32;
    f32x4 acc[2][NT];
    tx_load_res<C>(p.res, mbase, M, lr, lg, acc);

    // ---- the projection: acc = x + ao . Wp^T, ao's rows one k-step ahead
    {
        WcRows<C> ar;
        ar.init(p.a, mbase, M, lr);
        f32x4 pre[2][2];
        ar.load(0, lg, pre);
#pragma unroll
        for (int c = 0; c < 6; ++c) {
            __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of chunk c (and its rows) have landed
            __syncthreads();                // everyone's have, and everyone is done with chunk c - 1
            if (c + 1 < 6) wc_issue<NLP, TX_WAVES>(c & 1 ? Ws0 : Ws1, p.w + (size_t)(c + 1) * MX180_SLOT, wave, lane);
            else wc_issue<NL1, TX_WAVES>(Ws0, p.wm, wave, lane);  // the MLP's first chunk
            u32x4 xb[2][3];
            split_pre(pre, xb);
            if (c + 1 < 6) ar.load(c + 1, lg, pre);
            ws_mma<NT, 16 * NT>(c & 1 ? Ws1 : Ws0, lr, lg, xb, acc);
        }
    }
    // x' = acc (+ conv2's output times gate * cscale) + bias, kept in acc;
    // norm2's statistics from it
    float2 st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int m = mbase + mt * 16 + lr;
        const float* arow = HAB && m < M ? p.aux + (size_t)m * C + lg * 4 : hat_zero_row;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f32x4 b4 = *(const f32x4*)(Cp + nt * 16 + lg * 4);
            if constexpr (HAB) {
                const f32x4 a4 = *(const f32x4*)(m < M && tx_live<C>(nt, lg) ? arow + nt * 16 : hat_zero_row);
                const f32x4 g4 = *(const f32x4*)(Cp + 192 + nt * 16 + lg * 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[mt][nt][j] += a4[j] * g4[j];
            }
            acc[mt][nt] += b4;
        }
        st[mt] = tx_row_stats<C>(acc[mt], lg, p.eps);
        // an opaque copy of the mean: otherwise the compiler reuses the
        // statistics' x' - mean in part 0's norm and keeps those 48 values
        // live beside x' through part 0 (35 VGPRs spilled)
        asm volatile("" : "+v"(st[mt].x));
    }

    // ---- the MLP on x' (acc), in six parts of 64 hidden units
    auto norm_pre = [&](int ks, f32x4 (&pre)[2][2]) {
        const float* wk = Cn + ks * 32 + lg * 8;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f32x4 w4 = *(const f32x4*)(wk + 4 * j), b4 = *(const f32x4*)(wk + 192 + 4 * j);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) pre[mt][j][i] = (pre[mt][j][i] - st[mt].x) * st[mt].y * w4[i] + b4[i];
        }
    };
    // y = norm2(x') in the fused order for k-step ks, at the lane's own
    // channels of the output rows (tile 11 only in lane group 0)
    float* yrow[2];
    bool yalive[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int m = mbase + mt * 16 + lr;
        yalive[mt] = m < M;
        yrow[mt] = p.out + (size_t)(yalive[mt] ? m : 0) * C + lg * 4;
    }
    auto load_y = [&](int ks, f32x4 (&dst)[2][2]) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            dst[mt][0] = *(const f32x4*)(yalive[mt] ? yrow[mt] + 32 * ks : hat_zero_row);
            dst[mt][1] = *(const f32x4*)(yalive[mt] && (ks < 5 || lg == 0) ? yrow[mt] + 32 * ks + 16 : hat_zero_row);
        }
    };
    // fc2 over a part's units from registers: chunks 6, 7 of the part;
    // at_last runs in the last step, after its copies are issued (the next
    // part's first rows: read there, not in fc1's last step, so that fc2's
    // first wait is not for them)
    auto fc2_part = [&](int q, const unsigned short* wq, f32x4 (&h)[2][4], auto&& at_last) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (s == 0) wc_issue<NL2, TX_WAVES>(Ws1, wq + (size_t)7 * MX180_SLOT, wave, lane);
            else if (q < NP - 1) wc_issue<NL1, TX_WAVES>(Ws0, wq + (size_t)8 * MX180_SLOT, wave, lane);
            if (s == 1) at_last();
            if (s == 0) {
                // + b1 (the lane's four units of each tile, in the part's
                // permuted row order), then GELU
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const f32x4 b = *(const f32x4*)(p.b1x + q * MX180_HID + 16 * nt + 4 * lg);
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                        for (int j = 0; j < 4; ++j) h[mt][nt][j] = gelu(h[mt][nt][j] + b[j]);
                }
            }
            u32x4 xb[2][3];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const float f[8] = {h[mt][2 * s][0],     h[mt][2 * s][1],     h[mt][2 * s][2],
                                    h[mt][2 * s][3],     h[mt][2 * s + 1][0], h[mt][2 * s + 1][1],
                                    h[mt][2 * s + 1][2], h[mt][2 * s + 1][3]};
                split3_x8(f, xb[mt]);
            }
            ws_mma<NT, 16 * NT>(s == 0 ? Ws0 : Ws1, lr, lg, xb, acc);
        }
    };
    // part 0: fc1's input from the registers
    {
        const unsigned short* wq = p.wm;
        f32x4 h[2][4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) h[0][nt] = h[1][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 6; ++ks) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (ks < 5) wc_issue<NL1, TX_WAVES>(ks & 1 ? Ws0 : Ws1, wq + (size_t)(ks + 1) * MX180_SLOT, wave, lane);
            else wc_issue<NL2, TX_WAVES>(Ws0, wq + (size_t)6 * MX180_SLOT, wave, lane);
            f32x4 pre[2][2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                pre[mt][0] = acc[mt][2 * ks];
                pre[mt][1] = acc[mt][2 * ks + 1];
            }
            norm_pre(ks, pre);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                // y for parts 1..5 (rows past M: the sink)
                float* yr = yalive[mt] ? yrow[mt] + 32 * ks : hat_sink_row;
                *(f32x4*)yr = pre[mt][0];
                if (ks < 5 || lg == 0) *(f32x4*)(yr + (yalive[mt] ? 16 : 4)) = pre[mt][1];
            }
            u32x4 xb[2][3];
            split_pre(pre, xb);
            ws_mma<4, MX180_HID>(ks & 1 ? Ws1 : Ws0, lr, lg, xb, h);
        }
        fc2_part(0, wq, h, [] {});
    }
    // parts 1..5: fc1's input read back from the output rows, one k-step ahead
    f32x4 pre[2][2];
    load_y(0, pre);
#pragma unroll 1
    for (int q = 1; q < NP; ++q) {
        const unsigned short* wq = p.wm + (size_t)(8 * q) * MX180_SLOT;
        f32x4 h[2][4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) h[0][nt] = h[1][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        auto fc1_step = [&](int ks, auto parv) {
            constexpr int PAR = decltype(parv)::value;  // = ks & 1
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (ks < 5) wc_issue<NL1, TX_WAVES>(PAR ? Ws0 : Ws1, wq + (size_t)(ks + 1) * MX180_SLOT, wave, lane);
            else wc_issue<NL2, TX_WAVES>(Ws0, wq + (size_t)6 * MX180_SLOT, wave, lane);
            u32x4 xb[2][3];
            split_pre(pre, xb);
            if (ks < 5) load_y(ks + 1, pre);
            ws_mma<4, MX180_HID>(PAR ? Ws1 : Ws0, lr, lg, xb, h);
        };
#pragma unroll 1
        for (int ks = 0; ks < 6; ks += 2) {
            fc1_step(ks, CInt<0>{});
            fc1_step(ks + 1, CInt<1>{});
        }
        fc2_part(q, wq, h, [&] {
            if (q < NP - 1) load_y(0, pre);
        });
    }
    tx_store_rows<C>(acc, Cs, mbase, M, lr, lg, p.eps, p.out, LN ? p.xn : nullptr);
}

extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_projx_cab(TailXArgs p) { projx_body<true>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_projx(TailXArgs p) { projx_body<false>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_mlpx_ln(TailXArgs p) { mlpx_body<true>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_mlpx(TailXArgs p) { mlpx_body<false>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_mlpx180_ln(TailXArgs p) { mlpx180_body<true>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_mlpx180(TailXArgs p) { mlpx180_body<false>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_projx180_hab(TailXArgs p) { projx180_body<true>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_projx180(TailXArgs p) { projx180_body<false>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_habx_cab_ln(TailXArgs p) { habx_body<true, true>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_habx(TailXArgs p) { habx_body<false, false>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_habx180_hab_ln(TailXArgs p) { habx180_body<true, true>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_habx180(TailXArgs p) { habx180_body<false, false>(p); }
