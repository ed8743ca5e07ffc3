// The second half of a HAB (and of an OCAB), C = 144, on split-bf16 MFMA, as
// two kernels (hat_arch.py HAB.forward / OCAB.forward; cpu.rs hab 1090-1166,
// ocab 983-1055; the reference GPU graph's proj, CAB conv2 and channel scale,
// adds, norm2, fc1 + GELU + fc2 and the next norm1, src/gpu.rs:469-588):
//
//   hat_projx_cab / hat_projx:  x' = x + ao . Wp^T (+ nb(t1) . W2g^T) + bias
//                               out = x',  xn = LN2(x')
//   hat_mlpx_ln / hat_mlpx:     out = x' + fc2(gelu(fc1(LN2(x')))) + b2
//                               (xn = LN_next(out))
//
// ao is the attention output, nb(t1) the 3x3 neighbourhood of the CAB's conv1
// output (k = tap*6 + ci, 54 values) and W2g / bias the gate-scaled conv2
// weights and combined bias written by the gate (hat_cab_gate's work); the
// OCAB form has no conv2 and its bias is the projection's. Products are the
// six-term split-bf16 ones of attnx.hip on v_mfma_f32_16x16x32_bf16, weights as
// the A operand, tokens as B; a lane's four accumulators are four consecutive
// output channels of one token.
//
// One fused kernel would need the three-plane weights of all four linears
// (677 KB) to stream through LDS in double-buffered chunks next to epilogue
// staging, which 160 KB does not hold at a useful chunk size; split in two,
// each kernel takes 256-token row tiles through weight slices pre-split on
// the host (the projection's 144 rows: 121.5 KB; the MLP's: 88 KB per slice)
// with global_load_lds into one LDS buffer, at the cost of writing and
// re-reading x' and LN2(x').
//
// The MLP walks the hidden layer in thirds of 96 units, so that fc1's
// output of a third (48 registers) and fc2's accumulators (72) fit a lane
// next to the operands: per third, fc1's slice, then fc2's slice on those
// units. fc1's output stays in registers and is fc2's B operand: fc1's rows
// are permuted on the host so that output tile t, row 4g + r (lane group g,
// register r) is unit 32(t/2) + 8g + 4(t%2) + r of the third; fc2's 32-k
// step s then finds units 32s + 8g .. +7 in tiles 2s and 2s+1 of lane group
// g, its weights in natural order.
//
// Included after gemmx.hip (GX_* slice constants, the MFMA helpers).

#define TX_WAVES 8
#define TX_ROWS (TX_WAVES * 32)
#define TX_K2S 72                 // LDS row stride of the conv2 planes (64 k + 8)
#define TX_K2PLANE (144 * TX_K2S)

// This wave's 32 token rows of a [M][144] plane, 8 values at k = 32 ks + 8 lg
// per token, for the B operand (zeros past M and past k = 144).
struct TxRows {
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
};

// A pre-split slice of CHUNKS x 512 bf16 into LDS, every load in flight
// (lane l of a load writes 16 bytes at the load's LDS base + 16 l).
template <int CHUNKS>
__device__ __forceinline__ void tx_load_slice(unsigned short* Ws, const unsigned short* src, int wave, int lane)
{
    for (int c = wave; c < CHUNKS; c += TX_WAVES)
        __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)(c * 64 + lane) * 8),
                                         (__attribute__((address_space(3))) void*)(Ws + c * 512), 16, 0, 0);
}

// acc[mt][nt] += W[rows 16 nt .. +15][k 32 ks + 8 lg .. +7] . xb[mt]: the
// three weight planes (row stride KS, plane stride PLANE) of tile nt + 1 are
// read while tile nt's 12 MFMAs run (the barriers keep the scheduler from
// hoisting every tile's reads, which costs more registers than there are).
template <int NT, int KS, int PLANE>
__device__ __forceinline__ void tx_mma_step(const unsigned short* Ws, int ks, int lr, int lg, const u32x4 (&xb)[2][3],
                                            f32x4 (&acc)[2][NT])
{
    const unsigned short* wr = Ws + lr * KS + ks * 32 + lg * 8;
    u32x4 wa[2][3];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) wa[0][pl] = *(const u32x4*)(wr + pl * PLANE);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        __builtin_amdgcn_sched_barrier(0);
        if (nt + 1 < NT) {
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) wa[(nt + 1) & 1][pl] = *(const u32x4*)(wr + (nt + 1) * 16 * KS + pl * PLANE);
        }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) acc[mt][nt] = mfma16x6(wa[nt & 1], xb[mt], acc[mt][nt]);
    }
}

// acc[mt][nt] += W(slice) . X^T over K = 144 in five 32-k steps, X read from
// global rows one step ahead and split.
template <int NT, int KS, int PLANE>
__device__ __forceinline__ void tx_mma_rows(const unsigned short* Ws, const TxRows& xr, int lr, int lg,
                                            f32x4 (&acc)[2][NT])
{
    f32x4 pre[2][2];
    xr.load(0, lg, pre);
#pragma unroll 1
    for (int ks = 0; ks < 5; ++ks) {
        u32x4 xb[2][3];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const float f[8] = {pre[mt][0][0], pre[mt][0][1], pre[mt][0][2], pre[mt][0][3],
                                pre[mt][1][0], pre[mt][1][1], pre[mt][1][2], pre[mt][1][3]};
            split3_x8(f, xb[mt]);
        }
        if (ks + 1 < 5) xr.load(ks + 1, lg, pre);
        tx_mma_step<NT, KS, PLANE>(Ws, ks, lr, lg, xb, acc);
    }
}

// Row statistics of a token over its 144 channels (36 per lane, the four lane
// groups of the token reducing with shuffles): two-pass mean, biased variance
// (cpu.rs:563-581); returns (mean, rstd).
__device__ __forceinline__ float2 tx_row_stats(const f32x4 (&v)[9], float eps)
{
    float s = 0.0f;
#pragma unroll
    for (int nt = 0; nt < 9; ++nt)
#pragma unroll
        for (int j = 0; j < 4; ++j) s += v[nt][j];
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    const float mean = s / 144.0f;
    float q = 0.0f;
#pragma unroll
    for (int nt = 0; nt < 9; ++nt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float d = v[nt][j] - mean;
            q += d * d;
        }
    q += __shfl_xor(q, 16, 64);
    q += __shfl_xor(q, 32, 64);
    return make_float2(mean, 1.0f / sqrtf(q / 144.0f + eps));
}

// x' = x + ao . Wp^T (+ nb(t1) . W2g^T) + bias; out = x', xn = LN2(x').
template <bool CAB>
__device__ __forceinline__ void projx_body(const TailXArgs& p)
{
    __shared__ __attribute__((aligned(16))) unsigned short Ws[GX_SLICE_PAD];
    __shared__ __attribute__((aligned(16))) float Cs[3 * 144];  // bias, norm2 w, b
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    const int ntiles = (M + TX_ROWS - 1) / TX_ROWS;
    if ((int)blockIdx.x >= ntiles) return;  // whole block, before any barrier
    for (int i = tid; i < 3 * 144; i += TX_WAVES * 64)
        Cs[i] = i < 144 ? p.bias[i] : (i < 288 ? p.nw[i - 144] : p.nb[i - 288]);
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int mbase = tile * TX_ROWS + wave * 32;
        if (CAB || tile == (int)blockIdx.x) {
            // (the CAB form's conv2 planes take the slice's place every tile)
            __syncthreads();  // every wave is done with the previous tile's conv2 planes
            tx_load_slice<GX_SLICE_PAD / 512>(Ws, p.w, wave, lane);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
        f32x4 acc[2][9];
#pragma unroll
        for (int nt = 0; nt < 9; ++nt) {
            const f32x4 b4 = *(const f32x4*)(Cs + nt * 16 + lg * 4);
            acc[0][nt] = b4;
            acc[1][nt] = b4;
        }
        TxRows ar;
        ar.init(p.a, mbase, M, lr);
        tx_mma_rows<9, GX_KS, GX_PLANE>(Ws, ar, lr, lg, acc);
        if (CAB) {
            // The gated conv2: its fp32 weights [144][56], split into three
            // planes [144][TX_K2S] (k 56..71 zero), then two 32-k steps over
            // the t1 neighbourhood (k 54..63 of the activations zero).
            __syncthreads();  // the projection slice is no longer read
            for (int e = tid; e < 144 * 36; e += TX_WAVES * 64) {
                const int n = e / 36, k2 = (e - n * 36) * 2;
                const float a = k2 < CAB_K2 ? p.w2g[n * CAB_K2 + k2] : 0.0f;
                const float b = k2 + 1 < CAB_K2 ? p.w2g[n * CAB_K2 + k2 + 1] : 0.0f;
                unsigned q0, q1, q2;
                split3_pk(a, b, q0, q1, q2);
                *(unsigned*)(Ws + n * TX_K2S + k2) = q0;
                *(unsigned*)(Ws + TX_K2PLANE + n * TX_K2S + k2) = q1;
                *(unsigned*)(Ws + 2 * TX_K2PLANE + n * TX_K2S + k2) = q2;
            }
            __syncthreads();
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                u32x4 xb[2][3];
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const int m = mbase + mt * 16 + lr;
                    const bool alive = m < M;
                    const int y = m / p.W, x = m - y * p.W;
                    float f[8];
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        // k even: (ci, ci+1) of one tap; taps outside the plane and k >= 54 read zeros
                        const int k = ks * 32 + lg * 8 + j, tap = k / 6, ci = k - tap * 6;
                        const int yy = y + tap / 3 - 1, xx = x + tap % 3 - 1;
                        const bool ok = alive && tap < 9 && yy >= 0 && yy < p.H && xx >= 0 && xx < p.W;
                        const float2 v = *(const float2*)(ok ? p.t1 + ((size_t)yy * p.W + xx) * CAB_CS + ci : hat_zero_row);
                        f[j] = v.x;
                        f[j + 1] = v.y;
                    }
                    split3_x8(f, xb[mt]);
                }
#pragma unroll
                for (int nt = 0; nt < 9; ++nt) {
                    u32x4 wa[3];
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl)
                        wa[pl] = *(const u32x4*)(Ws + pl * TX_K2PLANE + (nt * 16 + lr) * TX_K2S + ks * 32 + lg * 8);
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) acc[mt][nt] = mfma16x6(wa, xb[mt], acc[mt][nt]);
                }
            }
        }
        // x' = x + acc; out = x'; xn = LN2(x')
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int m = mbase + mt * 16 + lr;
            const bool alive = m < M;
            const float* xrow = alive ? p.res + (size_t)m * 144 + lg * 4 : hat_zero_row;
            f32x4 v[9];
#pragma unroll
            for (int nt = 0; nt < 9; ++nt) v[nt] = *(const f32x4*)(xrow + (alive ? nt * 16 : 0)) + acc[mt][nt];
            const float2 st = tx_row_stats(v, p.eps);
            if (!alive) continue;
            float* orow = p.out + (size_t)m * 144 + lg * 4;
            float* nrow = p.xn + (size_t)m * 144 + lg * 4;
#pragma unroll
            for (int nt = 0; nt < 9; ++nt) {
                *(f32x4*)(orow + nt * 16) = v[nt];
                const f32x4 w4 = *(const f32x4*)(Cs + 144 + nt * 16 + lg * 4);
                const f32x4 b4 = *(const f32x4*)(Cs + 288 + nt * 16 + lg * 4);
                f32x4 y;
#pragma unroll
                for (int j = 0; j < 4; ++j) y[j] = (v[nt][j] - st.x) * st.y * w4[j] + b4[j];
                *(f32x4*)(nrow + nt * 16) = y;
            }
        }
    }
}

// out = x' + fc2(gelu(fc1(y))) + b2 (+ xn = LN_next(out)); y = p.a, x' = p.res.
// p.w: six MX_SLICE slots (per third: fc1's 96 permuted rows, fc2 on those
// units); p.bias: b1 in fc1's permuted row order.
template <bool LN>
__device__ __forceinline__ void mlpx_body(const TailXArgs& p)
{
    constexpr int P1 = MX_HID * MX_KS1, P2 = 144 * MX_KS2;  // plane strides
    __shared__ __attribute__((aligned(16))) unsigned short Ws[MX_SLICE];
    __shared__ __attribute__((aligned(16))) float Cs[288 + 3 * 144];  // b1, b2, next norm w, b
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int M = p.M;
    const int ntiles = (M + TX_ROWS - 1) / TX_ROWS;
    if ((int)blockIdx.x >= ntiles) return;  // whole block, before any barrier
    for (int i = tid; i < 288 + 3 * 144; i += TX_WAVES * 64) {
        float v;
        if (i < 288) v = p.bias[i];
        else if (i < 432) v = p.b2[i - 288];
        else if (i < 576) v = LN ? p.nw[i - 432] : 0.0f;
        else v = LN ? p.nb[i - 576] : 0.0f;
        Cs[i] = v;
    }
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int mbase = tile * TX_ROWS + wave * 32;
        TxRows yr;
        yr.init(p.a, mbase, M, lr);
        f32x4 acc2[2][9];
#pragma unroll
        for (int nt = 0; nt < 9; ++nt) acc2[0][nt] = acc2[1][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
        for (int q = 0; q < 3; ++q) {
            // fc1: the third's 96 hidden units (permuted rows)
            __syncthreads();
            tx_load_slice<MX_SLICE / 512>(Ws, p.w + (size_t)(2 * q) * MX_SLICE, wave, lane);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            f32x4 h[2][6];
#pragma unroll
            for (int nt = 0; nt < 6; ++nt) {
                const f32x4 b4 = *(const f32x4*)(Cs + q * MX_HID + nt * 16 + lg * 4);
                h[0][nt] = b4;
                h[1][nt] = b4;
            }
            tx_mma_rows<6, MX_KS1, P1>(Ws, yr, lr, lg, h);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 6; ++nt)
#pragma unroll
                    for (int j = 0; j < 4; ++j) h[mt][nt][j] = gelu(h[mt][nt][j]);
            // fc2 over the third's units, from registers
            __syncthreads();
            tx_load_slice<MX_SLICE / 512>(Ws, p.w + (size_t)(2 * q + 1) * MX_SLICE, wave, lane);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
#pragma unroll
            for (int ks = 0; ks < 3; ++ks) {
                u32x4 xb[2][3];
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const float f[8] = {h[mt][2 * ks][0],     h[mt][2 * ks][1],     h[mt][2 * ks][2],
                                        h[mt][2 * ks][3],     h[mt][2 * ks + 1][0], h[mt][2 * ks + 1][1],
                                        h[mt][2 * ks + 1][2], h[mt][2 * ks + 1][3]};
                    split3_x8(f, xb[mt]);
                }
                tx_mma_step<9, MX_KS2, P2>(Ws, ks, lr, lg, xb, acc2);
            }
        }
        // out = x' + acc2 + b2; xn = LN_next(out)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int m = mbase + mt * 16 + lr;
            const bool alive = m < M;
            const float* rrow = alive ? p.res + (size_t)m * 144 + lg * 4 : hat_zero_row;
            f32x4 v[9];
#pragma unroll
            for (int nt = 0; nt < 9; ++nt) {
                const f32x4 b4 = *(const f32x4*)(Cs + 288 + nt * 16 + lg * 4);
                v[nt] = *(const f32x4*)(rrow + (alive ? nt * 16 : 0)) + (acc2[mt][nt] + b4);
            }
            float2 st = make_float2(0.f, 0.f);
            if (LN) st = tx_row_stats(v, p.eps);
            if (!alive) continue;
            float* orow = p.out + (size_t)m * 144 + lg * 4;
#pragma unroll
            for (int nt = 0; nt < 9; ++nt) *(f32x4*)(orow + nt * 16) = v[nt];
            if (LN) {
                float* nrow = p.xn + (size_t)m * 144 + lg * 4;
#pragma unroll
                for (int nt = 0; nt < 9; ++nt) {
                    const f32x4 w4 = *(const f32x4*)(Cs + 432 + nt * 16 + lg * 4);
                    const f32x4 b4 = *(const f32x4*)(Cs + 576 + nt * 16 + lg * 4);
                    f32x4 y;
#pragma unroll
                    for (int j = 0; j < 4; ++j) y[j] = (v[nt][j] - st.x) * st.y * w4[j] + b4[j];
                    *(f32x4*)(nrow + nt * 16) = y;
                }
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_projx_cab(TailXArgs p) { projx_body<true>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_projx(TailXArgs p) { projx_body<false>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_mlpx_ln(TailXArgs p) { mlpx_body<true>(p); }
extern "C" __global__ __launch_bounds__(TX_WAVES * 64, 2) void hat_mlpx(TailXArgs p) { mlpx_body<false>(p); }
