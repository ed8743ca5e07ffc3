// Token GEMM on FP32 MFMA: out[m][n] = epi( A[m][:] . W[n][:] + bias[n] ).
//
// Replaces the reference's lg_linear / lg_conv1x1_rb launches (src/cuda.rs:
// 162-169, 440-453) together with the elementwise passes around them: the
// GELU (cuda.rs:195-199), the q/k/v split (lg_extract_rows, cuda.rs:428-434),
// the residual adds (lg_add / lg_add_scaled, cuda.rs:227-248) and - when one
// block holds whole rows (N <= 16*NT) - the LayerNorm that follows
// (lg_channel_layer_norm, cuda.rs:185-191) are folded into the epilogue.
//
// Tiling: 256 threads = 4 waves; block tile 128 rows (m) x 16*NT columns (n).
// Wave w owns rows [32w, 32w+32) as two 16-row MFMA tiles and all NT column
// tiles. The MFMA is v_mfma_f32_16x16x4_f32 with the weight rows as the A
// operand and the activation rows as the B operand, so each lane's 4
// accumulators are 4 consecutive output columns of one row (one 16-byte store),
// and the 4 lanes {l, l^16, l^32, l^48} together hold whole rows. K is walked
// in chunks of 16 through double-buffered LDS (one barrier per chunk); within a
// chunk lane group g (= lane/16) reduces k in {4g .. 4g+3}, one float4 read.
#include "common.h"

using namespace hatk;

#define GEMM_BM 128
#define GEMM_BK 16
#define GEMM_LDS_STRIDE 20  // 16 + 4 floats: conflict-free float4 rows

// EPI_QKV: for the block's columns n0 .. n0+BN-1, the head-major destination
// ((which*heads + head) << 8) | dim, so the epilogue scatters with no division.
template <int BN, int EPI>
__device__ __forceinline__ void build_colmap(const GemmArgs& p, int n0, int* colmap)
{
    if (EPI != EPI_QKV) return;
    const int C = p.heads * p.hdim;
    for (int j = threadIdx.x; j < BN; j += blockDim.x) {
        const int n = n0 + j;
        const int which = n / C, rem = n - which * C;
        const int hd = rem / p.hdim, dim = rem - hd * p.hdim;
        colmap[j] = ((which * p.heads + hd) << 8) | dim;
    }
}

// Column constants of a block's n0.. columns, indexed from n0 (global memory
// or an LDS copy).
struct EpiConsts {
    const float* bias;
    const float* nw;
    const float* nb;
};

__device__ __forceinline__ EpiConsts global_consts(const GemmArgs& p, int n0)
{
    return EpiConsts{p.bias + n0, p.nw ? p.nw + n0 : nullptr, p.nb ? p.nb + n0 : nullptr};
}

// Epilogue shared by the GEMM kernels: lane (lr, lg) holds out[m][n .. n+3]
// for m = mbase + 16*mt + lr and n = n0 + 16*nt + 4*lg. With pres, the
// residual values were loaded ahead by the caller (same layout as acc).
// Stores 16 consecutive whole rows of NT*16 floats (lane (lr, lg) holding
// columns 16 nt + 4 lg .. +3 of row mbase + lr) through the wave's LDS region
// `stage` (8 rows of NT*16 + 4 floats): 8 rows at a time go to LDS and leave as
// one contiguous run, every lane storing whole 16-byte pieces of it, instead of
// 64-byte pieces one row apart. Rows from M on are not stored.
template <int NT>
__device__ __forceinline__ void stage_store_rows(float* stage, const f32x4 (&v)[NT], int mbase, int M, float* dst,
                                                 int lr, int lg)
{
    constexpr int BN = 16 * NT, SS = BN + 4, NF4 = 8 * BN / 4;
    const int lane = lg * 16 + lr;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        if ((lr >> 3) == half) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) *(f32x4*)(stage + (lr & 7) * SS + nt * 16 + lg * 4) = v[nt];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
#pragma unroll
        for (int i = 0; i < (NF4 + 63) / 64; ++i) {
            const int f = lane + 64 * i;
            if (f < NF4) {
                const int row = f / (BN / 4), c4 = f - row * (BN / 4);
                const int m = mbase + half * 8 + row;
                const f32x4 x = *(const f32x4*)(stage + row * SS + c4 * 4);
                if (m < M) *(f32x4*)(dst + (size_t)m * BN + c4 * 4) = x;
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // the reads are done before the region is rewritten
    }
}

// STAGE: MT = 1, whole contiguous rows (n0 = 0, N = ldo = 16*NT), and `stage`
// is the wave's LDS region for stage_store_rows. NTSTORE: `out` (not xn) goes
// out with non-temporal stores.
template <int MT, int NT, int EPI, bool BIAS_IN_ACC = false, bool STAGE = false, bool NTSTORE = false>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& p, const EpiConsts& k, f32x4 (&acc)[MT][NT],
                                              int mbase, int n0, int lr, int lg, const int* colmap,
                                              const f32x4 (*pres)[NT] = nullptr, float* stage = nullptr)
{
    static_assert(!STAGE || (MT == 1 && EPI != EPI_QKV), "staged stores are for whole rows of one row tile");
    const int M = p.M, N = p.N;
    constexpr bool LNOUT = EPI == EPI_RESID_LN || EPI == EPI_HAB_LN || EPI == EPI_STORE_LN;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mbase + mt * 16 + lr;
        const bool mlive = m < M;
        // Without a preloaded residual, the row's residual loads are all issued
        // here, before any is used (one at a time, each would wait in turn).
        constexpr bool RES = EPI == EPI_RESID || EPI == EPI_RESID_LN || EPI == EPI_HAB || EPI == EPI_HAB_LN;
        f32x4 rl[RES ? NT : 1];
        if (RES && !pres) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int n = n0 + nt * 16 + lg * 4;
                rl[nt] = load_or_zero(p.res + (size_t)m * p.ldo + n, mlive && n < N);
            }
        }
        // Values (bias + residual combine) in place. N is a multiple of 4, so a
        // lane's four columns are all live or all padding: whole float4 accesses.
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n = n0 + nt * 16 + lg * 4;
            const bool live = mlive && n < N;
            f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
            if (live) {
                // BIAS_IN_ACC: the accumulators started from the bias
                if (BIAS_IN_ACC) {
                    v = acc[mt][nt];
                } else {
                    const float4 b4 = *(const float4*)(k.bias + (n - n0));
                    v = acc[mt][nt] + (f32x4){b4.x, b4.y, b4.z, b4.w};
                }
                if (EPI == EPI_GELU) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = gelu(v[j]);
                }
                if (EPI == EPI_RESID || EPI == EPI_RESID_LN || EPI == EPI_HAB || EPI == EPI_HAB_LN) {
                    v = (pres ? pres[mt][nt] : rl[RES ? nt : 0]) + v;
                }
                if (EPI == EPI_HAB || EPI == EPI_HAB_LN) {
                    const float4 a4 = *(const float4*)(p.aux + (size_t)m * p.ldo + n);
                    const float4 g4 = *(const float4*)(p.gate + n);
                    v[0] = v[0] + (a4.x * g4.x) * p.cscale;
                    v[1] = v[1] + (a4.y * g4.y) * p.cscale;
                    v[2] = v[2] + (a4.z * g4.z) * p.cscale;
                    v[3] = v[3] + (a4.w * g4.w) * p.cscale;
                }
            }
            acc[mt][nt] = v;
        }
        float mean = 0.0f, rstd = 0.0f;
        if (LNOUT) {
            // Row statistics over the 4 lanes that share the row: two-pass mean
            // then biased variance, as the reference's layer_norm (cpu.rs:563-581).
            float s = 0.0f;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int j = 0; j < 4; ++j) s += acc[mt][nt][j];
            s += __shfl_xor(s, 16, 64);
            s += __shfl_xor(s, 32, 64);
            mean = s / (float)N;
            float q = 0.0f;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int n = n0 + nt * 16 + lg * 4 + j;
                    const float d = n < N ? acc[mt][nt][j] - mean : 0.0f;
                    q += d * d;
                }
            q += __shfl_xor(q, 16, 64);
            q += __shfl_xor(q, 32, 64);
            rstd = 1.0f / sqrtf(q / (float)N + p.eps);
        }
        if constexpr (STAGE) {
            stage_store_rows<NT>(stage, acc[0], mbase, M, p.out, lr, lg);
            if (LNOUT) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const int j = nt * 16 + lg * 4;
                    const float4 w4 = *(const float4*)(k.nw + j);
                    const float4 b4 = *(const float4*)(k.nb + j);
                    const f32x4 v = acc[0][nt];
                    acc[0][nt] = (f32x4){(v[0] - mean) * rstd * w4.x + b4.x, (v[1] - mean) * rstd * w4.y + b4.y,
                                         (v[2] - mean) * rstd * w4.z + b4.z, (v[3] - mean) * rstd * w4.w + b4.w};
                }
                stage_store_rows<NT>(stage, acc[0], mbase, M, p.xn, lr, lg);
            }
            continue;
        }
        if (!mlive) continue;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n = n0 + nt * 16 + lg * 4;
            if (n >= N) continue;
            const f32x4 v = acc[mt][nt];
            if (EPI == EPI_QKV) {
                // colmap[n - n0] = ((which*heads + head) << 8) | dim, built per block.
                // With hdim % 4 == 0 the four columns n .. n+3 (n % 4 == 0) are one
                // head's dims d .. d+3, d % 4 == 0: one aligned 16-byte store.
                if ((p.hdim & 3) == 0) {
                    const int cm = colmap[n - n0];
                    *(float4*)(p.out + ((size_t)(cm >> 8) * M + m) * p.hdim + (cm & 255)) =
                        make_float4(v[0], v[1], v[2], v[3]);
                    continue;
                }
                // With hdim even, column pairs (n, n+1), (n+2, n+3) are one
                // head's dims d, d+1 with d even (n and d share parity): two
                // aligned 8-byte stores.
                if ((p.hdim & 1) == 0) {
#pragma unroll
                    for (int j = 0; j < 4; j += 2) {
                        const int cm = colmap[n - n0 + j];
                        *(float2*)(p.out + ((size_t)(cm >> 8) * M + m) * p.hdim + (cm & 255)) = make_float2(v[j], v[j + 1]);
                    }
                    continue;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int cm = colmap[n - n0 + j];
                    p.out[((size_t)(cm >> 8) * M + m) * p.hdim + (cm & 255)] = v[j];
                }
                continue;
            }
            if (NTSTORE)
                __builtin_nontemporal_store(v, (f32x4*)(p.out + (size_t)m * p.ldo + n));
            else
                *(float4*)(p.out + (size_t)m * p.ldo + n) = make_float4(v[0], v[1], v[2], v[3]);
            if (LNOUT) {
                const float4 w4 = *(const float4*)(k.nw + (n - n0));
                const float4 b4 = *(const float4*)(k.nb + (n - n0));
                *(float4*)(p.xn + (size_t)m * p.ldo + n) =
                    make_float4((v[0] - mean) * rstd * w4.x + b4.x, (v[1] - mean) * rstd * w4.y + b4.y,
                                (v[2] - mean) * rstd * w4.z + b4.z, (v[3] - mean) * rstd * w4.w + b4.w);
            }
        }
    }
}

template <int NT, int EPI>
__device__ __forceinline__ void gemm_body(const GemmArgs& p)
{
    constexpr int BN = 16 * NT;
    constexpr int ABUF = GEMM_BM * GEMM_LDS_STRIDE, WBUF = BN * GEMM_LDS_STRIDE;
    __shared__ float As[2 * ABUF];
    __shared__ float Ws[2 * WBUF];
    __shared__ int s_colmap[EPI == EPI_QKV ? BN : 1];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;  // row within a 16-tile
    const int lg = lane >> 4;  // k group
    const int m0 = blockIdx.x * GEMM_BM;
    const int n0 = blockIdx.y * BN;
    const int M = p.M, N = p.N, K = p.K;

    f32x4 acc[2][NT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // Global -> register staging. A: 128 rows x 16 floats = 512 float4, 2 per
    // thread. W: BN rows x 16 floats = 4*BN float4.
    constexpr int WV = (BN * 4 + 255) / 256;
    float4 ra[2];
    float4 rw[WV];
    const int nchunks = p.Kp / GEMM_BK;

    auto load_chunk = [&](int kc) {
        const int k0 = kc * GEMM_BK;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int idx = tid + j * 256;
            const int r = idx >> 2, c4 = (idx & 3) * 4;
            const int m = m0 + r, k = k0 + c4;
            const bool ok = m < M && k < K;
            const f32x4 v = load_or_zero(p.a + (size_t)m * p.lda + k, ok);
            ra[j] = make_float4(v.x, v.y, v.z, v.w);
        }
#pragma unroll
        for (int j = 0; j < WV; ++j) {
            const int idx = tid + j * 256;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (idx < BN * 4) {
                const int r = idx >> 2, c4 = (idx & 3) * 4;
                const int n = n0 + r;
                if (n < N) v = *(const float4*)(p.w + (size_t)n * p.Kp + k0 + c4);
            }
            rw[j] = v;
        }
    };

    auto store_chunk = [&](int buf) {
        float* as = As + buf * ABUF;
        float* ws = Ws + buf * WBUF;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int idx = tid + j * 256;
            const int r = idx >> 2, c4 = (idx & 3) * 4;
            *(float4*)(as + r * GEMM_LDS_STRIDE + c4) = ra[j];
        }
#pragma unroll
        for (int j = 0; j < WV; ++j) {
            const int idx = tid + j * 256;
            if (idx < BN * 4) {
                const int r = idx >> 2, c4 = (idx & 3) * 4;
                *(float4*)(ws + r * GEMM_LDS_STRIDE + c4) = rw[j];
            }
        }
    };

    build_colmap<BN, EPI>(p, n0, s_colmap);
    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    for (int kc = 0; kc < nchunks; ++kc) {
        const bool more = kc + 1 < nchunks;
        if (more) load_chunk(kc + 1);
        const float* as = As + (kc & 1) * ABUF;
        const float* ws = Ws + (kc & 1) * WBUF;
        f32x4 xv[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
            xv[mt] = *(const f32x4*)(as + (wave * 32 + mt * 16 + lr) * GEMM_LDS_STRIDE + lg * 4);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f32x4 wv = *(const f32x4*)(ws + (nt * 16 + lr) * GEMM_LDS_STRIDE + lg * 4);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) acc[mt][nt] = mfma16(wv[s], xv[mt][s], acc[mt][nt]);
            }
        }
        if (more) store_chunk((kc + 1) & 1);
        __syncthreads();
    }

    gemm_epilogue<2, NT, EPI>(p, global_consts(p, n0), acc, m0 + wave * 32, n0, lr, lg, s_colmap);
}

#define GEMM_INST(NAME, NT, EPI)                                                             \
    extern "C" __global__ __launch_bounds__(256) void NAME(GemmArgs p) { gemm_body<NT, EPI>(p); }

// ---------------------------------------------------------------------------
// Weight-stationary variant for K = 144 (the C = 144 family's qkv, proj and fc1).
//
// A block holds a 144 x 144 weight slice (one column block) in LDS and loops
// over row tiles. The work is the sequence of (column slice, row tile) units,
// slice-major; block b takes units b, b + G, b + 2G, ... (G = gridDim.x, one
// block per CU), so every CU gets the same number of tiles to within one and
// the blocks running at one time work on neighbouring rows; a block reloads the
// weights where its units cross into the next slice (slices - 1 times at most).
// Each of the WAVES waves owns 16*MT rows of
// a tile and streams its A rows from global memory straight into registers,
// three K-chunks ahead of the MFMAs, so the K loop has no barrier and no LDS
// traffic for A; waves drift apart freely, and one wave's epilogue stores
// overlap the other waves' MFMAs. The MFMA arrangement and the epilogue are
// the ones of gemm_body (a lane's four accumulators are four consecutive
// columns).
// KP: the weight rows' padded K (144, or 192 for K = 180), a multiple of 48;
// NT: 16-column tiles per block (9, or 12 for the C = 180 family).
template <int EPI, int MT, int WAVES, bool CAB, int KP, int NT>
__device__ __forceinline__ void gemm_ws_body(const GemmArgs& p)
{
    constexpr int ROWS = WAVES * 16 * MT;  // rows per tile
    constexpr int BN = 16 * NT, NCH = KP / 16;
    constexpr int WS_K = KP, WS_KS = KP + 4;  // LDS row stride of the weight slice
    static_assert(NCH % 3 == 0, "the K loop walks groups of three chunks");
    static_assert(!CAB || (KP == 144 && NT == 9), "the folded CAB is the C = 144 family's");
    constexpr int S2 = CAB_K2 + 4;         // LDS row stride of the conv2 slice
    __shared__ __attribute__((aligned(16))) float Wsm[BN * WS_KS];
    __shared__ __attribute__((aligned(16))) float W2s[CAB ? BN * S2 : 1];
    __shared__ int s_colmap[EPI == EPI_QKV ? BN : 1];
    constexpr bool LNOUT = EPI == EPI_RESID_LN || EPI == EPI_HAB_LN;
    // bias (+ LayerNorm weight and bias) of the block's columns
    __shared__ __attribute__((aligned(16))) float Cs[(LNOUT ? 3 : 1) * BN];
    // q/k/v staging of the 144-column, head_dim 24 shape: per wave 16 rows x 48
    // columns (two heads), row stride QS_S.
    constexpr bool QSTAGE = EPI == EPI_QKV && BN == 144 && MT == 1;
    constexpr int QS_S = 52;
    __shared__ __attribute__((aligned(16))) float Qs[QSTAGE ? WAVES * 16 * QS_S : 1];
    // row staging of the whole-row epilogues (N = 144 in one column block)
    constexpr bool RSTAGE = (EPI == EPI_RESID || EPI == EPI_RESID_LN || EPI == EPI_HAB_LN) && BN == 144 && MT == 1;
    __shared__ __attribute__((aligned(16))) float Rs[RSTAGE ? WAVES * 8 * (BN + 4) : 1];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int M = p.M, N = p.N;

    // The weight slice of the columns from n0: BN rows x KP/4 float4, with the
    // conv2 slice, the QKV column map and the epilogue constants.
    auto load_slice = [&](int n0) {
        for (int idx = tid; idx < BN * (WS_K / 4); idx += WAVES * 64) {
            const int r = idx / (WS_K / 4), c4 = (idx - r * (WS_K / 4)) * 4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (n0 + r < N) v = *(const float4*)(p.w + (size_t)(n0 + r) * p.Kp + c4);
            *(float4*)(Wsm + r * WS_KS + c4) = v;
        }
        if (CAB) {
            for (int idx = tid; idx < BN * (CAB_K2 / 4); idx += WAVES * 64) {
                const int r = idx / (CAB_K2 / 4), c4 = (idx - r * (CAB_K2 / 4)) * 4;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (n0 + r < N) v = *(const float4*)(p.w2g + (size_t)(n0 + r) * CAB_K2 + c4);
                *(float4*)(W2s + r * S2 + c4) = v;
            }
        }
        build_colmap<BN, EPI>(p, n0, s_colmap);
        for (int i = tid; i < (LNOUT ? 3 : 1) * BN; i += WAVES * 64) {
            const int j = i % BN, n = n0 + j;
            const float* src = i < BN ? p.bias : (i < 2 * BN ? p.nw : p.nb);
            Cs[i] = n < N ? src[n] : 0.0f;
        }
    };
    const EpiConsts kc{Cs, LNOUT ? Cs + BN : nullptr, LNOUT ? Cs + 2 * BN : nullptr};

    const int ntiles = (M + ROWS - 1) / ROWS;
    const long units = (long)ntiles * ((N + BN - 1) / BN);

    // The A rows of unit u's row tile, clamped to row 0 past M.
    auto rows_of = [&](long u, const float* (&ar)[MT], bool (&al)[MT]) {
        const int tile = (int)(u % ntiles);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = tile * ROWS + wave * 16 * MT + mt * 16 + lr;
            al[mt] = m < M;
            ar[mt] = al[mt] ? p.a + (size_t)m * p.lda + lg * 4 : hat_zero_row;  // + kc*16 stays in it
        }
    };
    // A operands in three register slots, streamed three chunks ahead of the
    // MFMAs that use them (the chunk loop is rolled over groups of 3 so the
    // slots are fixed registers). The stream runs across units: the last three
    // chunks of a unit load the first three of the block's next unit (or
    // reload its own after its last unit), so every step issues exactly one
    // load per slot and the compiler's waits name the oldest one only.
    f32x4 xa[3][MT];
    // k beyond K (K = 180 in 192) reads as zero: past it lies the next row
    const bool kin_last = (NCH - 1) * 16 + lg * 4 < p.K;
    auto load_a = [&](int slot, int kc, const float* const (&ar)[MT]) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const bool kin = KP == 144 || kc < NCH - 1 || kin_last;
            xa[slot][mt] = load_or_zero(ar[mt] + kc * 16, kin);
        }
    };
    const float* arow[MT];
    bool alive[MT];
    rows_of(blockIdx.x, arow, alive);
#pragma unroll
    for (int s = 0; s < 3; ++s) load_a(s, s, arow);

    int slice = -1;
    for (long u = blockIdx.x; u < units; u += gridDim.x) {
        const int us = (int)(u / ntiles), tile = (int)(u - (long)us * ntiles);
        if (us != slice) {  // block-uniform
            if (slice >= 0) __syncthreads();  // every wave is done with the old slice
            load_slice(us * BN);
            __syncthreads();
            slice = us;
        }
        const int n0 = slice * BN;
        const int mbase = tile * ROWS + wave * 16 * MT;
        const float* arow_n[MT];
        bool alive_n[MT];
        rows_of(u + gridDim.x < units ? u + gridDim.x : u, arow_n, alive_n);
        // CAB: the 3x3 neighbourhood of t1 at each row's pixel, k = tap*6 + ci
        // (54 values, 2 zero): three 16-k chunks, lane group g holding k =
        // 16 kc2 + 4g .. +3 (two float2 of one or two taps), and an 8-k tail,
        // g holding k = 48 + 2g, 49 + 2g (tap 8's channels 2g, 2g+1; zero for g = 3).
        constexpr int K2F = CAB_K2 / 16;
        f32x4 xg[CAB ? MT : 1][K2F];
        float2 xh[CAB ? MT : 1];
        if (CAB) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = mbase + mt * 16 + lr;
                const int y = m / p.W, x = m - y * p.W;
                // t1[neighbour at tap][ci, ci+1], zero outside the plane
                // out-of-plane taps read zeros
                auto pair = [&](int tap, int ci) -> float2 {
                    const int yy = y + tap / 3 - 1, xx = x + tap % 3 - 1;
                    const bool ok = alive[mt] && tap < 9 && yy >= 0 && yy < p.H && xx >= 0 && xx < p.W;
                    return *(const float2*)(ok ? p.t1 + ((size_t)yy * p.W + xx) * CAB_CS + ci : hat_zero_row);
                };
#pragma unroll
                for (int kc2 = 0; kc2 < K2F; ++kc2) {
                    const int k0 = kc2 * 16 + lg * 4, ta = k0 / CAB_CC, ca = k0 - ta * CAB_CC;  // ca: 0, 2 or 4
                    const float2 lo = pair(ta, ca);
                    const bool same = ca + 2 < CAB_CC;
                    const float2 hi = pair(same ? ta : ta + 1, same ? ca + 2 : 0);
                    xg[mt][kc2] = (f32x4){lo.x, lo.y, hi.x, hi.y};
                }
                xh[mt] = pair(lg < 3 ? 8 : 9, 2 * lg);
            }
        }
        // The residual for the epilogue, loaded now so its latency hides under
        // the K loop.
        constexpr bool PRE = EPI == EPI_RESID_LN || EPI == EPI_RESID;
        f32x4 rres[PRE ? MT : 1][NT];
        if (PRE) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = mbase + mt * 16 + lr;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const int n = n0 + nt * 16 + lg * 4;
                    const bool ok = alive[mt] && n < N;
                    rres[mt][nt] = load_or_zero(p.res + (size_t)m * p.ldo + n, ok);
                }
            }
        }
        // The accumulators start from the bias (cpu.rs linear's order: bias,
        // then the products); Cs is zero past N.
        f32x4 acc[MT][NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const f32x4 b4 = *(const f32x4*)(Cs + j * 16 + lg * 4);
#pragma unroll
            for (int i = 0; i < MT; ++i) acc[i][j] = b4;
        }
#pragma unroll
        for (int kg = 0; kg < NCH; kg += 3) {
#pragma unroll
            for (int slot = 0; slot < 3; ++slot) {
                const int kc = kg + slot;
                f32x4 cur[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) cur[mt] = xa[slot][mt];
                if (kc + 3 < NCH) load_a(slot, kc + 3, arow);  // compile-time choice
                else load_a(slot, kc + 3 - NCH, arow_n);
                // the load stays here, three chunks ahead of its MFMAs (the
                // scheduler would otherwise sink it next to them)
                __builtin_amdgcn_sched_barrier(0);
                const float* wrow = Wsm + lr * WS_KS + kc * 16 + lg * 4;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const f32x4 wv = *(const f32x4*)(wrow + nt * 16 * WS_KS);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            acc[mt][nt] = mfma16(wv[s], cur[mt][s], acc[mt][nt]);
                }
            }
        }
        // the slots now hold the next unit's first chunks
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            arow[mt] = arow_n[mt];
            alive[mt] = alive_n[mt];
        }
        if (CAB) {
#pragma unroll
            for (int kc2 = 0; kc2 <= K2F; ++kc2) {
                // keep each chunk's weight reads next to its MFMAs (hoisting
                // all of them costs more registers than there are)
                __builtin_amdgcn_sched_barrier(0);
                if (kc2 < K2F) {
                    const float* wrow = W2s + lr * S2 + kc2 * 16 + lg * 4;
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const f32x4 wv = *(const f32x4*)(wrow + nt * 16 * S2);
#pragma unroll
                        for (int s = 0; s < 4; ++s)
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt)
                                acc[mt][nt] = mfma16(wv[s], xg[mt][kc2][s], acc[mt][nt]);
                    }
                } else {
                    // the 8-k tail: two MFMAs, lane group g's k = 48 + 2g + s
                    const float* wrow = W2s + lr * S2 + K2F * 16 + lg * 2;
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const float2 wv = *(const float2*)(wrow + nt * 16 * S2);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            acc[mt][nt] = mfma16(wv.x, xh[mt].x, acc[mt][nt]);
                            acc[mt][nt] = mfma16(wv.y, xh[mt].y, acc[mt][nt]);
                        }
                    }
                }
            }
        }
        if (QSTAGE && p.hdim == 24 && p.heads * 24 == BN) {
            // A slice is one of q, k, v (6 heads x 24). Two heads at a time go
            // through the wave's LDS region and leave as 16 consecutive rows of
            // each head: 1536 contiguous bytes per head, every lane storing
            // 16 bytes of one run, instead of 16-byte pieces 96 bytes apart.
            // The stores are non-temporal (measured faster, for this kernel
            // and for the attention that reads q, k, v next).
            float* Q = Qs + wave * 16 * QS_S;
            const int mrows = M - mbase;  // rows of this wave that exist (may exceed 16)
#pragma unroll
            for (int ph = 0; ph < 3; ++ph) {
#pragma unroll
                for (int t = 0; t < 3; ++t) *(f32x4*)(Q + lr * QS_S + t * 16 + lg * 4) = acc[0][3 * ph + t];
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
#pragma unroll
                for (int i = 0; i < 3; ++i) {
                    const int f = lane + 64 * i, hh = f / 96, r = (f - hh * 96) / 6, d4 = f - hh * 96 - r * 6;
                    const f32x4 v = *(const f32x4*)(Q + r * QS_S + hh * 24 + d4 * 4);
                    if (r < mrows) {
                        const int head = 2 * ph + hh;
                        __builtin_nontemporal_store(v, (f32x4*)(p.out + ((size_t)(slice * p.heads + head) * M + mbase + r) * 24 + d4 * 4));
                    }
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next phase's writes
            }
            continue;
        }
        if constexpr (RSTAGE) {
            if (N == BN && p.ldo == BN) {
                gemm_epilogue<MT, NT, EPI, true, true>(p, kc, acc, mbase, n0, lr, lg, s_colmap, PRE ? rres : nullptr,
                                                       Rs + wave * 8 * (BN + 4));
                continue;
            }
        }
        gemm_epilogue<MT, NT, EPI, true>(p, kc, acc, mbase, n0, lr, lg, s_colmap, PRE ? rres : nullptr);
    }
}

#define GEMM_WS_INST(NAME, EPI, KP, NT)                                                      \
    extern "C" __global__ __launch_bounds__(ws_waves(EPI) * 64) void NAME(GemmArgs p)          \
    {                                                                                          \
        gemm_ws_body<EPI, ws_mt(EPI), ws_waves(EPI), false, KP, NT>(p);                        \
    }

// NT = 9: 144-wide column blocks (HAT-S: N = 144, 288, 432 divide exactly).
GEMM_INST(hat_gemm_n9_store, 9, EPI_STORE)
GEMM_INST(hat_gemm_n9_gelu, 9, EPI_GELU)
GEMM_INST(hat_gemm_n9_qkv, 9, EPI_QKV)
GEMM_INST(hat_gemm_n9_resid, 9, EPI_RESID)
GEMM_INST(hat_gemm_n9_resid_ln, 9, EPI_RESID_LN)
GEMM_INST(hat_gemm_n9_hab_ln, 9, EPI_HAB_LN)
// NT = 12: 192-wide column blocks (C = 180 models: 180, 360, 540 -> 1, 2, 3 blocks).
GEMM_INST(hat_gemm_n12_store, 12, EPI_STORE)
GEMM_INST(hat_gemm_n12_gelu, 12, EPI_GELU)
GEMM_INST(hat_gemm_n12_qkv, 12, EPI_QKV)
GEMM_INST(hat_gemm_n12_resid, 12, EPI_RESID)
GEMM_INST(hat_gemm_n12_resid_ln, 12, EPI_RESID_LN)
GEMM_INST(hat_gemm_n12_hab_ln, 12, EPI_HAB_LN)

// K = 144 weight-stationary instances (HAT-S: qkv N = 432, fc1 N = 288, attention
// proj and OCAB proj N = 144).
GEMM_WS_INST(hat_gemmws_qkv, EPI_QKV, 144, 9)
GEMM_WS_INST(hat_gemmws_gelu, EPI_GELU, 144, 9)
GEMM_WS_INST(hat_gemmws_resid_ln, EPI_RESID_LN, 144, 9)
GEMM_WS_INST(hat_gemmws_hab_ln, EPI_HAB_LN, 144, 9)
// K = 180 (padded to 192), 192-wide column blocks: the C = 180 family's qkv
// (N = 540 in 3 blocks), fc1 (N = 360 in 2) and projections (N = 180).
GEMM_WS_INST(hat_gemmws12_qkv, EPI_QKV, 192, 12)
GEMM_WS_INST(hat_gemmws12_gelu, EPI_GELU, 192, 12)
GEMM_WS_INST(hat_gemmws12_resid_ln, EPI_RESID_LN, 192, 12)
GEMM_WS_INST(hat_gemmws12_hab_ln, EPI_HAB_LN, 192, 12)

// HAB attention projection with the CAB's conv2 folded in as 56 more K (the
// block input as residual, bias = proj bias + folded conv2 bias), then norm2.
extern "C" __global__ __launch_bounds__(ws_waves(EPI_RESID_LN) * 64) void hat_gemmws_cab_ln(GemmArgs p)
{
    gemm_ws_body<EPI_RESID_LN, ws_mt(EPI_RESID_LN), ws_waves(EPI_RESID_LN), true, 144, 9>(p);
}
