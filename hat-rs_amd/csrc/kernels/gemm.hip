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

template <int NT, int EPI>
__device__ __forceinline__ void gemm_body(const GemmArgs& p)
{
    constexpr int BN = 16 * NT;
    constexpr int ABUF = GEMM_BM * GEMM_LDS_STRIDE, WBUF = BN * GEMM_LDS_STRIDE;
    __shared__ float As[2 * ABUF];
    __shared__ float Ws[2 * WBUF];

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
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < M && k < K) v = *(const float4*)(p.a + (size_t)m * p.lda + k);
            ra[j] = v;
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

    // Epilogue: lane holds out[m][n .. n+3] for n = n0 + 16*nt + 4*lg.
    constexpr bool LNOUT = EPI == EPI_RESID_LN || EPI == EPI_HAB_LN;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int m = m0 + wave * 32 + mt * 16 + lr;
        const bool mlive = m < M;
        // Values (bias + residual combine) in place. N is a multiple of 4, so a
        // lane's four columns are all live or all padding: whole float4 accesses.
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n = n0 + nt * 16 + lg * 4;
            const bool live = mlive && n < N;
            f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
            if (live) {
                const float4 b4 = *(const float4*)(p.bias + n);
                v = acc[mt][nt] + (f32x4){b4.x, b4.y, b4.z, b4.w};
                if (EPI == EPI_GELU) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = gelu(v[j]);
                }
                if (EPI == EPI_RESID || EPI == EPI_RESID_LN || EPI == EPI_HAB || EPI == EPI_HAB_LN) {
                    const float4 r4 = *(const float4*)(p.res + (size_t)m * p.ldo + n);
                    v = (f32x4){r4.x, r4.y, r4.z, r4.w} + v;
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
        if (!mlive) continue;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n = n0 + nt * 16 + lg * 4;
            if (n >= N) continue;
            const f32x4 v = acc[mt][nt];
            if (EPI == EPI_QKV) {
                const int C = p.heads * p.hdim;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int nn = n + j;
                    if (nn >= N) break;
                    const int which = nn / C, rem = nn - which * C;
                    const int hd = rem / p.hdim, dim = rem - hd * p.hdim;
                    p.out[((size_t)(which * p.heads + hd) * M + m) * p.hdim + dim] = v[j];
                }
                continue;
            }
            *(float4*)(p.out + (size_t)m * p.ldo + n) = make_float4(v[0], v[1], v[2], v[3]);
            if (LNOUT) {
                const float4 w4 = *(const float4*)(p.nw + n);
                const float4 b4 = *(const float4*)(p.nb + n);
                *(float4*)(p.xn + (size_t)m * p.ldo + n) =
                    make_float4((v[0] - mean) * rstd * w4.x + b4.x, (v[1] - mean) * rstd * w4.y + b4.y,
                                (v[2] - mean) * rstd * w4.z + b4.z, (v[3] - mean) * rstd * w4.w + b4.w);
            }
        }
    }
}

#define GEMM_INST(NAME, NT, EPI)                                                             \
    extern "C" __global__ __launch_bounds__(256) void NAME(GemmArgs p) { gemm_body<NT, EPI>(p); }

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
