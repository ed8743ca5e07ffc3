// Token GEMM on FP32 MFMA: out[m][n] = epi( pro(A)[m][:] . W[n][:] + bias[n] ).
//
// Replaces the reference's lg_linear / lg_conv1x1_rb launches (src/cuda.rs:
// 162-169, 440-453) together with the elementwise passes around them: the
// LayerNorm prologue (lg_channel_layer_norm, cuda.rs:185-191), the GELU
// (cuda.rs:195-199), the q/k/v split (lg_extract_rows, cuda.rs:428-434) and the
// residual adds (lg_add / lg_add_scaled, cuda.rs:227-248) are folded in.
//
// Tiling: 256 threads = 4 waves; block tile 128 rows (m) x 16*NT columns (n).
// Wave w owns rows [32w, 32w+32) as two 16-row MFMA tiles and all NT column
// tiles. The MFMA is v_mfma_f32_16x16x4_f32 with the weight rows as the A
// operand and the activation rows as the B operand, so each lane's 4
// accumulators are 4 consecutive output columns of one row (one 16-byte store).
// K is walked in chunks of 16, staged in LDS; within a chunk lane group g
// (= lane/16) reduces k in {4g .. 4g+3}, read as one float4.
#include "common.h"

using namespace hatk;

#define GEMM_BM 128
#define GEMM_BK 16
#define GEMM_LDS_STRIDE 20  // 16 + 4 floats: conflict-free float4 rows

template <int NT, int EPI, bool LN>
__device__ __forceinline__ void gemm_body(const GemmArgs& p)
{
    constexpr int BN = 16 * NT;
    __shared__ float As[GEMM_BM * GEMM_LDS_STRIDE];
    __shared__ float Ws[BN * GEMM_LDS_STRIDE];
    __shared__ float s_mean[LN ? GEMM_BM : 1];
    __shared__ float s_rstd[LN ? GEMM_BM : 1];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;  // row within a 16-tile
    const int lg = lane >> 4;  // k group
    const int m0 = blockIdx.x * GEMM_BM;
    const int n0 = blockIdx.y * BN;
    const int M = p.M, N = p.N, K = p.K;

    if (LN) {
        // Per-row LayerNorm statistics, two-pass (mean, then biased variance),
        // one wave per row; each wave covers its own 32 rows.
        for (int rr = 0; rr < 32; ++rr) {
            const int r = wave * 32 + rr;
            const int m = m0 + r;
            float mean = 0.0f, rstd = 0.0f;
            if (m < M) {
                const float* row = p.a + (size_t)m * p.lda;
                float s = 0.0f;
                for (int k = lane; k < K; k += 64) s += row[k];
                mean = wave_sum(s) / (float)K;
                float v = 0.0f;
                for (int k = lane; k < K; k += 64) {
                    float d = row[k] - mean;
                    v += d * d;
                }
                float var = wave_sum(v) / (float)K;
                rstd = 1.0f / sqrtf(var + p.eps);
            }
            if (lane == 0) {
                s_mean[r] = mean;
                s_rstd[r] = rstd;
            }
        }
        __syncthreads();
    }

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

    auto store_chunk = [&](int kc) {
        const int k0 = kc * GEMM_BK;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int idx = tid + j * 256;
            const int r = idx >> 2, c4 = (idx & 3) * 4;
            float4 v = ra[j];
            if (LN) {
                const int k = k0 + c4;
                if (k < K) {
                    const float mu = s_mean[r], rs = s_rstd[r];
                    v.x = (v.x - mu) * rs * p.lnw[k + 0] + p.lnb[k + 0];
                    v.y = (v.y - mu) * rs * p.lnw[k + 1] + p.lnb[k + 1];
                    v.z = (v.z - mu) * rs * p.lnw[k + 2] + p.lnb[k + 2];
                    v.w = (v.w - mu) * rs * p.lnw[k + 3] + p.lnb[k + 3];
                }
            }
            *(float4*)(As + r * GEMM_LDS_STRIDE + c4) = v;
        }
#pragma unroll
        for (int j = 0; j < WV; ++j) {
            const int idx = tid + j * 256;
            if (idx < BN * 4) {
                const int r = idx >> 2, c4 = (idx & 3) * 4;
                *(float4*)(Ws + r * GEMM_LDS_STRIDE + c4) = rw[j];
            }
        }
    };

    load_chunk(0);
    for (int kc = 0; kc < nchunks; ++kc) {
        __syncthreads();
        store_chunk(kc);
        __syncthreads();
        if (kc + 1 < nchunks) load_chunk(kc + 1);
        f32x4 xv[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
            xv[mt] = *(const f32x4*)(As + (wave * 32 + mt * 16 + lr) * GEMM_LDS_STRIDE + lg * 4);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f32x4 wv = *(const f32x4*)(Ws + (nt * 16 + lr) * GEMM_LDS_STRIDE + lg * 4);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) acc[mt][nt] = mfma16(wv[s], xv[mt][s], acc[mt][nt]);
            }
        }
    }

    // Epilogue: lane holds out[m][n .. n+3].
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int m = m0 + wave * 32 + mt * 16 + lr;
        if (m >= M) continue;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n = n0 + nt * 16 + lg * 4;
            if (n >= N) continue;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = acc[mt][nt][j] + (n + j < N ? p.bias[n + j] : 0.0f);
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
            float* o = p.out + (size_t)m * p.ldo + n;
            if (EPI == EPI_GELU) {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = gelu(v[j]);
            } else if (EPI == EPI_RESID) {
                const float* r = p.res + (size_t)m * p.ldo + n;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (n + j < N) v[j] = r[j] + v[j];
            } else if (EPI == EPI_HAB) {
                const float* r = p.res + (size_t)m * p.ldo + n;
                const float* a = p.aux + (size_t)m * p.ldo + n;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (n + j < N) v[j] = (r[j] + v[j]) + (a[j] * p.gate[n + j]) * p.cscale;
            }
            if (n + 3 < N && ((p.ldo & 3) == 0)) {
                *(float4*)o = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (n + j < N) o[j] = v[j];
            }
        }
    }
}

#define GEMM_INST(NAME, NT, EPI, LN)                                                         \
    extern "C" __global__ __launch_bounds__(256) void NAME(GemmArgs p)                      \
    {                                                                                        \
        gemm_body<NT, EPI, LN>(p);                                                           \
    }

// NT = 9: 144-wide column blocks (HAT-S: N = 144, 288, 432 divide exactly).
GEMM_INST(hat_gemm_n9_store, 9, EPI_STORE, false)
GEMM_INST(hat_gemm_n9_gelu_ln, 9, EPI_GELU, true)
GEMM_INST(hat_gemm_n9_qkv, 9, EPI_QKV, false)
GEMM_INST(hat_gemm_n9_qkv_ln, 9, EPI_QKV, true)
GEMM_INST(hat_gemm_n9_resid, 9, EPI_RESID, false)
GEMM_INST(hat_gemm_n9_hab, 9, EPI_HAB, false)
// NT = 6: 96-wide column blocks (C = 180 models: 180, 360, 540 -> 2, 4, 6 blocks).
GEMM_INST(hat_gemm_n6_store, 6, EPI_STORE, false)
GEMM_INST(hat_gemm_n6_gelu_ln, 6, EPI_GELU, true)
GEMM_INST(hat_gemm_n6_qkv, 6, EPI_QKV, false)
GEMM_INST(hat_gemm_n6_qkv_ln, 6, EPI_QKV, true)
GEMM_INST(hat_gemm_n6_resid, 6, EPI_RESID, false)
GEMM_INST(hat_gemm_n6_hab, 6, EPI_HAB, false)
