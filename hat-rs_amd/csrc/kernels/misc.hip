// Bandwidth kernels: LayerNorm, input preparation, squeeze-excite gate.
#include "common.h"

using namespace hatk;

// The device memory of hat_backend_forward_noalloc: the per-plan buffers of a
// forward carved from one array of fixed size, for callers that cannot
// allocate. The host resolves its address with hipModuleGetGlobal when the
// module loads; no kernel names it, they receive pointers into it.
__device__ __align__(256) unsigned char hat_scratch[SCRATCH_BYTES];

// LayerNorm over C channels of each row (lg_channel_layer_norm, cuda.rs:185-191;
// cpu.rs:563-581): two-pass mean then biased variance, y = (x - mean) * rstd *
// w + b; y may alias x. For C % 4 == 0, C <= 192 (the models' 144 and 180): a
// row per 16 lanes, four rows per wave, each lane holding up to three float4 of
// its row, the sums reduced within the 16 lanes. y goes out with non-temporal
// stores (a streaming pass) when a wave's four rows are whole 128-byte lines
// (C % 8 == 0, C = 144); otherwise (C = 180: 2880 bytes, 22.5 lines) lines
// split between waves are written partially, which non-temporal stores turn
// into a loss (measured at 262144 rows: 124 us cold / 82 us warm against 72 /
// 66 us with ordinary stores). x comes in with ordinary loads: in the forward it
// was written by the kernel just before, and the part of it still held in
// MI355X's 256 MB last-level cache (MALL) is read from there (measured in the
// HAT-S 512 forward: 51 us against 56 us with non-temporal loads, which are
// faster only on data that is cold). Otherwise one wave per row.
// The 16-lanes-per-row form; NTS: non-temporal stores.
template <bool NTS>
__device__ __forceinline__ void ln_rows16(const LnArgs& p, int lane, int C)
{
    const int g = lane & 15;
    const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
    if (row >= p.rows) return;  // whole 16-lane groups leave together
    const int n4 = C >> 2;
    const f32x4* x = (const f32x4*)(p.x + (size_t)row * C);
    f32x4 v[3];
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        const int k = g + 16 * t;
        v[t] = k < n4 ? x[k] : (f32x4){0.f, 0.f, 0.f, 0.f};
        s += (v[t].x + v[t].y) + (v[t].z + v[t].w);
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    const float mean = s / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        if (g + 16 * t < n4) {
            const float a = v[t].x - mean, b = v[t].y - mean, c = v[t].z - mean, d = v[t].w - mean;
            q += (a * a + b * b) + (c * c + d * d);
        }
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
    const float rstd = 1.0f / sqrtf(q / (float)C + p.eps);
    f32x4* y = (f32x4*)(p.y + (size_t)row * C);
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        const int k = g + 16 * t;
        if (k < n4) {
            const f32x4 w = ((const f32x4*)p.w)[k], b = ((const f32x4*)p.b)[k];
            const f32x4 o = {(v[t].x - mean) * rstd * w.x + b.x, (v[t].y - mean) * rstd * w.y + b.y,
                             (v[t].z - mean) * rstd * w.z + b.z, (v[t].w - mean) * rstd * w.w + b.w};
            if (NTS)
                __builtin_nontemporal_store(o, y + k);
            else
                y[k] = o;
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void hat_layernorm(LnArgs p)
{
    const int lane = threadIdx.x & 63;
    const int C = p.C;
    if ((C & 3) == 0 && C <= 192) {
        if ((C & 7) == 0)
            ln_rows16<true>(p, lane, C);
        else
            ln_rows16<false>(p, lane, C);
        return;
    }
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const float* x = p.x + (size_t)row * C;
    float* y = p.y + (size_t)row * C;
    float v[8];
    int n = 0;
    float s = 0.0f;
    for (int k = lane; k < C; k += 64) {
        v[n] = x[k];
        s += v[n];
        ++n;
    }
    const float mean = wave_sum(s) / (float)C;
    float q = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float d = v[i] - mean;
        q += d * d;
    }
    const float var = wave_sum(q) / (float)C;
    const float rstd = 1.0f / sqrtf(var + p.eps);
    n = 0;
    for (int k = lane; k < C; k += 64, ++n) y[k] = (v[n] - mean) * rstd * p.w[k] + p.b[k];
}

// Pre::adjust (backend.rs:71-89): edge-replicated padding to the window grid and
// (x - mean) * img_range, written NHWC with a padded channel stride.
extern "C" __global__ __launch_bounds__(256) void hat_pre(PreArgs p)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= p.hp * p.wp) return;
    const int y = i / p.wp, x = i - (i / p.wp) * p.wp;
    const int sy = y < p.h - 1 ? y : p.h - 1;
    const int sx = x < p.w - 1 ? x : p.w - 1;
    const size_t hw = (size_t)p.h * p.w;
    const size_t src = (size_t)sy * p.w + sx;
    float* o = p.out + (size_t)i * p.cstride;
    o[0] = (p.in[src] - p.m0) * p.range;
    o[1] = (p.in[hw + src] - p.m1) * p.range;
    o[2] = (p.in[2 * hw + src] - p.m2) * p.range;
    for (int c = 3; c < p.cstride; ++c) o[c] = 0.0f;
}

// A plain copy of n float4 (the HBM reference point the traffic counters of the
// other kernels are scaled by; also the library's device-to-device copy). A
// block copies a contiguous run of 1024 float4, four per thread, all four loads
// issued before the stores (on MI355X this shape measured 5.7 TB/s over 1 GiB,
// a grid-stride loop 4.7). Grid: ceil(n / 1024) blocks.
extern "C" __global__ __launch_bounds__(256) void hat_copy(CopyArgs p)
{
    const f32x4* src = (const f32x4*)p.src;
    f32x4* dst = (f32x4*)p.dst;
    const long base = (long)blockIdx.x * 1024 + threadIdx.x;
    f32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (base + u * 256 < p.n4) v[u] = src[base + u * 256];
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (base + u * 256 < p.n4) dst[base + u * 256] = v[u];
}

// First stage of the channel-attention pool (lg_channel_mean, cuda.rs:259-272):
// the per-tile column sums of the second CAB conv, summed over row blocks in
// a fixed order (deterministic). One block per row block, one thread per column.
extern "C" __global__ __launch_bounds__(256) void hat_colsum_reduce(ReduceArgs p)
{
    const int r0 = blockIdx.x * p.rows_per;
    const int r1 = min(r0 + p.rows_per, p.nrows);
    for (int c = threadIdx.x; c < p.C; c += 256) {
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        int r = r0;
        for (; r + 3 < r1; r += 4) {
            a0 += p.in[(size_t)r * p.stride + c];
            a1 += p.in[(size_t)(r + 1) * p.stride + c];
            a2 += p.in[(size_t)(r + 2) * p.stride + c];
            a3 += p.in[(size_t)(r + 3) * p.stride + c];
        }
        for (; r < r1; ++r) a0 += p.in[(size_t)r * p.stride + c];
        p.out[(size_t)blockIdx.x * p.C + c] = (a0 + a1) + (a2 + a3);
    }
}

// The channel attention's gate (CAB, hat_arch.py:40-55; cpu.rs:940-955):
// mean over the plane from the column sums of the second CAB conv, 1x1 squeeze
// + ReLU, 1x1 excite + sigmoid. One block; partial sums are added in block
// order.
extern "C" __global__ __launch_bounds__(256) void hat_se_gate(SeArgs p)
{
    __shared__ float s_mean[512];
    __shared__ float s_sq[64];
    const int tid = threadIdx.x;
    for (int c = tid; c < p.C; c += 256) {
        float acc = 0.0f;
        for (int b = 0; b < p.nblk; ++b) acc += p.partial[(size_t)b * p.co_stride + c];
        s_mean[c] = acc / p.count;
    }
    __syncthreads();
    for (int j = tid; j < p.sq; j += 256) {
        float acc = p.b1[j];
        for (int c = 0; c < p.C; ++c) acc += s_mean[c] * p.w1[(size_t)j * p.C + c];
        s_sq[j] = acc < 0.0f ? 0.0f : acc;
    }
    __syncthreads();
    for (int c = tid; c < p.C; c += 256) {
        float acc = p.b2[c];
        for (int j = 0; j < p.sq; ++j) acc += s_sq[j] * p.w2[(size_t)c * p.sq + j];
        p.gate[c] = 1.0f / (1.0f + __expf(-acc));
    }
}
