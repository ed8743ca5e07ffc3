// The second half of a HAB in one kernel, C = 144 with the folded CAB
// (hat_arch.py HAB.forward; cpu.rs hab, 1090-1166; the reference's GPU path
// runs it as the attention projection, the CAB's conv2 / channel scale, three
// adds, norm2, the two MLP linears with GELU and the next block's norm1,
// src/gpu.rs:469-520):
//
//   x'  = x + ao . Wp^T + nb(t1) . W2g^T + bias2     (proj, gated conv2, shortcut)
//   out = x' + fc2(gelu(fc1(LN2(x'))))
//   xn  = LN_next(out)
//
// ao is the attention output, nb(t1) the 3x3 neighbourhood of the CAB's conv1
// output at the row's pixel (k = tap*6 + ci) and W2g / bias2 the gate-scaled
// conv2 weights and combined bias (hat_cab_gate). x' and LN2(x') never leave
// the registers: the projection's accumulators have the layout of the MLP's
// input (lane (r, g) holds columns 16 kc + 4g .. +3 of row r), so LN2 turns
// them into fc1's operand in place, and x' is the MLP's residual.
//
// hat_ocab_tail is the same without the conv2 chunk and the next norm (the
// OCAB: x' = x + ao . Wp^T + bp, out = x' + MLP(norm2(x'))).
//
// A block of 8 waves walks 128-row tiles (wave w owns rows 16w .. 16w+15). Per
// tile eight weight chunks pass through the double-buffered LDS of the fused
// MLP (global_load_lds_dwordx4, swizzled unpadded rows, one barrier per
// chunk): the projection in two, k 0..79 (144 x 20 float4) and k 80..143
// (144 x 16 float4), then the six 48-unit hidden chunks. The gated conv2's
// weights (144 x 16 float4: 56 K, 8 zero) stay in LDS for the whole launch
// and run in the second projection chunk. The attention rows of the next
// tile are loaded under the last chunk's fc2, the residual rows and the t1
// neighbourhood at the start of each tile, ahead of the chunks that use them.
//
// Included after gemm.hip and mlp.hip in the one translation unit.

// CAB: the HAB's tail (the gated conv2 chunk; EPI_RESID_LN writes the next
// norm1). Without it, the OCAB's (hat_arch.py OCAB.forward, cpu.rs ocab
// 983-1055): x' = x + a . Wp^T + bp, out = x' + MLP(norm2(x')), EPI_RESID.
template <bool CAB, int EPI>
__device__ __forceinline__ void hab_tail_body(const HabTailArgs& p)
{
    constexpr int C = HT_C, NT = C / 16, NH = 2 * C, NCH = NH / MLP_HC;
    constexpr int HT_NPC = 2;                   // projection chunks per tile
    constexpr int HT_NCT = HT_NPC + NCH;        // chunks per tile (8: every tile starts in buffer 0)
    constexpr int R1 = C / 4, R2 = MLP_HC / 4;  // MLP slices: fc1 [48][36], fc2 [144][12] float4
    constexpr int W1F4 = MLP_HC * R1, F4 = W1F4 + C * R2;
    // projection chunks [144][20] (k 0..79) and [144][16] (k 80..143), the
    // resident conv2 slice [144][16] float4
    constexpr int RA = 20, RB = 16, RC = 16, KA = 4 * RA;
    constexpr int AF4 = C * RA, BF4 = C * RB, CF4 = C * RC;
    constexpr int BUF = F4 * 4;
    constexpr int PER = (F4 + MLP_THREADS - 1) / MLP_THREADS;
    static_assert(HT_NCT % 2 == 0, "an even chunk count keeps the buffer parity static");
    static_assert(KA + 4 * RB == C, "the two projection chunks cover K");
    static_assert(AF4 <= F4 && BF4 <= F4 && AF4 % 64 == 0 && BF4 % 64 == 0 && CF4 % 64 == 0 && F4 % 64 == 0,
                  "chunk sizes");
    static_assert(CAB_K2 == 56 && CAB_C == C, "the conv2 slice holds 56 K");
    // The two chunk buffers are separate objects, and every access below names
    // one of them at compile time (the chunk parity is static): the compiler
    // then knows that reading one buffer does not depend on the DMA still
    // filling the other, and does not wait for that DMA before the read.
    __shared__ __attribute__((aligned(16))) float Wb0[BUF];
    __shared__ __attribute__((aligned(16))) float Wb1[BUF];
    __shared__ __attribute__((aligned(16))) float W2s[CAB ? CF4 * 4 : 4];
    // b1 [288], b2, next-norm w, b [144 each], bias2, norm2 w, b [144 each]
    __shared__ __attribute__((aligned(16))) float Cs[NH + 6 * C];
    float* const b1s = Cs;
    float* const b2s = Cs + NH;
    float* const bias2s = Cs + NH + 3 * C;
    float* const n2ws = Cs + NH + 4 * C;
    float* const n2bs = Cs + NH + 5 * C;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int M = p.M;
    const int ntiles = (M + MLP_ROWS - 1) / MLP_ROWS;
    int tile = blockIdx.x;
    if (tile >= ntiles) return;  // whole block: no barrier has been passed yet

    for (int i = tid; i < NH + 6 * C; i += MLP_THREADS) {
        float v;
        if (i < NH) v = p.b1[i];
        else if (i < NH + C) v = p.b2[i - NH];
        else if (i < NH + 2 * C) v = EPI == EPI_RESID_LN ? p.nw[i - NH - C] : 0.0f;
        else if (i < NH + 3 * C) v = EPI == EPI_RESID_LN ? p.nb[i - NH - 2 * C] : 0.0f;
        else if (i < NH + 4 * C) v = p.bias2[i - NH - 3 * C];
        else if (i < NH + 5 * C) v = p.n2w[i - NH - 4 * C];
        else v = p.n2b[i - NH - 5 * C];
        Cs[i] = v;
    }

    // The MLP chunks' global offsets (relative to the chunk bases), as in mlp_body.
    unsigned goff[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int idx = tid + i * MLP_THREADS;
        if (idx < W1F4) {
            const int r = idx / R1, c4 = (idx - r * R1) ^ mlp_swz<R1>(r);
            goff[i] = r * p.ldw1 + c4 * 4;
        } else {
            const int j = idx - W1F4;
            const int r = j / R2, c4 = (j - r * R2) ^ mlp_swz<R2>(r);
            goff[i] = r * p.ldw2 + c4 * 4;
        }
    }
    // Chunk cj of a tile into LDS buffer bufc (a CInt: 0 or 1): cj = 0, 1 the
    // projection's k 0..79 and 80..143, else hidden chunk cj - HT_NPC.
    auto fetch = [&](int cj, auto bufc) {
        float* B = decltype(bufc)::value ? Wb1 : Wb0;
        const int nf4 = cj == 0 ? AF4 : (cj == 1 ? BF4 : F4);
        const int h0 = (cj - HT_NPC) * MLP_HC;
        const float* w1c = p.w1 + (size_t)(h0 > 0 ? h0 : 0) * p.ldw1;
        const float* w2c = p.w2 + (h0 > 0 ? h0 : 0);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int base = i * MLP_THREADS + wave * 64;  // wave-uniform
            if (base >= nf4) break;
            const int idx = base + lane;
            const float* src;
            // the projection chunks' offsets are computed here, a few VALU ops
            // per slot, from an index the compiler cannot see through:
            // otherwise it hoists every (chunk, slot) address out of the tile
            // loop, 64 bits each, and spills them
            int id = idx;
            asm volatile("" : "+v"(id));
            if (cj == 0) {
                const int r = id / RA, c4 = (id - r * RA) ^ mlp_swz<RA>(r);
                src = p.wp + r * C + c4 * 4;
            } else if (cj == 1) {
                const int r = id / RB, c4 = (id - r * RB) ^ mlp_swz<RB>(r);
                src = p.wp + r * C + KA + c4 * 4;
            } else {
                src = (base < W1F4 ? w1c : w2c) + goff[i];
            }
            __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(B + base * 4),
                                             16, 0, 0);
        }
    };

    // Registers: xa = the attention rows (projection phase), then LN2(x') (MLP
    // phase); xr = the residual rows x, then x'.
    f32x4 xa[NT], xr[NT];
    auto load_rows = [&](f32x4 (&dst)[NT], const float* src, int t) {
        const int m = t * MLP_ROWS + wave * 16 + lr;
        const float* row = m < M ? src + (size_t)m * C + lg * 4 : hat_zero_row;  // + kc*16 stays in it
#pragma unroll
        for (int kc = 0; kc < NT; ++kc) {
            dst[kc] = *(const f32x4*)(row + kc * 16);
        }
    };

    GemmArgs g{};
    g.out = p.out;
    g.xn = p.xn;
    g.M = M;
    g.N = C;
    g.ldo = C;
    g.eps = p.eps;
    const EpiConsts kc_out{b2s, Cs + NH + C, Cs + NH + 2 * C};

    // Swizzled operand columns (rows nt*16 + lr: (row >> 2) & 3 == (lr >> 2) & 3,
    // row & 15 == lr).
    const int sg = lg ^ mlp_swz<R1>(lr), sg2 = lg ^ mlp_swz<R2>(lr), sga = lg ^ mlp_swz<RA>(lr);
    fetch(0, CInt<0>{});
    if (CAB) {
        // the gated conv2 slice, once per launch: k 56..63 of a row are zero
#pragma unroll
        for (int i = 0; i < (CF4 + MLP_THREADS - 1) / MLP_THREADS; ++i) {
            const int base = i * MLP_THREADS + wave * 64;  // wave-uniform
            if (base >= CF4) break;
            const int idx = base + lane;
            const int r = idx / RC, c4 = (idx - r * RC) ^ mlp_swz<RC>(r);
            const float* src = c4 < CAB_K2 / 4 ? p.w2g + r * CAB_K2 + c4 * 4 : hat_zero_row;
            __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(W2s + base * 4),
                                             16, 0, 0);
        }
    }
    load_rows(xa, p.a, tile);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // One tile: chunk cj in buffer cj & 1 (the chunk count per tile is even).
    for (; tile < ntiles; tile += gridDim.x) {
        const bool last_tile = tile + (int)gridDim.x >= ntiles;
        const int mbase = tile * MLP_ROWS + wave * 16;
        // The residual rows and (CAB) the t1 neighbourhood, loaded while
        // projection chunk 0 computes (first used after the projection / by
        // the conv2 MFMAs in chunk 1).
        f32x4 xg[CAB_K2 / 16];
        float2 xh;
        auto load_tail_inputs = [&]() {
            load_rows(xr, p.res, tile);
            if (!CAB) return;
            const int m = mbase + lr;
            const bool alive = m < M;
            const int y = m / p.W, x = m - y * p.W;
            // taps outside the plane read zeros
            auto pair = [&](int tap, int ci) -> float2 {
                const int yy = y + tap / 3 - 1, xx = x + tap % 3 - 1;
                const bool ok = alive && tap < 9 && yy >= 0 && yy < p.H && xx >= 0 && xx < p.W;
                return *(const float2*)(ok ? p.t1 + ((size_t)yy * p.W + xx) * CAB_CS + ci : hat_zero_row);
            };
#pragma unroll
            for (int kc2 = 0; kc2 < CAB_K2 / 16; ++kc2) {
                const int k0 = kc2 * 16 + lg * 4, ta = k0 / CAB_CC, ca = k0 - ta * CAB_CC;
                const float2 lo = pair(ta, ca);
                const bool same = ca + 2 < CAB_CC;
                const float2 hi = pair(same ? ta : ta + 1, same ? ca + 2 : 0);
                xg[kc2] = (f32x4){lo.x, lo.y, hi.x, hi.y};
            }
            xh = pair(lg < 3 ? 8 : 9, 2 * lg);
        };

        // ---- projection (+ gated conv2), accumulators starting from bias2
        f32x4 acc[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt] = *(const f32x4*)(bias2s + nt * 16 + lg * 4);
        // chunk 0 (buffer 0): k 0..79, five 16-k steps
        fetch(1, CInt<1>{});
        load_tail_inputs();
#pragma unroll
        for (int k3 = 0; k3 < KA / 16; ++k3) {
            // A operand: the attention rows' 16-k chunk k3; each step's weight
            // reads stay next to their MFMAs
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f32x4 wv = *(const f32x4*)(Wb0 + (nt * 16 + lr) * (4 * RA) + (k3 * 4 + sga) * 4);
#pragma unroll
                for (int s = 0; s < 4; ++s) acc[nt] = mfma16(wv[s], xa[k3][s], acc[nt]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // chunk 1 (buffer 1): k 80..143, four 16-k steps, then the gated conv2
        // from its resident slice
        fetch(HT_NPC, CInt<0>{});
#pragma unroll
        for (int k3 = 0; k3 < RB / 4; ++k3) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int pc = (k3 * 4 + lg) ^ lr;  // 4-bit swizzle of the 16-float4 rows
                const f32x4 wv = *(const f32x4*)(Wb1 + (nt * 16 + lr) * (4 * RB) + pc * 4);
#pragma unroll
                for (int s = 0; s < 4; ++s) acc[nt] = mfma16(wv[s], xa[KA / 16 + k3][s], acc[nt]);
            }
        }
        if (CAB) {
#pragma unroll
            for (int k3 = 0; k3 < 3; ++k3) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const int pc = (k3 * 4 + lg) ^ lr;
                    const f32x4 wv = *(const f32x4*)(W2s + (nt * 16 + lr) * (4 * RC) + pc * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s) acc[nt] = mfma16(wv[s], xg[k3][s], acc[nt]);
                }
            }
            // the 8-k tail: lane group g's k = 48 + 2g + s, float4 12 + g/2
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int pc = (12 + (lg >> 1)) ^ lr;
                const float2 wv = *(const float2*)(W2s + (nt * 16 + lr) * (4 * RC) + pc * 4 + (lg & 1) * 2);
                acc[nt] = mfma16(wv.x, xh.x, acc[nt]);
                acc[nt] = mfma16(wv.y, xh.y, acc[nt]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();

        // ---- x' = x + acc (rows past M are zero); xa = LN2(x') (two-pass, biased
        // variance, cpu.rs:563-581), the four lanes of a row reducing with shuffles.
        float s = 0.0f;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            xr[nt] = xr[nt] + acc[nt];
#pragma unroll
            for (int j = 0; j < 4; ++j) s += xr[nt][j];
        }
        s += __shfl_xor(s, 16, 64);
        s += __shfl_xor(s, 32, 64);
        const float mean = s / (float)C;
        float q = 0.0f;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float d = xr[nt][j] - mean;
                q += d * d;
            }
        q += __shfl_xor(q, 16, 64);
        q += __shfl_xor(q, 32, 64);
        const float rstd = 1.0f / sqrtf(q / (float)C + p.eps);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f32x4 w4 = *(const f32x4*)(n2ws + nt * 16 + lg * 4);
            const f32x4 b4 = *(const f32x4*)(n2bs + nt * 16 + lg * 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) xa[nt][j] = (xr[nt][j] - mean) * rstd * w4[j] + b4[j];
        }

        // ---- the MLP (mlp_body's chunk loop), residual x'
        f32x4 acc2[1][NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) acc2[0][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
        // hidden chunk c (cj = HT_NPC + c) from buffer bufc, fetching the next
        // chunk (or the next tile's chunk 0) into the other one
        auto mlp_chunk = [&](int c, auto bufc) {
            constexpr int Q = decltype(bufc)::value;
            const float* B = Q ? Wb1 : Wb0;
            const int cj = HT_NPC + c;
            const bool more = c + 1 < NCH || !last_tile;  // block-uniform
            if (more) fetch(c + 1 < NCH ? cj + 1 : 0, CInt<Q ^ 1>{});
            f32x4 h[MLP_HC / 16];
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt) h[nt] = *(const f32x4*)(b1s + c * MLP_HC + nt * 16 + lg * 4);
            // fc1, per 16-k step: the three weight reads, then their 12 MFMAs
#pragma unroll
            for (int kc = 0; kc < NT; ++kc) {
                __builtin_amdgcn_sched_barrier(0);
                f32x4 wv[MLP_HC / 16];
#pragma unroll
                for (int nt = 0; nt < MLP_HC / 16; ++nt)
                    wv[nt] = *(const f32x4*)(B + (nt * 16 + lr) * C + (kc * 4 + sg) * 4);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int nt = 0; nt < MLP_HC / 16; ++nt) h[nt] = mfma16(wv[nt][s], xa[kc][s], h[nt]);
            }
            // the MLP input is dead after the last chunk's fc1: the next tile's
            // attention rows load under this chunk's fc2 and the epilogue
            if (c == NCH - 1 && !last_tile) load_rows(xa, p.a, tile + gridDim.x);
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt)
#pragma unroll
                for (int j = 0; j < 4; ++j) h[nt][j] = gelu(h[nt][j]);
            // fc2, per 16-unit step of the hidden chunk and three output
            // column tiles: the three weight reads, then their 12 MFMAs (the
            // reads in flight together, not one read's latency per four MFMAs;
            // the scheduler is free within a step)
#pragma unroll
            for (int nt = 0; nt < MLP_HC / 16; ++nt)
#pragma unroll
                for (int g3 = 0; g3 < NT; g3 += 3) {
                    if (g3 == 0) __builtin_amdgcn_sched_barrier(0);
                    f32x4 wv[3];
#pragma unroll
                    for (int j = 0; j < 3; ++j)
                        wv[j] = *(const f32x4*)(B + W1F4 * 4 + ((g3 + j) * 16 + lr) * MLP_HC + nt * 16 + sg2 * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int j = 0; j < 3; ++j) acc2[0][g3 + j] = mfma16(wv[j][s], h[nt][s], acc2[0][g3 + j]);
                }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        };
        static_assert(NCH % 2 == 0, "hidden chunks go in pairs, one per buffer");
        static_assert(HT_NPC % 2 == 0, "hidden chunk c sits in buffer c & 1");
#pragma unroll 1
        for (int c = 0; c < NCH; c += 2) {
            mlp_chunk(c, CInt<0>{});
            mlp_chunk(c + 1, CInt<1>{});
        }
        // the residual x' straight from xr (one row tile: pres[0][nt] = xr[nt])
        gemm_epilogue<1, NT, EPI>(g, kc_out, acc2, mbase, 0, lr, lg, nullptr,
                                           (const f32x4(*)[NT])xr);
    }
}

extern "C" __global__ __launch_bounds__(MLP_THREADS) void hat_hab_tail(HabTailArgs p)
{
    hab_tail_body<true, EPI_RESID_LN>(p);
}
extern "C" __global__ __launch_bounds__(MLP_THREADS) void hat_ocab_tail(HabTailArgs p)
{
    hab_tail_body<false, EPI_RESID>(p);
}
