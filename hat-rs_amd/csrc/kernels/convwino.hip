// 3x3 convolution (stride 1, zero padding 1, NHWC) by Winograd's minimal
// filtering F(2x2, 3x3) (Lavin & Gray, "Fast Algorithms for Convolutional
// Neural Networks", 2016), input channels in chunks of 16 and output channels
// in blocks of 16 NT (channels past CI read as zeros, past CO not stored):
//   - the 144 -> 144 trunk convs with the bias and the residual in the
//     epilogue: the reference's RHAG conv and conv_after_body,
//     lg_conv3x3_winograd (gpu.rs:605, 742) then lg_add (cuda.rs:227-248).
//     The RHAG conv's LayerNorm (lg_channel_layer_norm, cuda.rs:185-191)
//     follows as hat_layernorm: in this kernel it runs where no MFMA work
//     overlaps it (one block per CU) and costs more than the separate,
//     HBM-bound pass over rows still in the last-level cache (measured:
//     461 us fused against 375 + 52);
//   - the head's conv_before_upsample (144 -> 64, LeakyReLU) and upsample
//     convs (64 -> 256 into the PixelShuffle'd plane, two 128-channel column
//     blocks), gpu.rs:622-653;
//   - the C = 180 family's trunk convs (180 -> 180 + residual, two 96-channel
//     column blocks) and its unfolded CAB: conv1 180 -> 60 + GELU and conv2
//     60 -> 180 with per-tile column sums for the squeeze-excite gate
//     (lg_conv3x3 + lg_channel_mean's first stage, cuda.rs:171-183, 259-272).
//
// For each 2x2 output tile with the 4x4 input patch d (rows y-1 .. y+2):
//   Y = A^T [ U (.) V ] A,   U = G g G^T (per co, ci),   V = B^T d B (per ci)
// so each of the 16 transform points xi = 4i + j is an independent GEMM
// M[xi] (co x tile) = U[xi] (co x ci) . V[xi] (ci x tile): 16 * 144 * 144
// MACs per tile against 4 * 9 * 144 * 144 for the direct form (2.25x fewer).
//
// A block owns an 8 x 16 output tile (32 Winograd tiles, two 16-wide MFMA
// column tiles) and 16 NT output channels (the column-sum kernel walks several
// such tiles, one block a CU, fetching the next tile's first patch chunk under
// the current tile's epilogue). Wave w computes the two transform
// points xi = 2w, 2w + 1 (B^T row i = w / 2, columns j = 2 (w % 2) + {0, 1}),
// accumulating M[xi] (co 16 NT x tile 32) in 16 NT registers per lane (144
// for the trunk convs), on split-bf16 MFMA (v_mfma_f32_16x16x32_bf16, each
// fp32 operand as three bf16 parts and each product as the six terms of
// order <= 2, as accurate as FP32 MFMA; the split-bf16 attention explains the
// arithmetic). Input channels go in chunks of 32: the chunk's 10 x 18 halo
// patch is staged in LDS (global_load_lds, double-buffered, channel-quad-major);
// each lane forms V for its (tile, eight channels) from the patch, splits it
// and feeds it to the MFMAs as the B operand. U (pre-transformed and split on
// the host, 2.2 MB at 144 -> 144 with the channels padded to 160, L2-resident)
// streams from global memory as the A operand, two or three steps ahead of its
// MFMAs (a ring of three or four registers sets, whichever divides the 2 NT
// steps of a chunk; three ahead measured up to 2% faster than two at NT = 4).
//
// Epilogue, per 16-channel slice: the waves write their M slices to LDS, then
// each thread forms the 2x2 outputs of one (tile, channel) from the 16 points.
// A thread ends with 4 pixels x NT channels.
//
// Included after gemm.hip in the one translation unit.

#define WG_TH 8                            // output tile rows
#define WG_TW 16                           // output tile columns
#define WG_PH (WG_TH + 2)                  // 10 halo rows
#define WG_PW (WG_TW + 2)                  // 18 halo columns
#define WG_PPX (WG_PH * WG_PW)             // 180 halo pixels
#define WG_SLOTS 1536                      // float4 slots per patch buffer (1440 used)
#define WG_MS 20                           // LDS row stride of an M slice entry (16 used)

// NT: output channel tiles per block (column block cb), NTT: all of
// them (the U layout), NKC: 32-channel input chunks; CI, CO: the real channel
// counts (CO is also the row width of the residual epilogue's planes). HEAD
// -1 adds the bias and the residual; CEPI_STORE applies p.act (1 GELU, 2
// LeakyReLU 0.01); CEPI_SHUFFLE writes into the shuffled plane (channels
// pre-permuted as for the direct convs); CEPI_COLSUM stores and leaves the
// 8 x 16 tile's column sums, one partial row per tile.
template <int NT, int NTT, int NKC, int CI, int CO, int HEAD>
__device__ __forceinline__ void convwino_body(const ConvArgs& p)
{
    // Persistent over tiles only for the column-sum epilogue (CAB conv2 60 ->
    // 180: two input chunks, a six-slice epilogue and the sums), where fetching
    // the next tile under the epilogue measured 254.5 -> 244.8 us. For the
    // others the wait at the top of a tile (one memory counter, completing in
    // order: for the previous tile's stores as well as the next patch) and the
    // barrier cost more than the overlap gains (same box: 4-9% slower), and the
    // NT = 8 and 9 kernels spill 120-300 bytes more in the loop.
    constexpr bool PERSIST = HEAD == CEPI_COLSUM;
    static_assert(HEAD == -1 || HEAD == CEPI_STORE || HEAD == CEPI_SHUFFLE || HEAD == CEPI_COLSUM,
                  "residual, store, shuffle or column-sum epilogues");
    static_assert(NTT % NT == 0 && 16 * NTT >= CO && 16 * (NTT - 1) < CO, "the column blocks cover CO");
    static_assert(32 * NKC >= CI && 32 * (NKC - 1) < CI && CI % 4 == 0, "the 32-channel chunks cover CI");
    // PACK: the last chunk holds at most 16 real channels (CI = 144), so it is
    // packed as the K = 144 linears' last step (common.h half_operands, the
    // host's pack_wino): each lane forms V for four channels (quad lg), and
    // three MFMAs per step give the six products.
    constexpr bool PACK = CI % 32 != 0 && CI % 32 <= 16;
    __shared__ __attribute__((aligned(16))) float Pb0[WG_SLOTS * 4];
    __shared__ __attribute__((aligned(16))) float Pb1[WG_SLOTS * 4];
    __shared__ __attribute__((aligned(16))) float Ms0[16 * 32 * WG_MS];
    __shared__ __attribute__((aligned(16))) float Ms1[16 * 32 * WG_MS];
    __shared__ __attribute__((aligned(16))) float Cs[16 * NT];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int H = p.H, W = p.W;
    const int tiles_x = W / WG_TW;
    // Persistent over the launch's virtual blocks vb = blockIdx.x + i
    // gridDim.x, p.nblk of them (0: the grid's own, one a block): tile vb / NCB
    // (after a band's first tile tile0, 0 for the whole plane), column block
    // vb % NCB, the same for all of a block's tiles (the host makes gridDim.x
    // a multiple of NCB). A tile's column blocks are consecutive virtual
    // blocks, so they read its patch from L2 at about the same time.
    constexpr int NCB = NTT / NT;
    const int nvb = PERSIST && p.nblk > 0 ? p.nblk : (int)gridDim.x;
    int vb = (int)blockIdx.x;
    const int cb = vb % NCB;
    int tile, y0, x0;
    auto set_tile = [&](int v) {
        tile = p.tile0 + v / NCB;
        y0 = (tile / tiles_x) * WG_TH;
        x0 = (tile % tiles_x) * WG_TW;
    };
    set_tile(vb);

    for (int i = tid; i < 16 * NT; i += 512) Cs[i] = 16 * NT * cb + i < CO ? p.bias[16 * NT * cb + i] : 0.0f;

    // The patch of a 32-channel chunk is channel-quad-major: float4 slot
    // q * 180 + 18 hy + c holds channels 4q .. 4q+3 of halo pixel (hy, hx),
    // 1440 of WG_SLOTS used. With PSPLIT the even columns come first (c = hx
    // / 2) and then the odd ones (c = 9 + hx / 2), so that the 8 lanes that
    // LDS serves together (tiles tx = 0 .. 7 of a row, columns 2 tx + j) read
    // 8 consecutive slots, free of bank conflicts; without it c = hx and the
    // reads are 2-way conflicted. The 144-channel trunk conv (NT = 9, 144
    // accumulator registers) keeps c = hx: with the split columns the compiler
    // spills 32 registers there instead of 16, which costs more than the
    // conflicts. A lane's reads sit at one lane offset plus wave-uniform ones. The three slots this thread stages per chunk (the
    // third for waves 0..6 only): element offsets of the quad in chunk 0, or
    // -1 for slots outside the plane or past the 1440 used.
    constexpr bool PSPLIT = NT != 9;
    int soff[3], squad[3];
    auto set_offsets = [&](int ty0, int tx0) {  // for the tile at (ty0, tx0)
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int s = r * 512 + tid;
            const int q = s / WG_PPX, pix = s - q * WG_PPX;
            const int hy = pix / WG_PW, c = pix - hy * WG_PW, hx = !PSPLIT ? c : c < 9 ? 2 * c : 2 * c - 17;
            const int gy = ty0 - 1 + hy, gx = tx0 - 1 + hx;
            const bool ok = s < WG_PPX * 8 && gy >= 0 && gy < H && gx >= 0 && gx < W;
            soff[r] = ok ? (gy * W + gx) * p.cin_stride + q * 4 : -1;
            squad[r] = 4 * q;
        }
    };
    set_offsets(y0, x0);
    auto fetch = [&](int kc, auto bufc) {
        float* B = decltype(bufc)::value ? Pb1 : Pb0;
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            if (r == 2 && wave >= 7) break;  // wave-uniform: slots 1472.. are not used
            // quads past CI (the last chunk of CI = 60, 144, 180) read zeros
            const bool cin = CI % 32 == 0 || kc * 32 + squad[r] < CI;
            const float* src = soff[r] >= 0 && cin ? p.in + soff[r] + kc * 32 : hat_zero_row;
            __builtin_amdgcn_global_load_lds((const void*)src,
                                             (__attribute__((address_space(3))) void*)(B + (r * 512 + wave * 64) * 4),
                                             16, 0, 0);
        }
    };

    // U, split on the host and arranged [kc][xi][nt][part][lane][8] bf16: lane
    // (r, g) of step (e, nt) holds part `part` of U[2w + e][16 nt + r][32 kc +
    // 8 g .. +7], the MFMA A operand.
    const unsigned short* ubase = p.wu + ((size_t)(2 * wave) * NTT + NT * cb) * 3 * 512 + lane * 8;
    struct U3 {
        u32x4 v[3];
    };
    auto ldu = [&](int kc, int t) -> U3 {
        const int e = t / NT, nt = t - e * NT;
        const unsigned short* u = ubase + ((size_t)(kc * 16 + e) * NTT + nt) * 3 * 512;
        U3 r;
#pragma unroll
        for (int part = 0; part < 3; ++part) r.v[part] = *(const u32x4*)(u + part * 512);
        return r;
    };

    // The lane's B^T row / column pattern: R(col) = d[ra][col] + sr d[rb][col],
    // V[2w] = R(cA) - R(cB), V[2w+1] = R(cC) + sc R(cD).
    const int bi = wave >> 1, jp = wave & 1;
    const int ra = bi == 0 ? 0 : (bi == 2 ? 2 : 1);
    const int rb = bi == 0 ? 2 : (bi == 1 ? 2 : (bi == 2 ? 1 : 3));
    const float sr = bi == 1 ? 1.0f : -1.0f;
    const int cA = jp ? 2 : 0, cB = jp ? 1 : 2, cC = 1, cD = jp ? 3 : 2;
    const float sc = jp ? -1.0f : 1.0f;
    // LDS float offsets: the lane's tile origin (tile 16 nt2 + lr, quads 2 lg
    // and 2 lg + 1, 180 slots apart) and the wave's rows / columns
    int pbase[2];
#pragma unroll
    for (int nt2 = 0; nt2 < 2; ++nt2) {
        const int n = nt2 * 16 + lr, ty = n >> 3, tx = n & 7;
        pbase[nt2] = (2 * lg * WG_PPX + 2 * ty * WG_PW + (PSPLIT ? tx : 2 * tx)) * 4;
    }
    const int cols[4] = {cA, cB, cC, cD};
    int uoff[4][2];  // [column A..D][row a / b]
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        // column 2 tx + cols[c]'s slot, less the lane's part
        const int cs = PSPLIT ? (cols[c] & 1) * 9 + (cols[c] >> 1) : cols[c];
        uoff[c][0] = (ra * WG_PW + cs) * 4;
        uoff[c][1] = (rb * WG_PW + cs) * 4;
    }

    f32x4 acc[2][NT][2];

    // U loads RING - 1 steps ahead (2 NT steps a chunk, a multiple of RING, so
    // slot t % RING lines up across chunks)
    constexpr int RING = (2 * NT) % 3 == 0 ? 3 : 4;
    static_assert((2 * NT) % RING == 0 && 2 * NT >= RING, "the ring lines up across chunks");
    U3 ur[RING];
    fetch(0, CInt<0>{});
#pragma unroll
    for (int t = 0; t < RING - 1; ++t) ur[t] = ldu(0, t);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // Chunk kc from patch buffer Q. Transform point e's V (the lane's tile, 8
    // channels) is formed and split just before its NT steps t = e * NT + nt;
    // the U load of step t + 2 (the next chunk's first two at the end) is
    // issued ahead of step t.
    auto chunk = [&](int kc, auto bufc, auto lastc) {
        constexpr int Q = decltype(bufc)::value;
        constexpr bool LAST = decltype(lastc)::value;
        const float* B = Q ? Pb1 : Pb0;
        // the chunk after this one; after the last, chunk 0 of the block's next
        // tile (U is the same for every tile of the column block)
        const int kn = LAST ? 0 : kc + 1;
        constexpr bool HALF = PACK && LAST;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            u32x4 vb[2][3];
#pragma unroll
            for (int nt2 = 0; nt2 < 2; ++nt2) {
                float f[8];
#pragma unroll
                for (int hq = 0; hq < (HALF ? 1 : 2); ++hq) {
                    // HALF: quad lg (the lane's four channels), not 2 lg + hq
                    const float* P = B + pbase[nt2] + (HALF ? -lg : hq) * WG_PPX * 4;
                    const int c0 = e == 0 ? 0 : 2, c1 = c0 + 1;
                    const f32x4 r0 = *(const f32x4*)(P + uoff[c0][0]) + sr * *(const f32x4*)(P + uoff[c0][1]);
                    const f32x4 r1 = *(const f32x4*)(P + uoff[c1][0]) + sr * *(const f32x4*)(P + uoff[c1][1]);
                    const f32x4 v = e == 0 ? r0 - r1 : r0 + sc * r1;
#pragma unroll
                    for (int j = 0; j < 4; ++j) f[4 * hq + j] = v[j];
                }
                if (HALF) half_operands((f32x4){f[0], f[1], f[2], f[3]}, vb[nt2]);
                else split3_x8(f, vb[nt2]);
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int t = e * NT + nt;
                if (!LAST && t == 0) fetch(kc + 1, CInt<Q ^ 1>{});
#pragma unroll
                for (int nt2 = 0; nt2 < 2; ++nt2)
                    acc[e][nt][nt2] = HALF ? mfma16x3(ur[t % RING].v, vb[nt2], acc[e][nt][nt2])
                                           : mfma16x6(ur[t % RING].v, vb[nt2], acc[e][nt][nt2]);
                // step t + RING - 1's load into the slot step t - 1's MFMAs
                // have read
                {
                    constexpr int A = RING - 1;  // steps ahead
                    ur[(t + A) % RING] = t + A < 2 * NT ? ldu(kc, t + A) : ldu(kn, t + A - 2 * NT);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (LAST) {
            __builtin_amdgcn_s_waitcnt(0);
        } else {
            // The next chunk's patch copies landed: they were issued at step 0,
            // before this chunk's 6 NT U loads, and the memory counter
            // completes in order, so vmcnt(6 NT) covers them while the U loads
            // for the next chunk's first steps stay in flight under its V
            // transform.
            constexpr int VM = 6 * NT;
            static_assert(VM <= 63, "the 6-bit vmcnt field");
            __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
        }
        __syncthreads();
    };
#pragma unroll 1
    for (;;) {  // the block's tiles
        // an opaque copy of the U base each tile: otherwise the compiler keeps
        // every step's U address live across the tiles and spills
        if constexpr (PERSIST) asm volatile("" : "+v"(ubase));
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int nt2 = 0; nt2 < 2; ++nt2) acc[e][nt][nt2] = (f32x4){0.f, 0.f, 0.f, 0.f};
        // unrolled (at most six chunks): at a loop's back edge the compiler's
        // memory-counter waits merge to vmcnt(0), which would wait for the U
        // loads in flight as well
#pragma unroll
        for (int kc = 0; kc + 2 < NKC; kc += 2) {
            chunk(kc, CInt<0>{}, CInt<0>{});
            chunk(kc + 1, CInt<1>{}, CInt<0>{});
        }
        if constexpr (NKC % 2 == 1) {
            chunk(NKC - 1, CInt<0>{}, CInt<1>{});
        } else {
            chunk(NKC - 2, CInt<0>{}, CInt<0>{});
            chunk(NKC - 1, CInt<1>{}, CInt<1>{});
        }
        // The next tile's first patch chunk, in flight under this tile's epilogue:
        // the last chunk ended at a barrier, so no wave still reads the patch
        // buffers, and the epilogue uses Ms0 / Ms1 only.
        const int vn = vb + (int)gridDim.x;
        const bool more = PERSIST && vn < nvb;  // block-uniform
        if (more) {
            const int nt_tile = p.tile0 + vn / NCB;
            set_offsets((nt_tile / tiles_x) * WG_TH, (nt_tile % tiles_x) * WG_TW);
            fetch(0, CInt<0>{});
        }

        // ---- epilogue. Thread (tile = tid / 16, c = tid % 16): outputs of tile
        // (ty, tx) for channels 16 nt + c.
        const int et = tid >> 4, ec = tid & 15;
        // An M slice entry (a row of 16 floats) keeps its four float4s at slots
        // ws_slot(row, g), so that the waves' writes (8 lanes: rows r0 .. r0 + 7)
        // and the reads here (16 lanes a row, two rows at a time) meet no bank
        // conflicts; row x * 32 + et has (row >> 1) & 3 == (et >> 1) & 3.
        // (The NT = 9 trunk conv keeps plain rows of WG_MS floats, 2-way conflicted
        // reads: the swizzle's offset register makes the compiler spill more.)
        constexpr int MS = PSPLIT ? 16 : WG_MS;
        const int moff = PSPLIT ? 4 * ws_slot(et, ec >> 2) + (ec & 3) : ec;
        const int ety = et >> 3, etx = et & 7;
        const int py = y0 + 2 * ety, px = x0 + 2 * etx;
        // element offsets of the thread's four pixels in the residual epilogue's
        // planes (below 2^31 elements: checked at launch)
        const int pix0 = ((py * W) + px) * CO, prow = W * CO;
        const int ocb = 16 * NT * cb + ec;  // the thread's channel in slice 0
        constexpr bool PADCO = 16 * NTT != CO;  // channels past CO in the last column block
        float y[NT][4];
        auto out_slice = [&](int nt, auto bufc) {
            float* Ms = decltype(bufc)::value ? Ms1 : Ms0;
            // the slice's residual, loaded under the barrier and the transforms
            const bool live = PADCO ? ocb + 16 * nt < CO : true;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                y[nt][q] = HEAD < 0 ? p.res[live ? pix0 + (q >> 1) * prow + (q & 1) * CO + ocb + nt * 16 : 0] : 0.0f;
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int nt2 = 0; nt2 < 2; ++nt2)
                    *(f32x4*)(Ms + ((2 * wave + e) * 32 + nt2 * 16 + lr) * MS + 4 * (PSPLIT ? ws_slot(lr, lg) : lg)) =
                        acc[e][nt][nt2];
            __syncthreads();
            float m[16];
#pragma unroll
            for (int x = 0; x < 16; ++x) m[x] = Ms[(x * 32 + et) * MS + moff];
            float t0[4], t1[4];  // T[i][0], T[i][1] = M[i] A
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                t0[i] = m[4 * i] + m[4 * i + 1] + m[4 * i + 2];
                t1[i] = m[4 * i + 1] - m[4 * i + 2] - m[4 * i + 3];
            }
            const float bias = Cs[nt * 16 + ec];
            y[nt][0] += (t0[0] + t0[1] + t0[2]) + bias;
            y[nt][1] += (t1[0] + t1[1] + t1[2]) + bias;
            y[nt][2] += (t0[1] - t0[2] - t0[3]) + bias;
            y[nt][3] += (t1[1] - t1[2] - t1[3]) + bias;
        };
#pragma unroll
        for (int nt = 0; nt + 1 < NT; nt += 2) {
            out_slice(nt, CInt<0>{});
            out_slice(nt + 1, CInt<1>{});
        }
        if constexpr (NT % 2 == 1) out_slice(NT - 1, CInt<0>{});

        if constexpr (HEAD >= 0) {
            // Channel o = 16 NT cb + 16 nt + c of pixel (y, x): CEPI_STORE and
            // CEPI_COLSUM write it there (CEPI_STORE after p.act); CEPI_SHUFFLE
            // writes o = (i r + jj) Cf + c' to pixel (y r + i, x r + jj), channel c'
            // of the r-times larger plane.
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int o = ocb + 16 * nt;
                if (PADCO && o >= CO) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int yy = py + (q >> 1), xx = px + (q & 1);
                    float v = y[nt][q];
                    if (HEAD == CEPI_STORE || HEAD == CEPI_COLSUM) {
                        if (HEAD == CEPI_STORE && p.act == 2) v = v < 0.0f ? v * 0.01f : v;
                        if (HEAD == CEPI_STORE && p.act == 1) v = gelu(v);
                        p.out[(yy * W + xx) * p.co_stride + o] = v;
                    } else {
                        const int r = p.r, Cf = p.CO / (r * r);
                        const int sub = o / Cf, c = o - sub * Cf, i = sub / r, jj = sub - i * r;
                        p.out[((yy * r + i) * (W * r) + xx * r + jj) * p.co_stride + c] = v;
                    }
                }
            }
            if constexpr (HEAD == CEPI_COLSUM) {
                // Column sums of the tile's 128 pixels: the thread's four, the four
                // tiles of the wave with this channel (lanes ec + 16 k), then the
                // eight waves in order through LDS (Ms0, free after this barrier);
                // one partial row per 8 x 16 tile, [tile][co_stride].
                float cs[NT];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    float v = (y[nt][0] + y[nt][1]) + (y[nt][2] + y[nt][3]);
                    v += __shfl_xor(v, 16, 64);
                    v += __shfl_xor(v, 32, 64);
                    cs[nt] = v;
                }
                __syncthreads();
                if (lane < 16) {
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) Ms0[wave * 16 * NT + nt * 16 + ec] = cs[nt];
                }
                __syncthreads();
                if (tid < 16 * NT) {
                    const int o = 16 * NT * cb + tid;
                    float v = 0.0f;
#pragma unroll
                    for (int w = 0; w < 8; ++w) v += Ms0[w * 16 * NT + tid];
                    if (o < CO) p.partial[(size_t)tile * p.co_stride + o] = v;
                }
            }
        } else {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                if (PADCO && ocb + 16 * nt >= CO) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) p.out[pix0 + (q >> 1) * prow + (q & 1) * CO + ocb + nt * 16] = y[nt][q];
            }
        }
        if (!more) break;
        vb = vn;
        set_tile(vb);
        // this wave's copies of the next patch have landed; everyone's have, and
        // everyone is done with this tile's Ms
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }  // the block's tiles
}

extern "C" __global__ __launch_bounds__(512) void hat_convwino_resid(ConvArgs p)
{
    convwino_body<9, 9, 5, 144, 144, -1>(p);
}
// conv_before_upsample: 144 -> 64, LeakyReLU
extern "C" __global__ __launch_bounds__(512) void hat_convwino_n4_store(ConvArgs p)
{
    convwino_body<4, 4, 5, 144, 64, CEPI_STORE>(p);
}
// upsample convs: 64 -> 256 in two 128-channel column blocks, PixelShuffle(2)
extern "C" __global__ __launch_bounds__(512) void hat_convwino_n8_shuffle(ConvArgs p)
{
    convwino_body<8, 16, 2, 64, 256, CEPI_SHUFFLE>(p);
}
// The C = 180 family: trunk convs 180 -> 180 + residual (two 96-channel column
// blocks), conv_before_upsample 180 -> 64, CAB conv1 180 -> 60 (+ GELU) and
// conv2 60 -> 180 with column sums (two column blocks).
extern "C" __global__ __launch_bounds__(512) void hat_convwino_resid180(ConvArgs p)
{
    convwino_body<6, 12, 6, 180, 180, -1>(p);
}
extern "C" __global__ __launch_bounds__(512) void hat_convwino_n4_store180(ConvArgs p)
{
    convwino_body<4, 4, 6, 180, 64, CEPI_STORE>(p);
}
extern "C" __global__ __launch_bounds__(512) void hat_convwino_cab1_180(ConvArgs p)
{
    convwino_body<4, 4, 6, 180, 60, CEPI_STORE>(p);
}
extern "C" __global__ __launch_bounds__(512) void hat_convwino_cab2_180(ConvArgs p)
{
    convwino_body<6, 12, 2, 60, 180, CEPI_COLSUM>(p);
}
