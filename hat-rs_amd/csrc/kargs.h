// Kernel argument blocks shared by the host runtime (g++) and the gfx950
// kernels (hipcc). Every kernel takes exactly one of these structs by value,
// so the host packs the kernarg segment by copying the struct: the layout is
// plain C (pointers 8 bytes, int/float 4 bytes) and identical on both sides.
#pragma once
#include <stdint.h>

namespace hatk {

// The fixed device array behind hat_backend_forward_noalloc (hat_scratch in
// misc.hip): 256 MiB, enough for the per-plan buffers of a HAT-S or HAT x4
// forward up to 128 x 128 input pixels. Every process that loads the library
// holds it on the device until it exits.
constexpr unsigned long long SCRATCH_BYTES = 256ull << 20;

// Activation layout everywhere on the device: token-major NHWC, [pixel][channel],
// pixels in image row-major order over the padded plane (hp x wp).

// out[m][n] = epilogue( A[m][:] . W[n][:] + bias[n] )
enum GemmEpi : int {
    EPI_STORE = 0,       // out[m][n] = v
    EPI_GELU = 1,        // out[m][n] = gelu(v)
    EPI_QKV = 2,         // head-major scatter: out[which][head][m][dim]
    EPI_RESID = 3,       // out[m][n] = res[m][n] + v
    EPI_HAB = 4,         // out[m][n] = (res[m][n] + v) + (aux[m][n] * gate[n]) * cscale
    EPI_RESID_LN = 5,    // EPI_RESID, and xn[m][:] = LayerNorm(out[m][:]) (full rows)
    EPI_HAB_LN = 6,      // EPI_HAB, and xn[m][:] = LayerNorm(out[m][:]) (full rows)
    EPI_STORE_LN = 7,    // EPI_STORE, and xn[m][:] = LayerNorm(out[m][:]) (full rows)
};

// Weight-stationary K = 144 GEMM launch geometry per epilogue: ws_waves waves
// per block, each owning ws_mt 16-row MFMA tiles of a ws_rows-row tile. One
// 16-row tile per wave keeps the plain epilogues at 4 waves per SIMD, so one
// wave's stores overlap the others' MFMAs; the LayerNorm epilogues need the
// registers of 2 waves per SIMD.
constexpr int ws_mt(int /*epi*/) { return 1; }
constexpr int ws_waves(int epi) { return epi == EPI_RESID_LN || epi == EPI_HAB_LN ? 8 : 16; }
constexpr int ws_rows(int epi) { return ws_waves(epi) * 16 * ws_mt(epi); }

// Waves per block of the wide-tile 3x3 conv instances (convw.hip): 8 own two
// 16-pixel tile rows each (2 waves per SIMD), 16 own one (4 per SIMD, where
// the registers allow it; measured faster for these three).
#define CONVW_WAVES_N9_STORE_LN 16
#define CONVW_WAVES_N9_RESID_LN 8
#define CONVW_WAVES_N9_RESID 8
#define CONVW_WAVES_N6_RESID 8
#define CONVW_WAVES_N6_COLSUM 8
#define CONVW_WAVES_N4_STORE 16
#define CONVW_WAVES_N8_SHUFFLE 16

struct GemmArgs {
    const float* a;      // [M][lda]
    const float* w;      // [N][Kp] row-major, K contiguous, zero-padded to Kp
    const float* bias;   // [N]
    float* out;
    const float* res;    // residual input (EPI_RESID*, EPI_HAB*)
    const float* aux;    // EPI_HAB*: conv branch [M][N]
    const float* gate;   // EPI_HAB*: channel gate [N]
    float* xn;           // EPI_*_LN: LayerNorm of the output rows [M][ldo]
    const float* nw;     // EPI_*_LN: LayerNorm weight [N]
    const float* nb;     // EPI_*_LN: LayerNorm bias [N]
    int M, N, K;         // logical sizes
    int Kp;              // K rounded up to 16 (W rows are Kp long)
    int lda, ldo;        // row strides of A and out (floats)
    int heads, hdim;     // EPI_QKV geometry (N = 3 * heads * hdim)
    float cscale;        // EPI_HAB* conv scale
    float eps;           // LayerNorm eps
    // hat_gemmws_cab_ln only: the CAB's second conv as an extra K segment,
    // A = 3x3 neighbourhood of t1 on the H x W plane, W = w2g [144][CAB_K2].
    const float* t1;     // [H*W][CAB_CS]
    const float* w2g;    // [N][CAB_K2]
    int H, W;
};

// CAB of the compress-to-6 family (HAT-S: 144 -> 6 -> 144), restated by the
// linearity of its second conv: conv2 becomes a K segment of the attention
// projection GEMM and its pixel mean comes from per-tile sums of conv1's output.
#define CAB_C 144
#define CAB_CC 6             // compressed channels
#define CAB_CS 8             // t1 channel stride (channels 6, 7 are zero)
#define CAB_K2 56            // 9 taps x 6 channels (k = tap*6 + ci), 2 zero: 3 x 16 + 8
// conv1's weights split for hat_cab_conv1*: per 16-channel step ks (9), row
// tile nt (2 x 32 rows, row tap*6 + co, rows 54.. zero) and part (3), the
// 32x32x16 A operand of each lane (row l % 32, channels 16 ks + 8 (l / 32) .. +7)
#define CX_WPACK (9 * 2 * 3 * 64 * 8)
#define CAB_NSUM 5           // per-tile sums: whole tile, row 0, row H-1, col 0, col W-1

struct CabConvArgs {
    const float* xn;     // [H*W][144]
    const unsigned short* w;  // [9][2][3][64][8] bf16: step ks, row tile nt, part, lane (CX_WPACK)
    const float* bias;   // [6]
    float* t1;           // [H*W][8]: gelu(conv1(xn))
    float* partial;      // [CAB_NSUM * 8][tiles] (value-major)
    int H, W;            // multiples of 16
};

struct CabGateArgs {
    const float* partial;  // [CAB_NSUM * 8][tiles] (value-major)
    const float* t1;       // corner pixels
    int tiles, H, W;
    const float* w2;     // conv2 weight [144][6][3][3]
    const float* b2;     // [144]
    const float* wa;     // channel attention squeeze [sq][144]
    const float* ba;     // [sq]
    const float* wb;     // excite [144][sq]
    const float* bb;     // [144]
    const float* bproj;  // attention projection bias [144]
    float* w2g;          // out: cscale * gate[c] * conv2 weight, [144][CAB_K2] (k = tap*6 + ci)
    float* bias2;        // out: bproj + cscale * gate * b2, [144]
    float* gate;         // out: the gate itself [144]
    float cscale;
    int sq;
    unsigned short* w2gx;  // out (if set): w2g as 2 weight chunks [3][144][32] (swizzled) for hat_projx_cab
};

// Implicit-GEMM 3x3 convolution, stride 1, zero padding 1, NHWC.
enum ConvEpi : int {
    CEPI_STORE = 0,      // out[p][co] = v (+ act)
    CEPI_RESID = 1,      // out[p][co] = v + res[p][co]
    CEPI_SHUFFLE = 2,    // pixel shuffle by r into [H*r][W*r][co/(r*r)] (channels pre-permuted)
    CEPI_FINAL = 3,      // planar [3][ch][cw] with crop, / img_range + mean
    CEPI_COLSUM = 4,     // store + per-block column sums into partial[blk][co]
};

struct ConvArgs {
    const float* in;     // [H][W][cin_stride]
    const float* w;      // repacked: [CIp/16][9][COp][16] (chunk, tap, co, 16 ci)
    const float* bias;   // [COp]
    float* out;
    const float* res;    // CEPI_RESID
    float* partial;      // CEPI_COLSUM: [gridDim.x*gridDim.y][co_stride]
    int H, W;
    int CI, CIp, cin_stride;
    int CO, COp, co_stride;   // co_stride = channel stride of out (NHWC)
    int act;             // 0 none, 1 gelu, 2 leaky(0.01)
    int r;               // CEPI_SHUFFLE factor
    int crop_h, crop_w;  // CEPI_FINAL crop (output size)
    float img_range;     // CEPI_FINAL: out = v / img_range + mean
    float mean0, mean1, mean2;
    // hat_convw_* (all output channels per block, GEMM epilogues):
    float* xn;           // LayerNorm of the output rows [H*W][co_stride]
    const float* nw;
    const float* nb;
    float eps;
    // hat_convwino_*: Winograd F(2x2,3x3) weights U = G g G^T split into three
    // bf16 parts, arranged [kc][xi 16][nt][part 3][lane 64][8] (lane r + 16 g:
    // co 16 nt + r, ci 32 kc + 8 g .. +7; channels padded to 16s and 32s)
    const unsigned short* wu;
    // hat_convwino_* and hat_conv_last3 launched over a band of tile rows (the
    // host-memory forward's head): the band's first tile; 0 for a whole plane
    int tile0;
    // hat_convwino_*: the launch's virtual blocks (tiles x column blocks),
    // walked by a grid of at most one block per CU; 0: one per block
    int nblk;
};

// Squeeze-excite gate: gate[c] = sigmoid(b2 + W2 relu(b1 + W1 mean)).
struct SeArgs {
    const float* partial; // [nblk][co_stride]
    int nblk, co_stride;
    float count;          // pixel count (mean = sum / count)
    const float* w1;      // [sq][C]
    const float* b1;      // [sq]
    const float* w2;      // [C][sq]
    const float* b2;      // [C]
    float* gate;          // [C]
    int C, sq;
};

// Fused window attention: one block per (window, head) (grid nw x heads), or,
// for OCA with head_dim 24, persistent blocks walking the (window, head) items
// head-major (grid: at most one block per CU, gridDim.y = 1).
constexpr bool attn_persistent(int D, bool oca) { return oca && D == 24; }
// The split-bf16 kernels (attnx.hip) run one item per block, SW and OCA.
struct AttnArgs {
    const float* qkv;    // head-major [3][heads][T][D]
    const float* table;  // relative-position bias table [rows][heads]
    float* out;          // [T][C] token-major, image order
    int hp, wp, nx, ny;  // padded plane and window grid
    int heads, D, C;
    int shift;           // SW: cyclic shift (0 or win/2); mask applied iff shift > 0
    int owin, opad;      // OCA: unfold window and padding
    int T;
    float qscale;        // head_dim^-0.5 * log2(e)
    // with_gate: block (0, 0) of the item grid first computes the folded CAB's
    // gate (hat_cab_gate's work), which the HAB tail after this launch needs
    int with_gate;
    CabGateArgs gate;
    // with_se: the same for the unfolded CAB's squeeze-excite gate (C = 180)
    int with_se;
    SeArgs se;
};

// Fused MLP (C = 144, hidden 288; C = 180, hidden 360):
//   out[m][:] = res[m][:] + fc2(gelu(fc1(a[m][:])))   (+ xn = LayerNorm(out) for EPI_RESID_LN)
#define MLP_WAVES 8
#define MLP_ROWS (MLP_WAVES * 16)

struct MlpArgs {
    const float* a;      // [M][K]
    const float* w1;     // [H][ldw1] (K used)
    const float* b1;     // [H]
    const float* w2;     // [N][ldw2] (H used)
    const float* b2;     // [N]
    const float* res;    // [M][N] (may alias out)
    float* out;          // [M][N]
    float* xn;           // EPI_RESID_LN: [M][N] (may alias a)
    const float* nw;
    const float* nb;
    int M;
    float eps;
    int K, H, N;         // input width (= N), hidden width, output width
    int ldw1, ldw2;      // packed weight row strides
};

// The fused block tails' width.
#define HT_C 144

// The second half of a HAB, C = 144 with the folded CAB (hat_hab_tail):
//   x' = res + a . wp^T + nb(t1) . w2g^T + bias2,  out = x' + fc2(gelu(fc1(LN2(x')))),
//   xn = LN_next(out).
struct HabTailArgs {
    const float* a;      // [M][144] attention output
    const float* res;    // [M][144] block input
    float* out;          // [M][144] (may alias res)
    float* xn;           // [M][144] LN_next(out)
    const float* wp;     // [144][144] attention projection (packed, Kp = 144)
    const float* w2g;    // [144][CAB_K2] gate-scaled conv2 weights
    const float* bias2;  // [144] projection bias + gated conv2 bias
    const float* t1;     // [H*W][CAB_CS] CAB conv1 output
    const float* n2w;    // norm2
    const float* n2b;
    const float* w1;     // [288][ldw1]
    const float* b1;
    const float* w2;     // [144][ldw2]
    const float* b2;
    const float* nw;     // the next block's norm1
    const float* nb;
    int M, H, W;         // rows = the H x W plane
    float eps;
    int ldw1, ldw2;
};

// The C = 144 HAB / OCAB tail on split-bf16 MFMA as two kernels (tailx.hip):
// hat_projx(_cab): out = x' = res + a . Wp^T (+ nb(t1) . W2g^T) + bias,
//                  xn = LN(x') with nw / nb;
// hat_mlpx(_ln):   out = res + fc2(gelu(fc1(a))) + b2 (+ xn = LN(out)).
// Weight chunks of the split-bf16 tails (tailx.hip): one 32-k step of up to
// 192 rows as three bf16 planes [rows][32], each row's four 16-byte k-groups g
// stored at slot ws_slot(row, g) (ws_mma), WC_CHUNK elements apart (zeros after
// the planes). A chunk is copied as loads of 1 KB, the same number from every
// wave of a block: 144 rows take 27 (28 to share them out evenly), 96 rows 18
// (20), 192 rows 36.
#define WC_CHUNK 20480  // 40 x 512 >= 3 x 192 x 32
// The slot of row r's 16-byte k-group g in a 64-byte row of those planes. An
// MFMA fragment read has lane i take rows r0 + i at one k-group, 16 bytes a
// lane, and the LDS serves such reads 8 consecutive lanes at a time over its
// 32 four-byte banks; two 64-byte rows fill the banks once, so the XOR by
// (r >> 1) & 3 gives the four row pairs of every 8 lanes four distinct slots
// and the reads have no bank conflicts without padding (measured: none).
constexpr int ws_slot(int r, int g) { return g ^ ((r >> 1) & 3); }
// The MLP walks the hidden layer in thirds of MX_HID units: per third five
// fc1 chunks (96 permuted rows, k = input channel) then three fc2 chunks (144
// rows, k = the third's hidden units), 24 chunks in all.
#define MX_HID 96
// The C = 180 MLP (hat_mlpx180*) walks its 360 hidden units (384 with 24
// zero units) in six parts of MX180_HID: per part six fc1 chunks (64 permuted
// rows, k = input channel, b1 at k = 180) and two fc2 chunks (192 rows, 180
// real, k = the part's units), 48 chunks in the swizzled [rows][32] layout of
// the weight-stationary kernels, MX180_SLOT elements apart.
#define MX180_HID 64
#define MX180_SLOT (3 * 192 * 32)
// Their launch geometry (tailx): blocks of 4 waves, one 128-token row tile a block.
#define WX_THREADS 256
#define WX_ROWS 128
constexpr int wx_tiles(int M) { return (M + WX_ROWS - 1) / WX_ROWS; }

// The qkv linear (hat_gemmx_qkv, hat_gemmx_qkv180) keeps one column slice in
// LDS for the whole launch: per 32-k step three bf16 planes [rows][32],
// unpadded, each row's four 16-byte k-groups stored at slot ws_slot(row, g)
// (so that reads of one k-group down the rows are free of bank conflicts),
// WS_CHUNK elements apart. C = 144: three slices (q, k, v) of 144 rows, five
// k-steps; C = 180: six slices of 96 rows (three heads of 30, rows 90..95
// zero), six k-steps (WS_CHUNK180). Groups of NS blocks (one per slice, on one
// XCD) walk the same 32-token subtiles: gemmx_qkv_groups(cus, NS) groups.
#define WS_CHUNK (3 * 144 * 32)
#define WS_CHUNK180 (3 * 96 * 32)
#define GX_THREADS 512
constexpr int gemmx_qkv_groups(int cus, int ns) { return cus >= 8 * ns ? cus / (8 * ns) * 8 : 1; }

struct TailXArgs {
    const float* a;            // projx: attention output; mlpx (C = 144): x' rows, normed in the kernel by
                               // (inw, inb); mlpx180: LN2(x') rows
    const float* res;          // projx: block input; mlpx: x'
    float* out;                // [M][144] (may alias res)
    float* xn;                 // projx: LN2(x') when non-null; mlpx (LN): the next norm1 (may alias a)
    const unsigned short* w;   // weight chunks (projx: 5, mlpx: 24)
    const float* bias;         // projx: bias2 or the projection bias (mlpx: b1 is in its chunks)
    const float* b2;           // mlpx: fc2 bias
    const unsigned short* w2gx;  // projx_cab: the gate-scaled conv2 weights as 2 chunks (k = tap*6 + ci)
    const float* t1;           // projx_cab: [M][CAB_CS] CAB conv1 output
    const float* nw;
    const float* nb;
    int M, H, W;               // rows = the H x W plane
    float eps;
    // hat_projx180_hab (the unfolded CAB of the C = 180 family): out = x +
    // proj + bias + aux * gate * cscale (aux: conv2's output [M][180])
    const float* aux;
    const float* gate;
    float cscale;
    // hat_mlpx(_ln): norm2's weight and bias, applied to the x' rows of a
    const float* inw;
    const float* inb;
    // hat_habx*: the MLP's 24 weight chunks in the fused input order (w holds
    // the projection's)
    const unsigned short* wm;
    // hat_habx*: fc1's bias in the thirds' permuted row order (added to fc1's
    // output before the GELU)
    const float* b1x;
};

struct LnArgs {
    const float* x;
    float* y;
    const float* w;
    const float* b;
    int rows, C;
    float eps;
};

struct PreArgs {
    const float* in;     // [3][h][w]
    float* out;          // [hp][wp][cstride], channels >= 3 zeroed
    int h, w, hp, wp, cstride;
    float m0, m1, m2, range;
};

// dst[i] = src[i] for n4 float4 (16-byte aligned buffers).
struct CopyArgs {
    const float* src;
    float* dst;
    long n4;
};

// Column sums of a [nrows][stride] matrix in row blocks: out[blk][c] = sum of
// rows [blk*rows_per, blk*rows_per + rows_per) of column c.
struct ReduceArgs {
    const float* in;
    float* out;
    int nrows, C, stride, rows_per;
};

}  // namespace hatk
