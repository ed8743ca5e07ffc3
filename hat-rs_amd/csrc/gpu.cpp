#include "gpu.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <atomic>
#include <thread>

#include "kargs.h"
#include "tile.h"

namespace hat {

using namespace hatk;

// ---------------------------------------------------------------------------
// Weight repacking

std::vector<float> pack_linear(const float* w, int N, int K, int* Kp)
{
    const int kp = (K + 15) / 16 * 16;
    std::vector<float> out((size_t)N * kp, 0.0f);
    for (int n = 0; n < N; ++n) memcpy(&out[(size_t)n * kp], w + (size_t)n * K, sizeof(float) * K);
    *Kp = kp;
    return out;
}

namespace {
// float -> bf16, round to nearest even (NaN kept a NaN)
unsigned short bf16_rne(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}
float bf16_float(unsigned short h)
{
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
}  // namespace

// Rows [N][K] of w (row stride ldw), N <= 192, as weight chunks at dst: the
// value at (n, k) is column kbase + k, which lands in 32-k step s = (kbase +
// k) / 32, WC_CHUNK elements apart, as three bf16 planes [N][32] (plane stride
// N * 32) with row n's 16-byte k-groups g stored at slot ws_slot(n, g) (so that
// reads of one k-group down the rows are free of bank conflicts): x = h0 + h1 +
// h2, each part the RNE of what the parts before it leave; the rest stays zero.
static void split_chunks(const float* w, int N, int K, int ldw, unsigned short* dst, int kbase = 0)
{
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) {
            const float x = w[(size_t)n * ldw + k];
            const unsigned short h0 = bf16_rne(x);
            const float r1 = x - bf16_float(h0);
            const unsigned short h1 = bf16_rne(r1);
            const unsigned short h2 = bf16_rne(r1 - bf16_float(h1));
            const int s = (kbase + k) / 32, kk = (kbase + k) % 32;
            unsigned short* d = dst + (size_t)s * WC_CHUNK + (size_t)n * 32 + hatk::ws_slot(n, kk / 8) * 8 + kk % 8;
            d[0] = h0;
            d[(size_t)N * 32] = h1;
            d[(size_t)2 * N * 32] = h2;
        }
}

// The last k-step of a K = 144 split linear in the packed form (common.h
// ws_mma_half): only k = 128 .. 143 are real, so lane group g's slots j < 4
// hold k = 128 + 4 g + j and slots 4 + j the same k, and the three planes hold
// the part pairs (a0 | a0), (a1 | a0), (a1 | a2): against the activation pairs
// (b0 | b1), (b0 | b2), (b1 | b0) they give the six products of order <= 2 in
// three MFMAs. Row n of w (ldw apart) goes to row n of the chunk at dst, whose
// planes are N * 32 elements apart.
static void split_half_step(const float* w, int N, int ldw, unsigned short* dst)
{
    for (int n = 0; n < N; ++n)
        for (int kk = 0; kk < 16; ++kk) {
            const float x = w[(size_t)n * ldw + 128 + kk];
            const unsigned short h0 = bf16_rne(x);
            const float r1 = x - bf16_float(h0);
            const unsigned short h1 = bf16_rne(r1);
            const unsigned short h2 = bf16_rne(r1 - bf16_float(h1));
            const int g = kk / 4, j = kk % 4;
            unsigned short* d = dst + (size_t)n * 32 + hatk::ws_slot(n, g) * 8 + j;
            const size_t pl = (size_t)N * 32;
            d[0] = h0, d[4] = h0;            // (a0 | a0)
            d[pl] = h1, d[pl + 4] = h0;      // (a1 | a0)
            d[2 * pl] = h1, d[2 * pl + 4] = h2;  // (a1 | a2)
        }
}

std::vector<unsigned short> pack_linear_x(const float* w, int N, int K)
{
    constexpr int BN = 144;
    if (K != 144 || N % BN != 0) throw Error("pack_linear_x: needs K = 144 and N a multiple of 144");
    const int steps = (K + 31) / 32;
    std::vector<unsigned short> out((size_t)(N / BN) * steps * WC_CHUNK, 0);
    for (int sl = 0; sl < N / BN; ++sl) {
        unsigned short* dst = &out[(size_t)sl * steps * WC_CHUNK];
        // four whole k-steps, then k = 128 .. 143 packed (split_half_step);
        // the tails add the bias in fp32
        split_chunks(w + (size_t)sl * BN * K, BN, 128, K, dst);
        split_half_step(w + (size_t)sl * BN * K, BN, K, dst + (size_t)4 * WC_CHUNK);
    }
    return out;
}

std::vector<unsigned short> pack_linear_ws(const float* w, const float* bias, int N, int K)
{
    // C = 144: slices of 144 rows (q, k, v), five k-steps; C = 180: slices of
    // 90 rows (three heads of 30) padded to 96, six k-steps
    if (!((K == 144 && N == 432) || (K == 180 && N == 540)))
        throw Error("pack_linear_ws: needs the qkv shapes K = 144, N = 432 or K = 180, N = 540");
    const int real = K == 144 ? 144 : 90, rows = K == 144 ? 144 : 96, ks_n = (K + 32) / 32;
    const size_t chunk = (size_t)3 * rows * 32;
    std::vector<unsigned short> out((size_t)(N / real) * ks_n * chunk, 0);
    if (K == 144) {
        // four whole k-steps, then k = 128 .. 143 packed (split_half_step);
        // the bias is the accumulators' start value (hat_gemmx_qkv reads it)
        for (int sl = 0; sl < N / real; ++sl) {
            for (int n = 0; n < real; ++n)
                for (int k = 0; k < 128; ++k) {
                    const float x = w[((size_t)sl * real + n) * K + k];
                    const unsigned short h0 = bf16_rne(x);
                    const float r1 = x - bf16_float(h0);
                    const unsigned short h1 = bf16_rne(r1);
                    const unsigned short h2 = bf16_rne(r1 - bf16_float(h1));
                    const int s = k / 32, g = (k % 32) / 8, j = k % 8;
                    unsigned short* d = &out[((size_t)sl * ks_n + s) * chunk + (size_t)n * 32 + hatk::ws_slot(n, g) * 8 + j];
                    d[0] = h0;
                    d[(size_t)rows * 32] = h1;
                    d[(size_t)2 * rows * 32] = h2;
                }
            split_half_step(w + (size_t)sl * real * K, real, K, &out[((size_t)sl * ks_n + 4) * chunk]);
        }
        return out;
    }
    for (int n = 0; n < N; ++n)
        for (int k = 0; k <= K; ++k) {
            if (k == K && !bias) break;
            const float x = k < K ? w[(size_t)n * K + k] : bias[n];  // k = K: the bias column
            const unsigned short h0 = bf16_rne(x);
            const float r1 = x - bf16_float(h0);
            const unsigned short h1 = bf16_rne(r1);
            const unsigned short h2 = bf16_rne(r1 - bf16_float(h1));
            const int r = n % real, s = k / 32, g = (k % 32) / 8, j = k % 8;
            unsigned short* d = &out[((size_t)(n / real) * ks_n + s) * chunk + (size_t)r * 32 + hatk::ws_slot(r, g) * 8 + j];
            d[0] = h0;
            d[(size_t)rows * 32] = h1;
            d[(size_t)2 * rows * 32] = h2;
        }
    return out;
}

// fc1 output tile t, row 4g + r (lane group g, register r) -> hidden unit
// within a 96-unit third (tailx.hip): fc2's 32-k step s then finds units
// 32 s + 8 g .. +7 in tiles 2 s and 2 s + 1 of lane group g.
static int mlpx_unit(int row)
{
    const int t = row / 16, g = (row % 16) / 4, r = row % 4;
    return 32 * (t / 2) + 8 * g + 4 * (t % 2) + r;
}

void pack_mlp_x(const float* w1, const float* b1, const float* w2, std::vector<unsigned short>* w)
{
    constexpr int C = 144, H = 288;
    static_assert(3 * C * 32 <= WC_CHUNK && WC_CHUNK % 512 == 0 && H % MX_HID == 0, "chunks");
    std::vector<float> f1((size_t)MX_HID * C), fb((size_t)MX_HID);
    w->assign((size_t)24 * WC_CHUNK, 0);
    for (int q = 0; q < H / MX_HID; ++q) {
        for (int row = 0; row < MX_HID; ++row) {
            const int u = q * MX_HID + mlpx_unit(row);
            memcpy(&f1[(size_t)row * C], w1 + (size_t)u * C, C * sizeof(float));
            fb[row] = b1[u];
        }
        unsigned short* dst = &(*w)[(size_t)(8 * q) * WC_CHUNK];
        split_chunks(f1.data(), MX_HID, C, C, dst);
        // b1 as fc1's column k = 144 (step 4, j = 16)
        split_chunks(fb.data(), MX_HID, 1, 1, dst, C);
        split_chunks(w2 + q * MX_HID, C, MX_HID, H, &(*w)[(size_t)(8 * q + 5) * WC_CHUNK]);
    }
}

// Fused tail input position k = 32 ks + 8 g + j (ks: 32-k step, g: lane group,
// j < 8) -> channel of x': steps 0..3 hold the lane's accumulator tiles 2 ks
// and 2 ks + 1 (channels 32 ks + 4 g + j and 32 ks + 16 + 4 g + j - 4), step 4
// tile 8 (128 + 4 g + j) and b1's 1 at g = 0, j = 4 (-1); -2: an empty position.
// The device twin is habx_channel (tailx.hip).
int mlpx_fused_channel(int k)
{
    const int ks = k >> 5, g = (k >> 3) & 3, j = k & 7;
    if (ks < 4) return 32 * ks + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
    if (j < 4) return 128 + 4 * g + j;
    return g == 0 && j == 4 ? -1 : -2;
}

void pack_mlp_xf(const float* w1, const float* b1, const float* w2, std::vector<unsigned short>* w,
                 std::vector<float>* b1x)
{
    // per third: fc1's steps 0..3 in the fused input order, step 4 (channels
    // 128 .. 143, whose fused positions are 128 + 4 g + j) packed
    // (split_half_step), b1 added in fp32 before the GELU (b1x, in the
    // third's permuted row order), then fc2's three steps
    constexpr int C = 144, H = 288, KF = 128;
    std::vector<float> f1((size_t)MX_HID * KF), rows((size_t)MX_HID * C);
    w->assign((size_t)24 * WC_CHUNK, 0);
    b1x->assign(H, 0.0f);
    for (int q = 0; q < H / MX_HID; ++q) {
        for (int row = 0; row < MX_HID; ++row) {
            const int u = q * MX_HID + mlpx_unit(row);
            for (int k = 0; k < KF; ++k) f1[(size_t)row * KF + k] = w1[(size_t)u * C + mlpx_fused_channel(k)];
            memcpy(&rows[(size_t)row * C], w1 + (size_t)u * C, C * sizeof(float));
            (*b1x)[(size_t)q * MX_HID + row] = b1[u];
        }
        split_chunks(f1.data(), MX_HID, KF, KF, &(*w)[(size_t)(8 * q) * WC_CHUNK]);
        split_half_step(rows.data(), MX_HID, C, &(*w)[(size_t)(8 * q + 4) * WC_CHUNK]);
        split_chunks(w2 + q * MX_HID, C, MX_HID, H, &(*w)[(size_t)(8 * q + 5) * WC_CHUNK]);
    }
}

// One 32-k step of `rows` weight rows (value(r, kk), kk < 32) split into three
// bf16 planes [rows][32] in the swizzled layout of the weight-stationary
// kernels (row r's k-group g at slot ws_slot(r, g)).
template <typename F>
static void split_ws_step(int rows, F value, unsigned short* dst)
{
    for (int r = 0; r < rows; ++r)
        for (int kk = 0; kk < 32; ++kk) {
            const float x = value(r, kk);
            const unsigned short h0 = bf16_rne(x);
            const float r1 = x - bf16_float(h0);
            const unsigned short h1 = bf16_rne(r1);
            const unsigned short h2 = bf16_rne(r1 - bf16_float(h1));
            unsigned short* d = dst + (size_t)r * 32 + hatk::ws_slot(r, kk / 8) * 8 + kk % 8;
            d[0] = h0;
            d[(size_t)rows * 32] = h1;
            d[(size_t)2 * rows * 32] = h2;
        }
}

// The C = 180 projection [180][180] for hat_projx180*: six 32-k steps of 192
// rows (180 real; the bias is added in the epilogue), MX180_SLOT apart.
std::vector<unsigned short> pack_linear_x180(const float* w)
{
    constexpr int C = 180;
    std::vector<unsigned short> out((size_t)6 * MX180_SLOT, 0);
    for (int ks = 0; ks < 6; ++ks)
        split_ws_step(192, [&](int n, int kk) {
            const int k = ks * 32 + kk;
            return n < C && k < C ? w[(size_t)n * C + k] : 0.0f;
        }, &out[(size_t)ks * MX180_SLOT]);
    return out;
}

// The C = 180 MLP (fc1 [360][180] + b1, fc2 [180][360]) for hat_mlpx180: per
// part of 64 hidden units, six fc1 k-steps (rows permuted by mlpx_unit, b1 at
// k = 180) and two fc2 k-steps (192 rows, 180 real, the part's units in
// natural order), MX180_SLOT elements apart.
void pack_mlp_x180(const float* w1, const float* b1, const float* w2, std::vector<unsigned short>* w)
{
    constexpr int C = 180, H = 360, NP = 6;
    w->assign((size_t)8 * NP * MX180_SLOT, 0);
    for (int q = 0; q < NP; ++q) {
        for (int ks = 0; ks < 6; ++ks)
            split_ws_step(MX180_HID, [&](int r, int kk) {
                const int u = q * MX180_HID + mlpx_unit(r), k = ks * 32 + kk;
                if (u >= H) return 0.0f;
                return k < C ? w1[(size_t)u * C + k] : (k == C ? b1[u] : 0.0f);
            }, &(*w)[(size_t)(8 * q + ks) * MX180_SLOT]);
        for (int st = 0; st < 2; ++st)
            split_ws_step(192, [&](int n, int kk) {
                const int u = q * MX180_HID + st * 32 + kk;
                return n < C && u < H ? w2[(size_t)n * H + u] : 0.0f;
            }, &(*w)[(size_t)(8 * q + 6 + st) * MX180_SLOT]);
    }
}

// Fused C = 180 tail input position k = 32 ks + 8 g + j (ks < 6: 32-k step, g:
// lane group, j < 8) -> channel of x': the lane's accumulator tiles 2 ks and
// 2 ks + 1 (channels 32 ks + 4 g + j and 32 ks + 16 + 4 g + j - 4); -1 past
// channel 179. The device twin is habx180_channel (tailx.hip).
int mlpx180_fused_channel(int k)
{
    const int ks = k >> 5, g = (k >> 3) & 3, j = k & 7;
    const int c = 32 * ks + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
    return c < 180 ? c : -1;
}

void pack_mlp_xf180(const float* w1, const float* b1, const float* w2, std::vector<unsigned short>* w,
                    std::vector<float>* b1x)
{
    // per part: fc1's six steps with rows permuted by mlpx_unit and input
    // columns in the fused order, b1 in b1x (the same row order, added in
    // fp32 before the GELU), then fc2's two steps as in pack_mlp_x180
    constexpr int C = 180, H = 360, NP = 6;
    w->assign((size_t)8 * NP * MX180_SLOT, 0);
    b1x->assign((size_t)NP * MX180_HID, 0.0f);
    for (int q = 0; q < NP; ++q) {
        for (int r = 0; r < MX180_HID; ++r) {
            const int u = q * MX180_HID + mlpx_unit(r);
            if (u < H) (*b1x)[(size_t)q * MX180_HID + r] = b1[u];
        }
        for (int ks = 0; ks < 6; ++ks)
            split_ws_step(MX180_HID, [&](int r, int kk) {
                const int u = q * MX180_HID + mlpx_unit(r), c = mlpx180_fused_channel(ks * 32 + kk);
                return u < H && c >= 0 ? w1[(size_t)u * C + c] : 0.0f;
            }, &(*w)[(size_t)(8 * q + ks) * MX180_SLOT]);
        for (int st = 0; st < 2; ++st)
            split_ws_step(192, [&](int n, int kk) {
                const int u = q * MX180_HID + st * 32 + kk;
                return n < C && u < H ? w2[(size_t)n * H + u] : 0.0f;
            }, &(*w)[(size_t)(8 * q + 6 + st) * MX180_SLOT]);
    }
}

// [CO][CI][3][3] -> [CIp/16][9][COp][16]; with r > 0 the output channels are
// permuted so that channel o = c*r*r + i*r + j lands at o' = (i*r + j)*Cf + c
// (Cf = CO / r^2), which lets the conv store four consecutive o' as four
// consecutive channels of one pixel of the shuffled plane.
std::vector<float> pack_conv(const float* w, const float* b, int CO, int CI, int r,
                             std::vector<float>* bias_out, int* CIp, int* COp)
{
    const int cip = (CI + 15) / 16 * 16, cop = (CO + 15) / 16 * 16;
    const int Cf = r > 0 ? CO / (r * r) : 0;
    auto src_channel = [&](int o2) -> int {
        if (r <= 0) return o2;
        const int sub = o2 / Cf, c = o2 % Cf;
        const int i = sub / r, j = sub % r;
        return c * r * r + i * r + j;
    };
    std::vector<float> out((size_t)cip * 9 * cop, 0.0f);
    bias_out->assign(cop, 0.0f);
    for (int o2 = 0; o2 < CO; ++o2) {
        const int o = src_channel(o2);
        (*bias_out)[o2] = b[o];
        for (int ci = 0; ci < CI; ++ci)
            for (int tap = 0; tap < 9; ++tap) {
                const int cc = ci / 16, c16 = ci % 16;
                out[(((size_t)cc * 9 + tap) * cop + o2) * 16 + c16] = w[((size_t)o * CI + ci) * 9 + tap];
            }
    }
    *CIp = cip;
    *COp = cop;
    return out;
}

// [CO][CI][3][3] -> the Winograd F(2x2, 3x3) weights U[xi] = G g G^T of the
// hat_convwino_* kernels, G = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1],
// formed in double, rounded to fp32 and split into three bf16 parts, arranged
// [kc][xi][nt][part][lane][8]: lane r + 16 g of (kc, xi, nt) holds part `part`
// of U[xi][16 nt + r][32 kc + 8 g .. +7]; channels past CO and CI are zero
// (CO padded to 16s, CI to 32s). With r > 0 the output channels are permuted
// as pack_conv permutes them. When the last chunk holds at most 16 real
// channels (CI = 144), it is packed as the K = 144 linears' last step
// (split_half_step): lane r + 16 g, slots j < 4 hold channel 32 kc + 4 g + j,
// slots 4 + j the same channel, the parts as (0 | 0), (1 | 0), (1 | 2).
std::vector<unsigned short> pack_wino(const float* w, int CO, int CI, int r)
{
    if (r > 0 && CO % 16 != 0) throw Error("pack_wino: shuffled output channels must come in 16s");
    static const double G[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
    const int NTT = (CO + 15) / 16, NKC = (CI + 31) / 32, Cf = r > 0 ? CO / (r * r) : 0;
    const bool packed = CI % 32 != 0 && CI % 32 <= 16;  // the kernels' PACK
    std::vector<unsigned short> out((size_t)NKC * 16 * NTT * 3 * 512, 0);
    for (int o2 = 0; o2 < CO; ++o2) {
        int o = o2;
        if (r > 0) {
            const int sub = o2 / Cf, c = o2 % Cf;
            o = c * r * r + (sub / r) * r + sub % r;
        }
        for (int ci = 0; ci < CI; ++ci) {
            const float* g = w + ((size_t)o * CI + ci) * 9;
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 4; ++j) {
                    double u = 0.0;
                    for (int a = 0; a < 3; ++a)
                        for (int b = 0; b < 3; ++b) u += G[i][a] * (double)g[a * 3 + b] * G[j][b];
                    const float x = (float)u;
                    const unsigned short h0 = bf16_rne(x);
                    const float r1 = x - bf16_float(h0);
                    const unsigned short h1 = bf16_rne(r1);
                    const unsigned short h2 = bf16_rne(r1 - bf16_float(h1));
                    const int xi = 4 * i + j, kc = ci / 32, c32 = ci % 32, nt = o2 / 16, rr = o2 % 16;
                    if (packed && kc == NKC - 1) {
                        const int lane = rr + 16 * (c32 / 4);
                        const size_t at = ((((size_t)kc * 16 + xi) * NTT + nt) * 3 * 64 + lane) * 8 + c32 % 4;
                        out[at] = h0, out[at + 4] = h0;
                        out[at + 512] = h1, out[at + 512 + 4] = h0;
                        out[at + 1024] = h1, out[at + 1024 + 4] = h2;
                        continue;
                    }
                    const int lane = rr + 16 * (c32 / 8);
                    const size_t at = ((((size_t)kc * 16 + xi) * NTT + nt) * 3 * 64 + lane) * 8 + c32 % 8;
                    out[at] = h0;
                    out[at + 512] = h1;
                    out[at + 1024] = h2;
                }
        }
    }
    return out;
}

// Which convs have a Winograd kernel (hat_convwino_*): the 144 -> 144 and
// 180 -> 180 trunk convs, conv_before_upsample 144 / 180 -> 64, the x2
// upsample convs 64 -> 256 and the unfolded CAB's 180 -> 60 and 60 -> 180.
static bool wino_conv(int CO, int CI, int r)
{
    return (r == 0 && (CI == 144 || CI == 180) && (CO == CI || CO == 64)) || (r == 2 && CI == 64 && CO == 256) ||
           (r == 0 && CI == 180 && CO == 60) || (r == 0 && CI == 60 && CO == 180);
}

// conv1 [6][144][3][3] as the split A operands of hat_cab_conv1* (CX_WPACK):
// row r = tap * 6 + co (rows 54..63 zero), each weight as three bf16 parts.
std::vector<unsigned short> pack_cab_conv1(const float* w)
{
    std::vector<unsigned short> out(CX_WPACK, 0);
    for (int ks = 0; ks < 9; ++ks)
        for (int nt = 0; nt < 2; ++nt)
            for (int lane = 0; lane < 64; ++lane)
                for (int j = 0; j < 8; ++j) {
                    const int r = nt * 32 + lane % 32, ci = ks * 16 + 8 * (lane / 32) + j;
                    if (r >= 9 * CAB_CC) continue;
                    const int tap = r / CAB_CC, co = r % CAB_CC;
                    const float x = w[((size_t)co * CAB_C + ci) * 9 + tap];
                    const unsigned short h0 = bf16_rne(x);
                    const float r1 = x - bf16_float(h0);
                    const unsigned short h1 = bf16_rne(r1);
                    const unsigned short h2 = bf16_rne(r1 - bf16_float(h1));
                    const unsigned short parts[3] = {h0, h1, h2};
                    for (int part = 0; part < 3; ++part)
                        out[((size_t)((ks * 2 + nt) * 3 + part) * 64 + lane) * 8 + j] = parts[part];
                }
    return out;
}

// ---------------------------------------------------------------------------
// Launch helpers shared by the backend and the op entry points.

namespace {

// Column-block width of the GEMM for an output width N: 144 for the C = 144
// family, 192 for C = 180 (N = 180, 360, 540 in 1, 2, 3 blocks).
int gemm_bn(int N) { return N % 144 == 0 ? 144 : 192; }

const char* gemm_kernel(int N, int epi)
{
    const bool n9 = gemm_bn(N) == 144;
    switch (epi) {
    case EPI_STORE: return n9 ? "hat_gemm_n9_store" : "hat_gemm_n12_store";
    case EPI_GELU: return n9 ? "hat_gemm_n9_gelu" : "hat_gemm_n12_gelu";
    case EPI_QKV: return n9 ? "hat_gemm_n9_qkv" : "hat_gemm_n12_qkv";
    case EPI_RESID: return n9 ? "hat_gemm_n9_resid" : "hat_gemm_n12_resid";
    case EPI_RESID_LN: return n9 ? "hat_gemm_n9_resid_ln" : "hat_gemm_n12_resid_ln";
    case EPI_HAB_LN: return n9 ? "hat_gemm_n9_hab_ln" : "hat_gemm_n12_hab_ln";
    }
    throw Error("unknown GEMM epilogue");
}

// The weight-stationary kernels hold a block's whole weight row slice in LDS:
// K = 144 with 144-wide column blocks (N a multiple of 144), and K = 180
// (rows padded to 192) with 192-wide blocks, for the epilogues the blocks use.
// Returns the kernel and sets *bn to its column-block width.
const char* gemm_ws_kernel(const DevLinear& L, int epi, int* bn)
{
    const bool k144 = L.K == 144 && L.Kp == 144 && L.N % 144 == 0;
    const bool k180 = L.K == 180 && L.Kp == 192;
    if (!k144 && !k180) return nullptr;
    *bn = k144 ? 144 : 192;
    switch (epi) {
    case EPI_QKV: return k144 ? "hat_gemmws_qkv" : "hat_gemmws12_qkv";
    case EPI_GELU: return k144 ? "hat_gemmws_gelu" : "hat_gemmws12_gelu";
    case EPI_RESID_LN: return k144 ? "hat_gemmws_resid_ln" : "hat_gemmws12_resid_ln";
    case EPI_HAB_LN: return k144 ? "hat_gemmws_hab_ln" : "hat_gemmws12_hab_ln";
    }
    return nullptr;
}

struct GemmEpilogue {
    const float* res = nullptr;   // residual
    const float* aux = nullptr;   // conv branch (HAB)
    const float* gate = nullptr;  // channel gate (HAB)
    float* xn = nullptr;          // LayerNorm output of the result rows
    const float* nw = nullptr;
    const float* nb = nullptr;
};

void run_gemm(hipStream_t s, const DevLinear& L, const float* a, int lda, long M, float* out,
              int ldo, int epi, const GemmEpilogue& e, int heads, int hdim, float cscale)
{
    if (L.K % 4 != 0 || lda % 4 != 0 || lda < L.K)
        throw Error("GEMM: K and lda must be multiples of 4 with lda >= K");
    if (L.N % 4 != 0 || (epi != EPI_QKV && (ldo % 4 != 0 || ldo < L.N)))
        throw Error("GEMM: N and ldo must be multiples of 4 with ldo >= N");
    if (M > 0x7fffffffL) throw Error("GEMM: too many rows");
    const int BN = gemm_bn(L.N);
    if ((epi == EPI_RESID_LN || epi == EPI_HAB_LN) && L.N > BN)
        throw Error("GEMM: a LayerNorm epilogue needs whole rows in one block");
    GemmArgs p{};
    p.a = a;
    p.w = L.w;
    p.bias = L.b;
    p.out = out;
    p.res = e.res;
    p.aux = e.aux;
    p.gate = e.gate;
    p.xn = e.xn;
    p.nw = e.nw;
    p.nb = e.nb;
    p.M = (int)M;
    p.N = L.N;
    p.K = L.K;
    p.Kp = L.Kp;
    p.lda = lda;
    p.ldo = ldo;
    p.heads = heads;
    p.hdim = hdim;
    p.cscale = cscale;
    p.eps = 1e-5f;
    if (epi == EPI_QKV && L.wx && L.K == 144 && L.N == 432 && heads == 6 && hdim == 24 && lda == 144) {
        // split-bf16 qkv (gemmx.hip): weight-stationary, groups of three blocks
        static const int cus = std::max(1, Runtime::get().cu_count());
        p.w = (const float*)L.wx;
        launch(s, "hat_gemmx_qkv", (unsigned)(3 * gemmx_qkv_groups(cus, 3)), 1, 1, GX_THREADS, p);
        return;
    }
    if (epi == EPI_QKV && L.wx && L.K == 180 && L.N == 540 && heads == 6 && hdim == 30 && lda == 180) {
        // the same for C = 180: groups of six blocks (96-column slices)
        static const int cus = std::max(1, Runtime::get().cu_count());
        p.w = (const float*)L.wx;
        launch(s, "hat_gemmx_qkv180", (unsigned)(6 * gemmx_qkv_groups(cus, 6)), 1, 1, GX_THREADS, p);
        return;
    }
    int wbn = 0;
    if (const char* ws = gemm_ws_kernel(L, epi, &wbn)) {
        // One block per CU (its 85 or 150 KB weight slice fills the LDS); the
        // (column slice, row tile) units are dealt out round-robin over the blocks.
        static const int cus = std::max(1, Runtime::get().cu_count());
        const long ntiles = (M + ws_rows(epi) - 1) / ws_rows(epi);
        const long units = ntiles * ((L.N + wbn - 1) / wbn);
        launch(s, ws, (unsigned)std::max(1L, std::min<long>(units, cus)), 1, 1, ws_waves(epi) * 64, p);
        return;
    }
    launch(s, gemm_kernel(L.N, epi), (unsigned)((M + 127) / 128), (unsigned)((L.N + BN - 1) / BN), 1,
           256, p);
}

// The MLP of one block: x_out = res + fc2(gelu(fc1(a))), for EPI_RESID_LN also
// xn = LayerNorm(x_out). One fused kernel for C = 144 (hidden 288) and
// C = 180 (hidden 360), else fc1 and fc2 as two GEMMs through the hidden buffer.
// The fused MLP kernels: C = 144 (hidden 288) and C = 180 (hidden 360). Other
// shapes run fc1 and fc2 as two GEMMs through a T x hidden buffer.
bool mlp_c144(const DevLinear& fc1, const DevLinear& fc2)
{
    return fc1.K == 144 && fc1.Kp == 144 && fc1.N == 288 && fc2.K == 288 && fc2.N == 144;
}
bool mlp_c180(const DevLinear& fc1, const DevLinear& fc2)
{
    return fc1.K == 180 && fc1.Kp == 192 && fc1.N == 360 && fc2.K == 360 && fc2.N == 180;
}
bool mlp_fused(const DevLinear& fc1, const DevLinear& fc2) { return mlp_c144(fc1, fc2) || mlp_c180(fc1, fc2); }

void run_mlp(hipStream_t s, const DevLinear& fc1, const DevLinear& fc2, const float* a, long M,
             const float* res, float* out, int epi, const GemmEpilogue& ln, float* hidden)
{
    if (epi != EPI_RESID && epi != EPI_RESID_LN) throw Error("MLP: bad epilogue");
    const bool c144 = mlp_c144(fc1, fc2);
    if (mlp_fused(fc1, fc2)) {
        if (M > 0x7fffffffL) throw Error("MLP: too many rows");
        MlpArgs p{};
        p.a = a;
        p.w1 = fc1.w;
        p.b1 = fc1.b;
        p.w2 = fc2.w;
        p.b2 = fc2.b;
        p.res = res;
        p.out = out;
        p.xn = ln.xn;
        p.nw = ln.nw;
        p.nb = ln.nb;
        p.M = (int)M;
        p.eps = 1e-5f;
        p.K = fc1.K;
        p.H = fc1.N;
        p.N = fc2.N;
        p.ldw1 = fc1.Kp;
        p.ldw2 = fc2.Kp;
        // One block per CU (113 or 151 KB of LDS), persistent over the 128-row tiles.
        static const int cus = std::max(1, Runtime::get().cu_count());
        const long ntiles = (M + MLP_ROWS - 1) / MLP_ROWS;
        const long rounds = (ntiles + cus - 1) / cus;
        const long g = std::max(1L, (ntiles + rounds - 1) / rounds);
        const char* name = epi == EPI_RESID_LN ? (c144 ? "hat_mlp_resid_ln" : "hat_mlp12_resid_ln")
                                               : (c144 ? "hat_mlp_resid" : "hat_mlp12_resid");
        launch(s, name, (unsigned)g, 1, 1, MLP_WAVES * 64, p);
        return;
    }
    if (!hidden) throw Error("MLP: the unfused form needs a hidden buffer");
    GemmEpilogue e = ln;
    e.res = res;
    run_gemm(s, fc1, a, fc1.K, M, hidden, fc1.N, EPI_GELU, GemmEpilogue{}, 0, 0, 0.f);
    run_gemm(s, fc2, hidden, fc1.N, M, out, fc2.N, epi, e, 0, 0, 0.f);
}

// Folded CAB, first half: t1 = gelu(conv1(xn)) with its per-tile sums, then
// the gate and the gate-scaled conv2 weights (w2g) and combined bias (bias2 =
// bproj + cscale * gate * b2) for the projection GEMM. With `defer`, the gate
// is not launched: its arguments go to *defer, for the attention launch to run.
void run_cab(hipStream_t s, const DevCab& cb, const float* xn, int H, int W, const float* bproj,
             float cscale, int sq, float* t1, float* partial, float* w2g, float* bias2, float* gate,
             unsigned short* w2gx, CabGateArgs* defer = nullptr)
{
    if (H % 16 != 0 || W % 16 != 0 || H < 16 || W < 16) throw Error("CAB: plane must be 16-aligned");
    if (sq < 1 || sq > 64) throw Error("CAB: squeeze width must be 1..64");
    static const int cus = std::max(1, Runtime::get().cu_count());
    CabConvArgs a{xn, cb.w1, cb.b1, t1, partial, H, W};
    // Persistent over the output tiles, one block of 4 waves per CU: 16 wide x
    // 32 tall when the height allows, else 16 x 16.
    const bool t32 = H % 32 == 0;
    const int tiles = (H / (t32 ? 32 : 16)) * (W / 16);
    launch(s, t32 ? "hat_cab_conv1_t32" : "hat_cab_conv1", (unsigned)std::min(tiles, cus), 1, 1, 256, a);
    CabGateArgs g{};
    g.partial = partial;
    g.t1 = t1;
    g.tiles = tiles;
    g.H = H;
    g.W = W;
    g.w2 = cb.w2;
    g.b2 = cb.b2;
    g.wa = cb.wa;
    g.ba = cb.ba;
    g.wb = cb.wb;
    g.bb = cb.bb;
    g.bproj = bproj;
    g.w2g = w2g;
    g.bias2 = bias2;
    g.gate = gate;
    g.cscale = cscale;
    g.sq = sq;
    g.w2gx = w2gx;
    if (defer) {
        *defer = g;
        return;
    }
    launch(s, "hat_cab_gate", 1, 1, 1, 1024, g);
}

// x' = res + a . proj^T + conv2-segment + bias2; out = x' + MLP(norm2(x'));
// xn = norm_next(out). out may alias res; a, t1 and xn must not overlap out.
// Without t1 (the OCAB): x' = res + a . proj^T + bias2 (the projection bias),
// out = x' + MLP(norm2(x')), no xn.
bool hab_tail_fits(const DevLinear& proj, const DevLinear& fc1, const DevLinear& fc2)
{
    return proj.K == HT_C && proj.Kp == HT_C && proj.N == HT_C && fc1.K == HT_C && fc1.Kp == HT_C &&
           fc1.N == 2 * HT_C && fc2.K == 2 * HT_C && fc2.N == HT_C;
}

void run_hab_tail(hipStream_t s, const DevLinear& proj, const DevLinear& fc1, const DevLinear& fc2,
                  const float* a, const float* res, float* out, float* xn, const float* t1, const float* w2g,
                  const float* bias2, const float* n2w, const float* n2b, const float* nw, const float* nb,
                  int H, int W)
{
    const bool cab = t1 != nullptr;
    if (cab && (!w2g || !xn || !nw || !nb)) throw Error("HAB tail: the CAB form needs w2g and the next norm");
    if (!hab_tail_fits(proj, fc1, fc2)) throw Error("HAB tail: needs the 144 x 144 projection and 144 -> 288 -> 144 MLP");
    const long M = (long)H * W;
    if (M > 0x7fffffffL) throw Error("HAB tail: too many rows");
    HabTailArgs p{};
    p.a = a;
    p.res = res;
    p.out = out;
    p.xn = xn;
    p.wp = proj.w;
    p.w2g = w2g;
    p.bias2 = bias2;
    p.t1 = t1;
    p.n2w = n2w;
    p.n2b = n2b;
    p.w1 = fc1.w;
    p.b1 = fc1.b;
    p.w2 = fc2.w;
    p.b2 = fc2.b;
    p.nw = nw;
    p.nb = nb;
    p.M = (int)M;
    p.H = H;
    p.W = W;
    p.eps = 1e-5f;
    p.ldw1 = fc1.Kp;
    p.ldw2 = fc2.Kp;
    // One block per CU (113 KB of LDS), persistent over the 128-row tiles.
    static const int cus = std::max(1, Runtime::get().cu_count());
    const long ntiles = (M + MLP_ROWS - 1) / MLP_ROWS;
    const long rounds = (ntiles + cus - 1) / cus;
    const long g = std::max(1L, (ntiles + rounds - 1) / rounds);
    launch(s, cab ? "hat_hab_tail" : "hat_ocab_tail", (unsigned)g, 1, 1, MLP_WAVES * 64, p);
}

// The tail on split-bf16 (tailx.hip): x' = res + a . Wp^T (+ CAB: the gated
// conv2 of t1) + bias [hat_projx(_cab)]; out = x' + MLP(norm2(x')), norm2
// formed in the MLP kernel (+ with nw: xn = norm_next(out)) [hat_mlpx(_ln)].
// out may alias res.
void run_tailx(hipStream_t s, bool cab, const DevLinear& proj, const DevMlpX& mlp, const float* b2, const float* a,
               const float* res, float* out, float* xn, const float* t1, const unsigned short* w2gx, const float* bias,
               const float* n2w, const float* n2b, const float* nw, const float* nb, int H, int W)
{
    if (!proj.wx || proj.K != 144 || proj.N != 144) throw Error("tailx: needs the pre-split 144 x 144 projection");
    if (cab && (!t1 || !w2gx)) throw Error("tailx: the CAB form needs t1 and the gated conv2 weight chunks");
    const long M = (long)H * W;
    if (M > 0x7fffffffL) throw Error("tailx: too many rows");
    const unsigned g = (unsigned)wx_tiles((int)M);  // a block per 128-token tile
    if (mlp.wf && cab == (nw != nullptr)) {
        // one kernel, x' kept on the chip (the forms the network runs: the HAB's
        // with the next norm, the OCAB's without)
        TailXArgs f{};
        f.a = a;
        f.res = res;
        f.out = out;
        f.xn = nw ? xn : nullptr;
        f.w = proj.wx;
        f.wm = mlp.wf;
        f.b1x = mlp.b1x;
        f.bias = bias;
        f.b2 = b2;
        f.w2gx = w2gx;
        f.t1 = t1;
        f.inw = n2w;
        f.inb = n2b;
        f.nw = nw;
        f.nb = nb;
        f.M = (int)M;
        f.H = H;
        f.W = W;
        f.eps = 1e-5f;
        launch(s, cab ? "hat_habx_cab_ln" : "hat_habx", g, 1, 1, WX_THREADS, f);
        return;
    }
    // the projection writes x' only: the MLP forms norm2(x') from the x'
    // rows it reads
    TailXArgs p{};
    p.a = a;
    p.res = res;
    p.out = out;
    p.xn = nullptr;
    p.w = proj.wx;
    p.bias = bias;
    p.w2gx = w2gx;
    p.t1 = t1;
    p.nw = n2w;
    p.nb = n2b;
    p.M = (int)M;
    p.H = H;
    p.W = W;
    p.eps = 1e-5f;
    launch(s, cab ? "hat_projx_cab" : "hat_projx", g, 1, 1, WX_THREADS, p);
    TailXArgs q{};
    q.a = out;
    q.res = out;
    q.out = out;
    q.xn = nw ? xn : nullptr;
    q.w = mlp.w;
    q.b2 = b2;
    q.nw = nw;
    q.nb = nb;
    q.inw = n2w;
    q.inb = n2b;
    q.M = (int)M;
    q.H = H;
    q.W = W;
    q.eps = 1e-5f;
    launch(s, nw ? "hat_mlpx_ln" : "hat_mlpx", g, 1, 1, WX_THREADS, q);
}

// The channel-attention gate from the CAB conv's per-tile column sums:
// reduce in fixed row blocks, then squeeze-excite.
// With `defer` (C <= 192, sq <= 64), nothing is launched: *defer gets the
// arguments for the attention launch's first block, which adds the nblk
// partial rows itself.
void run_se(hipStream_t s, const float* partial, int nblk, int C, float* red, float count,
            const float* w1, const float* b1, const float* w2, const float* b2, int sq, float* gate,
            SeArgs* defer = nullptr)
{
    if (defer && C <= 192 && sq >= 1 && sq <= 64) {
        SeArgs se{};
        se.partial = partial;
        se.nblk = nblk;
        se.co_stride = C;
        se.count = count;
        se.w1 = w1;
        se.b1 = b1;
        se.w2 = w2;
        se.b2 = b2;
        se.gate = gate;
        se.C = C;
        se.sq = sq;
        *defer = se;
        return;
    }
    if (defer) defer->gate = nullptr;  // not deferred: launched here
    const int rows_per = 32;
    const int nred = (nblk + rows_per - 1) / rows_per;
    ReduceArgs r{partial, red, nblk, C, C, rows_per};
    launch(s, "hat_colsum_reduce", (unsigned)nred, 1, 1, 256, r);
    SeArgs se{};
    se.partial = red;
    se.nblk = nred;
    se.co_stride = C;
    se.count = count;
    se.w1 = w1;
    se.b1 = b1;
    se.w2 = w2;
    se.b2 = b2;
    se.gate = gate;
    se.C = C;
    se.sq = sq;
    launch(s, "hat_se_gate", 1, 1, 1, 256, se);
}

// The C = 180 CAB conv2 60 -> 180 and its column sums run on the Winograd
// kernel (hat_convwino_cab2_180, one partial row per 8x16 tile); other CO in
// (144, 192] on the wide-tile kernel (one per 16x16 tile); every other
// CEPI_COLSUM conv leaves one per 8x16 tile.
bool colsum_wide(int CO, int H, int W, int co_stride)
{
    return CO > 144 && CO <= 192 && CO != 180 && H % 16 == 0 && W % 16 == 0 && CO % 4 == 0 && co_stride % 4 == 0;
}
int colsum_rows(int CO, int H, int W, int co_stride)
{
    return colsum_wide(CO, H, W, co_stride) ? (W / 16) * (H / 16) : (W / 16) * (H / 8);
}

// [band_r0, band_r1): with band_r1 >= 0, only that band of tile rows is
// launched (the host-memory forward's head): 8 input rows of the Winograd
// upsample conv (hat_convwino_n8_shuffle), 16 output rows of conv_last
// (hat_conv_last3), the same band indices for the two since the shuffle
// doubles the rows. Other convs are always whole planes.
void run_conv(hipStream_t s, const DevConv& C, const float* in, int cin_stride, int H, int W,
              float* out, int co_stride, int epi, int act, const float* res, float* partial,
              int crop_h, int crop_w, float img_range, const float* mean, int band_r0, int band_r1)
{
    if (H % 8 != 0 || W % 16 != 0) throw Error("conv: plane must be a multiple of 8x16");
    const bool band = band_r1 >= 0;
    if (band && (band_r0 < 0 || band_r0 >= band_r1)) throw Error("conv: empty band");
    if (cin_stride % 4 != 0 || cin_stride < C.CI) throw Error("conv: bad input channel stride");
    // The wide-tile kernel (16x16 pixels, a whole 64-, 96- or 128-channel
    // column block per block) for the head convs, the 60-channel CAB conv and
    // the C = 180 trunk convs.
    const char* wide = nullptr;
    int wbn = 0, wwaves = 0;
    if (H % 16 == 0 && W % 16 == 0 && C.CO % 4 == 0 && co_stride % 4 == 0) {
        if (epi == CEPI_STORE && C.CO > 16 && C.CO <= 64) {
            wide = "hat_convw_n4_store";
            wbn = 64;
            wwaves = CONVW_WAVES_N4_STORE;
        } else if (epi == CEPI_SHUFFLE) {
            wide = "hat_convw_n8_shuffle";
            wbn = 128;
            wwaves = CONVW_WAVES_N8_SHUFFLE;
        } else if (epi == CEPI_RESID && C.CO > 144 && C.CO <= 192) {
            wide = "hat_convw_n6_resid";  // C = 180 trunk convs, two 96-channel blocks
            wbn = 96;
            wwaves = CONVW_WAVES_N6_RESID;
        } else if (epi == CEPI_COLSUM && colsum_wide(C.CO, H, W, co_stride)) {
            wide = "hat_convw_n6_colsum";  // C = 180 CAB conv2
            wbn = 96;
            wwaves = CONVW_WAVES_N6_COLSUM;
        }
    }
    const char* name = nullptr;
    int BN = 16;
    switch (epi) {
    case CEPI_STORE:
        if (C.CO <= 16) { name = "hat_conv_n1_store"; BN = 16; }
        else if (C.CO <= 64) { name = "hat_conv_n4_store"; BN = 64; }
        else { name = "hat_conv_n3_store"; BN = 48; }
        break;
    case CEPI_RESID: name = "hat_conv_n3_resid"; BN = 48; break;
    case CEPI_COLSUM: name = "hat_conv_n3_colsum"; BN = 48; break;
    case CEPI_SHUFFLE:
        name = "hat_conv_n4_shuffle";
        BN = 64;
        if ((C.CO / (C.r * C.r)) % 4 != 0) throw Error("conv: shuffled width must be a multiple of 4");
        break;
    case CEPI_FINAL: name = "hat_conv_n1_final"; BN = 16; break;
    default: throw Error("conv: unknown epilogue");
    }
    ConvArgs p{};
    p.in = in;
    p.w = C.w;
    p.bias = C.b;
    p.out = out;
    p.res = res;
    p.partial = partial;
    p.H = H;
    p.W = W;
    p.CI = C.CI;
    p.CIp = C.CIp;
    p.cin_stride = cin_stride;
    p.CO = C.CO;
    p.COp = C.COp;
    p.co_stride = co_stride;
    p.act = act;
    p.r = C.r;
    p.crop_h = crop_h;
    p.crop_w = crop_w;
    p.img_range = img_range;
    if (mean) {
        p.mean0 = mean[0];
        p.mean1 = mean[1];
        p.mean2 = mean[2];
    }
    // conv_before_upsample and the x2 upsample convs by Winograd F(2x2, 3x3):
    // 8 x 16 output tiles, 32-bit element offsets into both planes
    p.wu = C.wu;
    auto wino = [&](const char* name, unsigned tiles, unsigned ncb) { launch_wino(s, name, tiles, ncb, p); };
    const size_t rr = C.r > 0 ? (size_t)C.r * C.r : 1;
    if (C.wu && H % 16 == 0 && W % 16 == 0 && cin_stride % 4 == 0 && cin_stride >= C.CI &&
        (size_t)H * W * cin_stride < ((size_t)1 << 31) && (size_t)H * W * rr * co_stride < ((size_t)1 << 31)) {
        const unsigned tiles = (unsigned)((W / 16) * (H / 8));
        if (epi == CEPI_STORE && act == 2 && C.CO == 64 && C.CI == 144 && co_stride >= 64) {
            wino("hat_convwino_n4_store", tiles, 1);
            return;
        }
        if (epi == CEPI_SHUFFLE && C.r == 2 && C.CO == 256 && C.CI == 64 && co_stride >= 64) {
            unsigned nt = tiles;
            if (band) {
                if (band_r1 > H / 8) throw Error("conv: band past the plane");
                p.tile0 = band_r0 * (W / 16);
                nt = (unsigned)((band_r1 - band_r0) * (W / 16));
            }
            wino("hat_convwino_n8_shuffle", nt, 2);
            return;
        }
        if (band) throw Error("conv: only the Winograd upsample conv and conv_last run in bands");
        // the C = 180 family (the residual epilogue's planes are 180 wide)
        if (epi == CEPI_STORE && act == 2 && C.CO == 64 && C.CI == 180 && co_stride >= 64) {
            wino("hat_convwino_n4_store180", tiles, 1);
            return;
        }
        if (epi == CEPI_STORE && act == 1 && C.CO == 60 && C.CI == 180 && co_stride >= 60) {
            wino("hat_convwino_cab1_180", tiles, 1);
            return;
        }
        if (epi == CEPI_COLSUM && C.CO == 180 && C.CI == 60 && co_stride >= 180) {
            wino("hat_convwino_cab2_180", tiles, 2);
            return;
        }
        if (epi == CEPI_RESID && C.CO == 180 && C.CI == 180 && co_stride == 180) {
            if (in == out) throw Error("conv: the output must not overlap the input");
            wino("hat_convwino_resid180", tiles, 2);
            return;
        }
    }
    if (band && !(epi == CEPI_FINAL && C.CO == 3 && C.CI == 64 && C.CIp == 64 && cin_stride >= 64))
        throw Error("conv: only the Winograd upsample conv and conv_last run in bands");
    if (wide) {
        launch(s, wide, (unsigned)((W / 16) * (H / 16)), (unsigned)((C.CO + wbn - 1) / wbn), 1,
               (unsigned)(wwaves * 64), p);
        return;
    }
    if (epi == CEPI_FINAL) {
        if (crop_h > H || crop_w > W || crop_h < 1 || crop_w < 1) throw Error("conv: bad crop");
        // conv_last 64 -> 3 by per-tap products, 16 x 32 output tiles
        if (C.CO == 3 && C.CI == 64 && C.CIp == 64 && cin_stride >= 64) {
            const int ntx = (W + 31) / 32, nty = (H + 15) / 16;  // 16 x 32 output tiles
            unsigned nt = (unsigned)(ntx * nty);
            if (band) {
                if (band_r1 > nty) throw Error("conv: band past the plane");
                p.tile0 = band_r0 * ntx;
                nt = (unsigned)((band_r1 - band_r0) * ntx);
            }
            launch(s, "hat_conv_last3", nt, 1, 1, 512, p);
            return;
        }
    }
    launch(s, name, (unsigned)((W / 16) * (H / 8)), (unsigned)((C.CO + BN - 1) / BN), 1, 256, p);
}

// A C -> 144 3x3 conv with every output channel in one block and a GEMM
// epilogue: EPI_STORE_LN (out, xn = LN(out)), EPI_RESID_LN (out = conv + res,
// xn = LN(out)) or EPI_RESID. out may alias res; in, out and xn must not overlap.
bool convw_fits(const DevConv& C) { return C.r == 0 && C.CO == 144 && C.COp == 144; }

void run_ln(hipStream_t s, const float* x, float* y, const float* w, const float* b, long rows, int C);

void run_convw(hipStream_t s, const DevConv& C, const float* in, int cin_stride, int H, int W,
               float* out, int epi, const float* res, float* xn, const float* nw, const float* nb)
{
    if (!convw_fits(C)) throw Error("convw: needs 144 output channels");
    if (H % 16 != 0 || W % 16 != 0) throw Error("convw: plane must be 16-aligned");
    if (cin_stride % 4 != 0 || cin_stride < C.CI) throw Error("convw: bad input channel stride");
    const char* name = epi == EPI_STORE_LN   ? "hat_convw_n9_store_ln"
                       : epi == EPI_RESID_LN ? "hat_convw_n9_resid_ln"
                       : epi == EPI_RESID    ? "hat_convw_n9_resid"
                                             : nullptr;
    if (!name) throw Error("convw: bad epilogue");
    const int waves = epi == EPI_STORE_LN   ? CONVW_WAVES_N9_STORE_LN
                      : epi == EPI_RESID_LN ? CONVW_WAVES_N9_RESID_LN
                                            : CONVW_WAVES_N9_RESID;
    ConvArgs p{};
    p.in = in;
    p.w = C.w;
    p.bias = C.b;
    p.out = out;
    p.res = res;
    p.H = H;
    p.W = W;
    p.CI = C.CI;
    p.CIp = C.CIp;
    p.cin_stride = cin_stride;
    p.CO = C.CO;
    p.COp = C.COp;
    p.co_stride = C.CO;
    p.xn = xn;
    p.nw = nw;
    p.nb = nb;
    p.eps = 1e-5f;
    p.wu = C.wu;
    // The 144 -> 144 residual convs by Winograd F(2x2, 3x3): 8 x 16 output
    // tiles, 32-bit element offsets into the input plane. The RHAG conv's
    // LayerNorm follows as its own HBM-bound pass over the just-written rows.
    if (C.wu && C.CI == 144 && (epi == EPI_RESID_LN || epi == EPI_RESID) && H % 8 == 0 &&
        (size_t)H * W * cin_stride < ((size_t)1 << 31)) {
        if (in == out) throw Error("convw: the output must not overlap the input");
        launch_wino(s, "hat_convwino_resid", (unsigned)((W / 16) * (H / 8)), 1, p);
        if (epi == EPI_RESID_LN) run_ln(s, out, xn, nw, nb, (long)H * W, C.CO);
        return;
    }
    launch(s, name, (unsigned)((W / 16) * (H / 16)), 1, 1, (unsigned)(waves * 64), p);
}

void run_attn(hipStream_t s, const float* qkv, const float* table, float* out, const Plan& pl,
              int heads, int D, bool oca, int shift, const CabGateArgs* gate = nullptr,
              const SeArgs* se = nullptr)
{
    if (se && oca) throw Error("attention: the SE gate rides on SW launches only");
    if (gate && oca) throw Error("attention: the CAB gate rides on SW launches only");
    if (pl.win != 16 || pl.owin != 24)
        throw Error("attention: the gfx950 kernels are built for window 16 / overlap window 24");
    // The kernels wrap a rolled coordinate once, upward, and build the SW-MSA
    // mask from bit 3 of the unrolled position: only the plan's half-window
    // shift (or none) is meaningful, and the OCAB has no shift.
    if (!(shift == 0 || (!oca && shift == pl.shift)))
        throw Error("attention: shift " + std::to_string(shift) + " is not supported (0" +
                    (oca ? "" : " or " + std::to_string(pl.shift)) + ")");
    const char* name = nullptr;
    // The split-bf16 kernels (attnx.hip), one (window, head) item per block.
    if (D == 24) {
        name = oca ? "hat_attnx_oca_d24" : "hat_attnx_sw_d24";
    } else if (D == 30) {
        // SW in four parts of 64 keys (two blocks per CU; the whole-item form
        // hat_attnx_sw_d30 needs 114 KB of LDS, one block per CU)
        name = oca ? "hat_attnx_oca_d30" : "hat_attnx_swp_d30";
    } else {
        throw Error("attention: head_dim " + std::to_string(D) + " has no kernel (24 and 30 do)");
    }
    AttnArgs p{};
    p.qkv = qkv;
    p.table = table;
    p.out = out;
    p.hp = pl.hp;
    p.wp = pl.wp;
    p.nx = pl.nx();
    p.ny = pl.ny();
    p.heads = heads;
    p.D = D;
    p.C = heads * D;
    p.shift = shift;
    p.owin = pl.owin;
    p.opad = pl.opad();
    p.T = (int)pl.tokens();
    p.qscale = (1.0f / sqrtf((float)D)) * 1.4426950408889634f;
    if (gate) {
        p.with_gate = 1;
        p.gate = *gate;
    }
    if (se && se->gate) {
        p.with_se = 1;
        p.se = *se;
    }
    launch(s, name, (unsigned)pl.nw(), (unsigned)heads, 1, 512, p);
}

void run_ln(hipStream_t s, const float* x, float* y, const float* w, const float* b, long rows, int C)
{
    if (C > 512) throw Error("layernorm: C > 512");
    LnArgs p{x, y, w, b, (int)rows, C, 1e-5f};
    // 16 rows per block when C % 4 == 0 and C <= 192, else 4 (one per wave)
    const long per = (C % 4 == 0 && C <= 192) ? 16 : 4;
    launch(s, "hat_layernorm", (unsigned)((rows + per - 1) / per), 1, 1, 256, p);
}

}  // namespace

bool convwino_persistent(const std::string& name)
{
    // convwino.hip: the column-sum kernel (the CAB's conv2 at C = 180)
    return name == "hat_convwino_cab2_180";
}

void launch_wino(hipStream_t s, const char* name, unsigned tiles, unsigned ncb, ConvArgs& p, unsigned max_blocks)
{
    static const unsigned cus = (unsigned)std::max(1, Runtime::get().cu_count());
    const unsigned nvb = tiles * ncb;
    if (nvb == 0 || nvb > 0x7fffffffu || ncb == 0) throw Error("convwino: bad tile count");
    const bool persist = convwino_persistent(name);
    const unsigned cap = max_blocks ? max_blocks : cus;
    const unsigned g = persist ? std::max(ncb, std::min(nvb, cap) / ncb * ncb) : nvb;
    p.nblk = persist ? (int)nvb : 0;
    launch(s, name, g, 1, 1, 512, p);
}


// ---------------------------------------------------------------------------
// GpuBackend

float* GpuBackend::upload(const float* src, size_t n)
{
    if (count_only_) {
        weight_bytes_ += n * sizeof(float);
        return nullptr;
    }
    Runtime& rt = Runtime::get();
    float* d = (float*)rt.alloc(n * sizeof(float));
    owned_.push_back(d);
    rt.h2d(d, src, n * sizeof(float));
    weight_bytes_ += n * sizeof(float);
    return d;
}

void* GpuBackend::upload_bytes(const void* src, size_t bytes)
{
    if (count_only_) {
        weight_bytes_ += bytes;
        return nullptr;
    }
    Runtime& rt = Runtime::get();
    void* d = rt.alloc(bytes);
    owned_.push_back(d);
    rt.h2d(d, src, bytes);
    weight_bytes_ += bytes;
    return d;
}

void GpuBackend::upload_raw(const std::string& name)
{
    const TensorInfo& ti = wt_.info(name);
    raw_[name] = upload(wt_.t(name), ti.numel());
}

void GpuBackend::upload_linear(const std::string& name)
{
    const TensorInfo& ti = wt_.info(name + ".weight");
    DevLinear L;
    L.N = (int)ti.shape[0];
    L.K = (int)ti.shape[1];
    std::vector<float> pk = pack_linear(wt_.t(name + ".weight"), L.N, L.K, &L.Kp);
    L.w = upload(pk.data(), pk.size());
    L.b = upload(wt_.t(name + ".bias"), L.N);
    auto ends = [&](const char* t) {
        const size_t n = strlen(t);
        return name.size() >= n && name.compare(name.size() - n, n, t) == 0;
    };
    if (L.K == 180 && L.N == 180 && ends("proj")) {
        // the C = 180 projection tails (hat_projx180*)
        std::vector<unsigned short> x = pack_linear_x180(wt_.t(name + ".weight"));
        L.wx = (unsigned short*)upload_bytes(x.data(), x.size() * sizeof(unsigned short));
    }
    if ((L.K == 180 && L.N == 540 && ends(".qkv")) || (L.K == 144 && ((L.N == 432 && ends(".qkv")) || (L.N == 144 && ends("proj"))))) {
        // qkv: the weight-stationary layout of hat_gemmx_qkv; proj: streamed chunks (tailx)
        std::vector<unsigned short> x = ends(".qkv") ? pack_linear_ws(wt_.t(name + ".weight"), wt_.t(name + ".bias"), L.N, L.K)
                                                     : pack_linear_x(wt_.t(name + ".weight"), L.N, L.K);
        L.wx = (unsigned short*)upload_bytes(x.data(), x.size() * sizeof(unsigned short));
    }
    lin_[name] = L;
}

// The C = 144 MLP, pre-split for hat_mlpx (other widths keep the FP32 kernels).
void GpuBackend::upload_mlpx(const std::string& name)
{
    const TensorInfo& t1 = wt_.info(name + ".fc1.weight");
    const TensorInfo& t2 = wt_.info(name + ".fc2.weight");
    std::vector<unsigned short> w;
    DevMlpX m;
    if (t1.shape == std::vector<size_t>{288, 144} && t2.shape == std::vector<size_t>{144, 288}) {
        pack_mlp_x(wt_.t(name + ".fc1.weight"), wt_.t(name + ".fc1.bias"), wt_.t(name + ".fc2.weight"), &w);
        m.C = 144;
        std::vector<unsigned short> wf;
        std::vector<float> b1x;
        pack_mlp_xf(wt_.t(name + ".fc1.weight"), wt_.t(name + ".fc1.bias"), wt_.t(name + ".fc2.weight"), &wf, &b1x);
        m.wf = (unsigned short*)upload_bytes(wf.data(), wf.size() * sizeof(unsigned short));
        m.b1x = upload(b1x.data(), b1x.size());
    } else if (t1.shape == std::vector<size_t>{360, 180} && t2.shape == std::vector<size_t>{180, 360}) {
        pack_mlp_x180(wt_.t(name + ".fc1.weight"), wt_.t(name + ".fc1.bias"), wt_.t(name + ".fc2.weight"), &w);
        m.C = 180;
        std::vector<unsigned short> wf;
        std::vector<float> b1x;
        pack_mlp_xf180(wt_.t(name + ".fc1.weight"), wt_.t(name + ".fc1.bias"), wt_.t(name + ".fc2.weight"), &wf,
                       &b1x);
        m.wf = (unsigned short*)upload_bytes(wf.data(), wf.size() * sizeof(unsigned short));
        m.b1x = upload(b1x.data(), b1x.size());
    } else {
        return;
    }
    m.w = (unsigned short*)upload_bytes(w.data(), w.size() * sizeof(unsigned short));
    mlpx_[name] = m;
}

void GpuBackend::upload_conv(const std::string& name, int r)
{
    const TensorInfo& ti = wt_.info(name + ".weight");
    DevConv C;
    C.CO = (int)ti.shape[0];
    C.CI = (int)ti.shape[1];
    C.r = r;
    std::vector<float> bias;
    std::vector<float> pk = pack_conv(wt_.t(name + ".weight"), wt_.t(name + ".bias"), C.CO, C.CI, r,
                                      &bias, &C.CIp, &C.COp);
    C.w = upload(pk.data(), pk.size());
    C.b = upload(bias.data(), bias.size());
    if (wino_conv(C.CO, C.CI, r)) {
        std::vector<unsigned short> wu = pack_wino(wt_.t(name + ".weight"), C.CO, C.CI, r);
        C.wu = (unsigned short*)upload_bytes(wu.data(), wu.size() * sizeof(unsigned short));
    }
    conv_[name] = C;
}

// Gpu::new (gpu.rs:372-386): bring up the runtime, then upload every tensor.
GpuBackend::GpuBackend(const Weights& wt) : wt_(wt)
{
    Runtime& rt = Runtime::get();
    check_gpu_weights(wt);
    if (wt.window != 16 || wt.owin != 24)
        throw Error("the gfx950 attention kernels are built for window 16 and overlap window 24");
    if (wt.head_dim != 24 && wt.head_dim != 30)
        throw Error("head_dim " + std::to_string(wt.head_dim) + " has no attention kernel (24, 30)");
    if (wt.embed % 4 != 0 || wt.embed > 512) throw Error("embed_dim must be a multiple of 4, <= 512");
    if (wt.squeezed > 64) throw Error("squeeze width above 64 is not supported");
    if (wt.head_feat % 4 != 0) throw Error("head width must be a multiple of 4");
    for (int d : wt.depths)
        if (d < 1) throw Error("every stage needs at least one HAB");
    cab_fold_ = cab_folded(wt);
    rt.check(rt.api().StreamCreate(&stream_), "hipStreamCreate");
    upload_all();
    if (!wt.device_bytes_cache) wt.device_bytes_cache = weight_bytes_;
}

GpuBackend::GpuBackend(const Weights& wt, CountOnly) : wt_(wt), count_only_(true)
{
    cab_fold_ = cab_folded(wt);
    upload_all();
}

size_t GpuBackend::device_weight_bytes(const Weights& wt)
{
    if (!wt.device_bytes_cache) wt.device_bytes_cache = GpuBackend(wt, CountOnly{}).weight_bytes_;
    return wt.device_bytes_cache;
}

// Every tensor of the network, packed as the kernels read it (Gpu::new's upload,
// gpu.rs:372-386).
void GpuBackend::upload_all()
{
    const Weights& wt = wt_;
    upload_conv("conv_first");
    upload_raw("patch_embed.norm.weight");
    upload_raw("patch_embed.norm.bias");
    for (size_t s = 0; s < wt.depths.size(); ++s) {
        const std::string L = "layers." + std::to_string(s);
        for (int b = 0; b < wt.depths[s]; ++b) {
            const std::string p = L + ".residual_group.blocks." + std::to_string(b);
            for (const char* n : {".norm1.weight", ".norm1.bias", ".norm2.weight", ".norm2.bias",
                                  ".attn.relative_position_bias_table",
                                  ".conv_block.cab.3.attention.1.weight",
                                  ".conv_block.cab.3.attention.1.bias",
                                  ".conv_block.cab.3.attention.3.weight",
                                  ".conv_block.cab.3.attention.3.bias"})
                upload_raw(p + n);
            upload_linear(p + ".attn.qkv");
            upload_linear(p + ".attn.proj");
            upload_linear(p + ".mlp.fc1");
            upload_linear(p + ".mlp.fc2");
            upload_mlpx(p + ".mlp");
            if (cab_fold_) {
                const std::string c = p + ".conv_block.cab.";
                for (const char* n : {"0.bias", "2.weight", "2.bias"}) upload_raw(c + n);
                std::vector<unsigned short> w1 = pack_cab_conv1(wt.t(c + "0.weight"));
                DevCab cb;
                cb.w1 = (unsigned short*)upload_bytes(w1.data(), w1.size() * sizeof(unsigned short));
                cb.b1 = raw_.at(c + "0.bias");
                cb.w2 = raw_.at(c + "2.weight");
                cb.b2 = raw_.at(c + "2.bias");
                cb.wa = raw_.at(c + "3.attention.1.weight");
                cb.ba = raw_.at(c + "3.attention.1.bias");
                cb.wb = raw_.at(c + "3.attention.3.weight");
                cb.bb = raw_.at(c + "3.attention.3.bias");
                cab_[p] = cb;
            } else {
                upload_conv(p + ".conv_block.cab.0");
                upload_conv(p + ".conv_block.cab.2");
            }
        }
        const std::string p = L + ".residual_group.overlap_attn";
        for (const char* n : {".norm1.weight", ".norm1.bias", ".norm2.weight", ".norm2.bias",
                              ".relative_position_bias_table"})
            upload_raw(p + n);
        upload_linear(p + ".qkv");
        upload_linear(p + ".proj");
        upload_linear(p + ".mlp.fc1");
        upload_linear(p + ".mlp.fc2");
        upload_mlpx(p + ".mlp");
        upload_conv(L + ".conv");
    }
    upload_raw("norm.weight");
    upload_raw("norm.bias");
    upload_conv("conv_after_body");
    upload_conv("conv_before_upsample.0");
    const auto blocks = wt.up_blocks();
    for (size_t b = 0; b < blocks.size(); ++b)
        upload_conv("upsample." + std::to_string(2 * b), blocks[b].first);
    upload_conv("conv_last");
}

GpuBackend::~GpuBackend()
{
    if (count_only_) return;
    try {
        Runtime& rt = Runtime::get();
        rt.api().StreamSynchronize(stream_);
        free_batch();
        free_plan();
        for (void* p : owned_) rt.free(p);
        for (hipEvent_t e : band_ev_) rt.api().EventDestroy(e);
        for (hipEvent_t e : copy_ev_) rt.api().EventDestroy(e);
        if (copy_stream_) rt.api().StreamDestroy(copy_stream_);
        rt.api().StreamDestroy(stream_);
    } catch (...) {
    }
}

void GpuBackend::free_plan()
{
    Runtime& rt = Runtime::get();
    free_stage();
    for (void* p : acts_) rt.free(p);
    acts_.clear();
    acts_bytes_ = 0;
    a_ = Acts{};
    have_plan_ = false;
}

// The compress-to-6 CAB at C = 144 (HAT-S) runs folded (cab.hip + habtail.hip).
bool GpuBackend::cab_folded(const Weights& wt) { return wt.embed == CAB_C && wt.compressed == CAB_CC; }

size_t GpuBackend::plan_bytes(const Weights& wt, int h, int w, bool host_io)
{
    Acts a;
    size_t n = 0;
    for (auto& b : layout(wt, Plan::make(h, w, wt.window, wt.embed), a, host_io)) n += b.second * sizeof(float);
    return n;
}

// Acts::new (gpu.rs:293-334): the buffer set of one plan.
std::vector<std::pair<float**, size_t>> GpuBackend::layout(const Weights& wt_, const Plan& p, Acts& a,
                                                           bool host_io)
{
    const size_t T = (size_t)p.tokens(), C = wt_.embed;
    const size_t t1_stride = (size_t)(wt_.compressed + 3) / 4 * 4;
    const size_t nblk = (size_t)colsum_rows((int)C, p.hp, p.wp, (int)C);
    const bool cab_fold_ = cab_folded(wt_);
    // The T x hidden buffer only for MLP shapes without a fused kernel (every
    // block of a network shares one shape: fc1 C -> mlp_ratio * C).
    const bool fused_mlp = wt_.mlp_ratio == 2 && (C == 144 || C == 180);
    // Head ping-pong: the plane at each resolution goes to alternate buffers.
    size_t need[2] = {T * (size_t)wt_.head_feat, 0};
    size_t res = 1;
    int which = 0;
    for (auto& b : wt_.up_blocks()) {
        res *= (size_t)b.first * b.first;
        which ^= 1;
        need[which] = std::max(need[which], T * res * (size_t)wt_.head_feat);
    }
    const size_t s2 = (size_t)wt_.scale * wt_.scale;
    return {
        {&a.x0, T * 4},
        {&a.body, T * C},
        {&a.xa, T * C},
        {&a.xb, T * C},
        {&a.xn, T * C},
        {&a.t1, T * t1_stride},
        {&a.cab_part, cab_fold_ ? (size_t)(p.hp / 16) * (p.wp / 16) * CAB_NSUM * CAB_CS : 0},
        {&a.w2g, cab_fold_ ? C * CAB_K2 : 0},
        {&a.w2gx, cab_fold_ ? WC_CHUNK : 0},  // 2 chunks of bf16
        {&a.bias2, cab_fold_ ? C : 0},
        {&a.t2, cab_fold_ ? 0 : T * C},
        {&a.partial, cab_fold_ ? 0 : nblk * C},
        {&a.red, cab_fold_ ? 0 : (nblk + 31) / 32 * C},
        {&a.gate, C},
        {&a.qkv, 3 * T * C},
        {&a.ao, T * C},
        {&a.hidden, fused_mlp ? 0 : T * C * wt_.mlp_ratio},
        {&a.head0, need[0]},
        {&a.head1, std::max<size_t>(need[1], 4)},
        {&a.din, host_io ? 3 * (size_t)p.h * p.w : 0},
        {&a.dout, host_io ? 3 * (size_t)p.h * p.w * s2 : 0},
    };
}

// One allocation set per plan, reused by every forward at that size. A new
// plan is admitted against the device's free memory first (gpu.rs:766-771).
void GpuBackend::ensure_plan(int h, int w)
{
    Plan p = Plan::make(h, w, wt_.window, wt_.embed);
    if (have_plan_ && p == plan_) return;
    check_gpu(wt_, (size_t)h, (size_t)w);
    free_plan();
    plan_ = p;
    Runtime& rt = Runtime::get();
    t1_stride_ = (wt_.compressed + 3) / 4 * 4;
    nblk_conv2_ = colsum_rows(wt_.embed, p.hp, p.wp, wt_.embed);
    a_ = Acts{};
    for (auto& b : layout(wt_, p, a_, true)) {
        if (b.second == 0) continue;
        float* d = (float*)rt.alloc(b.second * sizeof(float));
        acts_.push_back(d);
        acts_bytes_ += b.second * sizeof(float);
        *b.first = d;
    }
    have_plan_ = true;
}

void GpuBackend::layernorm(const float* x, float* y, const std::string& prefix, long rows)
{
    run_ln(stream_, x, y, raw_.at(prefix + ".weight"), raw_.at(prefix + ".bias"), rows, wt_.embed);
}

void GpuBackend::gemm(const DevLinear& L, const float* a, int lda, long M, float* out, int ldo,
                      int epi, const float* res, const float* aux, const float* gate, float* xn,
                      const std::string& norm)
{
    GemmEpilogue e;
    e.res = res;
    e.aux = aux;
    e.gate = gate;
    e.xn = xn;
    if (!norm.empty()) {
        e.nw = raw_.at(norm + ".weight");
        e.nb = raw_.at(norm + ".bias");
    }
    run_gemm(stream_, L, a, lda, M, out, ldo, epi, e, wt_.heads, wt_.head_dim, wt_.conv_scale);
}

// x = x + fc2(gelu(fc1(a_.xn))), in place; with a norm also a_.xn = norm(x).
// The split-bf16 C = 180 projection tail: out = res + ao . Wp^T + bias (with
// aux: + aux * gate * cscale), and with xn: xn = LN2(out) by (nw, nb).
void run_projx180(hipStream_t s, const DevLinear& proj, const float* ao, const float* res, float* out, float* xn,
                  const float* nw, const float* nb, const float* aux, const float* gate, float cscale, long M)
{
    if (!proj.wx || proj.K != 180 || proj.N != 180) throw Error("projx180: needs the pre-split 180 x 180 projection");
    if (M > 0x7fffffffL) throw Error("projx180: too many rows");
    TailXArgs q{};
    q.a = ao;
    q.res = res;
    q.out = out;
    q.xn = xn;
    q.w = proj.wx;
    q.bias = proj.b;
    q.nw = nw;
    q.nb = nb;
    q.M = (int)M;
    q.eps = 1e-5f;
    q.aux = aux;
    q.gate = gate;
    q.cscale = cscale;
    launch(s, aux ? "hat_projx180_hab" : "hat_projx180", (unsigned)wx_tiles((int)M), 1, 1, WX_THREADS, q);
}

// The split-bf16 C = 180 MLP: x = x + fc2(gelu(fc1(norm2(x)))) + b2 (+ xn =
// LN(x)), norm2 by (n2w, n2b) formed in the kernel from the x rows.
void run_mlpx180(hipStream_t s, const DevMlpX& m, const float* b2, const float* n2w, const float* n2b, float* x,
                 float* xn_out, const float* nw, const float* nb, long M)
{
    if (m.C != 180) throw Error("mlpx180: needs the pre-split C = 180 MLP");
    if (M > 0x7fffffffL) throw Error("mlpx180: too many rows");
    TailXArgs q{};
    q.a = x;
    q.inw = n2w;
    q.inb = n2b;
    q.res = x;
    q.out = x;
    q.xn = nw ? xn_out : nullptr;
    q.w = m.w;
    q.b2 = b2;
    q.nw = nw;
    q.nb = nb;
    q.M = (int)M;
    q.eps = 1e-5f;
    launch(s, nw ? "hat_mlpx180_ln" : "hat_mlpx180", (unsigned)wx_tiles((int)M), 1, 1, WX_THREADS, q);
}

// The C = 180 tail: with the fused weights and a form hat_habx180* has (the
// HAB's with the unfolded CAB's gated conv2 output aux and the next norm, the
// OCAB's with neither) one kernel with x' kept on the chip; otherwise the
// projection writes x' (hat_projx180*) and the MLP forms norm2(x') from the
// rows it reads (hat_mlpx180*). out may alias res.
void run_tailx180(hipStream_t s, const DevLinear& proj, const DevMlpX& mlp, const float* b2, const float* ao,
                  const float* res, float* out, float* xn, const float* n2w, const float* n2b, const float* aux,
                  const float* gate, float cscale, const float* nw, const float* nb, long M)
{
    if (!proj.wx || proj.K != 180 || proj.N != 180 || mlp.C != 180)
        throw Error("tailx180: needs the pre-split C = 180 projection and MLP");
    if (M > 0x7fffffffL) throw Error("tailx180: too many rows");
    if (mlp.wf && mlp.b1x && (aux != nullptr) == (nw != nullptr)) {
        TailXArgs f{};
        f.a = ao;
        f.res = res;
        f.out = out;
        f.xn = nw ? xn : nullptr;
        f.w = proj.wx;
        f.wm = mlp.wf;
        f.b1x = mlp.b1x;
        f.bias = proj.b;
        f.b2 = b2;
        f.aux = aux;
        f.gate = gate;
        f.cscale = cscale;
        f.inw = n2w;
        f.inb = n2b;
        f.nw = nw;
        f.nb = nb;
        f.M = (int)M;
        f.eps = 1e-5f;
        launch(s, aux ? "hat_habx180_hab_ln" : "hat_habx180", (unsigned)wx_tiles((int)M), 1, 1, WX_THREADS, f);
        return;
    }
    run_projx180(s, proj, ao, res, out, nullptr, n2w, n2b, aux, gate, cscale, M);
    run_mlpx180(s, mlp, b2, n2w, n2b, out, xn, nw, nb, M);
}

void GpuBackend::mlp(const std::string& prefix, float* x, int epi, const std::string& norm)
{
    GemmEpilogue e;
    if (!norm.empty()) {
        e.xn = a_.xn;
        e.nw = raw_.at(norm + ".weight");
        e.nb = raw_.at(norm + ".bias");
    }
    run_mlp(stream_, lin_.at(prefix + ".fc1"), lin_.at(prefix + ".fc2"), a_.xn, plan_.tokens(), x, x, epi,
            e, a_.hidden);
}

void GpuBackend::conv(const DevConv& C, const float* in, int cin_stride, int H, int W, float* out,
                      int co_stride, int epi, int act, const float* res, float* partial,
                      int crop_h, int crop_w, int band_r0, int band_r1)
{
    run_conv(stream_, C, in, cin_stride, H, W, out, co_stride, epi, act, res, partial, crop_h,
             crop_w, wt_.img_range, wt_.mean, band_r0, band_r1);
}

void GpuBackend::attention(const std::string& table, bool oca, int shift, const CabGateArgs* gate,
                           const SeArgs* se)
{
    run_attn(stream_, a_.qkv, raw_.at(table), a_.ao, plan_, wt_.heads, wt_.head_dim, oca, shift, gate, se);
}

// HAB.forward (hat_arch.py:266-309; cpu.rs:1090-1166):
//   x = shortcut + attn(norm1 x) + conv_x * conv_scale;  x = x + mlp(norm2 x)
// On entry a_.xn holds norm1(x_in); on exit x_out holds the block's result and
// a_.xn holds next_norm(x_out), the input of whatever block follows.
void GpuBackend::hab(int stage, int block, float* x_in, float* x_out, const std::string& next_norm)
{
    const std::string p = "layers." + std::to_string(stage) + ".residual_group.blocks." +
                          std::to_string(block);
    const long T = plan_.tokens();
    const int C = wt_.embed, H = plan_.hp, W = plan_.wp;
    if (cab_fold_) {
        // CAB, folded: conv1 + GELU here, the gate inside the attention
        // launch (its first block), conv2 inside the tail's projection.
        const DevLinear& proj = lin_.at(p + ".attn.proj");
        CabGateArgs gate{};
        run_cab(stream_, cab_.at(p), a_.xn, H, W, proj.b, wt_.conv_scale, wt_.squeezed, a_.t1, a_.cab_part,
                a_.w2g, a_.bias2, a_.gate, (unsigned short*)a_.w2gx, &gate);
        gemm(lin_.at(p + ".attn.qkv"), a_.xn, C, T, a_.qkv, 0, EPI_QKV);
        attention(p + ".attn.relative_position_bias_table", false, block % 2 == 1 ? plan_.shift : 0, &gate);
        auto mx = mlpx_.find(p + ".mlp");
        if (proj.wx && C == 144 && mx != mlpx_.end()) {
            // split-bf16: proj + gated conv2 + shortcut + norm2, then the MLP + next norm1
            run_tailx(stream_, true, proj, mx->second, lin_.at(p + ".mlp.fc2").b, a_.ao, x_in, x_out, a_.xn, a_.t1,
                      (const unsigned short*)a_.w2gx, a_.bias2, raw_.at(p + ".norm2.weight"), raw_.at(p + ".norm2.bias"),
                      raw_.at(next_norm + ".weight"), raw_.at(next_norm + ".bias"), H, W);
            return;
        }
        run_hab_tail(stream_, proj, lin_.at(p + ".mlp.fc1"), lin_.at(p + ".mlp.fc2"), a_.ao, x_in, x_out, a_.xn, a_.t1,
                     a_.w2g, a_.bias2, raw_.at(p + ".norm2.weight"), raw_.at(p + ".norm2.bias"),
                     raw_.at(next_norm + ".weight"), raw_.at(next_norm + ".bias"), H, W);
        return;
    }
    // CAB: conv3x3 -> GELU -> conv3x3 (+ per-tile channel sums) -> gate.
    conv(conv_.at(p + ".conv_block.cab.0"), a_.xn, C, H, W, a_.t1, t1_stride_, CEPI_STORE, 1);
    conv(conv_.at(p + ".conv_block.cab.2"), a_.t1, t1_stride_, H, W, a_.t2, C, CEPI_COLSUM, 0, nullptr,
         a_.partial);
    // The gate: computed by the attention launch's first block where it fits.
    SeArgs se{};
    run_se(stream_, a_.partial, nblk_conv2_, C, a_.red, (float)T,
           raw_.at(p + ".conv_block.cab.3.attention.1.weight"),
           raw_.at(p + ".conv_block.cab.3.attention.1.bias"),
           raw_.at(p + ".conv_block.cab.3.attention.3.weight"),
           raw_.at(p + ".conv_block.cab.3.attention.3.bias"), wt_.squeezed, a_.gate, &se);
    // Window attention, the roll and the partition folded into its addressing;
    // proj's epilogue adds the shortcut and the gated conv branch, then norm2.
    gemm(lin_.at(p + ".attn.qkv"), a_.xn, C, T, a_.qkv, 0, EPI_QKV);
    attention(p + ".attn.relative_position_bias_table", false, block % 2 == 1 ? plan_.shift : 0, nullptr, &se);
    const DevLinear& proj = lin_.at(p + ".attn.proj");
    auto mx = mlpx_.find(p + ".mlp");
    if (proj.wx && C == 180 && mx != mlpx_.end() && mx->second.C == 180) {
        // split-bf16: projection + gated conv branch + shortcut, norm2, the
        // MLP + residual + next norm
        run_tailx180(stream_, proj, mx->second, lin_.at(p + ".mlp.fc2").b, a_.ao, x_in, x_out, a_.xn,
                     raw_.at(p + ".norm2.weight"), raw_.at(p + ".norm2.bias"), a_.t2, a_.gate, wt_.conv_scale,
                     next_norm.empty() ? nullptr : raw_.at(next_norm + ".weight"),
                     next_norm.empty() ? nullptr : raw_.at(next_norm + ".bias"), T);
        return;
    }
    gemm(proj, a_.ao, C, T, x_out, C, EPI_HAB_LN, x_in, a_.t2, a_.gate, a_.xn, p + ".norm2");
    mlp(p + ".mlp", x_out, EPI_RESID_LN, next_norm);
}

// OCAB.forward (hat_arch.py:392-438; cpu.rs:1170-1198): x = proj(attn) + x;
// x = x + mlp(norm2 x). On entry a_.xn holds norm1(x).
void GpuBackend::ocab(int stage, float* x)
{
    const std::string p = "layers." + std::to_string(stage) + ".residual_group.overlap_attn";
    const long T = plan_.tokens();
    const int C = wt_.embed;
    gemm(lin_.at(p + ".qkv"), a_.xn, C, T, a_.qkv, 0, EPI_QKV);
    attention(p + ".relative_position_bias_table", true, 0);
    const DevLinear& proj = lin_.at(p + ".proj");
    const DevLinear &fc1 = lin_.at(p + ".mlp.fc1"), &fc2 = lin_.at(p + ".mlp.fc2");
    auto mx = mlpx_.find(p + ".mlp");
    if (proj.wx && C == 144 && mx != mlpx_.end()) {
        // split-bf16: projection + shortcut + norm2, then the MLP + residual
        run_tailx(stream_, false, proj, mx->second, fc2.b, a_.ao, x, x, a_.xn, nullptr, nullptr, proj.b,
                  raw_.at(p + ".norm2.weight"), raw_.at(p + ".norm2.bias"), nullptr, nullptr, plan_.hp, plan_.wp);
        return;
    }
    if (hab_tail_fits(proj, fc1, fc2)) {
        // projection + shortcut + norm2 + MLP + residual in one kernel
        run_hab_tail(stream_, proj, fc1, fc2, a_.ao, x, x, nullptr, nullptr,
                     nullptr, proj.b, raw_.at(p + ".norm2.weight"), raw_.at(p + ".norm2.bias"), nullptr, nullptr,
                     plan_.hp, plan_.wp);
        return;
    }
    if (proj.wx && C == 180 && mx != mlpx_.end() && mx->second.C == 180) {
        run_tailx180(stream_, proj, mx->second, fc2.b, a_.ao, x, x, nullptr, raw_.at(p + ".norm2.weight"),
                     raw_.at(p + ".norm2.bias"), nullptr, nullptr, 0.0f, nullptr, nullptr, T);
        return;
    }
    gemm(proj, a_.ao, C, T, x, C, EPI_RESID_LN, x, nullptr, nullptr, a_.xn, p + ".norm2");
    mlp(p + ".mlp", x, EPI_RESID, "");
}

// forward_planes (gpu.rs:714-748; cpu.rs:1318-1368) with Pre::adjust and finish
// (backend.rs:71-109) folded into the first and last kernels.
void GpuBackend::forward_device(int h, int w, const float* d_in, float* d_out)
{
    if (h <= 0 || w <= 0) throw Error(std::to_string(h) + "x" + std::to_string(w) + " is empty");
    ensure_plan(h, w);
    run_forward(h, w, d_in, d_out);
}

size_t GpuBackend::noalloc_bytes(int h, int w) const
{
    if (h <= 0 || w <= 0) throw Error(std::to_string(h) + "x" + std::to_string(w) + " is empty");
    Acts a;
    size_t off = 0;
    for (auto& b : layout(wt_, Plan::make(h, w, wt_.window, wt_.embed), a, false))
        if (b.second) off += (b.second * sizeof(float) + 255) / 256 * 256;
    return off;
}

// forward_device with the per-plan buffers carved, 256-byte aligned, from the
// scratch array the code object holds (hipModuleGetGlobal at start-up), in
// place of the plan's own allocations, which are left as they are.
void GpuBackend::forward_noalloc(int h, int w, const float* d_in, float* d_out)
{
    if (h <= 0 || w <= 0) throw Error(std::to_string(h) + "x" + std::to_string(w) + " is empty");
    if (!d_in || !d_out) throw Error("null argument");
    Runtime& rt = Runtime::get();
    const Plan p = Plan::make(h, w, wt_.window, wt_.embed);
    // 64 KiB of the array stay unused past the last buffer, so no buffer ends
    // at the array's end.
    const size_t need = noalloc_bytes(h, w), cap = rt.scratch_bytes() - (64u << 10);
    if (need > cap) {
        char m[192];
        snprintf(m, sizeof m, "forward_noalloc: a %dx%d forward needs %.1f MiB of scratch; the library's "
                 "fixed array holds %.1f MiB", h, w, need / 1048576.0, cap / 1048576.0);
        throw Error(m);
    }
    Acts a;
    char* base = (char*)rt.scratch();
    size_t off = 0;
    for (auto& b : layout(wt_, p, a, false)) {
        if (b.second == 0) continue;
        *b.first = (float*)(base + off);
        off += (b.second * sizeof(float) + 255) / 256 * 256;
    }
    const Acts saved = a_;
    const Plan saved_plan = plan_;
    const int saved_nblk = nblk_conv2_;
    a_ = a;
    plan_ = p;
    t1_stride_ = (wt_.compressed + 3) / 4 * 4;
    nblk_conv2_ = colsum_rows(wt_.embed, p.hp, p.wp, wt_.embed);
    try {
        run_forward(h, w, d_in, d_out);
    } catch (...) {
        a_ = saved;
        plan_ = saved_plan;
        nblk_conv2_ = saved_nblk;
        throw;
    }
    a_ = saved;
    plan_ = saved_plan;
    nblk_conv2_ = saved_nblk;
}

// The forward on the current plan's buffers (a_, plan_).
void GpuBackend::run_forward(int h, int w, const float* d_in, float* d_out, std::vector<std::pair<int, int>>* bands)
{
    const long T = plan_.tokens();
    const int C = wt_.embed, H = plan_.hp, W = plan_.wp;
    PreArgs pa{d_in, a_.x0, h, w, H, W, 4, wt_.mean[0], wt_.mean[1], wt_.mean[2], wt_.img_range};
    launch(stream_, "hat_pre", (unsigned)((T + 255) / 256), 1, 1, 256, pa);
    const DevConv& cf = conv_.at("conv_first");
    // With 144 channels the trunk convs carry the LayerNorm that follows them.
    const bool fused = convw_fits(cf);
    if ((C == 144 || C == 180) && cf.CI == 3 && cf.CIp == 16 && cf.CO == C && cf.r == 0 && H % 16 == 0 &&
        W % 16 == 0) {
        // conv_first + patch_embed.norm as one K = 27 GEMM (convfirst.hip)
        ConvArgs p{};
        p.in = a_.x0;
        p.w = cf.w;
        p.bias = cf.b;
        p.out = a_.body;
        p.xn = a_.xa;
        p.nw = raw_.at("patch_embed.norm.weight");
        p.nb = raw_.at("patch_embed.norm.bias");
        p.H = H;
        p.W = W;
        p.CI = cf.CI;
        p.CIp = cf.CIp;
        p.cin_stride = 4;
        p.CO = C;
        p.COp = cf.COp;
        p.co_stride = C;
        p.eps = 1e-5f;
        launch(stream_, C == 144 ? "hat_conv_first_ln144" : "hat_conv_first_ln180", (unsigned)((W / 16) * (H / 16)), 1,
               1, 256, p);
    } else if (fused) {
        run_convw(stream_, cf, a_.x0, 4, H, W, a_.body, EPI_STORE_LN, nullptr, a_.xa,
                  raw_.at("patch_embed.norm.weight"), raw_.at("patch_embed.norm.bias"));
    } else {
        conv(cf, a_.x0, 4, H, W, a_.body, C, CEPI_STORE, 0);
        layernorm(a_.body, a_.xa, "patch_embed.norm", T);
    }
    const size_t S = wt_.depths.size();
    for (size_t s = 0; s < S; ++s) {
        // RHAG (gpu.rs:592-610): conv3x3(blocks(x)) + x, with the stage input
        // kept in a_.xa and the blocks working in a_.xb. Each block's last GEMM
        // leaves the next block's norm1 in a_.xn; the first block's comes from
        // the previous stage's conv (or its own pass).
        const std::string L = "layers." + std::to_string(s) + ".residual_group.";
        if (!fused || s == 0) layernorm(a_.xa, a_.xn, L + "blocks.0.norm1", T);
        for (int b = 0; b < wt_.depths[s]; ++b) {
            const std::string next = b + 1 < wt_.depths[s]
                                         ? L + "blocks." + std::to_string(b + 1) + ".norm1"
                                         : L + "overlap_attn.norm1";
            hab((int)s, b, b == 0 ? a_.xa : a_.xb, a_.xb, next);
        }
        ocab((int)s, a_.xb);
        const DevConv& rc = conv_.at("layers." + std::to_string(s) + ".conv");
        if (fused) {
            // x = conv(blocks) + x, then the next stage's norm1 or the final
            // norm into a_.xn (a_.xb, the conv's input, is still being read).
            const std::string nn = s + 1 < S ? "layers." + std::to_string(s + 1) + ".residual_group.blocks.0.norm1"
                                             : std::string("norm");
            run_convw(stream_, rc, a_.xb, C, H, W, a_.xa, EPI_RESID_LN, a_.xa, a_.xn, raw_.at(nn + ".weight"),
                      raw_.at(nn + ".bias"));
        } else {
            conv(rc, a_.xb, C, H, W, a_.xa, C, CEPI_RESID, 0, a_.xa);
        }
    }
    if (fused) {
        run_convw(stream_, conv_.at("conv_after_body"), a_.xn, C, H, W, a_.xa, EPI_RESID, a_.body, nullptr,
                  nullptr, nullptr);
    } else {
        layernorm(a_.xa, a_.xb, "norm", T);
        conv(conv_.at("conv_after_body"), a_.xb, C, H, W, a_.xa, C, CEPI_RESID, 0, a_.body);
    }
    // Head (gpu.rs:622-653): conv + LeakyReLU, [conv + PixelShuffle] per block, conv_last.
    const int feat = wt_.head_feat;
    conv(conv_.at("conv_before_upsample.0"), a_.xa, C, H, W, a_.head0, feat, CEPI_STORE, 2);
    float* cur = a_.head0;
    float* nxt = a_.head1;
    int hh = H, ww = W;
    const auto blocks = wt_.up_blocks();
    const DevConv& last = conv_.at("conv_last");
    const int oh = h * wt_.scale, ow = w * wt_.scale;
    for (size_t b = 0; b < blocks.size(); ++b) {
        const DevConv& up = conv_.at("upsample." + std::to_string(2 * b));
        if (bands && b + 1 == blocks.size() && head_bands_fit(up, last, hh, ww, feat)) {
            // The last upsample conv and conv_last over bands of tile rows
            // (eighths of the plane, the last one split in two, so that the
            // first download starts early and the last one is short),
            // conv_last's band k after the upsample's band k + 1 (its halo
            // row below), an event after each conv_last band.
            const int R = hh / 8, step = (R + 7) / 8;  // at most 8 steps + the split: 10 bands
            std::vector<int> bnd{0};
            while (bnd.back() + step < R) bnd.push_back(bnd.back() + step);
            if (R - bnd.back() >= 2) bnd.push_back(bnd.back() + (R - bnd.back()) / 2);
            bnd.push_back(R);
            const int nb = (int)bnd.size() - 1;
            if (nb > (int)band_ev_.size()) throw Error("forward: too many output bands");
            bands->clear();
            conv(up, cur, feat, hh, ww, nxt, feat, CEPI_SHUFFLE, 0, nullptr, nullptr, 0, 0, bnd[0], bnd[1]);
            for (int k = 0; k < nb; ++k) {
                if (k + 1 < nb)
                    conv(up, cur, feat, hh, ww, nxt, feat, CEPI_SHUFFLE, 0, nullptr, nullptr, 0, 0, bnd[k + 1],
                         bnd[k + 2]);
                conv(last, nxt, feat, 2 * hh, 2 * ww, d_out, 0, CEPI_FINAL, 0, nullptr, nullptr, oh, ow, bnd[k],
                     bnd[k + 1]);
                Runtime::get().check(Runtime::get().api().EventRecord(band_ev_[k], stream_), "hipEventRecord");
                bands->emplace_back(std::min(oh, 16 * bnd[k]), std::min(oh, 16 * bnd[k + 1]));
            }
            return;
        }
        conv(up, cur, feat, hh, ww, nxt, feat, CEPI_SHUFFLE, 0);
        hh *= blocks[b].first;
        ww *= blocks[b].first;
        std::swap(cur, nxt);
    }
    conv(last, cur, feat, hh, ww, d_out, 0, CEPI_FINAL, 0, nullptr, nullptr, oh, ow);
    if (bands) {
        // one band: the whole output
        if (band_ev_.empty()) throw Error("forward: no band events");
        Runtime::get().check(Runtime::get().api().EventRecord(band_ev_[0], stream_), "hipEventRecord");
        bands->assign(1, {0, oh});
    }
}

// Whether the head's last upsample conv (input hh x ww) and conv_last run on
// the kernels that take bands of tile rows: the Winograd x2 upsample and the
// 64 -> 3 conv_last, whose 16-row tiles are the upsample's 8-row tiles doubled.
bool GpuBackend::head_bands_fit(const DevConv& up, const DevConv& last, int hh, int ww, int feat) const
{
    return up.wu && up.r == 2 && up.CO == 256 && up.CI == 64 && feat == 64 && hh % 16 == 0 && ww % 16 == 0 &&
           (size_t)hh * ww * feat < ((size_t)1 << 31) && (size_t)hh * ww * 4 * feat < ((size_t)1 << 31) &&
           last.CO == 3 && last.CI == 64 && last.CIp == 64;
}

void GpuBackend::op_hab(int stage, int block, int hp, int wp, const float* x, float* out, int iters,
                        float* ms)
{
    if (!x || !out) throw Error("hab: null argument");
    if (stage < 0 || stage >= (int)wt_.depths.size())
        throw Error("hab: stage " + std::to_string(stage) + " of " + std::to_string(wt_.depths.size()));
    if (block < 0 || block >= wt_.depths[stage])
        throw Error("hab: block " + std::to_string(block) + " of " + std::to_string(wt_.depths[stage]) +
                    " in stage " + std::to_string(stage));
    if (hp <= 0 || wp <= 0 || hp % wt_.window || wp % wt_.window)
        throw Error("hab: the plane must be a non-empty window multiple");
    ensure_plan(hp, wp);
    Runtime& rt = Runtime::get();
    const HipApi& api = rt.api();
    const long T = plan_.tokens();
    const size_t bytes = (size_t)T * wt_.embed * sizeof(float);
    const std::string p = "layers." + std::to_string(stage) + ".residual_group.blocks." + std::to_string(block);
    rt.h2d(a_.xa, x, bytes);
    // norm1 into a_.xn, then the block from a_.xa into a_.xb. The block also writes
    // the next norm's output into a_.xn; its own norm1 stands in for it.
    auto run = [&]() {
        layernorm(a_.xa, a_.xn, p + ".norm1", T);
        hab(stage, block, a_.xa, a_.xb, p + ".norm1");
    };
    run();
    rt.check(api.StreamSynchronize(stream_), "hab");
    rt.d2h(out, a_.xb, bytes);
    if (iters > 0 && ms) {
        hipEvent_t a = nullptr, b = nullptr;
        rt.check(api.EventCreate(&a), "hipEventCreate");
        rt.check(api.EventCreate(&b), "hipEventCreate");
        api.EventRecord(a, stream_);
        for (int i = 0; i < iters; ++i) run();
        api.EventRecord(b, stream_);
        rt.check(api.EventSynchronize(b), "hab timing");
        float e = 0.f;
        api.EventElapsedTime(&e, a, b);
        *ms = e / iters;
        api.EventDestroy(a);
        api.EventDestroy(b);
    }
}

void GpuBackend::free_batch()
{
    Runtime& rt = Runtime::get();
    for (BatchSlot& sl : batch_) {
        if (sl.s) {
            rt.api().StreamSynchronize(sl.s);
            rt.api().StreamDestroy(sl.s);
        }
        if (sl.hin) rt.api().HostFree(sl.hin);
        if (sl.hout) rt.api().HostFree(sl.hout);
    }
    batch_.clear();
    for (void* p : batch_dev_) rt.free(p);
    batch_dev_.clear();
}

void GpuBackend::forward_batch(int n, int h, int w, const float* in, float* out)
{
    if (n <= 0 || h <= 0 || w <= 0) throw Error("forward_batch: empty batch or image");
    if (!in || !out) throw Error("forward_batch: null argument");
    Runtime& rt = Runtime::get();
    const HipApi& api = rt.api();
    const size_t s2 = (size_t)wt_.scale * wt_.scale;
    const size_t isz = 3 * (size_t)h * w, osz = isz * s2;
    const int slots = std::min(n, kBatchSlots);
    const Plan p = Plan::make(h, w, wt_.window, wt_.embed);
    if (!(batch_plan_ == p) || (int)batch_.size() < slots) {
        free_batch();
        // admission for all the slots' buffers at once (the weights are already up)
        const MemPlan mp = gpu_plan(wt_, (size_t)h, (size_t)w);
        const uint64_t need = (uint64_t)((double)mp.activations * kSlack) * slots + mp.base;
        if (mp.have_avail && need > mp.avail)
            throw Error("not enough video memory for a batch of " + std::to_string(slots) + " concurrent " +
                        std::to_string(w) + "x" + std::to_string(h) + " passes: about " + fmt_bytes(need) +
                        " needed, " + fmt_bytes(mp.avail) + " free");
        batch_plan_ = p;
        batch_.resize(slots);
        for (BatchSlot& sl : batch_) {
            rt.check(api.StreamCreate(&sl.s), "hipStreamCreate");
            for (auto& b : layout(wt_, p, sl.a, true)) {
                if (b.second == 0) continue;
                float* d = (float*)rt.alloc(b.second * sizeof(float));
                batch_dev_.push_back(d);
                *b.first = d;
            }
            rt.check(api.HostMalloc((void**)&sl.hin, isz * sizeof(float), 0), "hipHostMalloc");
            rt.check(api.HostMalloc((void**)&sl.hout, osz * sizeof(float), 0), "hipHostMalloc");
        }
    }
    // Swap a slot's stream and buffers in for run_forward, which only enqueues.
    const hipStream_t own_stream = stream_;
    const Acts own_acts = a_;
    const Plan own_plan = plan_;
    const int own_nblk = nblk_conv2_;
    auto restore = [&]() {
        stream_ = own_stream;
        a_ = own_acts;
        plan_ = own_plan;
        nblk_conv2_ = own_nblk;
    };
    auto drain = [&](BatchSlot& sl) {
        if (sl.img < 0) return;
        rt.check(api.StreamSynchronize(sl.s), "forward_batch");
        memcpy(out + (size_t)sl.img * osz, sl.hout, osz * sizeof(float));
        sl.img = -1;
    };
    try {
        for (int i = 0; i < n; ++i) {
            BatchSlot& sl = batch_[i % slots];
            drain(sl);
            memcpy(sl.hin, in + (size_t)i * isz, isz * sizeof(float));
            rt.check(api.MemcpyAsync(sl.a.din, sl.hin, isz * sizeof(float), hipMemcpyHostToDevice, sl.s),
                     "hipMemcpyAsync H2D");
            stream_ = sl.s;
            a_ = sl.a;
            plan_ = p;
            t1_stride_ = (wt_.compressed + 3) / 4 * 4;
            nblk_conv2_ = colsum_rows(wt_.embed, p.hp, p.wp, wt_.embed);
            run_forward(h, w, sl.a.din, sl.a.dout);
            restore();
            rt.check(api.MemcpyAsync(sl.hout, sl.a.dout, osz * sizeof(float), hipMemcpyDeviceToHost, sl.s),
                     "hipMemcpyAsync D2H");
            sl.img = i;
        }
        for (BatchSlot& sl : batch_) drain(sl);
    } catch (...) {
        restore();
        for (BatchSlot& sl : batch_) {
            api.StreamSynchronize(sl.s);
            sl.img = -1;
        }
        throw;
    }
}

void GpuBackend::free_stage()
{
    Runtime& rt = Runtime::get();
    if (copy_stream_) rt.api().StreamSynchronize(copy_stream_);
    if (stage_in_) rt.api().HostFree(stage_in_);
    if (stage_out_) rt.api().HostFree(stage_out_);
    stage_in_ = stage_out_ = nullptr;
    stage_in_n_ = stage_out_n_ = 0;
}

namespace {
// Host threads of Backend::forward: each copies its share of the input into
// pinned memory, and of every output band out of it.
constexpr unsigned kStageThreads = 8;
constexpr int kMaxBands = 10;
}  // namespace

// Backend::forward (backend.rs:29-36, gpu.rs:759-803): host [3][h][w] in, host
// [3][h*s][w*s] out. Eight host threads copy the input into a pinned buffer
// (each an eighth), which goes up in one DMA. The head's last convs run in
// bands of output rows (run_forward), each band downloaded into a pinned buffer
// on a second stream as soon as its event fires, while the GPU computes the
// next bands; the threads copy each band to `out` as its download completes.
// So the 50 MB download of a 512 x 512 x4 forward overlaps the last upsample
// conv, and only the last band's download and copy (1/16 of the output) follow
// the forward. (A pageable hipMemcpy would stage through the runtime's own
// bounce buffers one piece at a time, after the whole forward.)
void GpuBackend::forward(int h, int w, const float* in, float* out)
{
    if (h <= 0 || w <= 0) throw Error(std::to_string(h) + "x" + std::to_string(w) + " is empty");
    if (!in || !out) throw Error("forward: null argument");
    ensure_plan(h, w);
    Runtime& rt = Runtime::get();
    const HipApi& api = rt.api();
    const size_t oh = (size_t)h * wt_.scale, ow = (size_t)w * wt_.scale;
    const size_t in_bytes = 3 * (size_t)h * w * sizeof(float), plane_bytes = oh * ow * sizeof(float);
    if (stage_in_n_ != in_bytes || stage_out_n_ != 3 * plane_bytes) {
        free_stage();
        rt.check(api.HostMalloc((void**)&stage_in_, in_bytes, 0), "hipHostMalloc");
        stage_in_n_ = in_bytes;
        rt.check(api.HostMalloc((void**)&stage_out_, 3 * plane_bytes, 0), "hipHostMalloc");
        stage_out_n_ = 3 * plane_bytes;
    }
    if (!copy_stream_) rt.check(api.StreamCreate(&copy_stream_), "hipStreamCreate");
    while (band_ev_.size() < (size_t)kMaxBands) {
        hipEvent_t a = nullptr, b = nullptr;
        rt.check(api.EventCreateWithFlags(&a, hipEventDisableTiming), "hipEventCreate");
        band_ev_.push_back(a);
        rt.check(api.EventCreateWithFlags(&b, hipEventDisableTiming), "hipEventCreate");
        copy_ev_.push_back(b);
    }

    constexpr unsigned T = kStageThreads;
    std::vector<std::pair<int, int>> bands;  // output rows, in the order they are written
    std::atomic<unsigned> in_done{0};
    std::atomic<int> queued{0};  // 1: every band's download is queued; -1: queueing failed
    std::vector<hipError_t> err(T, hipSuccess);
    // thread t's share [a, b) of n bytes, in 64-byte units
    auto share = [](size_t n, unsigned t) {
        const size_t u = (n + 63) / 64;
        return std::make_pair(std::min(n, u * t / T * 64), std::min(n, u * (t + 1) / T * 64));
    };
    auto copy_in = [&](unsigned t) {
        const auto r = share(in_bytes, t);
        memcpy((char*)stage_in_ + r.first, (const char*)in + r.first, r.second - r.first);
        in_done.fetch_add(1, std::memory_order_release);
    };
    auto copy_out = [&](unsigned t) {
        int q;
        while ((q = queued.load(std::memory_order_acquire)) == 0) std::this_thread::yield();
        if (q < 0) return;
        for (size_t k = 0; k < bands.size(); ++k) {
            const hipError_t e = api.EventSynchronize(copy_ev_[k]);
            if (e != hipSuccess) {
                err[t] = e;
                return;
            }
            const size_t row = ow * sizeof(float), len = (size_t)(bands[k].second - bands[k].first) * row;
            const auto r = share(len, t);
            for (int c = 0; c < 3; ++c) {
                const size_t off = c * plane_bytes + (size_t)bands[k].first * row + r.first;
                memcpy((char*)out + off, (const char*)stage_out_ + off, r.second - r.first);
            }
        }
    };
    auto worker = [&](unsigned t) {
        copy_in(t);
        copy_out(t);
    };
    std::vector<std::thread> pool;
    try {
        // inside the try: if a thread cannot be started, the ones that were are
        // released (queued = -1) and joined below, not destroyed while joinable
        for (unsigned t = 1; t < T; ++t) pool.emplace_back(worker, t);
        copy_in(0);
        while (in_done.load(std::memory_order_acquire) < T) std::this_thread::yield();
        rt.check(api.MemcpyAsync(a_.din, stage_in_, in_bytes, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync H2D");
        run_forward(h, w, a_.din, a_.dout, &bands);
        for (size_t k = 0; k < bands.size(); ++k) {
            rt.check(api.StreamWaitEvent(copy_stream_, band_ev_[k], 0), "hipStreamWaitEvent");
            // the band's rows of the three planes: one 2D copy (a copy per
            // plane measured 25-45 us apart on the copy engine)
            const size_t row = ow * sizeof(float), len = (size_t)(bands[k].second - bands[k].first) * row;
            const size_t off = (size_t)bands[k].first * row;
            if (len > 0)
                rt.check(api.Memcpy2DAsync((char*)stage_out_ + off, plane_bytes, (const char*)a_.dout + off,
                                           plane_bytes, len, 3, hipMemcpyDeviceToHost, copy_stream_),
                         "hipMemcpy2DAsync D2H");
            rt.check(api.EventRecord(copy_ev_[k], copy_stream_), "hipEventRecord");
        }
    } catch (...) {
        queued.store(-1, std::memory_order_release);
        for (std::thread& th : pool) th.join();
        api.StreamSynchronize(stream_);
        api.StreamSynchronize(copy_stream_);
        throw;
    }
    queued.store(1, std::memory_order_release);
    copy_out(0);
    for (std::thread& th : pool) th.join();
    rt.check(api.StreamSynchronize(stream_), "forward");
    rt.check(api.StreamSynchronize(copy_stream_), "forward: download");
    for (hipError_t e : err) rt.check(e, "forward: download");
}

// ---------------------------------------------------------------------------
// Isolated ops.

namespace {

struct DevBuf {
    float* p = nullptr;
    DevBuf(size_t n) { p = (float*)Runtime::get().alloc(n * sizeof(float)); }
    DevBuf(const float* src, size_t n) : DevBuf(n) { Runtime::get().h2d(p, src, n * sizeof(float)); }
    ~DevBuf() { Runtime::get().free(p); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
};

// Device copy of a host bf16 array (DevBuf's units are floats).
static std::unique_ptr<DevBuf> dev_u16(const std::vector<unsigned short>& v)
{
    std::unique_ptr<DevBuf> d(new DevBuf((v.size() + 1) / 2));
    Runtime::get().h2d(d->p, v.data(), v.size() * sizeof(unsigned short));
    return d;
}

// A linear of the op entry points, packed as the backend packs it
// (upload_linear): the FP32 rows, and for the shapes a split-bf16 kernel
// takes (the qkv of 144 / 180 channels, the 144 / 180 projection) the split
// weights too, so that an op runs the forward's kernels.
struct OpLinear {
    enum Split { kNone, kQkv, kProj };
    DevBuf w, b;
    std::unique_ptr<DevBuf> x;
    DevLinear L;
    OpLinear(const float* wt, const float* bias, int N, int K, Split sp = kNone) : w(1), b(bias, N)
    {
        L.N = N;
        L.K = K;
        std::vector<float> pk = pack_linear(wt, N, K, &L.Kp);
        Runtime::get().free(w.p);
        w.p = (float*)Runtime::get().alloc(pk.size() * sizeof(float));
        Runtime::get().h2d(w.p, pk.data(), pk.size() * sizeof(float));
        L.w = w.p;
        L.b = b.p;
        std::vector<unsigned short> xs;
        if (sp == kQkv && ((N == 432 && K == 144) || (N == 540 && K == 180)))
            xs = pack_linear_ws(wt, bias, N, K);
        else if (sp == kProj && N == 144 && K == 144)
            xs = pack_linear_x(wt, N, K);
        else if (sp == kProj && N == 180 && K == 180)
            xs = pack_linear_x180(wt);
        if (!xs.empty()) {
            x = dev_u16(xs);
            L.wx = (unsigned short*)x->p;
        }
    }
};

// An op's MLP pre-split for hat_mlpx (C = 144) or hat_mlpx180 (C = 180), as
// upload_mlpx packs it; other shapes leave m.w null (the FP32 kernels).
struct OpMlpX {
    std::unique_ptr<DevBuf> buf, fbuf, bbuf;
    DevMlpX m;
    OpMlpX(const float* w1, const float* b1, const float* w2, int c, size_t hid)
    {
        std::vector<unsigned short> w, wf;
        std::vector<float> b1x;
        if (c == 144 && hid == 288) {
            pack_mlp_x(w1, b1, w2, &w);
            pack_mlp_xf(w1, b1, w2, &wf, &b1x);
        } else if (c == 180 && hid == 360) {
            pack_mlp_x180(w1, b1, w2, &w);
            pack_mlp_xf180(w1, b1, w2, &wf, &b1x);
        } else {
            return;
        }
        fbuf = dev_u16(wf);
        m.wf = (unsigned short*)fbuf->p;
        bbuf.reset(new DevBuf(b1x.data(), b1x.size()));
        m.b1x = bbuf->p;
        m.C = c;
        buf = dev_u16(w);
        m.w = (unsigned short*)buf->p;
    }
};

struct Timer {
    hipEvent_t a = nullptr, b = nullptr;
    Timer()
    {
        const HipApi& api = Runtime::get().api();
        api.EventCreate(&a);
        api.EventCreate(&b);
    }
    ~Timer()
    {
        const HipApi& api = Runtime::get().api();
        api.EventDestroy(a);
        api.EventDestroy(b);
    }
};

}  // namespace

void op_swmsa(const float* x, float* out, int hp, int wp, int c, int heads, int shift,
              const float* qkv_w, const float* qkv_b, const float* proj_w, const float* proj_b,
              const float* table, int iters, float* ms, float* attn_ms)
{
    // Arguments are checked before the runtime is touched.
    if (!x || !out || !qkv_w || !qkv_b || !proj_w || !proj_b || !table) throw Error("swmsa: null argument");
    if (hp <= 0 || wp <= 0 || c <= 0 || heads <= 0) throw Error("swmsa: empty plane or no channels");
    if ((size_t)hp * wp > (1u << 26) || c > 4096) throw Error("swmsa: plane or channels too large");  // int token counts
    if (c % heads) throw Error("swmsa: c must be divisible by heads");
    const int D = c / heads;
    if (D != 24 && D != 30) throw Error("swmsa: head_dim " + std::to_string(D) + " has no kernel (24, 30)");
    Plan pl = Plan::make(hp, wp, 16, c);
    if (pl.hp != hp || pl.wp != wp) throw Error("swmsa: the plane must be a window multiple");
    if (shift != 0 && shift != pl.shift)
        throw Error("swmsa: shift " + std::to_string(shift) + " is not supported (0 or " +
                    std::to_string(pl.shift) + ")");
    Runtime& rt = Runtime::get();
    const HipApi& api = rt.api();
    const size_t T = (size_t)hp * wp;
    hipStream_t s = nullptr;
    rt.check(api.StreamCreate(&s), "hipStreamCreate");
    {
        DevBuf dx(x, T * c), dq(3 * T * c), dao(T * c), dout(T * c), dtab(table, 961 * (size_t)heads);
        // qkv as in the forward; the projection here has no residual, a form the
        // forward never runs, so it stays on the FP32 store epilogue
        OpLinear qkv(qkv_w, qkv_b, 3 * c, c, OpLinear::kQkv), proj(proj_w, proj_b, c, c);
        const GemmEpilogue none;
        auto run = [&]() {
            run_gemm(s, qkv.L, dx.p, c, (long)T, dq.p, 0, EPI_QKV, none, heads, D, 0.f);
            run_attn(s, dq.p, dtab.p, dao.p, pl, heads, D, false, shift);
            run_gemm(s, proj.L, dao.p, c, (long)T, dout.p, c, EPI_STORE, none, heads, D, 0.f);
        };
        run();
        rt.check(api.StreamSynchronize(s), "swmsa");
        if (iters > 0 && (ms || attn_ms)) {
            Timer t, ta;
            api.EventRecord(t.a, s);
            for (int i = 0; i < iters; ++i) run();
            api.EventRecord(t.b, s);
            api.EventRecord(ta.a, s);
            for (int i = 0; i < iters; ++i) run_attn(s, dq.p, dtab.p, dao.p, pl, heads, D, false, shift);
            api.EventRecord(ta.b, s);
            rt.check(api.EventSynchronize(ta.b), "swmsa timing");
            float e = 0.f;
            api.EventElapsedTime(&e, t.a, t.b);
            if (ms) *ms = e / iters;
            api.EventElapsedTime(&e, ta.a, ta.b);
            if (attn_ms) *attn_ms = e / iters;
        }
        rt.d2h(out, dout.p, T * c * sizeof(float));
    }
    api.StreamDestroy(s);
}

void op_ocab(const float* x, float* out, int hp, int wp, int c, int heads, int mlp_ratio,
             const float* n1w, const float* n1b, const float* qkv_w, const float* qkv_b,
             const float* proj_w, const float* proj_b, const float* table, const float* n2w,
             const float* n2b, const float* fc1_w, const float* fc1_b, const float* fc2_w,
             const float* fc2_b, int iters, float* ms, float* attn_ms)
{
    if (!x || !out || !n1w || !n1b || !qkv_w || !qkv_b || !proj_w || !proj_b || !table || !n2w || !n2b ||
        !fc1_w || !fc1_b || !fc2_w || !fc2_b)
        throw Error("ocab: null argument");
    if (hp <= 0 || wp <= 0 || c <= 0 || heads <= 0 || mlp_ratio <= 0) throw Error("ocab: empty plane or no channels");
    if ((size_t)hp * wp > (1u << 26) || c > 4096) throw Error("ocab: plane or channels too large");  // int token counts
    if (c % heads) throw Error("ocab: c must be divisible by heads");
    const int D = c / heads;
    if (D != 24 && D != 30) throw Error("ocab: head_dim " + std::to_string(D) + " has no kernel (24, 30)");
    Plan pl = Plan::make(hp, wp, 16, c);
    if (pl.hp != hp || pl.wp != wp) throw Error("ocab: the plane must be a window multiple");
    Runtime& rt = Runtime::get();
    const HipApi& api = rt.api();
    const size_t T = (size_t)hp * wp, hid = (size_t)c * mlp_ratio;
    hipStream_t s = nullptr;
    rt.check(api.StreamCreate(&s), "hipStreamCreate");
    {
        DevBuf dx(x, T * c), dwork(T * c), dxn(T * c), dq(3 * T * c), dao(T * c), dh(T * hid),
            dtab(table, 1521 * (size_t)heads), d1w(n1w, c), d1b(n1b, c), d2w(n2w, c), d2b(n2b, c);
        OpLinear qkv(qkv_w, qkv_b, 3 * c, c, OpLinear::kQkv), proj(proj_w, proj_b, c, c, OpLinear::kProj),
            fc1(fc1_w, fc1_b, (int)hid, c), fc2(fc2_w, fc2_b, c, (int)hid);
        const OpMlpX mx(fc1_w, fc1_b, fc2_w, c, hid);
        const GemmEpilogue none;
        GemmEpilogue resid_ln;
        resid_ln.res = dx.p;
        resid_ln.xn = dxn.p;
        resid_ln.nw = d2w.p;
        resid_ln.nb = d2b.p;
        // The backend's OCAB sequence (GpuBackend::ocab): norm1, qkv, attention,
        // proj + shortcut (which also writes norm2), then the MLP + residual.
        auto run = [&]() {
            run_ln(s, dx.p, dxn.p, d1w.p, d1b.p, (long)T, c);
            run_gemm(s, qkv.L, dxn.p, c, (long)T, dq.p, 0, EPI_QKV, none, heads, D, 0.f);
            run_attn(s, dq.p, dtab.p, dao.p, pl, heads, D, true, 0);
            if (proj.L.wx && mx.m.w && c == 144) {
                run_tailx(s, false, proj.L, mx.m, fc2.L.b, dao.p, dx.p, dwork.p, dxn.p, nullptr, nullptr, proj.L.b,
                          d2w.p, d2b.p, nullptr, nullptr, hp, wp);
            } else if (proj.L.wx && mx.m.w && c == 180) {
                run_tailx180(s, proj.L, mx.m, fc2.L.b, dao.p, dx.p, dwork.p, nullptr, d2w.p, d2b.p, nullptr, nullptr, 0.f,
                             nullptr, nullptr, (long)T);
            } else {
                run_gemm(s, proj.L, dao.p, c, (long)T, dwork.p, c, EPI_RESID_LN, resid_ln, heads, D, 0.f);
                run_mlp(s, fc1.L, fc2.L, dxn.p, (long)T, dwork.p, dwork.p, EPI_RESID, none, dh.p);
            }
        };
        run();
        rt.check(api.StreamSynchronize(s), "ocab");
        rt.d2h(out, dwork.p, T * c * sizeof(float));
        if (iters > 0 && (ms || attn_ms)) {
            Timer t, ta;
            api.EventRecord(t.a, s);
            for (int i = 0; i < iters; ++i) run();
            api.EventRecord(t.b, s);
            api.EventRecord(ta.a, s);
            for (int i = 0; i < iters; ++i) run_attn(s, dq.p, dtab.p, dao.p, pl, heads, D, true, 0);
            api.EventRecord(ta.b, s);
            rt.check(api.EventSynchronize(ta.b), "ocab timing");
            float e = 0.f;
            api.EventElapsedTime(&e, t.a, t.b);
            if (ms) *ms = e / iters;
            api.EventElapsedTime(&e, ta.a, ta.b);
            if (attn_ms) *attn_ms = e / iters;
        }
    }
    api.StreamDestroy(s);
}

}  // namespace hat
