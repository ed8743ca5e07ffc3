// The kernel selftest: every gfx950 kernel against a host twin on seeded
// inputs, the contract of the reference's `--cuda-selftest` (src/selftest.rs:
// 437-523). Movement and integer work is compared exactly; floating-point
// kernels against a double-precision twin within a stated tolerance. The twins
// use the reference's own geometry formulas (plan.rs: window_index with the
// roll, unfold_index, the calculate_mask bands, rpi_sa, rpi_oca) rather than
// the kernels' folded forms, so an addressing shortcut that is wrong fails here.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "gpu.h"
#include "kargs.h"

namespace hat {

using namespace hatk;

namespace {

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    float uni()  // [-1, 1)
    {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return (float)((s >> 40) * (1.0 / 16777216.0)) * 2.0f - 1.0f;
    }
    std::vector<float> vec(size_t n, float scale)
    {
        std::vector<float> v(n);
        for (auto& x : v) x = uni() * scale;
        return v;
    }
};

struct Dev {
    float* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t n_) : n(n_) { p = (float*)Runtime::get().alloc(n * sizeof(float)); }
    Dev(const std::vector<float>& v) : Dev(v.size()) { Runtime::get().h2d(p, v.data(), n * sizeof(float)); }
    ~Dev() { Runtime::get().free(p); }
    std::vector<float> get() const
    {
        std::vector<float> v(n);
        Runtime::get().sync();
        Runtime::get().d2h(v.data(), p, n * sizeof(float));
        return v;
    }
    Dev(const Dev&) = delete;
};

void check_close(const std::string& name, const std::vector<float>& got, const std::vector<double>& want,
                 double tol)
{
    if (got.size() != want.size()) throw Error(name + ": size mismatch");
    double worst = 0;
    size_t at = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        double d = std::fabs((double)got[i] - want[i]);
        if (!std::isfinite((double)got[i])) throw Error(name + ": non-finite value at " + std::to_string(i));
        if (d > worst) {
            worst = d;
            at = i;
        }
    }
    if (worst > tol) {
        char b[256];
        snprintf(b, sizeof b, "%s: worst |diff| %.3e at %zu (got %.9e, want %.9e), tolerance %.0e",
                 name.c_str(), worst, at, got[at], want[at], tol);
        throw Error(b);
    }
}

// mask_label (plan.rs:300-334): region of pixel (y, x) from the three bands.
int band(int v, int len, int win, int shift)
{
    const int a = len - win > 0 ? len - win : 0, b = len - shift > 0 ? len - shift : 0;
    return v < a ? 0 : (v < b ? 1 : 2);
}

// Host twin of the fused attention, in double.
std::vector<double> attn_twin(const std::vector<float>& qkv, const std::vector<float>& table,
                              int hp, int wp, int heads, int D, bool oca, int shift)
{
    const int C = heads * D, T = hp * wp, nx = wp / 16, ny = hp / 16;
    const int nk = oca ? 576 : 256;
    std::vector<double> out((size_t)T * C, 0.0);
    const double scale = 1.0 / std::sqrt((double)D);
    auto Q = [&](int which, int hd, int pix, int d) { return (double)qkv[(((size_t)which * heads + hd) * T + pix) * D + d]; };
    for (int wy = 0; wy < ny; ++wy)
        for (int wx = 0; wx < nx; ++wx)
            for (int hd = 0; hd < heads; ++hd)
                for (int q = 0; q < 256; ++q) {
                    const int qy = q / 16, qx = q % 16;
                    const int qpy = (wy * 16 + qy + shift) % hp, qpx = (wx * 16 + qx + shift) % wp;
                    const int qpix = qpy * wp + qpx;
                    std::vector<double> s(nk);
                    double mx = -1e300;
                    for (int k = 0; k < nk; ++k) {
                        int kpix = -1, bidx;
                        if (oca) {
                            const int ky = k / 24, kx = k % 24;
                            const int y = wy * 16 - 4 + ky, x = wx * 16 - 4 + kx;
                            if (y >= 0 && y < hp && x >= 0 && x < wp) kpix = y * wp + x;
                            int raw = (ky - qy - 7) * 39 + (kx - qx - 7);
                            bidx = ((raw % 1521) + 1521) % 1521;
                        } else {
                            const int ky = k / 16, kx = k % 16;
                            kpix = ((wy * 16 + ky + shift) % hp) * wp + (wx * 16 + kx + shift) % wp;
                            bidx = (qy - ky + 15) * 31 + (qx - kx + 15);
                        }
                        double dot = 0;
                        if (kpix >= 0)
                            for (int d = 0; d < D; ++d) dot += Q(0, hd, qpix, d) * Q(1, hd, kpix, d);
                        double v = dot * scale + table[(size_t)bidx * heads + hd];
                        if (!oca && shift > 0) {
                            const int ky = k / 16, kx = k % 16;
                            const int lq = band(wy * 16 + qy, hp, 16, shift) * 3 + band(wx * 16 + qx, wp, 16, shift);
                            const int lk = band(wy * 16 + ky, hp, 16, shift) * 3 + band(wx * 16 + kx, wp, 16, shift);
                            if (lq != lk) v -= 100.0;
                        }
                        s[k] = v;
                        if (v > mx) mx = v;
                    }
                    double sum = 0;
                    for (int k = 0; k < nk; ++k) sum += (s[k] = std::exp(s[k] - mx));
                    for (int d = 0; d < D; ++d) {
                        double acc = 0;
                        for (int k = 0; k < nk; ++k) {
                            int kpix = -1;
                            if (oca) {
                                const int y = wy * 16 - 4 + k / 24, x = wx * 16 - 4 + k % 24;
                                if (y >= 0 && y < hp && x >= 0 && x < wp) kpix = y * wp + x;
                            } else {
                                kpix = ((wy * 16 + k / 16 + shift) % hp) * wp + (wx * 16 + k % 16 + shift) % wp;
                            }
                            if (kpix >= 0) acc += s[k] * Q(2, hd, kpix, d);
                        }
                        out[(size_t)qpix * C + hd * D + d] = acc / sum;
                    }
                }
    return out;
}

double gelu_d(double v) { return 0.5 * v * (1.0 + std::erf(v / std::sqrt(2.0))); }

}  // namespace

int gpu_selftest(std::string* err)
{
    int passed = 0;
    auto note = [&](const std::string& n) {
        printf("  ok  %s\n", n.c_str());
        fflush(stdout);
        ++passed;
    };
    try {
        Runtime& rt = Runtime::get();
        hipStream_t s = nullptr;
        printf("gpu selftest - every kernel against a host twin (%s, %d CUs, %zu kernels)\n",
               rt.device_name().c_str(), rt.cu_count(), rt.kernel_names().size());
        Rng rng(7);

        // ---- attention: both head dims, SW plain / shifted (masked) and OCA,
        // on a non-square 2 x 3 window grid and a single-window plane.
        for (int D : {24, 30})
            for (auto geo : {std::pair<int, int>{32, 48}, std::pair<int, int>{16, 16}})
                for (int mode = 0; mode < 3; ++mode) {
                    const int hp = geo.first, wp = geo.second, heads = 2, T = hp * wp;
                    const bool oca = mode == 2;
                    const int shift = mode == 1 ? 8 : 0;
                    std::vector<float> qkv = rng.vec((size_t)3 * T * heads * D, 1.0f);
                    std::vector<float> tab = rng.vec((size_t)(oca ? 1521 : 961) * heads, 0.5f);
                    Dev dq(qkv), dt(tab), dout((size_t)T * heads * D);
                    Plan pl = Plan::make(hp, wp, 16, heads * D);
                    AttnArgs p{};
                    p.qkv = dq.p;
                    p.table = dt.p;
                    p.out = dout.p;
                    p.hp = hp;
                    p.wp = wp;
                    p.nx = pl.nx();
                    p.ny = pl.ny();
                    p.heads = heads;
                    p.D = D;
                    p.C = heads * D;
                    p.shift = shift;
                    p.owin = 24;
                    p.opad = 4;
                    p.T = T;
                    p.qscale = (float)(1.0 / std::sqrt((double)D) * 1.4426950408889634);
                    std::vector<double> want = attn_twin(qkv, tab, hp, wp, heads, D, oca, shift);
                    // the FP32-MFMA kernel and the split-bf16 ones (SW head_dim 30:
                    // the whole-item form and the part-staged one the forward runs)
                    for (const char* fam : {oca ? "hat_attn_oca_d" : "hat_attn_sw_d", oca ? "hat_attnx_oca_d" : "hat_attnx_sw_d",
                                            oca ? "" : "hat_attnx_swp_d"}) {
                        if (!*fam || (std::string(fam) == "hat_attnx_swp_d" && D != 30)) continue;
                        std::string k = std::string(fam) + std::to_string(D);
                        const bool xk = k.find("attnx") != std::string::npos;
                        if (!xk && attn_persistent(D, oca))  // 3 blocks, so a block walks several items
                            launch(s, k.c_str(), 3, 1, 1, 512, p);
                        else
                            launch(s, k.c_str(), pl.nw(), heads, 1, 512, p);
                        char nm[128];
                        snprintf(nm, sizeof nm, "%s %dx%d shift %d", k.c_str(), hp, wp, shift);
                        check_close(nm, dout.get(), want, 2e-5);
                        note(nm);
                    }
                }

        // ---- GEMM epilogues (n9: the C = 144 family; n12: C = 180). The
        // LayerNorm epilogues also check the normalised rows they write.
        const int epis[6] = {EPI_STORE, EPI_GELU, EPI_QKV, EPI_RESID, EPI_RESID_LN, EPI_HAB_LN};
        const char* enames[7] = {"store", "gelu", "qkv", "resid", "", "resid_ln", "hab_ln"};
        // ws: the weight-stationary kernels (K = 144; K = 180 padded to 192, whose
        // last K chunk must not read past a row's 180 values), on 600 rows (3 or
        // 5 row tiles, the last one partial) with two blocks per column slice, so
        // a block walks several tiles.
        auto gemm_case = [&](int C, int epi, bool ws) {
                const int heads = 6, hd = C / heads;
                const int M = ws ? 600 : 200;  // not a multiple of the row tile
                const int N = epi == EPI_QKV ? 3 * C : (epi == EPI_GELU ? 2 * C : C);
                const int K = epi == EPI_RESID ? 2 * C : C;  // RESID at the fc2 shape
                const bool lnout = epi == EPI_RESID_LN || epi == EPI_HAB_LN;
                std::vector<float> a = rng.vec((size_t)M * K, 1.0f), w = rng.vec((size_t)N * K, 0.05f),
                                   b = rng.vec(N, 0.1f), res = rng.vec((size_t)M * N, 1.0f),
                                   aux = rng.vec((size_t)M * N, 1.0f), gate = rng.vec(N, 1.0f),
                                   nw = rng.vec(N, 1.0f), nb = rng.vec(N, 0.1f);
                int Kp = 0;
                std::vector<float> pk = pack_linear(w.data(), N, K, &Kp);
                Dev da(a), dw(pk), db(b), dres(res), daux(aux), dg(gate), dnw(nw), dnb(nb),
                    dout((size_t)M * N), dxn((size_t)M * N);
                GemmArgs p{};
                p.a = da.p;
                p.w = dw.p;
                p.bias = db.p;
                p.out = dout.p;
                p.res = dres.p;
                p.aux = daux.p;
                p.gate = dg.p;
                p.xn = dxn.p;
                p.nw = dnw.p;
                p.nb = dnb.p;
                p.M = M;
                p.N = N;
                p.K = K;
                p.Kp = Kp;
                p.lda = K;
                p.ldo = N;
                p.heads = heads;
                p.hdim = hd;
                p.cscale = 0.01f;
                p.eps = 1e-5f;
                const bool n9 = N % 144 == 0;
                const int BN = n9 ? 144 : 192;
                std::string k;
                if (ws) {
                    const int wbn = C == 144 ? 144 : 192;
                    k = std::string(C == 144 ? "hat_gemmws_" : "hat_gemmws12_") + enames[epi];
                    // 2 blocks: with 3 column slices each block's units
                    // cross from slice to slice
                    (void)wbn;
                    launch(s, k.c_str(), 2, 1, 1, ws_waves(epi) * 64, p);
                } else {
                    k = std::string(n9 ? "hat_gemm_n9_" : "hat_gemm_n12_") + enames[epi];
                    launch(s, k.c_str(), (M + 127) / 128, (N + BN - 1) / BN, 1, 256, p);
                }
                std::vector<double> want((size_t)M * N), wxn((size_t)M * N);
                for (int m = 0; m < M; ++m) {
                    for (int n = 0; n < N; ++n) {
                        double v = b[n];
                        for (int kk = 0; kk < K; ++kk) v += (double)a[(size_t)m * K + kk] * w[(size_t)n * K + kk];
                        const size_t o = (size_t)m * N + n;
                        if (epi == EPI_GELU) v = gelu_d(v);
                        if (epi == EPI_RESID || epi == EPI_RESID_LN) v = res[o] + v;
                        if (epi == EPI_HAB_LN) v = (res[o] + v) + aux[o] * gate[n] * 0.01;
                        if (epi == EPI_QKV) {
                            const int which = n / C, rem = n % C, h = rem / hd, d = rem % hd;
                            want[(((size_t)which * heads + h) * M + m) * hd + d] = v;
                        } else {
                            want[o] = v;
                        }
                    }
                    if (lnout) {
                        double mean = 0, var = 0;
                        for (int n = 0; n < N; ++n) mean += want[(size_t)m * N + n];
                        mean /= N;
                        for (int n = 0; n < N; ++n) var += (want[(size_t)m * N + n] - mean) * (want[(size_t)m * N + n] - mean);
                        var /= N;
                        for (int n = 0; n < N; ++n)
                            wxn[(size_t)m * N + n] = (want[(size_t)m * N + n] - mean) / std::sqrt(var + 1e-5) * nw[n] + nb[n];
                    }
                }
                check_close(k + " C " + std::to_string(C), dout.get(), want, 3e-5);
                if (lnout) check_close(k + " C " + std::to_string(C) + " layernorm", dxn.get(), wxn, 5e-5);
                note(k + " C " + std::to_string(C) + " M " + std::to_string(M) + " K " + std::to_string(K));
                if (ws && epi == EPI_QKV) {
                    // the split-bf16 form on the same inputs (the last
                    // subtile partial: 600 rows are 18.75 subtiles of 32 at
                    // C = 144, 12.5 of 48 at C = 180), one group: its 8 waves
                    // walk them all
                    std::vector<unsigned short> px = pack_linear_ws(w.data(), b.data(), N, K);
                    Dev dwx(std::vector<float>((px.size() + 1) / 2)), dout2((size_t)M * N);
                    rt.h2d(dwx.p, px.data(), px.size() * sizeof(unsigned short));
                    GemmArgs px2 = p;
                    px2.w = dwx.p;
                    px2.out = dout2.p;
                    const char* kx = C == 144 ? "hat_gemmx_qkv" : "hat_gemmx_qkv180";
                    launch(s, kx, C == 144 ? 3 : 6, 1, 1, GX_THREADS, px2);
                    check_close(std::string(kx) + " C " + std::to_string(C), dout2.get(), want, 3e-5);
                    note(std::string(kx) + " C " + std::to_string(C) + " M " + std::to_string(M) + " K " + std::to_string(K));
                }
        };
        for (int C : {144, 180})
            for (int epi : epis) gemm_case(C, epi, false);
        for (int C : {144, 180})
            for (int epi : {EPI_QKV, EPI_GELU, EPI_RESID_LN, EPI_HAB_LN}) gemm_case(C, epi, true);

        // ---- fused MLP (C = 144, hidden 288; C = 180, hidden 360 padded to
        // 384), in place as the backend runs it: out aliases the residual, the
        // LayerNorm output aliases the input. 600 rows = 5 tiles of 128 (the
        // last partial) over 2 blocks.
        for (int C : {144, 180})
        for (int epi : {EPI_RESID, EPI_RESID_LN}) {
            const int M = 600, H = 2 * C;
            std::vector<float> a = rng.vec((size_t)M * C, 1.0f), w1 = rng.vec((size_t)H * C, 0.08f),
                               b1 = rng.vec(H, 0.1f), w2 = rng.vec((size_t)C * H, 0.06f), b2 = rng.vec(C, 0.1f),
                               res = rng.vec((size_t)M * C, 1.0f), nw = rng.vec(C, 1.0f), nb = rng.vec(C, 0.1f);
            int K1 = 0, K2 = 0;
            std::vector<float> p1 = pack_linear(w1.data(), H, C, &K1), p2 = pack_linear(w2.data(), C, H, &K2);
            Dev da(a), dw1(p1), db1(b1), dw2(p2), db2(b2), dx(res), dnw(nw), dnb(nb);
            MlpArgs p{};
            p.a = da.p;
            p.w1 = dw1.p;
            p.b1 = db1.p;
            p.w2 = dw2.p;
            p.b2 = db2.p;
            p.res = dx.p;
            p.out = dx.p;
            p.xn = epi == EPI_RESID_LN ? da.p : nullptr;
            p.nw = dnw.p;
            p.nb = dnb.p;
            p.M = M;
            p.eps = 1e-5f;
            p.K = C;
            p.H = H;
            p.N = C;
            p.ldw1 = K1;
            p.ldw2 = K2;
            const char* k = epi == EPI_RESID_LN ? (C == 144 ? "hat_mlp_resid_ln" : "hat_mlp12_resid_ln")
                                                : (C == 144 ? "hat_mlp_resid" : "hat_mlp12_resid");
            launch(s, k, 2, 1, 1, MLP_WAVES * 64, p);
            std::vector<double> want((size_t)M * C), wxn((size_t)M * C), hid(H);
            for (int m = 0; m < M; ++m) {
                for (int j = 0; j < H; ++j) {
                    double v = b1[j];
                    for (int c = 0; c < C; ++c) v += (double)a[(size_t)m * C + c] * w1[(size_t)j * C + c];
                    hid[j] = gelu_d(v);
                }
                double mean = 0, var = 0;
                for (int n = 0; n < C; ++n) {
                    double v = b2[n];
                    for (int j = 0; j < H; ++j) v += hid[j] * w2[(size_t)n * H + j];
                    want[(size_t)m * C + n] = res[(size_t)m * C + n] + v;
                    mean += want[(size_t)m * C + n];
                }
                mean /= C;
                for (int n = 0; n < C; ++n) var += (want[(size_t)m * C + n] - mean) * (want[(size_t)m * C + n] - mean);
                var /= C;
                for (int n = 0; n < C; ++n)
                    wxn[(size_t)m * C + n] = (want[(size_t)m * C + n] - mean) / std::sqrt(var + 1e-5) * nw[n] + nb[n];
            }
            check_close(std::string(k), dx.get(), want, 5e-5);
            if (epi == EPI_RESID_LN) check_close(std::string(k) + " layernorm", da.get(), wxn, 5e-5);
            note(std::string(k) + " C " + std::to_string(C) + " M 600 (in place)");
            if (C == 180) {
                // the split-bf16 form, in place the same way, 5 tiles of 128
                // (the last partial): its fc1 input is norm2 (n2w, n2b) of the
                // residual rows, formed in the kernel; against double
                std::vector<float> n2w = rng.vec(C, 1.0f), n2b = rng.vec(C, 0.1f);
                std::vector<unsigned short> mw;
                pack_mlp_x180(w1.data(), b1.data(), w2.data(), &mw);
                Dev dx2(res), dxn2((size_t)M * C), dn2w(n2w), dn2b(n2b), dmw((mw.size() + 1) / 2);
                Runtime::get().h2d(dmw.p, mw.data(), mw.size() * sizeof(unsigned short));
                TailXArgs q{};
                q.a = dx2.p;
                q.inw = dn2w.p;
                q.inb = dn2b.p;
                q.res = dx2.p;
                q.out = dx2.p;
                q.xn = epi == EPI_RESID_LN ? dxn2.p : nullptr;
                q.w = (const unsigned short*)dmw.p;
                q.b2 = db2.p;
                q.nw = dnw.p;
                q.nb = dnb.p;
                q.M = M;
                q.eps = 1e-5f;
                const char* kx = epi == EPI_RESID_LN ? "hat_mlpx180_ln" : "hat_mlpx180";
                launch(s, kx, (unsigned)wx_tiles(M), 1, 1, WX_THREADS, q);
                std::vector<double> want2((size_t)M * C), wxn2((size_t)M * C), y(C);
                for (int m = 0; m < M; ++m) {
                    const float* r = &res[(size_t)m * C];
                    double mu = 0, va = 0;
                    for (int c = 0; c < C; ++c) mu += r[c];
                    mu /= C;
                    for (int c = 0; c < C; ++c) va += (r[c] - mu) * (r[c] - mu);
                    va /= C;
                    for (int c = 0; c < C; ++c) y[c] = (r[c] - mu) / std::sqrt(va + 1e-5) * n2w[c] + n2b[c];
                    for (int j = 0; j < H; ++j) {
                        double v = b1[j];
                        for (int c = 0; c < C; ++c) v += y[c] * w1[(size_t)j * C + c];
                        hid[j] = gelu_d(v);
                    }
                    double mean = 0, var = 0;
                    for (int n = 0; n < C; ++n) {
                        double v = b2[n];
                        for (int j = 0; j < H; ++j) v += hid[j] * w2[(size_t)n * H + j];
                        want2[(size_t)m * C + n] = r[n] + v;
                        mean += want2[(size_t)m * C + n];
                    }
                    mean /= C;
                    for (int n = 0; n < C; ++n) var += (want2[(size_t)m * C + n] - mean) * (want2[(size_t)m * C + n] - mean);
                    var /= C;
                    for (int n = 0; n < C; ++n)
                        wxn2[(size_t)m * C + n] = (want2[(size_t)m * C + n] - mean) / std::sqrt(var + 1e-5) * nw[n] + nb[n];
                }
                check_close(kx, dx2.get(), want2, 5e-5);
                if (epi == EPI_RESID_LN) check_close(std::string(kx) + " layernorm", dxn2.get(), wxn2, 5e-5);
                note(std::string(kx) + " C 180 M 600 (split-bf16 with norm2 in the kernel, in place) vs double");
            }
        }

        // ---- the split-bf16 C = 180 projection tails against double: out =
        // res + a . Wp^T + b (+ aux * gate * cscale), xn = LN(out), in place
        // over the residual, 600 rows (the last tile partial).
        for (int hab : {1, 0}) {
            const int M = 600, C = 180;
            const float cscale = 0.01f;
            std::vector<float> a = rng.vec((size_t)M * C, 1.0f), w = rng.vec((size_t)C * C, 0.08f),
                               b = rng.vec(C, 0.1f), res = rng.vec((size_t)M * C, 1.0f), aux = rng.vec((size_t)M * C, 1.0f),
                               gate = rng.vec(C, 1.0f), nw = rng.vec(C, 1.0f), nb = rng.vec(C, 0.1f);
            std::vector<unsigned short> wx = pack_linear_x180(w.data());
            Dev da(a), db(b), dx(res), daux(aux), dg(gate), dnw(nw), dnb(nb), dxn((size_t)M * C), dw((wx.size() + 1) / 2);
            Runtime::get().h2d(dw.p, wx.data(), wx.size() * sizeof(unsigned short));
            TailXArgs q{};
            q.a = da.p;
            q.res = dx.p;
            q.out = dx.p;
            q.xn = dxn.p;
            q.w = (const unsigned short*)dw.p;
            q.bias = db.p;
            q.nw = dnw.p;
            q.nb = dnb.p;
            q.M = M;
            q.eps = 1e-5f;
            q.aux = hab ? daux.p : nullptr;
            q.gate = hab ? dg.p : nullptr;
            q.cscale = cscale;
            const char* k = hab ? "hat_projx180_hab" : "hat_projx180";
            launch(s, k, (unsigned)wx_tiles(M), 1, 1, WX_THREADS, q);
            std::vector<double> want((size_t)M * C), wxn((size_t)M * C);
            for (int m = 0; m < M; ++m) {
                double mean = 0, var = 0;
                for (int n = 0; n < C; ++n) {
                    double v = b[n];
                    for (int c = 0; c < C; ++c) v += (double)a[(size_t)m * C + c] * w[(size_t)n * C + c];
                    v += res[(size_t)m * C + n];
                    if (hab) v += (double)aux[(size_t)m * C + n] * gate[n] * cscale;
                    want[(size_t)m * C + n] = v;
                    mean += v / C;
                }
                for (int n = 0; n < C; ++n) var += (want[(size_t)m * C + n] - mean) * (want[(size_t)m * C + n] - mean) / C;
                for (int n = 0; n < C; ++n)
                    wxn[(size_t)m * C + n] = (want[(size_t)m * C + n] - mean) / std::sqrt(var + 1e-5) * nw[n] + nb[n];
            }
            check_close(k, dx.get(), want, 3e-5);
            check_close(std::string(k) + " layernorm", dxn.get(), wxn, 5e-5);
            note(std::string(k) + " C 180 M 600 (split-bf16, in place)");
        }

        // ---- the fused C = 180 tails (x' on the chip) against the two
        // kernels above on the same inputs, in place over the residual, 600
        // rows (the last tile partial): HAB form (gated conv2 output + next
        // norm) and OCAB form (neither).
        for (int hab : {1, 0}) {
            const int M = 600, C = 180, H = 360;
            const float cscale = 0.01f;
            std::vector<float> a = rng.vec((size_t)M * C, 1.0f), wp = rng.vec((size_t)C * C, 0.08f),
                               bp = rng.vec(C, 0.1f), res = rng.vec((size_t)M * C, 1.0f),
                               aux = rng.vec((size_t)M * C, 1.0f), gate = rng.vec(C, 1.0f),
                               n2w = rng.vec(C, 1.0f), n2b = rng.vec(C, 0.1f), w1 = rng.vec((size_t)H * C, 0.08f),
                               b1 = rng.vec(H, 0.1f), w2 = rng.vec((size_t)C * H, 0.05f), b2 = rng.vec(C, 0.1f),
                               nw = rng.vec(C, 1.0f), nb = rng.vec(C, 0.1f);
            std::vector<unsigned short> pwx = pack_linear_x180(wp.data()), mw, mwf;
            std::vector<float> mb1x;
            pack_mlp_x180(w1.data(), b1.data(), w2.data(), &mw);
            pack_mlp_xf180(w1.data(), b1.data(), w2.data(), &mwf, &mb1x);
            Dev da(a), dbp(bp), daux(aux), dg(gate), dn2w(n2w), dn2b(n2b), db2(b2), dnw(nw), dnb(nb), dmb1x(mb1x),
                dx2(res), dxn2((size_t)M * C), dxf(res), dxnf((size_t)M * C), dpw((pwx.size() + 1) / 2),
                dmw((mw.size() + 1) / 2), dmwf((mwf.size() + 1) / 2);
            Runtime::get().h2d(dpw.p, pwx.data(), pwx.size() * sizeof(unsigned short));
            Runtime::get().h2d(dmw.p, mw.data(), mw.size() * sizeof(unsigned short));
            Runtime::get().h2d(dmwf.p, mwf.data(), mwf.size() * sizeof(unsigned short));
            TailXArgs q{};
            q.a = da.p;
            q.res = dx2.p;
            q.out = dx2.p;
            q.w = (const unsigned short*)dpw.p;
            q.bias = dbp.p;
            q.M = M;
            q.eps = 1e-5f;
            q.aux = hab ? daux.p : nullptr;
            q.gate = hab ? dg.p : nullptr;
            q.cscale = cscale;
            launch(s, hab ? "hat_projx180_hab" : "hat_projx180", (unsigned)wx_tiles(M), 1, 1, WX_THREADS, q);
            TailXArgs m2{};
            m2.a = dx2.p;
            m2.inw = dn2w.p;
            m2.inb = dn2b.p;
            m2.res = dx2.p;
            m2.out = dx2.p;
            m2.xn = hab ? dxn2.p : nullptr;
            m2.w = (const unsigned short*)dmw.p;
            m2.b2 = db2.p;
            m2.nw = hab ? dnw.p : nullptr;
            m2.nb = hab ? dnb.p : nullptr;
            m2.M = M;
            m2.eps = 1e-5f;
            launch(s, hab ? "hat_mlpx180_ln" : "hat_mlpx180", (unsigned)wx_tiles(M), 1, 1, WX_THREADS, m2);
            TailXArgs f = q;
            f.res = dxf.p;
            f.out = dxf.p;
            f.xn = hab ? dxnf.p : nullptr;
            f.wm = (const unsigned short*)dmwf.p;
            f.b1x = dmb1x.p;
            f.b2 = db2.p;
            f.inw = dn2w.p;
            f.inb = dn2b.p;
            f.nw = hab ? dnw.p : nullptr;
            f.nb = hab ? dnb.p : nullptr;
            const char* k = hab ? "hat_habx180_hab_ln" : "hat_habx180";
            launch(s, k, (unsigned)wx_tiles(M), 1, 1, WX_THREADS, f);
            const std::vector<float> two = dx2.get();
            check_close(k, dxf.get(), std::vector<double>(two.begin(), two.end()), 2e-5);
            if (hab) {
                const std::vector<float> twon = dxn2.get();
                check_close(std::string(k) + " next norm", dxnf.get(), std::vector<double>(twon.begin(), twon.end()),
                            2e-5);
            }
            note(std::string(k) + " (fused split-bf16 C 180 tail, M 600, in place) vs the two-kernel path");
        }

        // ---- folded CAB (144 -> 6 -> 144) against the unfolded computation:
        // conv1 + GELU, conv2 in full, its pixel mean, squeeze-excite, gate, and
        // shortcut + proj + gated conv2 * cscale + LayerNorm - in double. A 32 x 48
        // plane (6 tiles over 2 blocks, so tiles on every border line and corner).
        {
            const int H = 32, W = 48, T = H * W, C = CAB_C, CC = CAB_CC, sq = 6;
            const float cscale = 0.01f;
            std::vector<float> xn = rng.vec((size_t)T * C, 1.0f), w1 = rng.vec((size_t)CC * C * 9, 0.05f),
                               b1 = rng.vec(CC, 0.1f), w2 = rng.vec((size_t)C * CC * 9, 0.2f),
                               b2 = rng.vec(C, 0.1f), wa = rng.vec((size_t)sq * C, 0.2f), ba = rng.vec(sq, 0.1f),
                               wb = rng.vec((size_t)C * sq, 0.5f), bb = rng.vec(C, 0.1f),
                               ao = rng.vec((size_t)T * C, 1.0f), wp = rng.vec((size_t)C * C, 0.05f),
                               bp = rng.vec(C, 0.1f), res = rng.vec((size_t)T * C, 1.0f),
                               nw = rng.vec(C, 1.0f), nb = rng.vec(C, 0.1f);
            std::vector<unsigned short> w1p = pack_cab_conv1(w1.data());
            int Kp = 0;
            std::vector<float> wpp = pack_linear(wp.data(), C, C, &Kp);
            const int tiles = (H / 16) * (W / 16);
            Dev dxn(xn), dw1(w1p.size() / 2), db1(b1), dw2(w2), db2(b2), dwa(wa), dba(ba), dwb(wb), dbb(bb), dao(ao),
                dwp(wpp), dbp(bp), dres(res), dnw(nw), dnb(nb), dt1((size_t)T * CAB_CS),
                dpart((size_t)tiles * CAB_NSUM * CAB_CS), dw2g((size_t)C * CAB_K2), dw2gx(WC_CHUNK), dbias2(C), dgate(C),
                dout((size_t)T * C), dxo((size_t)T * C);
            Runtime::get().h2d(dw1.p, w1p.data(), w1p.size() * sizeof(unsigned short));
            CabConvArgs ca{dxn.p, (const unsigned short*)dw1.p, db1.p, dt1.p, dpart.p, H, W};
            launch(s, "hat_cab_conv1", 2, 1, 1, 256, ca);
            CabGateArgs ga{};
            ga.partial = dpart.p;
            ga.t1 = dt1.p;
            ga.tiles = tiles;
            ga.H = H;
            ga.W = W;
            ga.w2 = dw2.p;
            ga.b2 = db2.p;
            ga.wa = dwa.p;
            ga.ba = dba.p;
            ga.wb = dwb.p;
            ga.bb = dbb.p;
            ga.bproj = dbp.p;
            ga.w2g = dw2g.p;
            ga.bias2 = dbias2.p;
            ga.gate = dgate.p;
            ga.cscale = cscale;
            ga.sq = sq;
            ga.w2gx = (unsigned short*)dw2gx.p;
            launch(s, "hat_cab_gate", 1, 1, 1, 1024, ga);
            GemmArgs gp{};
            gp.a = dao.p;
            gp.w = dwp.p;
            gp.bias = dbias2.p;
            gp.out = dout.p;
            gp.res = dres.p;
            gp.xn = dxo.p;
            gp.nw = dnw.p;
            gp.nb = dnb.p;
            gp.M = T;
            gp.N = C;
            gp.K = C;
            gp.Kp = Kp;
            gp.lda = C;
            gp.ldo = C;
            gp.eps = 1e-5f;
            gp.t1 = dt1.p;
            gp.w2g = dw2g.p;
            gp.H = H;
            gp.W = W;
            launch(s, "hat_gemmws_cab_ln", 3, 1, 1, ws_waves(EPI_RESID_LN) * 64, gp);

            auto inb = [&](int y, int x) { return y >= 0 && y < H && x >= 0 && x < W; };
            std::vector<double> t1((size_t)T * CAB_CS, 0.0), y2((size_t)T * C);
            for (int y = 0; y < H; ++y)
                for (int x = 0; x < W; ++x)
                    for (int co = 0; co < CC; ++co) {
                        double v = b1[co];
                        for (int tap = 0; tap < 9; ++tap) {
                            const int yy = y + tap / 3 - 1, xx = x + tap % 3 - 1;
                            if (!inb(yy, xx)) continue;
                            for (int ci = 0; ci < C; ++ci)
                                v += (double)w1[((size_t)co * C + ci) * 9 + tap] * xn[((size_t)yy * W + xx) * C + ci];
                        }
                        t1[((size_t)y * W + x) * CAB_CS + co] = gelu_d(v);
                    }
            std::vector<double> mean2(C, 0.0);
            for (int y = 0; y < H; ++y)
                for (int x = 0; x < W; ++x)
                    for (int c = 0; c < C; ++c) {
                        double v = b2[c];
                        for (int tap = 0; tap < 9; ++tap) {
                            const int yy = y + tap / 3 - 1, xx = x + tap % 3 - 1;
                            if (!inb(yy, xx)) continue;
                            for (int ci = 0; ci < CC; ++ci)
                                v += (double)w2[((size_t)c * CC + ci) * 9 + tap] * t1[((size_t)yy * W + xx) * CAB_CS + ci];
                        }
                        y2[((size_t)y * W + x) * C + c] = v;
                        mean2[c] += v / T;
                    }
            std::vector<double> z(sq), gate(C), bias2(C), w2g((size_t)C * CAB_K2, 0.0);
            for (int j = 0; j < sq; ++j) {
                double v = ba[j];
                for (int c = 0; c < C; ++c) v += (double)wa[(size_t)j * C + c] * mean2[c];
                z[j] = v < 0 ? 0 : v;
            }
            for (int c = 0; c < C; ++c) {
                double v = bb[c];
                for (int j = 0; j < sq; ++j) v += (double)wb[(size_t)c * sq + j] * z[j];
                gate[c] = 1.0 / (1.0 + std::exp(-v));
                bias2[c] = bp[c] + cscale * gate[c] * b2[c];
                for (int tap = 0; tap < 9; ++tap)
                    for (int ci = 0; ci < CC; ++ci)
                        w2g[(size_t)c * CAB_K2 + tap * CAB_CC + ci] = cscale * gate[c] * w2[((size_t)c * CC + ci) * 9 + tap];
            }
            std::vector<double> want((size_t)T * C), wxn((size_t)T * C);
            for (int m = 0; m < T; ++m) {
                double mean = 0, var = 0;
                for (int c = 0; c < C; ++c) {
                    double v = bp[c];
                    for (int k = 0; k < C; ++k) v += (double)ao[(size_t)m * C + k] * wp[(size_t)c * C + k];
                    v = res[(size_t)m * C + c] + v + y2[(size_t)m * C + c] * gate[c] * cscale;
                    want[(size_t)m * C + c] = v;
                    mean += v / C;
                }
                for (int c = 0; c < C; ++c) var += (want[(size_t)m * C + c] - mean) * (want[(size_t)m * C + c] - mean) / C;
                for (int c = 0; c < C; ++c)
                    wxn[(size_t)m * C + c] = (want[(size_t)m * C + c] - mean) / std::sqrt(var + 1e-5) * nw[c] + nb[c];
            }
            check_close("hat_cab_conv1 t1", dt1.get(), t1, 2e-5);
            note("hat_cab_conv1 144->6 + gelu, 32x48");
            check_close("hat_cab_gate gate", dgate.get(), gate, 2e-6);
            check_close("hat_cab_gate bias2", dbias2.get(), bias2, 2e-6);
            check_close("hat_cab_gate w2g", dw2g.get(), w2g, 1e-7);
            note("hat_cab_gate (mean by linearity) vs conv2 in full");
            // The 16 x 32 tile form (3 tiles over 2 blocks) and the gate from its
            // per-tile sums.
            {
                const int tiles32 = (H / 32) * (W / 16);
                Dev dt1b((size_t)T * CAB_CS), dpartb((size_t)tiles32 * CAB_NSUM * CAB_CS), dw2gb((size_t)C * CAB_K2),
                    dbias2b(C), dgateb(C);
                CabConvArgs cb2{dxn.p, (const unsigned short*)dw1.p, db1.p, dt1b.p, dpartb.p, H, W};
                launch(s, "hat_cab_conv1_t32", 2, 1, 1, 256, cb2);
                CabGateArgs gb = ga;
                gb.partial = dpartb.p;
                gb.t1 = dt1b.p;
                gb.tiles = tiles32;
                gb.w2g = dw2gb.p;
                gb.bias2 = dbias2b.p;
                gb.gate = dgateb.p;
                launch(s, "hat_cab_gate", 1, 1, 1, 1024, gb);
                check_close("hat_cab_conv1_t32 t1", dt1b.get(), t1, 2e-5);
                check_close("hat_cab_gate gate (16x32 tiles)", dgateb.get(), gate, 2e-6);
                note("hat_cab_conv1_t32 144->6 + gelu, 32x48, and its tile sums");
            }
            check_close("hat_gemmws_cab_ln", dout.get(), want, 5e-5);
            check_close("hat_gemmws_cab_ln layernorm", dxo.get(), wxn, 5e-5);
            note("hat_gemmws_cab_ln proj + folded conv2 + norm2");

            // The fused HAB tail against hat_gemmws_cab_ln followed by the fused
            // MLP (both checked above against double precision) on the same
            // inputs: out = x' + MLP(norm2(x')), xn = norm_next(out).
            {
                const int Hd = 2 * C;
                std::vector<float> f1 = rng.vec((size_t)Hd * C, 0.05f), fb1 = rng.vec(Hd, 0.1f),
                                   f2 = rng.vec((size_t)C * Hd, 0.05f), fb2 = rng.vec(C, 0.1f),
                                   mw = rng.vec(C, 1.0f), mb = rng.vec(C, 0.1f);
                int K1 = 0, K2 = 0;
                std::vector<float> f1p = pack_linear(f1.data(), Hd, C, &K1), f2p = pack_linear(f2.data(), C, Hd, &K2);
                Dev df1(f1p), dfb1(fb1), df2(f2p), dfb2(fb2), dmw(mw), dmb(mb), dxn_ref((size_t)T * C),
                    dout_t(res), dxn_t((size_t)T * C);
                MlpArgs mp{};
                mp.a = dxo.p;  // norm2(x') from hat_gemmws_cab_ln
                mp.w1 = df1.p;
                mp.b1 = dfb1.p;
                mp.w2 = df2.p;
                mp.b2 = dfb2.p;
                mp.res = dout.p;  // x', updated in place
                mp.out = dout.p;
                mp.xn = dxn_ref.p;
                mp.nw = dmw.p;
                mp.nb = dmb.p;
                mp.M = T;
                mp.eps = 1e-5f;
                mp.K = C;
                mp.H = Hd;
                mp.N = C;
                mp.ldw1 = K1;
                mp.ldw2 = K2;
                launch(s, "hat_mlp_resid_ln", 2, 1, 1, MLP_WAVES * 64, mp);
                HabTailArgs tp{};
                tp.a = dao.p;
                tp.res = dout_t.p;  // in place over the block input, as in the forward
                tp.out = dout_t.p;
                tp.xn = dxn_t.p;
                tp.wp = dwp.p;
                tp.w2g = dw2g.p;
                tp.bias2 = dbias2.p;
                tp.t1 = dt1.p;
                tp.n2w = dnw.p;
                tp.n2b = dnb.p;
                tp.w1 = df1.p;
                tp.b1 = dfb1.p;
                tp.w2 = df2.p;
                tp.b2 = dfb2.p;
                tp.nw = dmw.p;
                tp.nb = dmb.p;
                tp.M = T;
                tp.H = H;
                tp.W = W;
                tp.eps = 1e-5f;
                tp.ldw1 = K1;
                tp.ldw2 = K2;
                launch(s, "hat_hab_tail", 5, 1, 1, MLP_WAVES * 64, tp);  // 12 tiles: blocks walk 2 or 3
                const std::vector<float> ro = dout.get(), rx = dxn_ref.get();
                check_close("hat_hab_tail", dout_t.get(), std::vector<double>(ro.begin(), ro.end()), 2e-5);
                check_close("hat_hab_tail next norm", dxn_t.get(), std::vector<double>(rx.begin(), rx.end()), 2e-5);
                note("hat_hab_tail (proj + folded conv2 + norm2 + MLP + norm) vs the two-kernel path");

                // The OCAB's tail: hat_gemmws_resid_ln (proj + bias + shortcut +
                // norm2) then hat_mlp_resid, against hat_ocab_tail.
                Dev dref2(res), dxn2((size_t)T * C), dout_o(res);
                GemmArgs op{};
                op.a = dao.p;
                op.w = dwp.p;
                op.bias = dbp.p;
                op.out = dref2.p;
                op.res = dref2.p;
                op.xn = dxn2.p;
                op.nw = dnw.p;
                op.nb = dnb.p;
                op.M = T;
                op.N = C;
                op.K = C;
                op.Kp = Kp;
                op.lda = C;
                op.ldo = C;
                op.eps = 1e-5f;
                launch(s, "hat_gemmws_resid_ln", 3, 1, 1, ws_waves(EPI_RESID_LN) * 64, op);
                MlpArgs mo = mp;
                mo.a = dxn2.p;
                mo.res = dref2.p;
                mo.out = dref2.p;
                mo.xn = nullptr;
                launch(s, "hat_mlp_resid", 2, 1, 1, MLP_WAVES * 64, mo);
                HabTailArgs to = tp;
                to.res = dout_o.p;
                to.out = dout_o.p;
                to.xn = nullptr;
                to.t1 = nullptr;
                to.w2g = nullptr;
                to.bias2 = dbp.p;
                to.nw = nullptr;
                to.nb = nullptr;
                launch(s, "hat_ocab_tail", 5, 1, 1, MLP_WAVES * 64, to);
                const std::vector<float> r2 = dref2.get();
                check_close("hat_ocab_tail", dout_o.get(), std::vector<double>(r2.begin(), r2.end()), 2e-5);
                note("hat_ocab_tail (proj + norm2 + MLP) vs the two-kernel path");

                // The split-bf16 tails (tailx.hip) on the same inputs, in place
                // as the forward runs them (out over the block input, the next
                // norm over norm2's rows); 12 row tiles of 128.
                std::vector<unsigned short> pwx = pack_linear_x(wp.data(), C, C), mwx, mwf;
                std::vector<float> mb1x;
                pack_mlp_x(f1.data(), fb1.data(), f2.data(), &mwx);
                pack_mlp_xf(f1.data(), fb1.data(), f2.data(), &mwf, &mb1x);
                Dev dmb1x(mb1x);
                Dev dpwx(std::vector<float>((pwx.size() + 1) / 2)), dmwx(std::vector<float>((mwx.size() + 1) / 2)),
                    dmwf(std::vector<float>((mwf.size() + 1) / 2)), dout_x(res), dxn_x((size_t)T * C),
                    dout_f(res), dxn_f((size_t)T * C);
                Runtime::get().h2d(dpwx.p, pwx.data(), pwx.size() * sizeof(unsigned short));
                Runtime::get().h2d(dmwx.p, mwx.data(), mwx.size() * sizeof(unsigned short));
                Runtime::get().h2d(dmwf.p, mwf.data(), mwf.size() * sizeof(unsigned short));
                TailXArgs xa{};
                xa.a = dao.p;
                xa.res = dout_x.p;
                xa.out = dout_x.p;
                xa.xn = dxn_x.p;
                xa.w = (const unsigned short*)dpwx.p;
                xa.bias = dbias2.p;
                xa.w2gx = (const unsigned short*)dw2gx.p;
                xa.t1 = dt1.p;
                xa.nw = dnw.p;
                xa.nb = dnb.p;
                xa.M = T;
                xa.H = H;
                xa.W = W;
                xa.eps = 1e-5f;
                launch(s, "hat_projx_cab", (unsigned)wx_tiles(T), 1, 1, WX_THREADS, xa);
                check_close("hat_projx_cab", dout_x.get(), want, 5e-5);
                check_close("hat_projx_cab layernorm", dxn_x.get(), wxn, 5e-5);
                note("hat_projx_cab (split-bf16 proj + folded conv2 + norm2) vs double");
                TailXArgs xm{};
                xm.a = dout_x.p;  // x': the kernel forms norm2 from it
                xm.inw = dnw.p;
                xm.inb = dnb.p;
                xm.res = dout_x.p;
                xm.out = dout_x.p;
                xm.xn = dxn_x.p;
                xm.w = (const unsigned short*)dmwx.p;
                xm.b2 = dfb2.p;
                xm.nw = dmw.p;
                xm.nb = dmb.p;
                xm.M = T;
                xm.H = H;
                xm.W = W;
                xm.eps = 1e-5f;
                launch(s, "hat_mlpx_ln", (unsigned)wx_tiles(T), 1, 1, WX_THREADS, xm);
                check_close("hat_mlpx_ln", dout_x.get(), std::vector<double>(ro.begin(), ro.end()), 2e-5);
                check_close("hat_mlpx_ln next norm", dxn_x.get(), std::vector<double>(rx.begin(), rx.end()), 2e-5);
                note("hat_mlpx_ln (split-bf16 MLP + norm) vs the two-kernel path");
                // The fused tail (x' on the chip) on the same inputs, in place,
                // against the same references.
                TailXArgs xf = xa;
                xf.res = dout_f.p;
                xf.out = dout_f.p;
                xf.xn = dxn_f.p;
                xf.wm = (const unsigned short*)dmwf.p;
                xf.b1x = dmb1x.p;
                xf.b2 = dfb2.p;
                xf.inw = dnw.p;
                xf.inb = dnb.p;
                xf.nw = dmw.p;
                xf.nb = dmb.p;
                launch(s, "hat_habx_cab_ln", (unsigned)wx_tiles(T), 1, 1, WX_THREADS, xf);
                check_close("hat_habx_cab_ln", dout_f.get(), std::vector<double>(ro.begin(), ro.end()), 2e-5);
                check_close("hat_habx_cab_ln next norm", dxn_f.get(), std::vector<double>(rx.begin(), rx.end()), 2e-5);
                note("hat_habx_cab_ln (fused split-bf16 proj + conv2 + MLP + norm) vs the two-kernel path");
                // The OCAB form over a partial last tile: rows from Mo on stay
                // the block input.
                const int Mo = T - 100;
                Dev dout_ox(res), dxn_ox((size_t)T * C);
                TailXArgs xo = xa;
                xo.res = dout_ox.p;
                xo.out = dout_ox.p;
                xo.xn = dxn_ox.p;
                xo.bias = dbp.p;
                xo.w2gx = nullptr;
                xo.t1 = nullptr;
                xo.M = Mo;
                launch(s, "hat_projx", (unsigned)wx_tiles(Mo), 1, 1, WX_THREADS, xo);
                TailXArgs xo2 = xm;
                xo2.a = dout_ox.p;
                xo2.res = dout_ox.p;
                xo2.out = dout_ox.p;
                xo2.xn = nullptr;
                xo2.nw = nullptr;
                xo2.nb = nullptr;
                xo2.M = Mo;
                launch(s, "hat_mlpx", (unsigned)wx_tiles(Mo), 1, 1, WX_THREADS, xo2);
                std::vector<double> wo(r2.begin(), r2.end());
                for (size_t i = (size_t)Mo * C; i < wo.size(); ++i) wo[i] = res[i];
                check_close("hat_projx + hat_mlpx", dout_ox.get(), wo, 2e-5);
                note("hat_projx + hat_mlpx (split-bf16 OCAB tail, partial tile) vs the two-kernel path");
                Dev dout_of(res);
                TailXArgs xof = xo;
                xof.res = dout_of.p;
                xof.out = dout_of.p;
                xof.xn = nullptr;
                xof.wm = (const unsigned short*)dmwf.p;
                xof.b1x = dmb1x.p;
                xof.b2 = dfb2.p;
                xof.inw = dnw.p;
                xof.inb = dnb.p;
                xof.nw = nullptr;
                xof.nb = nullptr;
                launch(s, "hat_habx", (unsigned)wx_tiles(Mo), 1, 1, WX_THREADS, xof);
                check_close("hat_habx", dout_of.get(), wo, 2e-5);
                note("hat_habx (fused split-bf16 OCAB tail, partial tile) vs the two-kernel path");
            }
        }

        // ---- trunk convs with every output channel in a block (C -> 144):
        // residual (in place) + LayerNorm, conv_first's 3-channel input +
        // LayerNorm, and a plain residual; 32 x 48 plane = 6 tiles.
        {
            // wino: the Winograd F(2x2, 3x3) kernels (8 x 16 tiles, 512 threads)
            // the conv_first kernels (convfirst.hip): 16 x 16 tiles, 4 waves
            struct WCase { int CI, cin_stride, CO, epi; const char* k; int waves; bool wino; };
            const WCase wc[] = {{144, 144, 144, EPI_RESID_LN, "hat_convw_n9_resid_ln", CONVW_WAVES_N9_RESID_LN, false},
                                {3, 4, 144, EPI_STORE_LN, "hat_convw_n9_store_ln", CONVW_WAVES_N9_STORE_LN, false},
                                {3, 4, 144, EPI_STORE_LN, "hat_conv_first_ln144", 4, false},
                                {3, 4, 180, EPI_STORE_LN, "hat_conv_first_ln180", 4, false},
                                {144, 144, 144, EPI_RESID, "hat_convw_n9_resid", CONVW_WAVES_N9_RESID, false},
                                {144, 144, 144, EPI_RESID, "hat_convwino_resid", 8, true}};
            for (const WCase& c : wc) {
                const int H = 32, W = 48, HW = H * W, CO = c.CO;
                std::vector<float> in((size_t)HW * c.cin_stride, 0.0f);
                for (int q = 0; q < HW; ++q)
                    for (int ci = 0; ci < c.CI; ++ci) in[(size_t)q * c.cin_stride + ci] = rng.uni();
                std::vector<float> w = rng.vec((size_t)CO * c.CI * 9, 0.05f), b = rng.vec(CO, 0.1f),
                                   res = rng.vec((size_t)HW * CO, 1.0f), nw = rng.vec(CO, 1.0f),
                                   nb = rng.vec(CO, 0.1f);
                std::vector<float> bias;
                int CIp = 0, COp = 0;
                std::vector<float> pk = pack_conv(w.data(), b.data(), CO, c.CI, 0, &bias, &CIp, &COp);
                Dev din(in), dw(pk), db(bias), dres(res), dnw(nw), dnb(nb), dxn((size_t)HW * CO);
                const std::vector<unsigned short> wux = c.wino ? pack_wino(w.data(), CO, c.CI, 0)
                                                               : std::vector<unsigned short>(8, 0);
                Dev dwu((wux.size() + 1) / 2);
                Runtime::get().h2d(dwu.p, wux.data(), wux.size() * sizeof(unsigned short));
                ConvArgs p{};
                p.in = din.p;
                p.w = dw.p;
                p.bias = db.p;
                p.out = dres.p;  // in place over the residual
                p.res = c.epi == EPI_STORE_LN ? nullptr : dres.p;
                p.H = H;
                p.W = W;
                p.CI = c.CI;
                p.CIp = CIp;
                p.cin_stride = c.cin_stride;
                p.CO = CO;
                p.COp = COp;
                p.co_stride = CO;
                p.xn = dxn.p;
                p.nw = dnw.p;
                p.nb = dnb.p;
                p.eps = 1e-5f;
                p.wu = (const unsigned short*)dwu.p;
                if (c.wino) launch_wino(s, c.k, (W / 16) * (H / 8), 1, p, 5);  // persistent ones over 5 blocks
                else launch(s, c.k, (W / 16) * (H / 16), 1, 1, c.waves * 64, p);  // convw and conv_first: 16 x 16
                std::vector<double> want((size_t)HW * CO), wxn((size_t)HW * CO);
                for (int y = 0; y < H; ++y)
                    for (int x = 0; x < W; ++x) {
                        const size_t o = ((size_t)y * W + x) * CO;
                        double mean = 0, var = 0;
                        for (int co = 0; co < CO; ++co) {
                            double v = b[co];
                            for (int tap = 0; tap < 9; ++tap) {
                                const int yy = y + tap / 3 - 1, xx = x + tap % 3 - 1;
                                if (yy < 0 || yy >= H || xx < 0 || xx >= W) continue;
                                for (int ci = 0; ci < c.CI; ++ci)
                                    v += (double)w[((size_t)co * c.CI + ci) * 9 + tap] *
                                         in[((size_t)yy * W + xx) * c.cin_stride + ci];
                            }
                            if (c.epi != EPI_STORE_LN) v += res[o + co];
                            want[o + co] = v;
                            mean += v / CO;
                        }
                        for (int co = 0; co < CO; ++co) var += (want[o + co] - mean) * (want[o + co] - mean) / CO;
                        for (int co = 0; co < CO; ++co)
                            wxn[o + co] = (want[o + co] - mean) / std::sqrt(var + 1e-5) * nw[co] + nb[co];
                    }
                check_close(c.k, dres.get(), want, 5e-5);
                if (c.epi != EPI_RESID) check_close(std::string(c.k) + " layernorm", dxn.get(), wxn, 5e-5);
                note(std::string(c.k) + " " + std::to_string(c.CI) + "->" + std::to_string(CO) + ", 32x48");
            }
        }

        // ---- convolutions (all epilogues) on a non-square plane.
        struct CCase { int CI, CO, epi, act, r; const char* what; };
        const CCase cases[] = {
            {144, 6, CEPI_STORE, 1, 0, "cab conv1 144->6 + gelu"},
            {180, 60, CEPI_STORE, 1, 0, "cab conv1 180->60 + gelu"},
            {6, 144, CEPI_COLSUM, 0, 0, "cab conv2 6->144 + column sums"},
            {60, 180, CEPI_COLSUM, 0, 0, "cab conv2 60->180 + column sums"},
            {144, 144, CEPI_RESID, 0, 0, "rhag conv 144->144 + residual"},
            {180, 180, CEPI_RESID, 0, 0, "rhag conv 180->180 + residual"},
            {3, 144, CEPI_STORE, 0, 0, "conv_first 3->144"},
            {144, 64, CEPI_STORE, 2, 0, "conv_before_upsample 144->64 + leaky"},
            {180, 64, CEPI_STORE, 2, 0, "conv_before_upsample 180->64 + leaky"},
            {64, 256, CEPI_SHUFFLE, 0, 2, "upsample 64->256 + shuffle 2"},
            {64, 576, CEPI_SHUFFLE, 0, 3, "upsample 64->576 + shuffle 3"},
            {64, 3, CEPI_FINAL, 0, 0, "conv_last 64->3 + crop/denorm"},
        };
        for (const CCase& cc : cases) {
            const int H = 32, W = 48, HW = H * W;
            const int cin_stride = (cc.CI + 3) / 4 * 4;
            std::vector<float> in((size_t)HW * cin_stride, 0.0f);
            for (int p = 0; p < HW; ++p)
                for (int c = 0; c < cc.CI; ++c) in[(size_t)p * cin_stride + c] = rng.uni();
            std::vector<float> w = rng.vec((size_t)cc.CO * cc.CI * 9, 0.05f), b = rng.vec(cc.CO, 0.1f);
            std::vector<float> res = rng.vec((size_t)HW * cc.CO, 1.0f);
            std::vector<float> bias;
            int CIp = 0, COp = 0;
            std::vector<float> pk = pack_conv(w.data(), b.data(), cc.CO, cc.CI, cc.r, &bias, &CIp, &COp);
            const int nblk = (W / 16) * (H / 8);
            const int crop_h = 30, crop_w = 41;
            size_t out_n = cc.epi == CEPI_FINAL ? (size_t)3 * crop_h * crop_w : (size_t)HW * cc.CO;
            Dev din(in), dw(pk), db(bias), dres(res), dout(out_n), dpart((size_t)nblk * cc.CO);
            DevConv C;
            C.w = dw.p;
            C.b = db.p;
            C.CI = cc.CI;
            C.CIp = CIp;
            C.CO = cc.CO;
            C.COp = COp;
            C.r = cc.r;
            const float mean[3] = {0.4488f, 0.4371f, 0.4040f};
            ConvArgs p{};
            p.in = din.p;
            p.w = dw.p;
            p.bias = db.p;
            p.out = dout.p;
            p.res = dres.p;
            p.partial = dpart.p;
            p.H = H;
            p.W = W;
            p.CI = cc.CI;
            p.CIp = CIp;
            p.cin_stride = cin_stride;
            p.CO = cc.CO;
            p.COp = COp;
            p.co_stride = cc.epi == CEPI_SHUFFLE ? cc.CO / (cc.r * cc.r) : cc.CO;
            p.act = cc.act;
            p.r = cc.r;
            p.crop_h = crop_h;
            p.crop_w = crop_w;
            p.img_range = 1.0f;
            p.mean0 = mean[0];
            p.mean1 = mean[1];
            p.mean2 = mean[2];
            const char* name = nullptr;
            int BN = 16;
            switch (cc.epi) {
            case CEPI_STORE:
                name = cc.CO <= 16 ? "hat_conv_n1_store" : cc.CO <= 64 ? "hat_conv_n4_store" : "hat_conv_n3_store";
                BN = cc.CO <= 16 ? 16 : cc.CO <= 64 ? 64 : 48;
                break;
            case CEPI_RESID: name = "hat_conv_n3_resid"; BN = 48; break;
            case CEPI_COLSUM: name = "hat_conv_n3_colsum"; BN = 48; break;
            case CEPI_SHUFFLE: name = "hat_conv_n4_shuffle"; BN = 64; break;
            case CEPI_FINAL: name = "hat_conv_n1_final"; BN = 16; break;
            }
            launch(s, name, nblk, (cc.CO + BN - 1) / BN, 1, 256, p);
            std::vector<double> full((size_t)HW * cc.CO);
            for (int y = 0; y < H; ++y)
                for (int x = 0; x < W; ++x)
                    for (int o = 0; o < cc.CO; ++o) {
                        double v = b[o];
                        for (int ci = 0; ci < cc.CI; ++ci)
                            for (int dy = 0; dy < 3; ++dy)
                                for (int dx = 0; dx < 3; ++dx) {
                                    const int yy = y + dy - 1, xx = x + dx - 1;
                                    if (yy < 0 || yy >= H || xx < 0 || xx >= W) continue;
                                    v += (double)in[((size_t)yy * W + xx) * cin_stride + ci] *
                                         w[((size_t)o * cc.CI + ci) * 9 + dy * 3 + dx];
                                }
                        if (cc.act == 1) v = gelu_d(v);
                        if (cc.act == 2 && v < 0) v *= 0.01;
                        full[((size_t)y * W + x) * cc.CO + o] = v;
                    }
            std::vector<double> want(out_n);
            if (cc.epi == CEPI_STORE || cc.epi == CEPI_COLSUM) want = full;
            else if (cc.epi == CEPI_RESID)
                for (size_t i = 0; i < want.size(); ++i) want[i] = full[i] + res[i];
            else if (cc.epi == CEPI_SHUFFLE) {
                // PixelShuffle (cpu.rs:1285-1301): channel c*r*r + i*r + j -> (r*y+i, r*x+j).
                const int r = cc.r, Cf = cc.CO / (r * r);
                for (int y = 0; y < H; ++y)
                    for (int x = 0; x < W; ++x)
                        for (int c = 0; c < Cf; ++c)
                            for (int i = 0; i < r; ++i)
                                for (int j = 0; j < r; ++j)
                                    want[((size_t)(r * y + i) * (W * r) + r * x + j) * Cf + c] =
                                        full[((size_t)y * W + x) * cc.CO + c * r * r + i * r + j];
            } else if (cc.epi == CEPI_FINAL) {
                for (int c = 0; c < 3; ++c)
                    for (int y = 0; y < crop_h; ++y)
                        for (int x = 0; x < crop_w; ++x)
                            want[((size_t)c * crop_h + y) * crop_w + x] = full[((size_t)y * W + x) * 3 + c] + mean[c];
            }
            check_close(name + std::string(" ") + cc.what, dout.get(), want, 5e-5);
            if (cc.epi == CEPI_COLSUM) {
                std::vector<double> ps((size_t)nblk * cc.CO, 0.0);
                const int tiles_x = W / 16;
                for (int y = 0; y < H; ++y)
                    for (int x = 0; x < W; ++x) {
                        const int blk = (y / 8) * tiles_x + x / 16;
                        for (int o = 0; o < cc.CO; ++o) ps[(size_t)blk * cc.CO + o] += full[((size_t)y * W + x) * cc.CO + o];
                    }
                check_close(std::string(name) + " partial sums", dpart.get(), ps, 5e-4);
            }
            note(std::string(name) + "  " + cc.what + "  32x48");
            // The wide-tile kernel serves the same store / shuffle cases.
            const char* wide = cc.epi == CEPI_STORE && cc.CO > 16 && cc.CO <= 64 ? "hat_convw_n4_store"
                               : cc.epi == CEPI_SHUFFLE                           ? "hat_convw_n8_shuffle"
                               : cc.epi == CEPI_RESID && cc.CO > 144              ? "hat_convw_n6_resid"
                               : cc.epi == CEPI_COLSUM && cc.CO > 144             ? "hat_convw_n6_colsum"
                                                                                  : nullptr;
            if (wide) {
                const int wbn = cc.epi == CEPI_SHUFFLE ? 128 : (cc.epi == CEPI_RESID || cc.epi == CEPI_COLSUM) ? 96 : 64;
                const int wwaves = cc.epi == CEPI_SHUFFLE  ? CONVW_WAVES_N8_SHUFFLE
                                   : cc.epi == CEPI_RESID  ? CONVW_WAVES_N6_RESID
                                   : cc.epi == CEPI_COLSUM ? CONVW_WAVES_N6_COLSUM
                                                           : CONVW_WAVES_N4_STORE;
                Dev dout2(out_n), dpart2((size_t)(W / 16) * (H / 16) * cc.CO);
                p.out = dout2.p;
                p.partial = dpart2.p;
                launch(s, wide, (W / 16) * (H / 16), (cc.CO + wbn - 1) / wbn, 1, wwaves * 64, p);
                check_close(std::string(wide) + " " + cc.what, dout2.get(), want, 5e-5);
                if (cc.epi == CEPI_COLSUM) {
                    // one partial row per 16x16 tile
                    std::vector<double> ps((size_t)(W / 16) * (H / 16) * cc.CO, 0.0);
                    for (int y = 0; y < H; ++y)
                        for (int x = 0; x < W; ++x) {
                            const int blk = (y / 16) * (W / 16) + x / 16;
                            for (int o = 0; o < cc.CO; ++o) ps[(size_t)blk * cc.CO + o] += full[((size_t)y * W + x) * cc.CO + o];
                        }
                    check_close(std::string(wide) + " partial sums", dpart2.get(), ps, 5e-4);
                }
                note(std::string(wide) + "  " + cc.what + "  32x48");
            }
            // The Winograd kernels serve conv_before_upsample and the x2 upsample
            // convs (8 x 16 tiles; the shuffle in two 128-channel column blocks).
            // For the C = 180 family they serve the trunk conv and both CAB convs
            // (180 -> 180 and 60 -> 180 in two 96-channel column blocks).
            const char* wino = cc.epi == CEPI_STORE && cc.act == 2 && cc.CI == 144 && cc.CO == 64
                                   ? "hat_convwino_n4_store"
                               : cc.epi == CEPI_SHUFFLE && cc.r == 2 && cc.CI == 64 && cc.CO == 256
                                   ? "hat_convwino_n8_shuffle"
                               : cc.epi == CEPI_STORE && cc.act == 2 && cc.CI == 180 && cc.CO == 64
                                   ? "hat_convwino_n4_store180"
                               : cc.epi == CEPI_STORE && cc.act == 1 && cc.CI == 180 && cc.CO == 60
                                   ? "hat_convwino_cab1_180"
                               : cc.epi == CEPI_COLSUM && cc.CI == 60 && cc.CO == 180 ? "hat_convwino_cab2_180"
                               : cc.epi == CEPI_RESID && cc.CI == 180 && cc.CO == 180 ? "hat_convwino_resid180"
                                                                                      : nullptr;
            if (wino) {
                const int ncb = cc.CO == 256 ? 2 : cc.CO == 180 ? 2 : 1;
                const std::vector<unsigned short> wux = pack_wino(w.data(), cc.CO, cc.CI, cc.r);
                Dev dwu((wux.size() + 1) / 2), dout4(out_n), dpart4((size_t)nblk * cc.CO);
                Runtime::get().h2d(dwu.p, wux.data(), wux.size() * sizeof(unsigned short));
                p.out = dout4.p;
                p.partial = dpart4.p;
                p.wu = (const unsigned short*)dwu.p;
                // the persistent kernels over 5 ncb blocks (2 or 3 of the 12 tiles
                // each, the next tile's patch fetched under an epilogue)
                launch_wino(s, wino, (W / 16) * (H / 8), ncb, p, 5 * ncb);
                p.nblk = 0;
                check_close(std::string(wino) + " " + cc.what, dout4.get(), want, 5e-5);
                if (cc.epi == CEPI_COLSUM) {
                    // one partial row per 8x16 tile
                    std::vector<double> ps((size_t)nblk * cc.CO, 0.0);
                    for (int y = 0; y < H; ++y)
                        for (int x = 0; x < W; ++x) {
                            const int blk = (y / 8) * (W / 16) + x / 16;
                            for (int o = 0; o < cc.CO; ++o) ps[(size_t)blk * cc.CO + o] += full[((size_t)y * W + x) * cc.CO + o];
                        }
                    check_close(std::string(wino) + " partial sums", dpart4.get(), ps, 5e-4);
                }
                note(std::string(wino) + "  " + cc.what + "  32x48");
            }
            // conv_last by per-tap products: 16 x 32 tiles, so W = 48 leaves a
            // half tile whose pixels past W are zero halo and are not stored.
            if (cc.epi == CEPI_FINAL) {
                Dev dout3(out_n);
                p.out = dout3.p;
                launch(s, "hat_conv_last3", ((W + 31) / 32) * ((H + 15) / 16), 1, 1, 512, p);
                check_close(std::string("hat_conv_last3 ") + cc.what, dout3.get(), want, 5e-5);
                note(std::string("hat_conv_last3  ") + cc.what + "  32x48");
            }
        }

        // ---- LayerNorm, input preparation, squeeze-excite.
        // C = 144 and 180 take the 16-lanes-per-row path (16 rows per block),
        // C = 196 the one-wave-per-row path (4 rows per block); 300 rows leave
        // partial blocks in both.
        for (int C : {144, 180, 196}) {
            const int rows = 300;
            std::vector<float> x = rng.vec((size_t)rows * C, 2.0f), w = rng.vec(C, 1.0f), b = rng.vec(C, 0.5f);
            Dev dx(x), dw(w), db(b), dy((size_t)rows * C);
            LnArgs p{dx.p, dy.p, dw.p, db.p, rows, C, 1e-5f};
            const int per = (C % 4 == 0 && C <= 192) ? 16 : 4;
            launch(s, "hat_layernorm", (rows + per - 1) / per, 1, 1, 256, p);
            std::vector<double> want((size_t)rows * C);
            for (int r = 0; r < rows; ++r) {
                double mean = 0, var = 0;
                for (int c = 0; c < C; ++c) mean += x[(size_t)r * C + c];
                mean /= C;
                for (int c = 0; c < C; ++c) var += (x[(size_t)r * C + c] - mean) * (x[(size_t)r * C + c] - mean);
                var /= C;
                for (int c = 0; c < C; ++c)
                    want[(size_t)r * C + c] = (x[(size_t)r * C + c] - mean) / std::sqrt(var + 1e-5) * w[c] + b[c];
            }
            check_close("hat_layernorm C " + std::to_string(C), dy.get(), want, 1e-5);
            note("hat_layernorm 300x" + std::to_string(C));
        }
        {
            const int h = 21, w = 35, hp = 32, wp = 48;
            std::vector<float> in = rng.vec((size_t)3 * h * w, 1.0f);
            Dev din(in), dout((size_t)hp * wp * 4);
            PreArgs p{din.p, dout.p, h, w, hp, wp, 4, 0.4488f, 0.4371f, 0.4040f, 1.0f};
            launch(s, "hat_pre", (hp * wp + 255) / 256, 1, 1, 256, p);
            std::vector<float> got = dout.get();
            const float m[3] = {0.4488f, 0.4371f, 0.4040f};
            for (int y = 0; y < hp; ++y)
                for (int x = 0; x < wp; ++x)
                    for (int c = 0; c < 4; ++c) {
                        const int sy = y < h - 1 ? y : h - 1, sx = x < w - 1 ? x : w - 1;
                        const float want = c < 3 ? (in[(size_t)c * h * w + sy * w + sx] - m[c]) * 1.0f : 0.0f;
                        if (got[((size_t)y * wp + x) * 4 + c] != want)
                            throw Error("hat_pre: mismatch at (" + std::to_string(y) + ", " + std::to_string(x) + ")");
                    }
            note("hat_pre 21x35 -> 32x48 (exact)");
        }
        {
            const int nrows = 2048 + 17, C = 180, rows_per = 32, nred = (nrows + rows_per - 1) / rows_per;
            std::vector<float> in = rng.vec((size_t)nrows * C, 4.0f);
            Dev din(in), dout((size_t)nred * C);
            ReduceArgs p{din.p, dout.p, nrows, C, C, rows_per};
            launch(s, "hat_colsum_reduce", nred, 1, 1, 256, p);
            std::vector<double> want((size_t)nred * C, 0.0);
            for (int r = 0; r < nrows; ++r)
                for (int c = 0; c < C; ++c) want[(size_t)(r / rows_per) * C + c] += in[(size_t)r * C + c];
            check_close("hat_colsum_reduce", dout.get(), want, 1e-4);
            note("hat_colsum_reduce 2065x180 in blocks of 32 rows");
        }
        {
            const int C = 144, sq = 6, nblk = 37;
            std::vector<float> part = rng.vec((size_t)nblk * C, 10.0f), w1 = rng.vec((size_t)sq * C, 0.1f),
                               b1 = rng.vec(sq, 0.1f), w2 = rng.vec((size_t)C * sq, 0.1f), b2 = rng.vec(C, 0.1f);
            Dev dp(part), d1(w1), db1(b1), d2(w2), db2(b2), dg(C);
            SeArgs p{dp.p, nblk, C, 4096.0f, d1.p, db1.p, d2.p, db2.p, dg.p, C, sq};
            launch(s, "hat_se_gate", 1, 1, 1, 256, p);
            std::vector<double> mean(C), hid(sq), want(C);
            for (int c = 0; c < C; ++c) {
                double a = 0;
                for (int b = 0; b < nblk; ++b) a += part[(size_t)b * C + c];
                mean[c] = a / 4096.0;
            }
            for (int j = 0; j < sq; ++j) {
                double a = b1[j];
                for (int c = 0; c < C; ++c) a += mean[c] * w1[(size_t)j * C + c];
                hid[j] = a < 0 ? 0 : a;
            }
            for (int c = 0; c < C; ++c) {
                double a = b2[c];
                for (int j = 0; j < sq; ++j) a += hid[j] * w2[(size_t)c * sq + j];
                want[c] = 1.0 / (1.0 + std::exp(-a));
            }
            check_close("hat_se_gate", dg.get(), want, 1e-6);
            note("hat_se_gate C 144 sq 6");
        }
        printf("  gpu selftest: %d checks passed\n", passed);
        fflush(stdout);
    } catch (const Error& e) {
        if (err) *err = e.msg;
        printf("  FAIL %s\n", e.msg.c_str());
        fflush(stdout);
        return -1;
    }
    return passed;
}

}  // namespace hat
