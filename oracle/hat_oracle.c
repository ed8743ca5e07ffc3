/*
 * hat_oracle.c - TEST INFRASTRUCTURE ONLY (see hat_oracle.h).
 *
 * A C restatement of the reference CPU backend. Each function names the
 * reference file:line it follows. Arithmetic is written to reproduce the
 * reference's operation order exactly; this file is compiled with
 * -ffp-contract=off so that no multiply-add is fused (Rust does not contract).
 */
#include "hat_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* Parallel-for over output elements (the reference parallelises with rayon
 * over outputs; the reduction inside one output is serial, so the thread
 * count never changes a value). */
static int g_threads = 0;

void or_set_threads(int n) { g_threads = n; }

int or_get_threads(void)
{
    if (g_threads <= 0) {
        const char *e = getenv("HAT_ORACLE_THREADS");
        int n = e ? atoi(e) : 0;
        if (n <= 0) n = (int)sysconf(_SC_NPROCESSORS_ONLN);
        if (n <= 0) n = 1;
        g_threads = n;
    }
    return g_threads;
}

typedef void (*task_fn)(void *ctx, long begin, long end);
typedef struct {
    long n, grain;
    long next;
    task_fn fn;
    void *ctx;
} pf_job;

static void *pf_worker(void *arg)
{
    pf_job *j = (pf_job *)arg;
    for (;;) {
        long b = __atomic_fetch_add(&j->next, j->grain, __ATOMIC_RELAXED);
        if (b >= j->n) break;
        long e = b + j->grain < j->n ? b + j->grain : j->n;
        j->fn(j->ctx, b, e);
    }
    return NULL;
}

static void par_for(long n, long grain, task_fn fn, void *ctx)
{
    if (n <= 0) return;
    int t = or_get_threads();
    if (grain < 1) grain = 1;
    long chunks = (n + grain - 1) / grain;
    if (t > chunks) t = (int)chunks;
    pf_job j = {n, grain, 0, fn, ctx};
    if (t <= 1) {
        fn(ctx, 0, n);
        return;
    }
    pthread_t th[256];
    if (t > 256) t = 256;
    for (int i = 1; i < t; ++i) pthread_create(&th[i], NULL, pf_worker, &j);
    pf_worker(&j);
    for (int i = 1; i < t; ++i) pthread_join(th[i], NULL);
}

static long grain_for(long n) { long g = n / (or_get_threads() * 16L); return g < 1 ? 1 : g; }

static void *xmalloc(size_t n)
{
    void *p = calloc(n ? n : 1, 1);
    if (!p) {
        fprintf(stderr, "oracle: out of memory (%zu bytes)\n", n);
        abort();
    }
    return p;
}

/* ------------------------------------------------------------------------ */
/* Geometry: src/plan.rs */

/* Plan::new (plan.rs:53-66) */
void or_plan_new(or_plan *p, int h, int w, int win, int c)
{
    p->h = h;
    p->w = w;
    p->hp = (h + win - 1) / win * win;
    p->wp = (w + win - 1) / win * win;
    p->c = c;
    p->win = win;
    p->shift = win / 2;
    p->owin = win + win / 2;
}
int or_plan_nx(const or_plan *p) { return p->wp / p->win; }            /* plan.rs:83 */
int or_plan_ny(const or_plan *p) { return p->hp / p->win; }            /* plan.rs:87 */
int or_plan_nw(const or_plan *p) { return or_plan_nx(p) * or_plan_ny(p); }
int or_plan_opad(const or_plan *p) { return (p->owin - p->win) / 2; }  /* plan.rs:110 */

/* window_index (plan.rs:129-151): roll is out[i] = p[(i + shift) mod n]. */
void or_window_index(const or_plan *p, int shift, uint32_t *out)
{
    int win = p->win, wp = p->wp, hp = p->hp, ny = or_plan_ny(p), nx = or_plan_nx(p);
    long k = 0;
    for (int wy = 0; wy < ny; ++wy)
        for (int wx = 0; wx < nx; ++wx)
            for (int y = 0; y < win; ++y)
                for (int x = 0; x < win; ++x) {
                    int sy = (wy * win + y + shift) % hp;
                    int sx = (wx * win + x + shift) % wp;
                    out[k++] = (uint32_t)(sy * wp + sx);
                }
}

/* unfold_index (plan.rs:170-205): nn.Unfold(owin, stride win, pad opad); the
 * index is clamped into the plane and `keep` says whether it is real. */
void or_unfold_index(const or_plan *p, uint32_t *idx, uint8_t *keep)
{
    int win = p->win, wp = p->wp, hp = p->hp, owin = p->owin, pad = or_plan_opad(p);
    int ny = or_plan_ny(p), nx = or_plan_nx(p);
    long k = 0;
    for (int wy = 0; wy < ny; ++wy)
        for (int wx = 0; wx < nx; ++wx)
            for (int y = 0; y < owin; ++y)
                for (int x = 0; x < owin; ++x) {
                    int sy = wy * win + y - pad;
                    int sx = wx * win + x - pad;
                    int inside = sy >= 0 && sx >= 0 && sy < hp && sx < wp;
                    int cy = sy < 0 ? 0 : (sy > hp - 1 ? hp - 1 : sy);
                    int cx = sx < 0 ? 0 : (sx > wp - 1 ? wp - 1 : sx);
                    idx[k] = (uint32_t)(cy * wp + cx);
                    keep[k] = (uint8_t)inside;
                    ++k;
                }
}

static int sat_sub(int a, int b) { return a > b ? a - b : 0; }

static void label_plane(const or_plan *p, uint32_t *label)
{
    int hp = p->hp, wp = p->wp, win = p->win, shift = p->shift;
    int cy[3][2] = {{0, sat_sub(hp, win)}, {sat_sub(hp, win), sat_sub(hp, shift)},
                    {sat_sub(hp, shift), hp}};
    int cx[3][2] = {{0, sat_sub(wp, win)}, {sat_sub(wp, win), sat_sub(wp, shift)},
                    {sat_sub(wp, shift), wp}};
    uint32_t region = 0;
    for (int a = 0; a < 3; ++a)
        for (int b = 0; b < 3; ++b) {
            for (int y = cy[a][0]; y < cy[a][1]; ++y)
                for (int x = cx[b][0]; x < cx[b][1]; ++x) label[y * wp + x] = region;
            ++region;
        }
}

/* mask_label (plan.rs:300-334) */
void or_mask_label(const or_plan *p, uint32_t *out)
{
    int hp = p->hp, wp = p->wp, win = p->win, ny = or_plan_ny(p), nx = or_plan_nx(p);
    uint32_t *label = (uint32_t *)xmalloc(sizeof(uint32_t) * (size_t)hp * wp);
    label_plane(p, label);
    long k = 0;
    for (int wy = 0; wy < ny; ++wy)
        for (int wx = 0; wx < nx; ++wx)
            for (int y = 0; y < win; ++y)
                for (int x = 0; x < win; ++x) out[k++] = label[(wy * win + y) * wp + wx * win + x];
    free(label);
}

/* shift_mask (plan.rs:241-290): 0 where labels agree, -100 where they do not. */
void or_shift_mask(const or_plan *p, float *mask)
{
    int win = p->win, n = win * win, nw = or_plan_nw(p);
    uint32_t *lab = (uint32_t *)xmalloc(sizeof(uint32_t) * (size_t)nw * n);
    or_mask_label(p, lab);
    for (int w = 0; w < nw; ++w) {
        const uint32_t *l = lab + (size_t)w * n;
        float *m = mask + (size_t)w * n * n;
        for (int q = 0; q < n; ++q)
            for (int k = 0; k < n; ++k) m[(size_t)q * n + k] = l[q] == l[k] ? 0.0f : -100.0f;
    }
    free(lab);
}

/* rpi_sa (plan.rs:357-372): (query - key) + (win - 1) per axis. */
void or_rpi_sa(int win, uint32_t *out)
{
    int n = win * win;
    for (int qy = 0; qy < win; ++qy)
        for (int qx = 0; qx < win; ++qx)
            for (int ky = 0; ky < win; ++ky)
                for (int kx = 0; kx < win; ++kx) {
                    int dh = qy + win - 1 - ky;
                    int dw = qx + win - 1 - kx;
                    out[(qy * win + qx) * n + ky * win + kx] = (uint32_t)(dh * (2 * win - 1) + dw);
                }
}

/* rpi_oca (plan.rs:397-416): (key - query) + (win - owin + 1), folded with
 * rem_euclid into the (win+owin-1)^2-row table. */
void or_rpi_oca(int win, int owin, uint32_t *out)
{
    int nk = owin * owin;
    int shift = win - owin + 1;
    int side = win + owin - 1;
    int rows = side * side;
    for (int qy = 0; qy < win; ++qy)
        for (int qx = 0; qx < win; ++qx)
            for (int ky = 0; ky < owin; ++ky)
                for (int kx = 0; kx < owin; ++kx) {
                    int dh = ky - qy + shift;
                    int dw = kx - qx + shift;
                    int v = (dh * side + dw) % rows;
                    if (v < 0) v += rows;
                    out[(qy * win + qx) * nk + ky * owin + kx] = (uint32_t)v;
                }
}

/* ------------------------------------------------------------------------ */
/* conv3x3 (cpu.rs:304-422): per output, bias first, then for each input
 * channel ascending a per-channel subtotal over (dy, dx) that is added to the
 * accumulator. Blocked along x by BLK pixels like the reference; the
 * arithmetic per output is the same in the interior and edge paths. */
#define BLK 8
typedef struct {
    const float *in;
    float *out;
    const float *w, *b;
    int ci, co, h, wd, relu, blk;
} conv_ctx;

static float conv_one(const conv_ctx *c, int o, int y, int x)
{
    int h = c->h, wd = c->wd;
    long hw = (long)h * wd;
    float acc = c->b[o];
    const float *kb = c->w + (size_t)o * c->ci * 9;
    for (int ch = 0; ch < c->ci; ++ch) {
        const float *p = c->in + (size_t)ch * hw;
        const float *k = kb + ch * 9;
        float s = 0.0f;
        if (y > 0) {
            const float *r = p + (size_t)(y - 1) * wd;
            if (x > 0) s += r[x - 1] * k[0];
            s += r[x] * k[1];
            if (x + 1 < wd) s += r[x + 1] * k[2];
        }
        {
            const float *r = p + (size_t)y * wd;
            if (x > 0) s += r[x - 1] * k[3];
            s += r[x] * k[4];
            if (x + 1 < wd) s += r[x + 1] * k[5];
        }
        if (y + 1 < h) {
            const float *r = p + (size_t)(y + 1) * wd;
            if (x > 0) s += r[x - 1] * k[6];
            s += r[x] * k[7];
            if (x + 1 < wd) s += r[x + 1] * k[8];
        }
        acc += s;
    }
    return acc;
}

static void conv_task(void *vctx, long g0, long g1)
{
    const conv_ctx *c = (const conv_ctx *)vctx;
    int h = c->h, wd = c->wd;
    long hw = (long)h * wd;
    for (long gi = g0; gi < g1; ++gi) {
        long i0 = gi * c->blk;
        int o = (int)(i0 / hw);
        long p0 = i0 % hw;
        int y = (int)(p0 / wd), x0 = (int)(p0 % wd);
        float acc[BLK];
        if (c->blk == BLK && x0 >= 1 && x0 + BLK <= wd - 1) {
            /* interior fast path (cpu.rs:351-376) */
            const float *kb = c->w + (size_t)o * c->ci * 9;
            for (int j = 0; j < BLK; ++j) acc[j] = c->b[o];
            for (int ch = 0; ch < c->ci; ++ch) {
                const float *p = c->in + (size_t)ch * hw;
                const float *k = kb + ch * 9;
                float s[BLK] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int dy = 0; dy < 3; ++dy) {
                    if ((dy == 0 && y == 0) || (dy == 2 && y + 1 == h)) continue;
                    const float *r = p + (size_t)(y + dy - 1) * wd;
                    for (int dx = 0; dx < 3; ++dx) {
                        float kk = k[dy * 3 + dx];
                        const float *rb = r + x0 - 1 + dx;
                        for (int j = 0; j < BLK; ++j) s[j] += rb[j] * kk;
                    }
                }
                for (int j = 0; j < BLK; ++j) acc[j] += s[j];
            }
        } else {
            for (int j = 0; j < c->blk; ++j) acc[j] = conv_one(c, o, y, x0 + j);
        }
        float *d = c->out + i0;
        for (int j = 0; j < c->blk; ++j) d[j] = c->relu ? (acc[j] > 0.0f ? acc[j] : 0.0f) : acc[j];
    }
}

void or_conv3x3(const float *in, float *out, const float *w, const float *b, int ci, int co,
                int h, int wd, int relu)
{
    conv_ctx c = {in, out, w, b, ci, co, h, wd, relu, (wd % BLK == 0) ? BLK : 1};
    long n = (long)co * h * wd / c.blk;
    par_for(n, grain_for(n), conv_task, &c);
}

/* conv1x1 (cpu.rs:435-448): b + sum over c ascending. */
void or_conv1x1(const float *in, float *out, const float *w, const float *b, int ci, int co,
                int hw)
{
    for (int o = 0; o < co; ++o)
        for (int i = 0; i < hw; ++i) {
            float acc = b[o];
            for (int c = 0; c < ci; ++c) acc += in[(size_t)c * hw + i] * w[(size_t)o * ci + c];
            out[(size_t)o * hw + i] = acc;
        }
}

/* linear (cpu.rs:456-555): out = x W^T + b; acc = bias, then c ascending.
 * The 8x8 register tile only moves loads; each output's order is unchanged. */
typedef struct {
    const float *x;
    float *out;
    const float *w, *b;
    int ci, co;
    long rows;
} lin_ctx;

static void lin_task(void *vctx, long rb0, long rb1)
{
    const lin_ctx *L = (const lin_ctx *)vctx;
    int ci = L->ci, co = L->co;
    for (long rb = rb0; rb < rb1; ++rb) {
        long r0 = rb * 8;
        int nr = (int)(L->rows - r0 < 8 ? L->rows - r0 : 8);
        for (int o0 = 0; o0 < co; o0 += 8) {
            int nc = co - o0 < 8 ? co - o0 : 8;
            float acc[8][8];
            if (nr == 8 && nc == 8) {
                for (int i = 0; i < 8; ++i)
                    for (int j = 0; j < 8; ++j) acc[i][j] = L->b[o0 + j];
                for (int c = 0; c < ci; ++c) {
                    float xv[8], wv[8];
                    for (int i = 0; i < 8; ++i) xv[i] = L->x[(size_t)(r0 + i) * ci + c];
                    for (int j = 0; j < 8; ++j) wv[j] = L->w[(size_t)(o0 + j) * ci + c];
                    for (int i = 0; i < 8; ++i)
                        for (int j = 0; j < 8; ++j) acc[i][j] += xv[i] * wv[j];
                }
            } else {
                for (int i = 0; i < nr; ++i)
                    for (int j = 0; j < nc; ++j) acc[i][j] = L->b[o0 + j];
                for (int c = 0; c < ci; ++c)
                    for (int i = 0; i < nr; ++i)
                        for (int j = 0; j < nc; ++j)
                            acc[i][j] += L->x[(size_t)(r0 + i) * ci + c] * L->w[(size_t)(o0 + j) * ci + c];
            }
            for (int i = 0; i < nr; ++i)
                for (int j = 0; j < nc; ++j) L->out[(size_t)(r0 + i) * co + o0 + j] = acc[i][j];
        }
    }
}

void or_linear(const float *x, float *out, const float *w, const float *b, int ci, int co,
               long rows)
{
    lin_ctx L = {x, out, w, b, ci, co, rows};
    long nb = (rows + 7) / 8;
    par_for(nb, grain_for(nb), lin_task, &L);
}

/* layer_norm (cpu.rs:563-581): two-pass mean then biased variance, eps 1e-5,
 * y = (x - mean) * rstd * w + b. */
typedef struct {
    float *x;
    const float *w, *b;
    int c;
    float eps;
} ln_ctx;

static void ln_task(void *vctx, long r0, long r1)
{
    const ln_ctx *L = (const ln_ctx *)vctx;
    int c = L->c;
    for (long r = r0; r < r1; ++r) {
        float *row = L->x + (size_t)r * c;
        float mean = 0.0f;
        for (int i = 0; i < c; ++i) mean += row[i];
        mean /= (float)c;
        float var = 0.0f;
        for (int i = 0; i < c; ++i) {
            float d = row[i] - mean;
            var += d * d;
        }
        var /= (float)c;
        float rstd = 1.0f / sqrtf(var + L->eps);
        for (int i = 0; i < c; ++i) row[i] = (row[i] - mean) * rstd * L->w[i] + L->b[i];
    }
}

void or_layer_norm(float *x, const float *w, const float *b, int c, long rows, float eps)
{
    ln_ctx L = {x, w, b, c, eps};
    par_for(rows, grain_for(rows), ln_task, &L);
}

/* erf (cpu.rs:597-603): Abramowitz & Stegun 7.1.26. */
float or_erf(float x)
{
    float sign = x < 0.0f ? -1.0f : 1.0f;
    x = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * x);
    float poly = ((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t
                 + 0.254829592f;
    float y = 1.0f - poly * t * expf(-x * x);
    return sign * y;
}

/* gelu (cpu.rs:585-587): exact-erf form. */
float or_gelu(float v) { return 0.5f * v * (1.0f + or_erf(v * 0.70710677f)); }

typedef struct {
    float *x;
    int kind; /* 0 gelu, 1 leaky 0.01 */
} act_ctx;

static void act_task(void *vctx, long b, long e)
{
    const act_ctx *A = (const act_ctx *)vctx;
    for (long i = b; i < e; ++i) {
        float v = A->x[i];
        if (A->kind == 0)
            A->x[i] = or_gelu(v);
        else if (v < 0.0f)
            A->x[i] = v * 0.01f;
    }
}

static void apply_act(float *x, long n, int kind)
{
    act_ctx A = {x, kind};
    par_for(n, grain_for(n), act_task, &A);
}

/* channel_mean (cpu.rs:610-619): ascending sum over the plane, one divide. */
static void channel_mean(const float *x, float *out, int c, long hw)
{
    for (int ch = 0; ch < c; ++ch) {
        float acc = 0.0f;
        const float *p = x + (size_t)ch * hw;
        for (long i = 0; i < hw; ++i) acc += p[i];
        out[ch] = acc / (float)hw;
    }
}

/* channel_scale (cpu.rs:622-629) */
static void channel_scale(float *x, const float *gate, int c, long hw)
{
    for (int ch = 0; ch < c; ++ch) {
        float g = gate[ch];
        float *p = x + (size_t)ch * hw;
        for (long i = 0; i < hw; ++i) p[i] *= g;
    }
}

/* add_scaled (cpu.rs:632-634): dst += src * scale. */
static void add_scaled(float *dst, const float *src, float scale, long n)
{
    for (long i = 0; i < n; ++i) dst[i] += src[i] * scale;
}

/* gather_windows / scatter_windows (cpu.rs:643-680) */
static void gather_windows(const float *plane, const uint32_t *idx, float *out, int c, int win,
                           long hw, int nw)
{
    int wq = win * win;
    for (long t = 0; t < (long)nw * wq; ++t) {
        long s = idx[t];
        float *d = out + (size_t)t * c;
        for (int ch = 0; ch < c; ++ch) d[ch] = plane[(size_t)ch * hw + s];
    }
}

static void scatter_windows(const float *tok, const uint32_t *idx, float *plane, int c, int win,
                            long hw, int nw)
{
    int wq = win * win;
    for (long t = 0; t < (long)nw * wq; ++t) {
        long d = idx[t];
        for (int ch = 0; ch < c; ++ch) plane[(size_t)ch * hw + d] = tok[(size_t)t * c + ch];
    }
}

/* unfold_kv (cpu.rs:698-721): k channels [0,c), v channels [c,2c) of the 2c
 * plane; zero where keep is 0. */
static void unfold_kv(const float *plane, const uint32_t *idx, const uint8_t *keep, float *k,
                      float *v, int c, int wk, long hw, int nw)
{
    for (long t = 0; t < (long)nw * wk; ++t) {
        long s = idx[t];
        int live = keep[t] != 0;
        for (int ch = 0; ch < c; ++ch) {
            k[(size_t)t * c + ch] = live ? plane[(size_t)ch * hw + s] : 0.0f;
            v[(size_t)t * c + ch] = live ? plane[(size_t)c * hw + (size_t)ch * hw + s] : 0.0f;
        }
    }
}

/* split_qkv (cpu.rs:731-740) */
static void split_qkv(const float *qkv, float *q, float *k, float *v, int c, long rows)
{
    for (long r = 0; r < rows; ++r) {
        memcpy(q + r * c, qkv + r * 3 * c, sizeof(float) * c);
        memcpy(k + r * c, qkv + r * 3 * c + c, sizeof(float) * c);
        memcpy(v + r * c, qkv + r * 3 * c + 2 * c, sizeof(float) * c);
    }
}

static void to_plane(const float *tok, float *plane, int c, long hw)
{
    for (int ch = 0; ch < c; ++ch)
        for (long i = 0; i < hw; ++i) plane[(size_t)ch * hw + i] = tok[(size_t)i * c + ch];
}

static void to_tokens(const float *plane, float *tok, int c, long hw)
{
    for (long i = 0; i < hw; ++i)
        for (int ch = 0; ch < c; ++ch) tok[(size_t)i * c + ch] = plane[(size_t)ch * hw + i];
}

/* window_attention (cpu.rs:772-844): per (window, query) row, heads serial;
 * s = (q.k)*scale + bias (+ mask); max; e = exp(s - max); sum; inv = 1/sum;
 * out = sum_k (e*inv) * v. */
typedef struct {
    const float *q, *k, *v;
    const uint32_t *bias_idx;
    const float *bias_tab;
    const float *mask;
    float *out;
    int nw, nq, nk, heads, d, has_mask;
    float scale;
} attn_ctx;

static void attn_rows(const attn_ctx *A, long r, float *row, float *prob, int per_window_bias)
{
    int nq = A->nq, nk = A->nk, d = A->d, heads = A->heads, c = heads * d;
    long wi = r / nq;
    int qi = (int)(r % nq);
    const float *qw = A->q + (size_t)wi * nq * c;
    const float *kw = A->k + (size_t)wi * nk * c;
    const float *vw = A->v + (size_t)wi * nk * c;
    const float *mw = A->has_mask ? A->mask + (size_t)wi * nq * nq : NULL;
    float *orow = A->out + (size_t)r * c;
    (void)per_window_bias;
    for (int hd = 0; hd < heads; ++hd) {
        const float *qr = qw + (size_t)qi * c + hd * d;
        float mx = -INFINITY;
        for (int ki = 0; ki < nk; ++ki) {
            const float *kr = kw + (size_t)ki * c + hd * d;
            float acc = 0.0f;
            for (int i = 0; i < d; ++i) acc += qr[i] * kr[i];
            float bias = 0.0f;
            if (A->bias_idx && A->bias_tab) {
                uint32_t p = A->bias_idx[(size_t)qi * nk + ki];
                bias = A->bias_tab[(size_t)p * heads + hd];
            }
            float s = acc * A->scale + bias;
            if (mw) s += mw[(size_t)qi * nq + ki];
            row[ki] = s;
            if (s > mx) mx = s;
        }
        float sum = 0.0f;
        for (int ki = 0; ki < nk; ++ki) {
            float e = expf(row[ki] - mx);
            prob[ki] = e;
            sum += e;
        }
        float inv = 1.0f / sum;
        float *dst = orow + hd * d;
        for (int i = 0; i < d; ++i) dst[i] = 0.0f;
        for (int ki = 0; ki < nk; ++ki) {
            float p = prob[ki] * inv;
            const float *vr = vw + (size_t)ki * c + hd * d;
            for (int i = 0; i < d; ++i) dst[i] += p * vr[i];
        }
    }
}

static void attn_task(void *vctx, long r0, long r1)
{
    const attn_ctx *A = (const attn_ctx *)vctx;
    float *row = (float *)xmalloc(sizeof(float) * A->nk);
    float *prob = (float *)xmalloc(sizeof(float) * A->nk);
    for (long r = r0; r < r1; ++r) attn_rows(A, r, row, prob, 0);
    free(row);
    free(prob);
}

void or_window_attention(const float *q, const float *k, const float *v, const uint32_t *bias_idx,
                         const float *bias_tab, const float *mask, float *out, int nw, int nq,
                         int heads, int d, float scale, int has_mask)
{
    attn_ctx A = {q, k, v, bias_idx, bias_tab, mask, out, nw, nq, nq, heads, d, has_mask, scale};
    long n = (long)nw * nq;
    par_for(n, grain_for(n), attn_task, &A);
}

/* overlap_attention (cpu.rs:852-900): the same row arithmetic, nk keys, no
 * mask, bias through the OCA index map. */
void or_overlap_attention(const float *q, const float *k, const float *v,
                          const uint32_t *bias_idx, const float *bias_tab, float *out, int nw,
                          int nq, int nk, int heads, int d, float scale)
{
    attn_ctx A = {q, k, v, bias_idx, bias_tab, NULL, out, nw, nq, nk, heads, d, 0, scale};
    long n = (long)nw * nq;
    par_for(n, grain_for(n), attn_task, &A);
}

/* pixel_shuffle (cpu.rs:1285-1301): in channel c*r*r + i*r + j goes to
 * out channel c at (r*y + i, r*x + j). */
void or_pixel_shuffle(const float *src, float *dst, int c, int h, int w, int r)
{
    int ow = w * r, oh = h * r;
    long shw = (long)h * w, dhw = (long)oh * ow;
    for (int co = 0; co < c; ++co)
        for (int y = 0; y < h; ++y)
            for (int x = 0; x < w; ++x)
                for (int i = 0; i < r; ++i)
                    for (int j = 0; j < r; ++j)
                        dst[(size_t)co * dhw + (size_t)(r * y + i) * ow + (r * x + j)] =
                            src[(size_t)(co * r * r + i * r + j) * shw + (size_t)y * w + x];
}

/* ------------------------------------------------------------------------ */
/* The model: src/cpu.rs:918-1402 */

const float *or_t(const or_model *m, const char *name)
{
    for (int i = 0; i < m->n_tensors; ++i)
        if (strcmp(m->names[i], name) == 0) return m->data[i];
    fprintf(stderr, "oracle: weight `%s` missing\n", name);
    abort();
}

static const float *T(const or_model *m, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
#include <stdarg.h>
static const float *T(const or_model *m, const char *fmt, ...)
{
    char buf[256];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return or_t(m, buf);
}

typedef struct {
    or_plan plan;
    long hw;
    int c, nw, wq, wk;
    float *plane, *plane2, *tok, *tok2, *win, *win_out, *kw, *vw, *okv, *ovv, *oq, *oout, *qkv,
        *hidden, *mask, *hidden_plane, *mid_plane, *pooled, *seq_hidden, *gate, *qplane, *kvplane,
        *proj, *body, *resi;
    uint32_t *wi_shift, *wi_plain, *k_idx, *rpi_sa, *rpi_oca;
    uint8_t *k_keep;
} acts;

static void acts_new(acts *a, const or_plan *p, int mlp_ratio)
{
    memset(a, 0, sizeof *a);
    a->plan = *p;
    int c = p->c;
    long hw = (long)p->hp * p->wp;
    long tok = hw * c;
    a->hw = hw;
    a->c = c;
    a->nw = or_plan_nw(p);
    a->wq = p->win * p->win;
    a->wk = p->owin * p->owin;
    size_t F = sizeof(float);
    a->plane = xmalloc(F * tok);
    a->plane2 = xmalloc(F * tok);
    a->tok = xmalloc(F * tok);
    a->tok2 = xmalloc(F * tok);
    a->win = xmalloc(F * tok);
    a->win_out = xmalloc(F * tok);
    a->kw = xmalloc(F * tok);
    a->vw = xmalloc(F * tok);
    a->okv = xmalloc(F * (size_t)a->nw * a->wk * c);
    a->ovv = xmalloc(F * (size_t)a->nw * a->wk * c);
    a->oq = xmalloc(F * tok);
    a->oout = xmalloc(F * tok);
    a->qkv = xmalloc(F * 3 * tok);
    a->hidden = xmalloc(F * tok * mlp_ratio);
    a->mask = xmalloc(F * (size_t)a->nw * a->wq * a->wq);
    or_shift_mask(p, a->mask);
    a->hidden_plane = xmalloc(F * tok);
    a->mid_plane = xmalloc(F * tok);
    a->pooled = xmalloc(F * c);
    a->seq_hidden = xmalloc(F * c);
    a->gate = xmalloc(F * c);
    a->qplane = xmalloc(F * tok);
    a->kvplane = xmalloc(F * 2 * tok);
    a->proj = xmalloc(F * tok);
    a->body = xmalloc(F * tok);
    a->resi = xmalloc(F * tok);
    a->wi_shift = xmalloc(4 * (size_t)a->nw * a->wq);
    a->wi_plain = xmalloc(4 * (size_t)a->nw * a->wq);
    or_window_index(p, p->shift, a->wi_shift);
    or_window_index(p, 0, a->wi_plain);
    a->k_idx = xmalloc(4 * (size_t)a->nw * a->wk);
    a->k_keep = xmalloc((size_t)a->nw * a->wk);
    or_unfold_index(p, a->k_idx, a->k_keep);
    a->rpi_sa = xmalloc(4 * (size_t)a->wq * a->wq);
    or_rpi_sa(p->win, a->rpi_sa);
    a->rpi_oca = xmalloc(4 * (size_t)a->wq * a->wk);
    or_rpi_oca(p->win, p->owin, a->rpi_oca);
}

static void acts_free(acts *a)
{
    void *ps[] = {a->plane, a->plane2, a->tok, a->tok2, a->win, a->win_out, a->kw, a->vw,
                  a->okv, a->ovv, a->oq, a->oout, a->qkv, a->hidden, a->mask, a->hidden_plane,
                  a->mid_plane, a->pooled, a->seq_hidden, a->gate, a->qplane, a->kvplane,
                  a->proj, a->body, a->resi, a->wi_shift, a->wi_plain, a->k_idx, a->k_keep,
                  a->rpi_sa, a->rpi_oca};
    for (size_t i = 0; i < sizeof ps / sizeof ps[0]; ++i) free(ps[i]);
}

/* cab (cpu.rs:918-960): conv3x3 c->comp, GELU, conv3x3 comp->c, then the
 * channel attention gate; no residual. Result lands in a->plane. */
static void cab(acts *a, const or_model *m, const char *p, int h, int w)
{
    int c = m->embed, comp = m->compressed, sq = m->squeezed;
    long hw = (long)h * w;
    or_conv3x3(a->plane, a->hidden_plane, T(m, "%s.cab.0.weight", p), T(m, "%s.cab.0.bias", p),
               c, comp, h, w, 0);
    apply_act(a->hidden_plane, comp * hw, 0);
    or_conv3x3(a->hidden_plane, a->mid_plane, T(m, "%s.cab.2.weight", p),
               T(m, "%s.cab.2.bias", p), comp, c, h, w, 0);
    channel_mean(a->mid_plane, a->pooled, c, hw);
    or_conv1x1(a->pooled, a->seq_hidden, T(m, "%s.cab.3.attention.1.weight", p),
               T(m, "%s.cab.3.attention.1.bias", p), c, sq, 1);
    for (int i = 0; i < c; ++i)
        if (a->seq_hidden[i] < 0.0f) a->seq_hidden[i] = 0.0f;
    or_conv1x1(a->seq_hidden, a->gate, T(m, "%s.cab.3.attention.3.weight", p),
               T(m, "%s.cab.3.attention.3.bias", p), sq, c, 1);
    for (int i = 0; i < c; ++i) a->gate[i] = 1.0f / (1.0f + expf(-a->gate[i]));
    channel_scale(a->mid_plane, a->gate, c, hw);
    float *t = a->plane;
    a->plane = a->mid_plane;
    a->mid_plane = t;
}

/* hab (cpu.rs:1090-1166) */
static void hab(acts *a, const or_model *m, int stage, int block)
{
    const or_plan *pl = &a->plan;
    int c = m->embed;
    long hw = a->hw;
    int h = pl->hp, w = pl->wp, nw = a->nw, wq = a->wq;
    char p[128];
    snprintf(p, sizeof p, "layers.%d.residual_group.blocks.%d", stage, block);
    int shifted = block % 2 == 1;
    float scale = 1.0f / sqrtf((float)m->head_dim);
    long n = hw * c;

    memcpy(a->plane2, a->plane, sizeof(float) * n);
    to_tokens(a->plane, a->tok, c, hw);
    or_layer_norm(a->tok, T(m, "%s.norm1.weight", p), T(m, "%s.norm1.bias", p), c, hw, 1e-5f);
    to_plane(a->tok, a->mid_plane, c, hw);
    float *t = a->plane;
    a->plane = a->mid_plane;
    a->mid_plane = t;
    char cp[160];
    snprintf(cp, sizeof cp, "%s.conv_block", p);
    cab(a, m, cp, h, w);

    memcpy(a->mid_plane, a->plane, sizeof(float) * n); /* conv_x */
    memcpy(a->plane, a->plane2, sizeof(float) * n);    /* shortcut */

    to_plane(a->tok, a->qplane, c, hw);
    const uint32_t *idx = shifted ? a->wi_shift : a->wi_plain;
    gather_windows(a->qplane, idx, a->win, c, pl->win, hw, nw);
    or_linear(a->win, a->qkv, T(m, "%s.attn.qkv.weight", p), T(m, "%s.attn.qkv.bias", p), c,
              3 * c, (long)nw * wq);
    split_qkv(a->qkv, a->win, a->kw, a->vw, c, (long)nw * wq);
    or_window_attention(a->win, a->kw, a->vw, a->rpi_sa,
                        T(m, "%s.attn.relative_position_bias_table", p),
                        shifted ? a->mask : NULL, a->win_out, nw, wq, m->heads, m->head_dim,
                        scale, shifted);
    or_linear(a->win_out, a->tok2, T(m, "%s.attn.proj.weight", p), T(m, "%s.attn.proj.bias", p),
              c, c, (long)nw * wq);
    scatter_windows(a->tok2, idx, a->plane, c, pl->win, hw, nw);
    add_scaled(a->plane, a->plane2, 1.0f, n);
    add_scaled(a->plane, a->mid_plane, m->conv_scale, n);

    to_tokens(a->plane, a->tok, c, hw);
    or_layer_norm(a->tok, T(m, "%s.norm2.weight", p), T(m, "%s.norm2.bias", p), c, hw, 1e-5f);
    int hidden = m->mlp_ratio * c;
    or_linear(a->tok, a->hidden, T(m, "%s.mlp.fc1.weight", p), T(m, "%s.mlp.fc1.bias", p), c,
              hidden, hw);
    apply_act(a->hidden, hw * hidden, 0);
    or_linear(a->hidden, a->tok2, T(m, "%s.mlp.fc2.weight", p), T(m, "%s.mlp.fc2.bias", p),
              hidden, c, hw);
    to_plane(a->tok2, a->plane2, c, hw);
    add_scaled(a->plane, a->plane2, 1.0f, n);
}

/* ocab (cpu.rs:983-1055): qkv on the normed tokens in a->tok; q windows,
 * unfolded k/v; the projected result is scattered into a->plane2. */
static void ocab(acts *a, const or_model *m, int stage)
{
    const or_plan *pl = &a->plan;
    int c = m->embed;
    long hw = a->hw;
    int nw = a->nw, wq = a->wq, wk = a->wk;
    char p[128];
    snprintf(p, sizeof p, "layers.%d.residual_group.overlap_attn", stage);
    float scale = 1.0f / sqrtf((float)m->head_dim);
    or_linear(a->tok, a->qkv, T(m, "%s.qkv.weight", p), T(m, "%s.qkv.bias", p), c, 3 * c, hw);
    for (int ch = 0; ch < c; ++ch)
        for (long i = 0; i < hw; ++i) a->qplane[(size_t)ch * hw + i] = a->qkv[(size_t)i * 3 * c + ch];
    gather_windows(a->qplane, a->wi_plain, a->oq, c, pl->win, hw, nw);
    for (int ch = 0; ch < 2 * c; ++ch) {
        int src = ch < c ? c + ch : 2 * c + (ch - c);
        for (long i = 0; i < hw; ++i)
            a->kvplane[(size_t)ch * hw + i] = a->qkv[(size_t)i * 3 * c + src];
    }
    unfold_kv(a->kvplane, a->k_idx, a->k_keep, a->okv, a->ovv, c, wk, hw, nw);
    or_overlap_attention(a->oq, a->okv, a->ovv, a->rpi_oca,
                         T(m, "%s.relative_position_bias_table", p), a->oout, nw, wq, wk,
                         m->heads, m->head_dim, scale);
    or_linear(a->oout, a->proj, T(m, "%s.proj.weight", p), T(m, "%s.proj.bias", p), c, c,
              (long)nw * wq);
    scatter_windows(a->proj, a->wi_plain, a->plane2, c, pl->win, hw, nw);
}

/* ocab_block (cpu.rs:1170-1198) */
static void ocab_block(acts *a, const or_model *m, int stage)
{
    int c = m->embed;
    long hw = a->hw, n = hw * c;
    char p[128];
    snprintf(p, sizeof p, "layers.%d.residual_group.overlap_attn", stage);
    memcpy(a->plane2, a->plane, sizeof(float) * n);
    to_tokens(a->plane, a->tok, c, hw);
    or_layer_norm(a->tok, T(m, "%s.norm1.weight", p), T(m, "%s.norm1.bias", p), c, hw, 1e-5f);
    ocab(a, m, stage);
    add_scaled(a->plane, a->plane2, 1.0f, n);
    to_tokens(a->plane, a->tok, c, hw);
    or_layer_norm(a->tok, T(m, "%s.norm2.weight", p), T(m, "%s.norm2.bias", p), c, hw, 1e-5f);
    int hidden = m->mlp_ratio * c;
    or_linear(a->tok, a->hidden, T(m, "%s.mlp.fc1.weight", p), T(m, "%s.mlp.fc1.bias", p), c,
              hidden, hw);
    apply_act(a->hidden, hw * hidden, 0);
    or_linear(a->hidden, a->tok2, T(m, "%s.mlp.fc2.weight", p), T(m, "%s.mlp.fc2.bias", p),
              hidden, c, hw);
    to_plane(a->tok2, a->plane2, c, hw);
    add_scaled(a->plane, a->plane2, 1.0f, n);
}

/* rhag (cpu.rs:1206-1225) */
static void rhag(acts *a, const or_model *m, int stage)
{
    int c = m->embed;
    long n = a->hw * c;
    memcpy(a->resi, a->plane, sizeof(float) * n);
    for (int b = 0; b < m->depths[stage]; ++b) hab(a, m, stage, b);
    ocab_block(a, m, stage);
    or_conv3x3(a->plane, a->hidden_plane, T(m, "layers.%d.conv.weight", stage),
               T(m, "layers.%d.conv.bias", stage), c, c, a->plan.hp, a->plan.wp, 0);
    memcpy(a->plane, a->hidden_plane, sizeof(float) * n);
    add_scaled(a->plane, a->resi, 1.0f, n);
}

/* Weights::up_blocks (weights.rs:290-305): (factor, widened) per block. */
static int up_blocks(const or_model *m, int *r, int *widened)
{
    int feat = m->head_feat;
    if (m->scale == 3) {
        r[0] = 3;
        widened[0] = 9 * feat;
        return 1;
    }
    int s = m->scale, n = 0;
    while (s > 1 && s % 2 == 0) {
        ++n;
        s /= 2;
    }
    if (s != 1) return 0;
    for (int i = 0; i < n; ++i) {
        r[i] = 2;
        widened[i] = 4 * feat;
    }
    return n;
}

/* head (cpu.rs:1232-1271); returns the output plane [3][hh][ww] (malloc'd). */
static float *head(acts *a, const or_model *m, int *oh, int *ow)
{
    int c = m->embed, feat = m->head_feat;
    int h = a->plan.hp, w = a->plan.wp;
    long hw = (long)h * w;
    float *cur = xmalloc(sizeof(float) * feat * hw);
    or_conv3x3(a->plane, cur, or_t(m, "conv_before_upsample.0.weight"),
               or_t(m, "conv_before_upsample.0.bias"), c, feat, h, w, 0);
    apply_act(cur, (long)feat * hw, 1);
    int rr[8], wd[8];
    int nb = up_blocks(m, rr, wd);
    int hh = h, ww = w;
    for (int b = 0; b < nb; ++b) {
        float *wide = xmalloc(sizeof(float) * (size_t)wd[b] * hh * ww);
        or_conv3x3(cur, wide, T(m, "upsample.%d.weight", 2 * b), T(m, "upsample.%d.bias", 2 * b),
                   feat, wd[b], hh, ww, 0);
        int nh = hh * rr[b], nwd = ww * rr[b];
        float *next = xmalloc(sizeof(float) * (size_t)feat * nh * nwd);
        or_pixel_shuffle(wide, next, feat, hh, ww, rr[b]);
        free(wide);
        free(cur);
        cur = next;
        hh = nh;
        ww = nwd;
    }
    float *out = xmalloc(sizeof(float) * 3 * (size_t)hh * ww);
    or_conv3x3(cur, out, or_t(m, "conv_last.weight"), or_t(m, "conv_last.bias"), feat, 3, hh, ww,
               0);
    free(cur);
    *oh = hh;
    *ow = ww;
    return out;
}

/* forward_planes (cpu.rs:1318-1368) */
static float *forward_planes(acts *a, const or_model *m, int *oh, int *ow)
{
    int c = m->embed;
    long hw = a->hw, n = hw * c;
    int h = a->plan.hp, w = a->plan.wp;
    or_conv3x3(a->plane, a->hidden_plane, or_t(m, "conv_first.weight"), or_t(m, "conv_first.bias"),
               3, c, h, w, 0);
    memcpy(a->body, a->hidden_plane, sizeof(float) * n);
    memcpy(a->plane, a->hidden_plane, sizeof(float) * n);
    to_tokens(a->plane, a->tok, c, hw);
    or_layer_norm(a->tok, or_t(m, "patch_embed.norm.weight"), or_t(m, "patch_embed.norm.bias"), c,
                  hw, 1e-5f);
    to_plane(a->tok, a->plane, c, hw);
    for (int s = 0; s < m->n_stages; ++s) rhag(a, m, s);
    to_tokens(a->plane, a->tok, c, hw);
    or_layer_norm(a->tok, or_t(m, "norm.weight"), or_t(m, "norm.bias"), c, hw, 1e-5f);
    to_plane(a->tok, a->plane, c, hw);
    or_conv3x3(a->plane, a->hidden_plane, or_t(m, "conv_after_body.weight"),
               or_t(m, "conv_after_body.bias"), c, c, h, w, 0);
    memcpy(a->plane, a->hidden_plane, sizeof(float) * n);
    add_scaled(a->plane, a->body, 1.0f, n);
    return head(a, m, oh, ow);
}

/* Cpu::forward (cpu.rs:1381-1402) with Pre::adjust and finish
 * (backend.rs:71-109): edge-replicated padding, (x - mean) * img_range in,
 * crop and / img_range + mean out. */
int or_forward(const or_model *m, int h, int w, const float *in, float *out)
{
    if (h <= 0 || w <= 0) return 1;
    or_plan p;
    or_plan_new(&p, h, w, m->window, m->embed);
    acts a;
    acts_new(&a, &p, m->mlp_ratio);
    int hp = p.hp, wp = p.wp;
    long phw = (long)hp * wp, ihw = (long)h * w;
    for (int ch = 0; ch < 3; ++ch) {
        float mn = m->mean[ch];
        for (int y = 0; y < hp; ++y) {
            int sy = y < h - 1 ? y : h - 1;
            for (int x = 0; x < wp; ++x) {
                int sx = x < w - 1 ? x : w - 1;
                a.plane[(size_t)ch * phw + (size_t)y * wp + x] =
                    (in[(size_t)ch * ihw + (size_t)sy * w + sx] - mn) * m->img_range;
            }
        }
    }
    int oh, ow;
    float *planes = forward_planes(&a, m, &oh, &ow);
    int ch_ = h * m->scale, cw = w * m->scale;
    for (int ch = 0; ch < 3; ++ch) {
        float mn = m->mean[ch];
        for (int y = 0; y < ch_; ++y)
            for (int x = 0; x < cw; ++x)
                out[(size_t)ch * ch_ * cw + (size_t)y * cw + x] =
                    planes[(size_t)ch * oh * ow + (size_t)y * ow + x] / m->img_range + mn;
    }
    free(planes);
    acts_free(&a);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Isolated ops (token-major I/O). */

void or_swmsa_op(const float *x, float *out, int hp, int wp, int c, int heads, int win, int shift,
                 const float *qkv_w, const float *qkv_b, const float *proj_w, const float *proj_b,
                 const float *rpb_table)
{
    or_plan p;
    or_plan_new(&p, hp, wp, win, c);
    int nw = or_plan_nw(&p), wq = win * win, d = c / heads;
    long hw = (long)hp * wp, n = hw * c;
    float *plane = xmalloc(sizeof(float) * n), *wtok = xmalloc(sizeof(float) * n);
    float *qkv = xmalloc(sizeof(float) * 3 * n), *q = xmalloc(sizeof(float) * n),
          *k = xmalloc(sizeof(float) * n), *v = xmalloc(sizeof(float) * n),
          *o = xmalloc(sizeof(float) * n);
    uint32_t *idx = xmalloc(4 * (size_t)nw * wq), *rpi = xmalloc(4 * (size_t)wq * wq);
    float *mask = NULL;
    or_window_index(&p, shift, idx);
    or_rpi_sa(win, rpi);
    if (shift > 0) {
        mask = xmalloc(sizeof(float) * (size_t)nw * wq * wq);
        or_shift_mask(&p, mask);
    }
    to_plane(x, plane, c, hw);
    gather_windows(plane, idx, wtok, c, win, hw, nw);
    or_linear(wtok, qkv, qkv_w, qkv_b, c, 3 * c, (long)nw * wq);
    split_qkv(qkv, q, k, v, c, (long)nw * wq);
    or_window_attention(q, k, v, rpi, rpb_table, mask, o, nw, wq, heads, d,
                        1.0f / sqrtf((float)d), shift > 0);
    or_linear(o, wtok, proj_w, proj_b, c, c, (long)nw * wq);
    scatter_windows(wtok, idx, plane, c, win, hw, nw);
    to_tokens(plane, out, c, hw);
    free(plane); free(wtok); free(qkv); free(q); free(k); free(v); free(o); free(idx); free(rpi);
    free(mask);
}

void or_ocab_op(const float *x, float *out, int hp, int wp, int c, int heads, int win, int owin,
                int mlp_ratio, const float *n1w, const float *n1b, const float *qkv_w,
                const float *qkv_b, const float *proj_w, const float *proj_b,
                const float *rpb_table, const float *n2w, const float *n2b, const float *fc1_w,
                const float *fc1_b, const float *fc2_w, const float *fc2_b)
{
    const char *names[] = {"layers.0.residual_group.overlap_attn.norm1.weight",
                           "layers.0.residual_group.overlap_attn.norm1.bias",
                           "layers.0.residual_group.overlap_attn.qkv.weight",
                           "layers.0.residual_group.overlap_attn.qkv.bias",
                           "layers.0.residual_group.overlap_attn.proj.weight",
                           "layers.0.residual_group.overlap_attn.proj.bias",
                           "layers.0.residual_group.overlap_attn.relative_position_bias_table",
                           "layers.0.residual_group.overlap_attn.norm2.weight",
                           "layers.0.residual_group.overlap_attn.norm2.bias",
                           "layers.0.residual_group.overlap_attn.mlp.fc1.weight",
                           "layers.0.residual_group.overlap_attn.mlp.fc1.bias",
                           "layers.0.residual_group.overlap_attn.mlp.fc2.weight",
                           "layers.0.residual_group.overlap_attn.mlp.fc2.bias"};
    const float *data[] = {n1w, n1b, qkv_w, qkv_b, proj_w, proj_b, rpb_table,
                           n2w, n2b, fc1_w, fc1_b, fc2_w, fc2_b};
    or_model m;
    memset(&m, 0, sizeof m);
    m.window = win;
    m.owin = owin;
    m.embed = c;
    m.heads = heads;
    m.head_dim = c / heads;
    m.mlp_ratio = mlp_ratio;
    m.n_tensors = 13;
    m.names = names;
    m.data = data;
    or_plan p;
    or_plan_new(&p, hp, wp, win, c);
    p.owin = owin;
    acts a;
    acts_new(&a, &p, mlp_ratio);
    to_plane(x, a.plane, c, a.hw);
    ocab_block(&a, &m, 0);
    to_tokens(a.plane, out, c, a.hw);
    acts_free(&a);
}

void or_hab_op(const or_model *m, const float *x, float *out, int hp, int wp, int stage, int block)
{
    or_plan p;
    or_plan_new(&p, hp, wp, m->window, m->embed);
    acts a;
    acts_new(&a, &p, m->mlp_ratio);
    to_plane(x, a.plane, m->embed, a.hw);
    hab(&a, m, stage, block);
    to_tokens(a.plane, out, m->embed, a.hw);
    acts_free(&a);
}
