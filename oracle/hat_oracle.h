/*
 * hat_oracle.h - TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU path (jacobsparts/hat-rs
 * src/cpu.rs, src/plan.rs, src/backend.rs), written to be the parity checker
 * for the MI355X path and the timed CPU baseline. Only tests/, the smoke()
 * entry of __graft_entry__.py and bench.py's cpu_baseline leg may load it.
 * Nothing in hat-rs_amd/ links it or calls it.
 *
 * Every function keeps the reference's reduction order (channel-ascending
 * sums, two-pass LayerNorm, max-subtracted softmax with one reciprocal, ...)
 * so that a difference against it is a difference of the GPU path, not of
 * the checker. Parallelism is over output elements only, as the reference's
 * rayon loops are, so the thread count never changes a result.
 */
#ifndef HAT_ORACLE_H
#define HAT_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- threading ---------------------------------------------------------- */
void or_set_threads(int n);
int or_get_threads(void);

/* ---- geometry (src/plan.rs) --------------------------------------------- */
typedef struct {
    int h, w;    /* input size */
    int hp, wp;  /* padded to a window multiple */
    int c, win, shift, owin;
} or_plan;

void or_plan_new(or_plan *p, int h, int w, int win, int c);
int or_plan_nx(const or_plan *p);
int or_plan_ny(const or_plan *p);
int or_plan_nw(const or_plan *p);
int or_plan_opad(const or_plan *p);
void or_window_index(const or_plan *p, int shift, uint32_t *out);
void or_unfold_index(const or_plan *p, uint32_t *idx, uint8_t *keep);
void or_shift_mask(const or_plan *p, float *mask);
void or_mask_label(const or_plan *p, uint32_t *out);
void or_rpi_sa(int win, uint32_t *out);
void or_rpi_oca(int win, int owin, uint32_t *out);

/* ---- primitives (src/cpu.rs) -------------------------------------------- */
void or_conv3x3(const float *in, float *out, const float *w, const float *b, int ci, int co,
                int h, int wd, int relu);
void or_conv1x1(const float *in, float *out, const float *w, const float *b, int ci, int co,
                int hw);
void or_linear(const float *x, float *out, const float *w, const float *b, int ci, int co,
               long rows);
void or_layer_norm(float *x, const float *w, const float *b, int c, long rows, float eps);
float or_erf(float x);
float or_gelu(float v);
void or_pixel_shuffle(const float *src, float *dst, int c, int h, int w, int r);
void or_window_attention(const float *q, const float *k, const float *v, const uint32_t *bias_idx,
                         const float *bias_tab, const float *mask, float *out, int nw, int nq,
                         int heads, int d, float scale, int has_mask);
void or_overlap_attention(const float *q, const float *k, const float *v,
                          const uint32_t *bias_idx, const float *bias_tab, float *out, int nw,
                          int nq, int nk, int heads, int d, float scale);

/* ---- whole model --------------------------------------------------------- */
typedef struct {
    int scale, window, owin, embed, heads, head_dim, mlp_ratio;
    int n_stages;
    int depths[32];
    int compressed, squeezed, head_feat;
    float conv_scale, img_range;
    float mean[3];
    /* weight lookup table: names and f32 data pointers (owned by the caller) */
    int n_tensors;
    const char **names;
    const float **data;
} or_model;

const float *or_t(const or_model *m, const char *name);
/* Backend::forward: in [3][h][w] in [0,1], out [3][h*s][w*s]. */
int or_forward(const or_model *m, int h, int w, const float *in, float *out);

/* Isolated ops on token-major [hp*wp][c] feature maps.
 * SW-MSA: gather (with the roll when shift>0) -> qkv -> attention(+mask) -> proj ->
 * scatter; this is the attention branch of HAB.forward without norm1. */
void or_swmsa_op(const float *x, float *out, int hp, int wp, int c, int heads, int win, int shift,
                 const float *qkv_w, const float *qkv_b, const float *proj_w, const float *proj_b,
                 const float *rpb_table);
/* The whole OCAB block: norm1, qkv, unfold, attention, proj + shortcut, norm2, MLP. */
void or_ocab_op(const float *x, float *out, int hp, int wp, int c, int heads, int win, int owin,
                int mlp_ratio, const float *n1w, const float *n1b, const float *qkv_w,
                const float *qkv_b, const float *proj_w, const float *proj_b,
                const float *rpb_table, const float *n2w, const float *n2b, const float *fc1_w,
                const float *fc1_b, const float *fc2_w, const float *fc2_b);
/* One HAB on a token-major map, with the block's weights looked up under `prefix`. */
void or_hab_op(const or_model *m, const float *x, float *out, int hp, int wp, int stage,
               int block);

#ifdef __cplusplus
}
#endif
#endif
