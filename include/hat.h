/*
 * hat.h - the C ABI of the MI355X HAT backend (libhat.so).
 *
 * A drop-in for the reference's GPU backend (jacobsparts/hat-rs). Every entry
 * point names the reference interface it replaces. Plain pointers and sizes
 * only; no GPU runtime types cross this boundary. Errors: functions returning
 * int give 0 on success (or a count, where stated) and a negative value on
 * failure; functions returning a pointer give NULL on failure. In both cases
 * hat_last_error() holds the message (thread-local), the counterpart of the
 * reference's `Result<_, String>` printed as `hat: <msg>` (src/main.rs:189-195).
 */
#ifndef HAT_H
#define HAT_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hat_weights hat_weights;
typedef struct hat_backend hat_backend;

/* Library version string (the reference's hat::VERSION, src/lib.rs). */
const char *hat_version(void);

/* The last error message on this thread, or "" (main.rs:189-195). */
const char *hat_last_error(void);

/* ---- Weights (src/weights.rs) ------------------------------------------ */

/* Weights::load (weights.rs:60-129): mmap a converted .safetensors file, read
 * the architecture from __metadata__, validate every tensor shape
 * (weights.rs:133-265). */
hat_weights *hat_weights_open(const char *path);
void hat_weights_close(hat_weights *w);

/* The architecture fields of `Weights` (weights.rs:28-57). */
typedef struct {
    int scale, window, owin, embed, heads, head_dim, mlp_ratio;
    int n_stages;
    int depths[32];
    int compressed, squeezed, head_feat;
    float conv_scale, img_range;
    float mean[3];
} hat_model_info;
int hat_weights_info(const hat_weights *w, hat_model_info *out);

/* The checkpoint's `variant` metadata and its size in bytes (Weights.variant,
 * Weights.bytes, weights.rs:28-57; main.rs:205-206 prints both). */
const char *hat_weights_variant(const hat_weights *w);
unsigned long long hat_weights_file_bytes(const hat_weights *w);

/* Tensor listing and access (weights.rs:270-272 `t`, `--list-weights`). */
int hat_weights_count(const hat_weights *w);
const char *hat_weights_name(const hat_weights *w, int i);
/* F32 tensor data (owned by the weights object) and its element count. */
const float *hat_weights_tensor(const hat_weights *w, const char *name, size_t *numel);
/* Weights::i64 (weights.rs:331-346): copies up to n int64 values; returns the
 * element count. */
long hat_weights_index_i64(const hat_weights *w, const char *name, long long *out, size_t n);

/* A seeded checkpoint in tools/convert.py's format (convert.py:205-250): every
 * weight, bias and bias table ~ N(0, 0.02), LayerNorm weight 1 / bias 0, the
 * int64 relative-position index buffers from their closed forms. `variant` is
 * "hat-s", "hat" or "hat-l"; `depths` (may be NULL) overrides the variant's
 * per-stage block counts. No reference counterpart: the reference ships
 * converted checkpoints, and this writes the synthetic ones the benchmarks
 * and parity tests use. */
int hat_weights_generate(const char *path, const char *variant, int scale, unsigned long long seed,
                         const int *depths, int n_depths);

/* ---- Backend (src/backend.rs:29-36, src/gpu.rs:372-803) ------------------ */

/* 1 if the HIP runtime and a device can be brought up, else 0 (the probe
 * behind main.rs:148-174 `resolve_device`). Never fails. */
int hat_gpu_available(void);

/* Gpu::new (gpu.rs:372-386): brings up the runtime, checks that every kernel
 * resolves (cuda.rs:558-563) and uploads every weight. `device` must be "gpu"
 * (or NULL): this library has no CPU path, and asking for one is an error
 * rather than a silent fallback. The weights must outlive the backend. */
hat_backend *hat_backend_new(const hat_weights *w, const char *device);
/* Backend::name (backend.rs:30). */
const char *hat_backend_name(const hat_backend *b);
/* Backend::forward (backend.rs:32-35): in = [3][h][w] in [0,1] host memory;
 * out = caller-allocated [3][h*scale][w*scale] host memory. Synchronous. */
int hat_backend_forward(hat_backend *b, size_t h, size_t w, const float *in, float *out);
/* The same pass on device-resident buffers (from hat_device_alloc);
 * asynchronous on the backend's stream until hat_backend_synchronize. */
int hat_backend_forward_device(hat_backend *b, size_t h, size_t w, const float *d_in, float *d_out);
int hat_backend_synchronize(hat_backend *b);
/* hat_backend_forward_device without allocating: no reference counterpart. It
 * is for callers that cannot call hipMalloc (code under graph capture, serving
 * loops that forbid allocation). Every per-plan buffer of the pass is carved
 * from one fixed 256 MiB device array the library holds from load to process
 * exit (enough for HAT-S or HAT x4 up to 128 x 128 input pixels); a larger
 * plan is refused with an error and nothing runs. The caller passes device
 * input and output as for hat_backend_forward_device; the pass is asynchronous
 * on the backend's stream. All calls in a process share the one array: calls
 * that overlap on the GPU (two backends, two streams, two threads) race. */
int hat_backend_forward_noalloc(hat_backend *b, size_t h, size_t w, const float *d_in, float *d_out);
/* One HAB of the backend's network, `hab` (gpu.rs:469-520; HAB.forward,
 * hat_arch.py:266-309): x' = x + W-MSA(norm1 x) + conv_scale * CAB(norm1 x),
 * out = x' + MLP(norm2 x'), for layers.<stage>.residual_group.blocks.<block>,
 * shifted and masked when the block is odd. x/out: host token-major
 * [hp*wp][embed] on a plane whose sides are window multiples. iters > 0: *ms
 * (if non-NULL) = mean device time of the block over that many further runs. */
int hat_backend_hab(hat_backend *b, int stage, int block, size_t hp, size_t wp, const float *x,
                    float *out, int iters, float *ms);
/* Device bytes of the per-plan buffers and of the uploaded weights
 * (Acts/footprint, gpu.rs:78-290). */
size_t hat_backend_acts_bytes(const hat_backend *b);
size_t hat_backend_weight_bytes(const hat_backend *b);
void hat_backend_free(hat_backend *b);

/* ---- Batching, tiling and memory admission (src/tile.rs, src/memguard.rs) */

/* n images of one size through the backend: in = host [n][3][h][w], out =
 * host [n][3][h*scale][w*scale]. Up to 4 images are in flight at once, each on
 * its own stream with its own per-plan buffers, so the kernels of several
 * small images fill the device together (the single-GPU part of multi-image
 * batching). Synchronous; results identical to n calls of hat_backend_forward. */
int hat_backend_forward_batch(hat_backend *b, size_t n, size_t h, size_t w, const float *in, float *out);

/* tile::Tiling (tile.rs:34-45). */
typedef struct {
    size_t tile, margin, scale, tiles, largest_h, largest_w;
} hat_tiling;
/* tile::forward (tile.rs:50-107): the image in window-aligned cores of `tile`
 * input pixels, each run with a halo of `margin` pixels (both rounded up to
 * the window) on every side that is not the image's edge; only the cores are
 * copied to out. info (may be NULL) reports what ran. */
int hat_tile_forward(hat_backend *b, size_t h, size_t w, const float *in, float *out, size_t tile,
                     size_t margin, hat_tiling *info);
/* tile::auto_tile (tile.rs:140-184): the largest window-multiple core whose
 * sub-image (core plus both margins) fits budget_bytes at per_pixel_floats per
 * pixel plus constant_floats; 0 when not even one window fits (None). */
size_t hat_auto_tile(size_t h, size_t w, size_t win, unsigned long long budget_bytes,
                     unsigned long long per_pixel_floats, unsigned long long constant_floats, size_t margin);
/* memguard::Plan (memguard.rs:46-58). */
typedef struct {
    unsigned long long activations, weights, base, need, avail;
    int have_avail;
} hat_mem_plan;
/* memguard::gpu_plan (memguard.rs:147-160): the per-plan device buffers of an
 * h x w pass, the checkpoint's bytes and 128 MiB of runtime, with 5% slack,
 * against free device memory (have_avail = 0 when no device answers). The
 * backend refuses a plan that does not fit, with the reference's message
 * (memguard.rs:162-190), before allocating it. */
int hat_gpu_plan(const hat_weights *w, size_t h, size_t wd, hat_mem_plan *out);
/* main.rs:115-140 gpu_auto_tile: the tile a run without --tile/--mem uses,
 * halved from the larger image side until hat_gpu_plan fits. */
long hat_gpu_auto_tile(const hat_weights *w, size_t h, size_t wd);

/* ---- PNG I/O (src/image.rs) ------------------------------------------- */

/* image::load_rgb (image.rs:43-99): decode an 8- or 16-bit grey, grey+alpha,
 * RGB or RGBA PNG into planar [3][h][w] floats in [0,1]. Sets *w and *h; with
 * out non-NULL also writes the planes (cap >= 3*w*h floats). */
int hat_png_load(const char *path, size_t *w, size_t *h, float *out, size_t cap);
/* image::save_rgb of Image::to_rgb8 (image.rs:30-41,101-114): planar [3][h][w]
 * floats, clamped to [0,1], scaled by 255, rounded half up, as 8-bit RGB. */
int hat_png_save(const char *path, size_t w, size_t h, const float *planes);

/* Weights::shape (weights.rs:275-280, `--list-weights`): writes up to cap
 * dimensions of the named tensor; returns its rank. */
int hat_weights_shape(const hat_weights *w, const char *name, size_t *dims, int cap);

/* ---- Contracts (src/main.rs:312-326, src/selftest.rs:437-523) ----------- */

/* `--verify`: load a HATF v1 fixture (fixture.rs:44-78), run the backend,
 * print "  verify worst |diff| ... at (y, x, ch), mean |diff| ..." and return
 * 0 if the worst difference is within 1e-4, 1 if it is not, -1 on error. */
int hat_verify(const hat_weights *w, const char *device, const char *fixture_path);

/* `--cuda-selftest`: every gfx950 kernel against a host twin; prints
 * "  ok  <name>" per check and returns the number passed, or -1. */
int hat_gpu_selftest(void);

/* ---- Isolated ops (benchmark configs 2 and 3; host buffers) -------------- */

/* Shifted-window self-attention, the attention branch of HAB.forward
 * (hat_arch.py:266-309; cpu.rs:1117-1130): gather with the cyclic shift,
 * qkv linear, attention with relative-position bias and (shift > 0) the
 * SW-MSA mask, proj linear, scatter. x/out are token-major [hp*wp][c]; table is
 * [961][heads]. `iters` > 0 times that many extra runs: *ms = mean device time
 * of the op, *attn_ms = of its attention kernel alone (either may be NULL). */
int hat_op_swmsa(const float *x, float *out, int hp, int wp, int c, int heads, int shift,
                 const float *qkv_w, const float *qkv_b, const float *proj_w, const float *proj_b,
                 const float *table, int iters, float *ms, float *attn_ms);

/* The OCAB block (hat_arch.py:392-438; cpu.rs:1170-1198): norm1, qkv,
 * 24x24 unfold (stride 16, pad 4), attention with the [1521][heads] bias on
 * all 576 keys, proj + shortcut, norm2, GELU MLP + residual. */
int hat_op_ocab(const float *x, float *out, int hp, int wp, int c, int heads, int mlp_ratio,
                const float *n1w, const float *n1b, const float *qkv_w, const float *qkv_b,
                const float *proj_w, const float *proj_b, const float *table, const float *n2w,
                const float *n2b, const float *fc1_w, const float *fc1_b, const float *fc2_w,
                const float *fc2_b, int iters, float *ms, float *attn_ms);

/* ---- Device memory and timing (lightgpu::vm DevBuf, src/cuda.rs:528-555) -- */
void *hat_device_alloc(size_t bytes);
int hat_device_free(void *p);
int hat_memcpy_h2d(void *dst, const void *src, size_t bytes);
int hat_memcpy_d2h(void *dst, const void *src, size_t bytes);
/* Device-to-device copy with the library's plain copy kernel (bytes a multiple
 * of 16, 16-byte aligned pointers); asynchronous on the library's stream. It is
 * also the HBM reference point the benchmark scales traffic counters by. */
int hat_device_copy(void *dst, const void *src, size_t bytes);
int hat_device_synchronize(void);
/* Free and total device memory in bytes (hipMemGetInfo): the measured side
 * of the working-set figures (the reference's free-VRAM delta,
 * examples/bench.rs:110-184). */
int hat_device_mem_info(size_t *free_bytes, size_t *total_bytes);
/* Device name and compute-unit count; "" / 0 when no device. */
const char *hat_device_name(void);
int hat_device_cu_count(void);

/* Per-kernel HIP-event timing of every launch between begin and end, on the
 * stream each kernel is launched on. hat_profile_get returns 0 and fills the
 * i-th kernel's name, launch count and total milliseconds. */
int hat_profile_begin(void);
int hat_profile_end(void);
int hat_profile_count(void);
int hat_profile_get(int i, char *name, int cap, long *count, double *total_ms);

#ifdef __cplusplus
}
#endif
#endif
