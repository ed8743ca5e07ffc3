// The C ABI (include/hat.h): the boundary a Rust (or any FFI) caller binds.
#include "../../include/hat.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gpu.h"
#include "hip_rt.h"
#include "image.h"
#include "tile.h"
#include "kargs.h"
#include "weights.h"

struct hat_weights {
    std::unique_ptr<hat::Weights> w;
};
struct hat_backend {
    std::unique_ptr<hat::GpuBackend> b;
};

namespace {
thread_local std::string g_err;

template <class F>
int guard(F&& f)
{
    try {
        g_err.clear();
        return f();
    } catch (const hat::Error& e) {
        g_err = e.msg;
    } catch (const std::bad_alloc&) {
        g_err = "out of host memory";
    } catch (const std::exception& e) {
        g_err = e.what();
    }
    return -1;
}

// A side or count of the C ABI as the int the backend takes: refused past
// INT_MAX, not truncated to a smaller one the caller's buffers do not match.
int as_int(size_t v, const char* what)
{
    if (v > (size_t)INT32_MAX) throw hat::Error(std::string(what) + " " + std::to_string(v) + " is out of range");
    return (int)v;
}
}  // namespace

extern "C" {

const char* hat_version(void) { return "hat-mi355x 0.1.0"; }
const char* hat_last_error(void) { return g_err.c_str(); }

hat_weights* hat_weights_open(const char* path)
{
    hat_weights* out = nullptr;
    guard([&] {
        if (!path) throw hat::Error("null path");
        out = new hat_weights{std::unique_ptr<hat::Weights>(hat::Weights::load(path))};
        return 0;
    });
    return out;
}

void hat_weights_close(hat_weights* w) { delete w; }

int hat_weights_info(const hat_weights* w, hat_model_info* o)
{
    return guard([&] {
        if (!w || !o) throw hat::Error("null argument");
        const hat::Weights& x = *w->w;
        memset(o, 0, sizeof *o);
        o->scale = x.scale;
        o->window = x.window;
        o->owin = x.owin;
        o->embed = x.embed;
        o->heads = x.heads;
        o->head_dim = x.head_dim;
        o->mlp_ratio = x.mlp_ratio;
        if (x.depths.size() > 32) throw hat::Error("more than 32 stages");
        o->n_stages = (int)x.depths.size();
        for (size_t i = 0; i < x.depths.size(); ++i) o->depths[i] = x.depths[i];
        o->compressed = x.compressed;
        o->squeezed = x.squeezed;
        o->head_feat = x.head_feat;
        o->conv_scale = x.conv_scale;
        o->img_range = x.img_range;
        for (int i = 0; i < 3; ++i) o->mean[i] = x.mean[i];
        return 0;
    });
}

const char* hat_weights_variant(const hat_weights* w) { return w ? w->w->variant.c_str() : nullptr; }
unsigned long long hat_weights_file_bytes(const hat_weights* w) { return w ? w->w->file_bytes : 0; }

int hat_weights_count(const hat_weights* w) { return w ? (int)w->w->names.size() : -1; }

const char* hat_weights_name(const hat_weights* w, int i)
{
    if (!w || i < 0 || i >= (int)w->w->names.size()) return nullptr;
    return w->w->names[i].c_str();
}

const float* hat_weights_tensor(const hat_weights* w, const char* name, size_t* numel)
{
    const float* p = nullptr;
    guard([&] {
        if (!w || !name) throw hat::Error("null argument");
        p = w->w->t(name);
        if (numel) *numel = w->w->info(name).numel();
        return 0;
    });
    return p;
}

long hat_weights_index_i64(const hat_weights* w, const char* name, long long* out, size_t n)
{
    long r = -1;
    guard([&] {
        if (!w || !name) throw hat::Error("null argument");
        std::vector<int64_t> v = w->w->i64(name);
        for (size_t i = 0; i < v.size() && i < n && out; ++i) out[i] = v[i];
        r = (long)v.size();
        return 0;
    });
    return r;
}

int hat_weights_generate(const char* path, const char* variant, int scale, unsigned long long seed,
                         const int* depths, int n_depths)
{
    return guard([&] {
        if (!path || !variant) throw hat::Error("null argument");
        hat::Variant v;
        if (!hat::variant_by_name(variant, &v))
            throw hat::Error(std::string("unknown variant `") + variant + "` (hat-s, hat, hat-l)");
        if (depths && n_depths > 0) v.depths.assign(depths, depths + n_depths);
        hat::generate_weights(path, v, scale, seed);
        return 0;
    });
}

int hat_gpu_available(void)
{
    try {
        std::string why;
        return hat::gpu_available(&why) ? 1 : 0;
    } catch (...) {
        return 0;
    }
}

hat_backend* hat_backend_new(const hat_weights* w, const char* device)
{
    hat_backend* out = nullptr;
    guard([&] {
        if (!w) throw hat::Error("null weights");
        if (device && strcmp(device, "gpu") != 0)
            throw hat::Error(std::string("device `") + device +
                             "`: this library is the MI355X backend and has only `gpu`");
        out = new hat_backend{std::unique_ptr<hat::GpuBackend>(new hat::GpuBackend(*w->w))};
        return 0;
    });
    return out;
}

const char* hat_backend_name(const hat_backend* b) { return b ? b->b->name() : nullptr; }

int hat_backend_forward(hat_backend* b, size_t h, size_t w, const float* in, float* out)
{
    return guard([&] {
        if (!b || !in || !out) throw hat::Error("null argument");
        b->b->forward(as_int(h, "height"), as_int(w, "width"), in, out);
        return 0;
    });
}

int hat_backend_forward_device(hat_backend* b, size_t h, size_t w, const float* d_in, float* d_out)
{
    return guard([&] {
        if (!b || !d_in || !d_out) throw hat::Error("null argument");
        b->b->forward_device(as_int(h, "height"), as_int(w, "width"), d_in, d_out);
        return 0;
    });
}

int hat_backend_forward_noalloc(hat_backend* b, size_t h, size_t w, const float* d_in, float* d_out)
{
    return guard([&] {
        if (!b || !d_in || !d_out) throw hat::Error("null argument");
        if (h > 65536 || w > 65536) throw hat::Error("forward_noalloc: image too large");
        b->b->forward_noalloc(as_int(h, "height"), as_int(w, "width"), d_in, d_out);
        return 0;
    });
}

int hat_backend_synchronize(hat_backend* b)
{
    return guard([&] {
        if (!b) throw hat::Error("null backend");
        hat::Runtime& rt = hat::Runtime::get();
        rt.check(rt.api().StreamSynchronize(b->b->stream()), "hipStreamSynchronize");
        return 0;
    });
}

int hat_backend_hab(hat_backend* b, int stage, int block, size_t hp, size_t wp, const float* x, float* out,
                    int iters, float* ms)
{
    return guard([&] {
        if (!b || !x || !out) throw hat::Error("null argument");
        if (hp > 65536 || wp > 65536) throw hat::Error("hab: plane too large");
        b->b->op_hab(stage, block, as_int(hp, "height"), as_int(wp, "width"), x, out, iters, ms);
        return 0;
    });
}

size_t hat_backend_acts_bytes(const hat_backend* b) { return b ? b->b->acts_bytes() : 0; }
size_t hat_backend_weight_bytes(const hat_backend* b) { return b ? b->b->weight_bytes() : 0; }
void hat_backend_free(hat_backend* b) { delete b; }

int hat_backend_forward_batch(hat_backend* b, size_t n, size_t h, size_t w, const float* in, float* out)
{
    return guard([&] {
        if (!b || !in || !out) throw hat::Error("null argument");
        if (n > (1u << 20) || h > 65536 || w > 65536) throw hat::Error("forward_batch: too large");
        b->b->forward_batch(as_int(n, "image count"), as_int(h, "height"), as_int(w, "width"), in, out);
        return 0;
    });
}

int hat_tile_forward(hat_backend* b, size_t h, size_t w, const float* in, float* out, size_t tile,
                     size_t margin, hat_tiling* info)
{
    return guard([&] {
        if (!b || !in || !out) throw hat::Error("null argument");
        if (h > 65536 || w > 65536) throw hat::Error("tile: image too large");
        const hat::Weights& wt = b->b->weights();
        hat::Tiling t = hat::tile_forward(*b->b, h, w, in, out, tile, margin, (size_t)wt.scale,
                                          (size_t)wt.window);
        if (info) {
            info->tile = t.tile;
            info->margin = t.margin;
            info->scale = t.scale;
            info->tiles = t.tiles;
            info->largest_h = t.largest_h;
            info->largest_w = t.largest_w;
        }
        return 0;
    });
}

size_t hat_auto_tile(size_t h, size_t w, size_t win, unsigned long long budget_bytes,
                     unsigned long long per_pixel_floats, unsigned long long constant_floats, size_t margin)
{
    if (win == 0) return 0;
    return hat::auto_tile(h, w, win, budget_bytes, per_pixel_floats, constant_floats, margin);
}

int hat_gpu_plan(const hat_weights* w, size_t h, size_t wd, hat_mem_plan* out)
{
    return guard([&] {
        if (!w || !out) throw hat::Error("null argument");
        if (h == 0 || wd == 0 || h > 65536 || wd > 65536) throw hat::Error("gpu_plan: bad size");
        hat::MemPlan p = hat::gpu_plan(*w->w, h, wd);
        out->activations = p.activations;
        out->weights = p.weights;
        out->base = p.base;
        out->need = p.need;
        out->avail = p.avail;
        out->have_avail = p.have_avail ? 1 : 0;
        return 0;
    });
}

long hat_gpu_auto_tile(const hat_weights* w, size_t h, size_t wd)
{
    long r = -1;
    guard([&] {
        if (!w) throw hat::Error("null argument");
        if (h == 0 || wd == 0 || h > 65536 || wd > 65536) throw hat::Error("gpu_auto_tile: bad size");
        r = (long)hat::gpu_auto_tile(*w->w, h, wd);
        return 0;
    });
    return r;
}

int hat_png_load(const char* path, size_t* w, size_t* h, float* out, size_t cap)
{
    return guard([&] {
        if (!path || !w || !h) throw hat::Error("null argument");
        hat::Image img = hat::load_png(path);
        *w = img.w;
        *h = img.h;
        if (out) {
            if (cap < img.data.size())
                throw hat::Error(std::string(path) + ": " + std::to_string(img.data.size()) +
                                 " floats needed, room for " + std::to_string(cap));
            memcpy(out, img.data.data(), img.data.size() * sizeof(float));
        }
        return 0;
    });
}

int hat_png_save(const char* path, size_t w, size_t h, const float* planes)
{
    return guard([&] {
        if (!path || !planes) throw hat::Error("null argument");
        hat::save_png(path, w, h, planes);
        return 0;
    });
}

int hat_weights_shape(const hat_weights* w, const char* name, size_t* dims, int cap)
{
    return guard([&] {
        if (!w || !name) throw hat::Error("null argument");
        const hat::TensorInfo& ti = w->w->info(name);
        for (int i = 0; i < (int)ti.shape.size() && i < cap && dims; ++i) dims[i] = ti.shape[i];
        return (int)ti.shape.size();
    });
}

// main.rs:312-326 with the fixture format of fixture.rs:44-107.
int hat_verify(const hat_weights* w, const char* device, const char* fixture_path)
{
    int rc = guard([&] {
        if (!w || !fixture_path) throw hat::Error("null argument");
        FILE* f = fopen(fixture_path, "rb");
        if (!f) throw hat::Error(std::string(fixture_path) + ": " + strerror(errno));
        std::vector<unsigned char> b;
        unsigned char buf[65536];
        size_t n;
        while ((n = fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + n);
        fclose(f);
        auto u32 = [&](size_t off) {
            uint32_t v;
            memcpy(&v, &b[off], 4);
            return v;
        };
        if (b.size() < 36 || memcmp(b.data(), "HATF", 4) != 0)
            throw hat::Error(std::string(fixture_path) + ": not a hat fixture (want 4-byte magic HATF)");
        const uint32_t version = u32(4), h = u32(8), wd = u32(12), c = u32(16), scale = u32(20),
                       flags = u32(28);
        if (version != 1) throw hat::Error("fixture version " + std::to_string(version) + ", this engine reads 1");
        if (flags != 0) throw hat::Error("fixture flags are not zero");
        // The backend takes and returns 3-channel planes: a fixture of any
        // other width cannot be run, and sizing the buffers by it would read
        // and write past them.
        if (c != 3)
            throw hat::Error(std::string(fixture_path) + ": a " + std::to_string(c) +
                             "-channel fixture; the model takes 3-channel RGB input");
        if (h == 0 || wd == 0 || scale == 0) throw hat::Error(std::string(fixture_path) + ": empty fixture");
        if ((int)scale != w->w->scale)
            throw hat::Error(std::string(fixture_path) + " is a x" + std::to_string(scale) +
                             " fixture but the model is x" + std::to_string(w->w->scale));
        // Sides are 32-bit fields: bounded here, so that the sizes below cannot
        // wrap (a header whose products wrap to the file's length would size
        // the buffers for a few values and run the forward at its real sides)
        // and the sides fit the forward's int arguments.
        if (h > (1u << 20) || wd > (1u << 20))
            throw hat::Error(std::string(fixture_path) + ": a " + std::to_string(h) + "x" + std::to_string(wd) +
                             " fixture; sides above 2^20 are refused");
        const size_t need = 36 + 4 * ((size_t)h * wd * c + (size_t)h * scale * wd * scale * c);
        if (b.size() != need)
            throw hat::Error(std::string(fixture_path) + ": " + std::to_string(need) + " bytes expected, " +
                             std::to_string(b.size()) + " present");
        std::vector<float> in((size_t)h * wd * c), exp((size_t)h * scale * wd * scale * c);
        memcpy(in.data(), &b[36], in.size() * 4);
        memcpy(exp.data(), &b[36 + in.size() * 4], exp.size() * 4);
        if (device && strcmp(device, "gpu") != 0) throw hat::Error("only the gpu device exists here");
        hat::GpuBackend be(*w->w);
        std::vector<float> got(exp.size());
        be.forward((int)h, (int)wd, in.data(), got.data());
        float worst = 0.f;
        size_t at = 0;
        double mean = 0;
        for (size_t i = 0; i < got.size(); ++i) {
            float d = std::fabs(exp[i] - got[i]);
            mean += d;
            if (d > worst || std::isnan(d)) {
                worst = std::isnan(d) ? INFINITY : d;
                at = i;
            }
        }
        const size_t oh = (size_t)h * scale, ow = (size_t)wd * scale, plane = oh * ow;
        printf("  verify worst |diff| %.3e at (y %zu, x %zu, ch %zu), mean |diff| %.3e\n", worst,
               (at % plane) / ow, (at % plane) % ow, at / plane, mean / got.size());
        if (worst > 1e-4f) {
            char m[128];
            snprintf(m, sizeof m, "worst |diff| %.3e exceeds 1e-4", worst);
            g_err = m;
            return 1;
        }
        printf("  ok\n");
        return 0;
    });
    return rc;
}

int hat_gpu_selftest(void)
{
    return guard([&] {
        std::string err;
        int n = hat::gpu_selftest(&err);
        if (n < 0) throw hat::Error(err);
        return n;
    });
}

int hat_op_swmsa(const float* x, float* out, int hp, int wp, int c, int heads, int shift,
                 const float* qkv_w, const float* qkv_b, const float* proj_w, const float* proj_b,
                 const float* table, int iters, float* ms, float* attn_ms)
{
    return guard([&] {
        hat::op_swmsa(x, out, hp, wp, c, heads, shift, qkv_w, qkv_b, proj_w, proj_b, table, iters, ms,
                      attn_ms);
        return 0;
    });
}

int hat_op_ocab(const float* x, float* out, int hp, int wp, int c, int heads, int mlp_ratio,
                const float* n1w, const float* n1b, const float* qkv_w, const float* qkv_b,
                const float* proj_w, const float* proj_b, const float* table, const float* n2w,
                const float* n2b, const float* fc1_w, const float* fc1_b, const float* fc2_w,
                const float* fc2_b, int iters, float* ms, float* attn_ms)
{
    return guard([&] {
        hat::op_ocab(x, out, hp, wp, c, heads, mlp_ratio, n1w, n1b, qkv_w, qkv_b, proj_w, proj_b, table,
                     n2w, n2b, fc1_w, fc1_b, fc2_w, fc2_b, iters, ms, attn_ms);
        return 0;
    });
}

void* hat_device_alloc(size_t bytes)
{
    void* p = nullptr;
    guard([&] {
        p = hat::Runtime::get().alloc(bytes);
        return 0;
    });
    return p;
}

int hat_device_free(void* p)
{
    return guard([&] {
        hat::Runtime::get().free(p);
        return 0;
    });
}

int hat_memcpy_h2d(void* dst, const void* src, size_t bytes)
{
    return guard([&] {
        hat::Runtime::get().h2d(dst, src, bytes);
        return 0;
    });
}

int hat_memcpy_d2h(void* dst, const void* src, size_t bytes)
{
    return guard([&] {
        hat::Runtime::get().d2h(dst, src, bytes);
        return 0;
    });
}

int hat_device_copy(void* dst, const void* src, size_t bytes)
{
    return guard([&] {
        if (!dst || !src || bytes % 16 != 0 || ((uintptr_t)dst | (uintptr_t)src) % 16 != 0)
            throw hat::Error("hat_device_copy: 16-byte aligned pointers and a multiple of 16 bytes");
        hatk::CopyArgs p{(const float*)src, (float*)dst, (long)(bytes / 16)};
        const long blocks = (p.n4 + 1023) / 1024;
        if (blocks > 0x7fffffffL) throw hat::Error("hat_device_copy: too large");
        hat::launch(nullptr, "hat_copy", (unsigned)std::max<long>(blocks, 1), 1, 1, 256, p);
        return 0;
    });
}

int hat_device_synchronize(void)
{
    return guard([&] {
        hat::Runtime::get().sync();
        return 0;
    });
}

int hat_device_mem_info(size_t* free_bytes, size_t* total_bytes)
{
    return guard([&] {
        if (!free_bytes || !total_bytes) throw hat::Error("null argument");
        hat::Runtime& rt = hat::Runtime::get();
        rt.check(rt.api().MemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
        return 0;
    });
}

const char* hat_device_name(void)
{
    static std::string name;
    guard([&] {
        name = hat::Runtime::get().device_name();
        return 0;
    });
    return name.c_str();
}

int hat_device_cu_count(void)
{
    int n = 0;
    guard([&] {
        n = hat::Runtime::get().cu_count();
        return 0;
    });
    return n;
}

int hat_profile_begin(void)
{
    return guard([&] {
        hat::Runtime::get();
        hat::profile_begin();
        return 0;
    });
}

int hat_profile_end(void)
{
    return guard([&] {
        hat::profile_end();
        return 0;
    });
}

int hat_profile_count(void) { return (int)hat::profile_stats().size(); }

int hat_profile_get(int i, char* name, int cap, long* count, double* total_ms)
{
    return guard([&] {
        std::vector<hat::KernelStat> st = hat::profile_stats();
        if (i < 0 || i >= (int)st.size()) throw hat::Error("profile index out of range");
        if (name && cap > 0) snprintf(name, (size_t)cap, "%s", st[i].name.c_str());
        if (count) *count = st[i].count;
        if (total_ms) *total_ms = st[i].total_ms;
        return 0;
    });
}

}  // extern "C"
