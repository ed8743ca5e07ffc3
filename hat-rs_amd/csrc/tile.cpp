// Tiling and memory admission; see tile.h.
#include "tile.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "hip_rt.h"

namespace hat {

namespace {
size_t round_up(size_t v, size_t to) { return to == 0 ? v : (v + to - 1) / to * to; }
}  // namespace

Tiling tile_forward(Backend& be, size_t h, size_t w, const float* in, float* out, size_t tile,
                    size_t margin, size_t scale, size_t win)
{
    if (h == 0 || w == 0 || !in || !out)
        throw Error("tile: bad input " + std::to_string(h) + "x" + std::to_string(w));
    // The core starts on the whole image's window grid and the halo is a whole
    // number of windows, so each sub-image's windows, shifts, unfold and mask
    // are the whole image's at that offset (tile.rs:62-66).
    const size_t step = std::max(round_up(tile, win), win);
    margin = round_up(margin, win);
    const size_t oh = h * scale, ow = w * scale;
    const size_t tiles_y = (h + step - 1) / step, tiles_x = (w + step - 1) / step;
    Tiling info;
    info.tile = step;
    info.margin = margin;
    info.scale = scale;
    std::vector<float> sub, planes;
    for (size_t ty = 0; ty < tiles_y; ++ty)
        for (size_t tx = 0; tx < tiles_x; ++tx) {
            const size_t y0 = ty * step, x0 = tx * step;
            const size_t y1 = std::min(y0 + step, h), x1 = std::min(x0 + step, w);
            const size_t sy0 = y0 > margin ? y0 - margin : 0, sx0 = x0 > margin ? x0 - margin : 0;
            const size_t sy1 = std::min(y1 + margin, h), sx1 = std::min(x1 + margin, w);
            const size_t sh = sy1 - sy0, sw = sx1 - sx0;
            info.largest_h = std::max(info.largest_h, sh);
            info.largest_w = std::max(info.largest_w, sw);
            sub.resize(3 * sh * sw);
            for (size_t c = 0; c < 3; ++c)
                for (size_t y = 0; y < sh; ++y)
                    memcpy(&sub[(c * sh + y) * sw], &in[(c * h + sy0 + y) * w + sx0], sw * sizeof(float));
            planes.resize(3 * sh * scale * sw * scale);
            be.forward((int)sh, (int)sw, sub.data(), planes.data());
            // the core, not the halo, at the core's own position scaled by the model
            const size_t dy0 = (y0 - sy0) * scale, dx0 = (x0 - sx0) * scale;
            const size_t ch = (y1 - y0) * scale, cw = (x1 - x0) * scale;
            for (size_t c = 0; c < 3; ++c)
                for (size_t y = 0; y < ch; ++y)
                    memcpy(&out[c * oh * ow + (y0 * scale + y) * ow + x0 * scale],
                           &planes[c * sh * scale * sw * scale + (dy0 + y) * sw * scale + dx0], cw * sizeof(float));
            ++info.tiles;
        }
    return info;
}

size_t auto_tile(size_t h, size_t w, size_t win, uint64_t budget_bytes, uint64_t per_pixel_floats,
                 uint64_t constant_floats, size_t margin)
{
    const uint64_t bytes_per_pixel = std::max<uint64_t>(per_pixel_floats, 1) * 4;
    const uint64_t constant = constant_floats * 4;
    // The halo is part of what a tile runs a forward on, so it is part of the
    // budget (tile.rs:160-172).
    const uint64_t halo = 2 * (uint64_t)margin;
    const uint64_t one_window = (win + halo) * (win + halo) * bytes_per_pixel + constant;
    if (budget_bytes < one_window) return 0;
    const uint64_t pixels = (budget_bytes - constant) / bytes_per_pixel;
    size_t side = (size_t)std::sqrt((double)pixels);
    side = std::max((side > halo ? side - halo : 0) / win * win, win);
    return std::min(side, std::max(h, w));
}

std::string fmt_bytes(uint64_t n)
{
    const double mib = (double)n / 1048576.0;
    char b[64];
    if (mib >= 1024.0) snprintf(b, sizeof b, "%.1f GiB", mib / 1024.0);
    else snprintf(b, sizeof b, "%.0f MiB", mib);
    return b;
}

MemPlan gpu_plan(const Weights& wt, size_t h, size_t w)
{
    MemPlan p;
    p.activations = GpuBackend::plan_bytes(wt, (int)h, (int)w, true);
    // what the upload allocates: the packed tensors and their split-bf16 copies
    // (the reference's backend uploads the file's tensors as they are, wt.bytes)
    p.weights = GpuBackend::device_weight_bytes(wt);
    p.base = kBase;
    p.need = (uint64_t)((double)p.activations * kSlack) + p.weights + p.base;
    std::string why;
    if (gpu_available(&why)) {
        size_t fr = 0, tot = 0;
        Runtime& rt = Runtime::get();
        if (rt.api().MemGetInfo(&fr, &tot) == hipSuccess) {
            p.avail = fr;
            p.have_avail = true;
        }
    }
    return p;
}

void check_gpu(const Weights& wt, size_t h, size_t w)
{
    const MemPlan p = gpu_plan(wt, h, w);
    if (p.have_avail && p.need > p.avail) {
        throw Error("not enough video memory for a " + std::to_string(w) + "x" + std::to_string(h) +
                    " pass on the GPU\nhat: it needs about " + fmt_bytes(p.need) + " (" +
                    fmt_bytes(p.activations) + " of device buffers + " + fmt_bytes(p.weights) + " of weights + " +
                    fmt_bytes(p.base) + " of runtime, plus " +
                    std::to_string((int)std::lround((kSlack - 1.0) * 100.0)) + "% of slack); " +
                    fmt_bytes(p.avail) + " is free on the device\nhat: `--mem` runs it in tiles on the device "
                    "(each tile allocates its own buffers, so the tile's size is the number that must fit); "
                    "a smaller image does too");
    }
}

void check_gpu_weights(const Weights& wt)
{
    std::string why;
    if (!gpu_available(&why)) return;
    size_t fr = 0, tot = 0;
    if (Runtime::get().api().MemGetInfo(&fr, &tot) != hipSuccess) return;
    const uint64_t dev = GpuBackend::device_weight_bytes(wt);
    const uint64_t need = dev + kBase;
    if (need > fr)
        throw Error("not enough video memory for the checkpoint alone\nhat: " + wt.variant + " uploads as " +
                    fmt_bytes(dev) + " of tensors, and " + fmt_bytes(fr) +
                    " is free on the device\nhat: a smaller checkpoint is what fits");
}

size_t gpu_auto_tile(const Weights& wt, size_t h, size_t w)
{
    const size_t start = std::max({w, h, (size_t)wt.window});
    size_t t = start;
    for (;;) {
        const MemPlan p = gpu_plan(wt, t, t);
        if (!p.have_avail) return start;  // no basis to tile: run whole, let the guard refuse
        if (p.need <= p.avail) return t;
        if (t <= (size_t)wt.window)
            throw Error(fmt_bytes(p.avail) + " is free on the device, and one window does not fit it");
        t = std::max(t / 2, (size_t)wt.window);
    }
}

}  // namespace hat
