// Tiling and memory admission (src/tile.rs and src/memguard.rs of the reference).
//
// tile_forward runs an image too large for one pass in window-aligned cores,
// each with a halo of `margin` input pixels on every side that is not the
// image's edge, and copies back only the cores (tile.rs:50-107). The memory
// plan is the reference's (memguard.rs:60-225): the per-plan buffers with 5%
// allocator slack, plus the checkpoint, plus 128 MiB of runtime, against the
// device's free memory.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>

#include "gpu.h"
#include "weights.h"

namespace hat {

struct Tiling {
    size_t tile = 0, margin = 0, scale = 0, tiles = 0, largest_h = 0, largest_w = 0;
};

// tile::forward (tile.rs:50-107): in [3][h][w], out [3][h*scale][w*scale].
Tiling tile_forward(Backend& be, size_t h, size_t w, const float* in, float* out, size_t tile,
                    size_t margin, size_t scale, size_t win);

// tile::auto_tile (tile.rs:140-184): the largest window-multiple core whose
// sub-image (core + 2 margins) fits the budget; 0 when not even one window does.
size_t auto_tile(size_t h, size_t w, size_t win, uint64_t budget_bytes, uint64_t per_pixel_floats,
                 uint64_t constant_floats, size_t margin);

constexpr double kSlack = 1.05;                 // memguard::SLACK
constexpr uint64_t kBase = 128ull << 20;        // memguard::BASE

struct MemPlan {
    uint64_t activations = 0, weights = 0, base = 0, need = 0, avail = 0;
    bool have_avail = false;
};

// memguard::gpu_plan (memguard.rs:147-160): this backend's per-plan buffers for
// an h x w pass (host staging included) and the checkpoint's bytes, against
// the free device memory (have_avail false when no device answers).
MemPlan gpu_plan(const Weights& wt, size_t h, size_t w);
// memguard::check_gpu (memguard.rs:162-190): throws the reference's message
// when the plan does not fit.
void check_gpu(const Weights& wt, size_t h, size_t w);
// memguard::check_gpu_weights (memguard.rs:192-210).
void check_gpu_weights(const Weights& wt);
// main.rs:115-140 gpu_auto_tile: halve from the larger side until gpu_plan fits.
size_t gpu_auto_tile(const Weights& wt, size_t h, size_t w);
// memguard::fmt_bytes (memguard.rs:35-44).
std::string fmt_bytes(uint64_t n);

}  // namespace hat
