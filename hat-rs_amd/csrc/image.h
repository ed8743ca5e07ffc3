// PNG I/O for the `hat` CLI and the C ABI (src/image.rs of the reference).
#pragma once
#include <cstddef>
#include <string>
#include <vector>

namespace hat {

// A planar RGB image: data is [3][h][w], values in [0,1].
struct Image {
    size_t w = 0, h = 0;
    std::vector<float> data;
};

// image::load_rgb (image.rs:43-99): 8/16-bit grey, grey+alpha, RGB, RGBA.
Image load_png(const std::string& path);
// Image::to_rgb8 (image.rs:30-41): clamp to [0,1], scale by 255, round half up.
std::vector<unsigned char> to_rgb8(size_t w, size_t h, const float* planes);
// image::save_rgb (image.rs:101-114): 8-bit RGB from planar [3][h][w] floats.
void save_png(const std::string& path, size_t w, size_t h, const float* planes);

}  // namespace hat
