// The checkpoint: a .safetensors file plus the architecture its __metadata__
// records, validated against the tensors actually present.
//
// Mirrors src/weights.rs:28-347 of the reference: the metadata keys
// (weights.rs:64-66), the derived sizes (owin, head_dim, compressed, squeezed,
// head_feat), the shape table checked at load (weights.rs:133-265) and the
// head's block list (up_blocks, weights.rs:290-305). The file format is the one
// tools/convert.py writes (convert.py:205-250): F32 tensors and I64 index
// buffers, 4-byte-aligned payloads, architecture strings in __metadata__.
#pragma once
#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <utility>
#include <vector>

namespace hat {

struct TensorInfo {
    std::string dtype;           // "F32" or "I64"
    std::vector<size_t> shape;
    size_t begin = 0, end = 0;   // byte offsets into the data region
    size_t numel() const
    {
        size_t n = 1;
        for (size_t d : shape) n *= d;
        return n;
    }
};

class Weights {
public:
    static Weights* load(const std::string& path);  // throws hat::Error
    ~Weights();

    std::string variant, source;
    int scale = 0, window = 0, owin = 0, embed = 0, heads = 0, head_dim = 0, mlp_ratio = 0;
    std::vector<int> depths;
    int compressed = 0, squeezed = 0, head_feat = 0;
    float conv_scale = 0.f, img_range = 1.f;
    float mean[3] = {0.f, 0.f, 0.f};
    std::vector<std::string> names;  // file order (sorted, as convert.py writes)
    size_t file_bytes = 0;
    // What the GPU backend's upload of this checkpoint allocates on the device,
    // once computed (0 until then; GpuBackend::device_weight_bytes fills it).
    mutable size_t device_bytes_cache = 0;

    bool has(const std::string& name) const { return info_.count(name) != 0; }
    const TensorInfo& info(const std::string& name) const;
    const float* t(const std::string& name) const;        // F32 tensor data
    std::vector<int64_t> i64(const std::string& name) const;
    // (factor, widened) per upsampling block; empty if the scale is unsupported.
    std::vector<std::pair<int, int>> up_blocks() const;

private:
    Weights() = default;
    void validate(const std::string& path) const;
    void* map_ = nullptr;
    size_t map_len_ = 0;
    const unsigned char* data_ = nullptr;
    std::map<std::string, TensorInfo> info_;
};

// Architectures of the released checkpoints (tools/convert.py:62-71).
struct Variant {
    std::string name;
    int embed, heads, mlp_ratio, compress_ratio, squeeze_factor;
    std::vector<int> depths;
};
bool variant_by_name(const std::string& name, Variant* out);

// Writes a seeded checkpoint in the converter's format: every weight, bias and
// relative-position table ~ N(0, 0.02), LayerNorm weight 1 and bias 0, and the
// int64 relative_position_index_SA/OCA buffers from their closed forms.
// Normals come from splitmix64 (one stream per tensor, keyed by the seed and
// the tensor name) through the Box-Muller transform.
void generate_weights(const std::string& path, const Variant& v, int scale, uint64_t seed,
                      int window = 16, float overlap = 0.5f);

}  // namespace hat
