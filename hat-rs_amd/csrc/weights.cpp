#include "weights.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <sstream>

#include "hip_rt.h"
#include "plan.h"

namespace hat {

// ---------------------------------------------------------------------------
// A small JSON reader, enough for a safetensors header: objects, arrays,
// strings (with escapes), numbers, true/false/null.
namespace {

struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const std::string& k) const
    {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

// Whether s is well-formed UTF-8 (no overlong forms, no surrogates, at most
// U+10FFFF): a safetensors header is UTF-8 JSON, and its strings name tensors
// and end up in messages.
bool utf8_ok(const std::string& s)
{
    const unsigned char* q = (const unsigned char*)s.data();
    const unsigned char* end = q + s.size();
    while (q < end) {
        const unsigned c = *q++;
        if (c < 0x80) continue;
        int n;
        unsigned cp;
        if (c >= 0xC2 && c <= 0xDF) n = 1, cp = c & 0x1F;
        else if (c >= 0xE0 && c <= 0xEF) n = 2, cp = c & 0x0F;
        else if (c >= 0xF0 && c <= 0xF4) n = 3, cp = c & 0x07;
        else return false;
        if (end - q < n) return false;
        for (int i = 0; i < n; ++i) {
            if ((q[i] & 0xC0) != 0x80) return false;
            cp = cp << 6 | (q[i] & 0x3F);
        }
        q += n;
        if ((n == 2 && (cp < 0x800 || (cp >= 0xD800 && cp <= 0xDFFF))) || (n == 3 && (cp < 0x10000 || cp > 0x10FFFF)))
            return false;
    }
    return true;
}

struct JParser {
    const char* p;
    const char* e;
    void ws()
    {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    [[noreturn]] void fail(const char* what) { throw Error(std::string("safetensors header: ") + what); }
    std::string string()
    {
        if (p >= e || *p != '"') fail("expected a string");
        ++p;
        std::string s;
        while (p < e && *p != '"') {
            if (*p == '\\') {
                ++p;
                if (p >= e) fail("bad escape");
                char c = *p++;
                switch (c) {
                case 'n': s += '\n'; break;
                case 't': s += '\t'; break;
                case 'r': s += '\r'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'u': {
                    if (e - p < 4) fail("bad \\u escape");
                    unsigned cp = (unsigned)strtoul(std::string(p, 4).c_str(), nullptr, 16);
                    p += 4;
                    if (cp < 0x80) s += (char)cp;
                    else if (cp < 0x800) { s += (char)(0xC0 | (cp >> 6)); s += (char)(0x80 | (cp & 0x3F)); }
                    else { s += (char)(0xE0 | (cp >> 12)); s += (char)(0x80 | ((cp >> 6) & 0x3F)); s += (char)(0x80 | (cp & 0x3F)); }
                    break;
                }
                default: s += c;
                }
            } else {
                s += *p++;
            }
        }
        if (p >= e) fail("unterminated string");
        ++p;
        if (!utf8_ok(s)) fail("a string that is not UTF-8");
        return s;
    }
    JVal value()
    {
        ws();
        if (p >= e) fail("unexpected end");
        JVal v;
        if (*p == '{') {
            ++p;
            v.kind = JVal::Obj;
            ws();
            if (p < e && *p == '}') { ++p; return v; }
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p >= e || *p != ':') fail("expected ':'");
                ++p;
                v.obj.emplace_back(k, value());
                ws();
                if (p < e && *p == ',') { ++p; continue; }
                if (p < e && *p == '}') { ++p; break; }
                fail("expected ',' or '}'");
            }
        } else if (*p == '[') {
            ++p;
            v.kind = JVal::Arr;
            ws();
            if (p < e && *p == ']') { ++p; return v; }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (p < e && *p == ',') { ++p; continue; }
                if (p < e && *p == ']') { ++p; break; }
                fail("expected ',' or ']'");
            }
        } else if (*p == '"') {
            v.kind = JVal::Str;
            v.str = string();
        } else if (!strncmp(p, "true", 4) && e - p >= 4) { v.kind = JVal::Bool; v.num = 1; p += 4; }
        else if (!strncmp(p, "false", 5) && e - p >= 5) { v.kind = JVal::Bool; p += 5; }
        else if (!strncmp(p, "null", 4) && e - p >= 4) { p += 4; }
        else {
            char* end = nullptr;
            v.num = strtod(std::string(p, std::min<ptrdiff_t>(e - p, 64)).c_str(), &end);
            if (end == nullptr) fail("bad number");
            const char* q = p;
            while (q < e && (isdigit((unsigned char)*q) || *q == '-' || *q == '+' || *q == '.' || *q == 'e' || *q == 'E')) ++q;
            if (q == p) fail("bad token");
            v.kind = JVal::Num;
            p = q;
        }
        return v;
    }
};

std::string join_dims(const std::vector<size_t>& s)
{
    std::string o = "[";
    for (size_t i = 0; i < s.size(); ++i) o += (i ? ", " : "") + std::to_string(s[i]);
    return o + "]";
}

std::vector<std::string> split(const std::string& s, char c)
{
    std::vector<std::string> out;
    std::string cur;
    for (char ch : s) {
        if (ch == c) { out.push_back(cur); cur.clear(); }
        else cur += ch;
    }
    out.push_back(cur);
    return out;
}

std::string trim(const std::string& s)
{
    size_t a = s.find_first_not_of(" \t"), b = s.find_last_not_of(" \t");
    return a == std::string::npos ? "" : s.substr(a, b - a + 1);
}

}  // namespace

// ---------------------------------------------------------------------------

Weights::~Weights()
{
    if (map_) munmap(map_, map_len_);
}

const TensorInfo& Weights::info(const std::string& name) const
{
    auto it = info_.find(name);
    if (it == info_.end()) throw Error("weight `" + name + "` is not in the checkpoint");
    return it->second;
}

const float* Weights::t(const std::string& name) const
{
    const TensorInfo& ti = info(name);
    if (ti.dtype != "F32") throw Error("weight `" + name + "` is " + ti.dtype + ", not F32");
    return reinterpret_cast<const float*>(data_ + ti.begin);
}

std::vector<int64_t> Weights::i64(const std::string& name) const
{
    const TensorInfo& ti = info(name);
    if (ti.dtype != "I64") throw Error("`" + name + "` is " + ti.dtype + ", not I64");
    std::vector<int64_t> v(ti.numel());
    if (ti.end - ti.begin != v.size() * 8)
        throw Error("`" + name + "`: byte length does not match its shape");
    memcpy(v.data(), data_ + ti.begin, v.size() * 8);
    return v;
}

// Weights::up_blocks (weights.rs:290-305)
std::vector<std::pair<int, int>> Weights::up_blocks() const
{
    const int feat = head_feat;
    if (scale == 3) return {{3, 9 * feat}};
    int s = scale, n = 0;
    while (s > 1 && s % 2 == 0) {
        ++n;
        s /= 2;
    }
    if (s != 1 || n == 0) return {};
    return std::vector<std::pair<int, int>>(n, {2, 4 * feat});
}

// Weights::load (weights.rs:60-129)
Weights* Weights::load(const std::string& path)
{
    std::unique_ptr<Weights> w(new Weights());
    int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) throw Error(path + ": " + strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        throw Error(path + ": cannot stat");
    }
    w->map_len_ = (size_t)st.st_size;
    w->file_bytes = w->map_len_;
    if (w->map_len_ < 8) {
        close(fd);
        throw Error(path + ": too short to be a safetensors file");
    }
    w->map_ = mmap(nullptr, w->map_len_, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (w->map_ == MAP_FAILED) {
        w->map_ = nullptr;
        throw Error(path + ": mmap failed");
    }
    const unsigned char* b = (const unsigned char*)w->map_;
    uint64_t hlen = 0;
    memcpy(&hlen, b, 8);
    if (hlen > w->map_len_ - 8) throw Error(path + ": header length past the end of the file");
    JParser jp{(const char*)b + 8, (const char*)b + 8 + hlen};
    JVal root = jp.value();
    if (root.kind != JVal::Obj) throw Error(path + ": header is not a JSON object");
    w->data_ = b + 8 + hlen;
    const size_t data_len = w->map_len_ - 8 - hlen;
    std::map<std::string, std::string> meta;
    for (auto& kv : root.obj) {
        if (kv.first == "__metadata__") {
            for (auto& m : kv.second.obj) meta[m.first] = m.second.str;
            continue;
        }
        const JVal& v = kv.second;
        const JVal* dt = v.get("dtype");
        const JVal* sh = v.get("shape");
        const JVal* off = v.get("data_offsets");
        if (!dt || !sh || !off || off->arr.size() != 2)
            throw Error(path + ": tensor `" + kv.first + "` has an incomplete header entry");
        TensorInfo ti;
        ti.dtype = dt->str;
        // Dimensions and offsets are JSON numbers: only exact integers in
        // [0, 2^53) are taken (a cast of anything else to size_t is undefined),
        // and the element and byte counts are formed without wrapping, so that
        // no shape passes the length check below by overflowing to it.
        auto count = [&](const JVal& v, const char* what) -> size_t {
            if (v.kind != JVal::Num || !(v.num >= 0.0) || v.num >= 9007199254740992.0 || v.num != std::floor(v.num))
                throw Error(path + ": tensor `" + kv.first + "` has a " + what + " that is not a count");
            return (size_t)v.num;
        };
        size_t nbytes = ti.dtype == "F32" ? 4 : ti.dtype == "I64" ? 8 : 0;
        if (nbytes == 0) throw Error(path + ": tensor `" + kv.first + "` has unsupported dtype " + ti.dtype);
        for (auto& d : sh->arr) {
            ti.shape.push_back(count(d, "dimension"));
            if (__builtin_mul_overflow(nbytes, ti.shape.back(), &nbytes))
                throw Error(path + ": tensor `" + kv.first + "` is larger than any file");
        }
        ti.begin = count(off->arr[0], "data offset");
        ti.end = count(off->arr[1], "data offset");
        if (ti.end < ti.begin || ti.end > data_len || ti.end - ti.begin != nbytes)
            throw Error(path + ": tensor `" + kv.first + "` has inconsistent offsets");
        if (ti.dtype == "F32" && (ti.begin % 4) != 0)
            throw Error(path + ": tensor `" + kv.first + "` is not 4-byte aligned");
        w->info_[kv.first] = ti;
        w->names.push_back(kv.first);
    }
    const char* keys[] = {"variant", "scale", "window_size", "overlap_ratio", "embed_dim",
                          "num_heads", "mlp_ratio", "depths", "compress_ratio", "squeeze_factor",
                          "conv_scale", "img_range", "rgb_mean", "source"};
    for (const char* k : keys)
        if (!meta.count(k))
            throw Error(path + ": no `" + k +
                        "` in __metadata__ - convert the checkpoint with tools/convert.py, which "
                        "records the architecture; a plain state_dict cannot be checked");
    auto num = [&](const char* k) -> int {
        char* end = nullptr;
        long v = strtol(meta[k].c_str(), &end, 10);
        if (!end || *end != '\0' || meta[k].empty())
            throw Error(path + ": `" + k + "` = \"" + meta[k] + "\" is not an integer");
        return (int)v;
    };
    auto fnum = [&](const char* k) -> float {
        char* end = nullptr;
        float v = strtof(meta[k].c_str(), &end);
        if (!end || *end != '\0' || meta[k].empty())
            throw Error(path + ": `" + k + "` = \"" + meta[k] + "\" is not a number");
        return v;
    };
    for (const std::string& d : split(meta["depths"], ',')) {
        std::string t = trim(d);
        char* end = nullptr;
        long v = strtol(t.c_str(), &end, 10);
        if (t.empty() || *end != '\0' || v <= 0 || v > 1024) throw Error(path + ": depths: bad entry `" + t + "`");
        w->depths.push_back((int)v);
    }
    if (w->depths.empty() || w->depths.size() > 32)  // hat_model_info holds 32
        throw Error(path + ": depths: " + std::to_string(w->depths.size()) + " stages");
    std::vector<std::string> ms = split(meta["rgb_mean"], ',');
    if (ms.size() != 3) throw Error("rgb_mean has " + std::to_string(ms.size()) + " entries, expected 3");
    for (int i = 0; i < 3; ++i) w->mean[i] = strtof(trim(ms[i]).c_str(), nullptr);
    w->variant = meta["variant"];
    w->source = meta["source"];
    w->embed = num("embed_dim");
    w->heads = num("num_heads");
    if (w->heads <= 0 || w->embed % w->heads != 0)
        throw Error("embed_dim " + std::to_string(w->embed) + " is not divisible by num_heads " +
                    std::to_string(w->heads));
    w->window = num("window_size");
    const float overlap = fnum("overlap_ratio");
    if (!(overlap >= 0.0f && overlap <= 1.0f) || w->window <= 0 || w->window > 256)
        throw Error(path + ": window_size " + std::to_string(w->window) + " or overlap_ratio " + meta["overlap_ratio"] +
                    " out of range");
    // int(window_size * overlap_ratio) + window_size, a truncation (weights.rs:93-97)
    w->owin = w->window + (int)((float)w->window * overlap);
    w->scale = num("scale");
    w->head_dim = w->embed / w->heads;
    w->mlp_ratio = num("mlp_ratio");
    // far past every HAT configuration; what validate() sizes its shape table by
    if (w->embed <= 0 || w->embed > 4096 || w->heads > 64 || w->window <= 0 || w->window > 256 || w->owin > 512 ||
        w->mlp_ratio <= 0 || w->mlp_ratio > 16)
        throw Error(path + ": embed_dim, num_heads, window_size, overlap_ratio or mlp_ratio out of range");
    const int cr = num("compress_ratio"), sf = num("squeeze_factor");
    if (cr <= 0 || sf <= 0) throw Error(path + ": compress_ratio and squeeze_factor must be positive");
    w->compressed = w->embed / cr;
    w->squeezed = w->embed / sf;
    w->conv_scale = fnum("conv_scale");
    w->img_range = fnum("img_range");
    if (!w->has("conv_before_upsample.0.weight"))
        throw Error(path + ": the checkpoint has no `conv_before_upsample.0.weight`");
    const std::vector<size_t>& hs = w->info("conv_before_upsample.0.weight").shape;
    if (hs.empty() || hs[0] == 0 || hs[0] > 4096)
        throw Error(path + ": `conv_before_upsample.0.weight` is " + join_dims(hs));
    w->head_feat = (int)hs[0];
    w->validate(path);
    return w.release();
}

// Weights::validate (weights.rs:133-265)
void Weights::validate(const std::string& path) const
{
    const size_t c = embed, hd = heads, win = window, ow = owin, mr = mlp_ratio;
    std::vector<std::pair<std::string, std::vector<size_t>>> want = {
        {"conv_first.weight", {c, 3, 3, 3}},
        {"conv_first.bias", {c}},
        {"conv_after_body.weight", {c, c, 3, 3}},
        {"conv_after_body.bias", {c}},
        {"norm.weight", {c}},
        {"norm.bias", {c}},
        {"patch_embed.norm.weight", {c}},
        {"patch_embed.norm.bias", {c}},
        {"relative_position_index_SA", {win * win, win * win}},
        {"relative_position_index_OCA", {win * win, ow * ow}},
        {"conv_before_upsample.0.weight", {(size_t)head_feat, c, 3, 3}},
        {"conv_before_upsample.0.bias", {(size_t)head_feat}},
    };
    auto blocks = up_blocks();
    if (blocks.empty())
        throw Error("scale " + std::to_string(scale) +
                    " is not one the reference's own `Upsample` builds: it accepts a power of two "
                    "(one conv and a 2x shuffle per octave) and 3 (a single conv and a 3x shuffle)");
    for (size_t o = 0; o < blocks.size(); ++o) {
        want.push_back({"upsample." + std::to_string(2 * o) + ".weight",
                        {(size_t)blocks[o].second, (size_t)head_feat, 3, 3}});
        want.push_back({"upsample." + std::to_string(2 * o) + ".bias", {(size_t)blocks[o].second}});
    }
    want.push_back({"conv_last.weight", {3, (size_t)head_feat, 3, 3}});
    want.push_back({"conv_last.bias", {3}});
    for (size_t layer = 0; layer < depths.size(); ++layer) {
        const std::string L = "layers." + std::to_string(layer);
        want.push_back({L + ".conv.weight", {c, c, 3, 3}});
        want.push_back({L + ".conv.bias", {c}});
        for (int b = 0; b < depths[layer]; ++b) {
            const std::string p = L + ".residual_group.blocks." + std::to_string(b);
            want.push_back({p + ".norm1.weight", {c}});
            want.push_back({p + ".norm1.bias", {c}});
            want.push_back({p + ".norm2.weight", {c}});
            want.push_back({p + ".norm2.bias", {c}});
            want.push_back({p + ".attn.qkv.weight", {3 * c, c}});
            want.push_back({p + ".attn.qkv.bias", {3 * c}});
            want.push_back({p + ".attn.proj.weight", {c, c}});
            want.push_back({p + ".attn.proj.bias", {c}});
            want.push_back({p + ".attn.relative_position_bias_table", {(2 * win - 1) * (2 * win - 1), hd}});
            want.push_back({p + ".mlp.fc1.weight", {mr * c, c}});
            want.push_back({p + ".mlp.fc1.bias", {mr * c}});
            want.push_back({p + ".mlp.fc2.weight", {c, mr * c}});
            want.push_back({p + ".mlp.fc2.bias", {c}});
            want.push_back({p + ".conv_block.cab.0.weight", {(size_t)compressed, c, 3, 3}});
            want.push_back({p + ".conv_block.cab.0.bias", {(size_t)compressed}});
            want.push_back({p + ".conv_block.cab.2.weight", {c, (size_t)compressed, 3, 3}});
            want.push_back({p + ".conv_block.cab.2.bias", {c}});
            want.push_back({p + ".conv_block.cab.3.attention.1.weight", {(size_t)squeezed, c, 1, 1}});
            want.push_back({p + ".conv_block.cab.3.attention.1.bias", {(size_t)squeezed}});
            want.push_back({p + ".conv_block.cab.3.attention.3.weight", {c, (size_t)squeezed, 1, 1}});
            want.push_back({p + ".conv_block.cab.3.attention.3.bias", {c}});
        }
        const std::string p = L + ".residual_group.overlap_attn";
        want.push_back({p + ".norm1.weight", {c}});
        want.push_back({p + ".norm1.bias", {c}});
        want.push_back({p + ".norm2.weight", {c}});
        want.push_back({p + ".norm2.bias", {c}});
        want.push_back({p + ".qkv.weight", {3 * c, c}});
        want.push_back({p + ".qkv.bias", {3 * c}});
        want.push_back({p + ".proj.weight", {c, c}});
        want.push_back({p + ".proj.bias", {c}});
        want.push_back({p + ".relative_position_bias_table", {(win + ow - 1) * (win + ow - 1), hd}});
        want.push_back({p + ".mlp.fc1.weight", {mr * c, c}});
        want.push_back({p + ".mlp.fc1.bias", {mr * c}});
        want.push_back({p + ".mlp.fc2.weight", {c, mr * c}});
        want.push_back({p + ".mlp.fc2.bias", {c}});
    }
    std::string dstr;
    for (size_t i = 0; i < depths.size(); ++i) dstr += (i ? "," : "") + std::to_string(depths[i]);
    for (auto& kv : want) {
        auto it = info_.find(kv.first);
        if (it == info_.end())
            throw Error(path + ": the checkpoint has no `" + kv.first + "`; the metadata says " +
                        variant + " with embed " + std::to_string(embed) + " and depths " + dstr +
                        ", which does not describe these tensors");
        if (it->second.shape != kv.second)
            throw Error(path + ": `" + kv.first + "` is " + join_dims(it->second.shape) +
                        ", expected " + join_dims(kv.second) + " for " + variant + " at embed " +
                        std::to_string(embed));
    }
    // The attention kernels index the bias tables by closed forms. The
    // reference instead reads the checkpoint's index buffers, folded into the
    // table with rem_euclid (gpu.rs:59-62), and its tests hold those buffers to
    // its own construction (tests/parity.rs:114-149). A checkpoint whose
    // buffers, folded the same way, differ from the closed forms describes a
    // different network: refuse it rather than run it with other semantics.
    const int64_t rows_sa = (2 * (int64_t)win - 1) * (2 * (int64_t)win - 1);
    const int64_t rows_oca = ((int64_t)win + ow - 1) * ((int64_t)win + ow - 1);
    auto fold = [](int64_t v, int64_t rows) { return ((v % rows) + rows) % rows; };
    auto check_index = [&](const char* name, const std::vector<int64_t>& want, int64_t rows) {
        const std::vector<int64_t> got = i64(name);
        if (got.size() != want.size())
            throw Error(path + ": `" + name + "` has " + std::to_string(got.size()) + " entries, expected " +
                        std::to_string(want.size()));
        for (size_t i = 0; i < got.size(); ++i)
            if (fold(got[i], rows) != fold(want[i], rows))
                throw Error(path + ": `" + name + "`[" + std::to_string(i / (win * win)) + "][" +
                            std::to_string(i % (win * win)) + "] = " + std::to_string(got[i]) +
                            " but the window geometry gives " + std::to_string(want[i]) + " (mod " +
                            std::to_string(rows) + "): the checkpoint's relative-position index is not "
                            "the one this network's attention uses");
    };
    check_index("relative_position_index_SA", rpi_sa_raw((int)win), rows_sa);
    check_index("relative_position_index_OCA", rpi_oca_raw((int)win, (int)ow), rows_oca);
}

// ---------------------------------------------------------------------------
// Variants and the seeded generator.

bool variant_by_name(const std::string& name, Variant* out)
{
    // tools/convert.py:62-71 (options/test/HAT-S_SRx4.yml, HAT_SRx4.yml,
    // HAT-L_SRx4_ImageNet-pretrain.yml)
    if (name == "hat-s") { *out = {name, 144, 6, 2, 24, 24, std::vector<int>(6, 6)}; return true; }
    if (name == "hat") { *out = {name, 180, 6, 2, 3, 30, std::vector<int>(6, 6)}; return true; }
    if (name == "hat-l") { *out = {name, 180, 6, 2, 3, 30, std::vector<int>(12, 6)}; return true; }
    return false;
}

namespace {

uint64_t splitmix64(uint64_t& s)
{
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t fnv1a(const std::string& s)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char ch : s) {
        h ^= ch;
        h *= 0x100000001b3ull;
    }
    return h;
}

struct GenTensor {
    std::string name;
    std::vector<size_t> shape;
    std::vector<float> f;
    std::vector<int64_t> i;
};

void fill_normal(GenTensor& t, uint64_t seed, double std)
{
    uint64_t s = seed ^ fnv1a(t.name);
    splitmix64(s);
    size_t n = 1;
    for (size_t d : t.shape) n *= d;
    t.f.resize(n);
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t k = 0; k < n; ++k) {
        // u1 in (0, 1], u2 in [0, 1): Box-Muller, cosine branch.
        double u1 = ((splitmix64(s) >> 11) + 1) * (1.0 / 9007199254740992.0);
        double u2 = (splitmix64(s) >> 11) * (1.0 / 9007199254740992.0);
        double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
        t.f[k] = (float)(std * z);
    }
}

}  // namespace

void generate_weights(const std::string& path, const Variant& v, int scale, uint64_t seed,
                      int window, float overlap)
{
    const size_t c = v.embed, hd = v.heads, win = window, mr = v.mlp_ratio;
    const size_t ow = window + (int)((float)window * overlap);
    const size_t comp = c / v.compress_ratio, sq = c / v.squeeze_factor, feat = 64;
    std::vector<GenTensor> ts;
    auto W = [&](const std::string& n, std::vector<size_t> s) { ts.push_back({n, s, {}, {}}); };
    auto LN = [&](const std::string& n) {
        GenTensor w{n + ".weight", {c}, std::vector<float>(c, 1.0f), {}};
        GenTensor b{n + ".bias", {c}, std::vector<float>(c, 0.0f), {}};
        ts.push_back(w);
        ts.push_back(b);
    };
    W("conv_first.weight", {c, 3, 3, 3});
    W("conv_first.bias", {c});
    LN("patch_embed.norm");
    for (size_t layer = 0; layer < v.depths.size(); ++layer) {
        const std::string L = "layers." + std::to_string(layer);
        for (int b = 0; b < v.depths[layer]; ++b) {
            const std::string p = L + ".residual_group.blocks." + std::to_string(b);
            LN(p + ".norm1");
            W(p + ".attn.relative_position_bias_table", {(2 * win - 1) * (2 * win - 1), hd});
            W(p + ".attn.qkv.weight", {3 * c, c});
            W(p + ".attn.qkv.bias", {3 * c});
            W(p + ".attn.proj.weight", {c, c});
            W(p + ".attn.proj.bias", {c});
            W(p + ".conv_block.cab.0.weight", {comp, c, 3, 3});
            W(p + ".conv_block.cab.0.bias", {comp});
            W(p + ".conv_block.cab.2.weight", {c, comp, 3, 3});
            W(p + ".conv_block.cab.2.bias", {c});
            W(p + ".conv_block.cab.3.attention.1.weight", {sq, c, 1, 1});
            W(p + ".conv_block.cab.3.attention.1.bias", {sq});
            W(p + ".conv_block.cab.3.attention.3.weight", {c, sq, 1, 1});
            W(p + ".conv_block.cab.3.attention.3.bias", {c});
            LN(p + ".norm2");
            W(p + ".mlp.fc1.weight", {mr * c, c});
            W(p + ".mlp.fc1.bias", {mr * c});
            W(p + ".mlp.fc2.weight", {c, mr * c});
            W(p + ".mlp.fc2.bias", {c});
        }
        const std::string p = L + ".residual_group.overlap_attn";
        LN(p + ".norm1");
        W(p + ".qkv.weight", {3 * c, c});
        W(p + ".qkv.bias", {3 * c});
        W(p + ".relative_position_bias_table", {(win + ow - 1) * (win + ow - 1), hd});
        W(p + ".proj.weight", {c, c});
        W(p + ".proj.bias", {c});
        LN(p + ".norm2");
        W(p + ".mlp.fc1.weight", {mr * c, c});
        W(p + ".mlp.fc1.bias", {mr * c});
        W(p + ".mlp.fc2.weight", {c, mr * c});
        W(p + ".mlp.fc2.bias", {c});
        W(L + ".conv.weight", {c, c, 3, 3});
        W(L + ".conv.bias", {c});
    }
    LN("norm");
    W("conv_after_body.weight", {c, c, 3, 3});
    W("conv_after_body.bias", {c});
    W("conv_before_upsample.0.weight", {feat, c, 3, 3});
    W("conv_before_upsample.0.bias", {feat});
    {
        std::vector<std::pair<int, int>> blocks;
        if (scale == 3) blocks = {{3, 9 * (int)feat}};
        else {
            int s = scale, n = 0;
            while (s > 1 && s % 2 == 0) { ++n; s /= 2; }
            if (s != 1 || n == 0) throw Error("scale " + std::to_string(scale) + " is not 2^n or 3");
            blocks.assign(n, {2, 4 * (int)feat});
        }
        for (size_t o = 0; o < blocks.size(); ++o) {
            W("upsample." + std::to_string(2 * o) + ".weight", {(size_t)blocks[o].second, feat, 3, 3});
            W("upsample." + std::to_string(2 * o) + ".bias", {(size_t)blocks[o].second});
        }
    }
    W("conv_last.weight", {3, feat, 3, 3});
    W("conv_last.bias", {3});
    for (GenTensor& t : ts)
        if (t.f.empty()) fill_normal(t, seed, 0.02);
    {
        GenTensor sa{"relative_position_index_SA", {win * win, win * win}, {}, rpi_sa_raw((int)win)};
        GenTensor oca{"relative_position_index_OCA", {win * win, ow * ow}, {}, rpi_oca_raw((int)win, (int)ow)};
        ts.push_back(sa);
        ts.push_back(oca);
    }
    std::sort(ts.begin(), ts.end(), [](const GenTensor& a, const GenTensor& b) { return a.name < b.name; });

    // Header, as tools/convert.py:223-250 writes it.
    std::ostringstream h;
    h << "{";
    size_t off = 0;
    for (size_t k = 0; k < ts.size(); ++k) {
        const GenTensor& t = ts[k];
        size_t n = t.i.empty() ? t.f.size() * 4 : t.i.size() * 8;
        h << "\"" << t.name << "\":{\"dtype\":\"" << (t.i.empty() ? "F32" : "I64") << "\",\"shape\":[";
        for (size_t d = 0; d < t.shape.size(); ++d) h << (d ? "," : "") << t.shape[d];
        h << "],\"data_offsets\":[" << off << "," << off + n << "]},";
        off += (n + 3) & ~(size_t)3;
    }
    std::string depths;
    for (size_t i = 0; i < v.depths.size(); ++i) depths += (i ? "," : "") + std::to_string(v.depths[i]);
    char ovl[32];
    snprintf(ovl, sizeof ovl, "%g", (double)overlap);
    h << "\"__metadata__\":{\"variant\":\"" << v.name << "\",\"scale\":\"" << scale
      << "\",\"window_size\":\"" << window << "\",\"overlap_ratio\":\"" << ovl << "\",\"embed_dim\":\""
      << v.embed << "\",\"num_heads\":\"" << v.heads << "\",\"mlp_ratio\":\"" << v.mlp_ratio
      << "\",\"depths\":\"" << depths << "\",\"compress_ratio\":\"" << v.compress_ratio
      << "\",\"squeeze_factor\":\"" << v.squeeze_factor
      << "\",\"conv_scale\":\"0.01\",\"img_range\":\"1.0\",\"rgb_mean\":\"0.4488,0.4371,0.4040\","
         "\"source\":\"seeded:"
      << seed << "\",\"format\":\"pt\"}}";
    std::string hj = h.str();
    size_t pad = (8 - ((8 + hj.size()) % 8)) % 8;
    hj.append(pad, ' ');
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) throw Error(path + ": " + strerror(errno));
    uint64_t hl = hj.size();
    bool ok = fwrite(&hl, 8, 1, f) == 1 && fwrite(hj.data(), 1, hj.size(), f) == hj.size();
    for (const GenTensor& t : ts) {
        const void* d = t.i.empty() ? (const void*)t.f.data() : (const void*)t.i.data();
        size_t n = t.i.empty() ? t.f.size() * 4 : t.i.size() * 8;
        ok = ok && fwrite(d, 1, n, f) == n;
        size_t gap = ((n + 3) & ~(size_t)3) - n;
        static const char z[4] = {0, 0, 0, 0};
        if (gap) ok = ok && fwrite(z, 1, gap, f) == gap;
    }
    if (fclose(f) != 0 || !ok) throw Error(path + ": write failed");
}

}  // namespace hat
