// PNG I/O: decode to planar f32 RGB in [0,1], encode 8-bit RGB (src/image.rs).
//
// The reference decodes with the `png` crate and accepts 8- and 16-bit grey,
// grey+alpha, RGB and RGBA (image.rs:51-99); grey is replicated to three
// planes, alpha is dropped, samples are scaled by 1/255 or 1/65535. It writes
// 8-bit RGB from values clamped to [0,1], scaled by 255 and rounded half up
// (image.rs:30-41). This is the same contract on zlib: chunks are CRC-checked,
// IDAT is inflated, the five scanline filters are undone, Adam7 interlacing
// is de-interlaced.
#include "image.h"

#include <zlib.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "hip_rt.h"

namespace hat {

namespace {

const unsigned char kSig[8] = {0x89, 'P', 'N', 'G', '\r', '\n', 0x1a, '\n'};

uint32_t be32(const unsigned char* p) { return (uint32_t)p[0] << 24 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 8 | p[3]; }

// A chunk type for a message: its bytes come from the file, so anything
// outside printable ASCII is written as \xNN (messages stay valid text)
std::string chunk_name(const unsigned char* type)
{
    std::string s;
    for (int i = 0; i < 4; ++i) {
        if (type[i] >= 0x20 && type[i] < 0x7f) {
            s += (char)type[i];
        } else {
            char e[8];
            snprintf(e, sizeof e, "\\x%02x", type[i]);
            s += e;
        }
    }
    return s;
}

void put32(std::vector<unsigned char>& o, uint32_t v)
{
    o.push_back((unsigned char)(v >> 24));
    o.push_back((unsigned char)(v >> 16));
    o.push_back((unsigned char)(v >> 8));
    o.push_back((unsigned char)v);
}

std::vector<unsigned char> read_file(const std::string& path)
{
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) throw Error("open " + path + ": " + strerror(errno));
    std::vector<unsigned char> b;
    unsigned char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + n);
    fclose(f);
    return b;
}

int paeth(int a, int b, int c)
{
    const int p = a + b - c, pa = std::abs(p - a), pb = std::abs(p - b), pc = std::abs(p - c);
    if (pa <= pb && pa <= pc) return a;
    return pb <= pc ? b : c;
}

// Undo the filters of `rows` scanlines of `rowbytes` bytes (each preceded by
// its filter byte) in place; returns the unfiltered rows packed.
std::vector<unsigned char> unfilter(const unsigned char* src, size_t rows, size_t rowbytes, size_t bpp)
{
    std::vector<unsigned char> out(rows * rowbytes);
    for (size_t y = 0; y < rows; ++y) {
        const unsigned char ft = src[y * (rowbytes + 1)];
        const unsigned char* in = src + y * (rowbytes + 1) + 1;
        unsigned char* cur = &out[y * rowbytes];
        const unsigned char* prev = y ? &out[(y - 1) * rowbytes] : nullptr;
        for (size_t i = 0; i < rowbytes; ++i) {
            const int a = i >= bpp ? cur[i - bpp] : 0, b = prev ? prev[i] : 0,
                      c = (prev && i >= bpp) ? prev[i - bpp] : 0;
            int v = in[i];
            switch (ft) {
            case 0: break;
            case 1: v += a; break;
            case 2: v += b; break;
            case 3: v += (a + b) / 2; break;
            case 4: v += paeth(a, b, c); break;
            default: throw Error("png: scanline filter type " + std::to_string(ft) + " is not one PNG defines");
            }
            cur[i] = (unsigned char)v;
        }
    }
    return out;
}

}  // namespace

Image load_png(const std::string& path)
{
    std::vector<unsigned char> b = read_file(path);
    try {
        if (b.size() < 8 || memcmp(b.data(), kSig, 8) != 0) throw Error("not a PNG file (bad signature)");
        size_t off = 8;
        uint32_t w = 0, h = 0;
        int depth = 0, ctype = -1, interlace = 0;
        bool have_ihdr = false, have_iend = false;
        std::vector<unsigned char> idat;
        while (off + 12 <= b.size()) {
            const uint32_t len = be32(&b[off]);
            if (len > b.size() - off - 12) throw Error("truncated chunk");
            const unsigned char* type = &b[off + 4];
            const unsigned char* data = &b[off + 8];
            const uint32_t crc = be32(&b[off + 8 + len]);
            if ((uint32_t)crc32(crc32(0L, Z_NULL, 0), type, len + 4) != crc)
                throw Error(std::string("CRC error in chunk ") + chunk_name(type));
            if (!memcmp(type, "IHDR", 4)) {
                if (len != 13) throw Error("IHDR has the wrong length");
                w = be32(data);
                h = be32(data + 4);
                depth = data[8];
                ctype = data[9];
                if (data[10] != 0 || data[11] != 0) throw Error("unknown compression or filter method");
                interlace = data[12];
                if (interlace > 1) throw Error("unknown interlace method");
                have_ihdr = true;
            } else if (!memcmp(type, "IDAT", 4)) {
                idat.insert(idat.end(), data, data + len);
            } else if (!memcmp(type, "IEND", 4)) {
                have_iend = true;
                break;
            } else if (!(type[0] & 0x20)) {
                // an unknown critical chunk (PLTE is critical but only meaningful
                // for the indexed type, which is refused below)
                if (memcmp(type, "PLTE", 4) != 0)
                    throw Error(std::string("unknown critical chunk ") + chunk_name(type));
            }
            off += 12 + len;
        }
        if (!have_ihdr) throw Error("no IHDR chunk");
        if (!have_iend) throw Error("no IEND chunk (truncated file?)");
        int channels = 0;
        const char* cname = "?";
        switch (ctype) {
        case 0: channels = 1; cname = "Grayscale"; break;
        case 2: channels = 3; cname = "Rgb"; break;
        case 3: cname = "Indexed"; break;
        case 4: channels = 2; cname = "GrayscaleAlpha"; break;
        case 6: channels = 4; cname = "Rgba"; break;
        }
        if (channels == 0) throw Error(std::string("unsupported png colour type ") + cname);
        if (depth != 8 && depth != 16) throw Error("unsupported png bit depth " + std::to_string(depth));
        if (w == 0 || h == 0 || w > (1u << 20) || h > (1u << 20)) throw Error("image size out of range");
        const size_t bps = depth / 8, bpp = channels * bps;
        // Adam7 passes: (x0, y0, dx, dy); one full pass when not interlaced.
        static const int adam7[7][4] = {{0, 0, 8, 8}, {4, 0, 8, 8}, {0, 4, 4, 8}, {2, 0, 4, 4},
                                        {0, 2, 2, 4}, {1, 0, 2, 2}, {0, 1, 1, 2}};
        const int npass = interlace ? 7 : 1;
        size_t raw_size = 0;
        for (int ps = 0; ps < npass; ++ps) {
            const int x0 = interlace ? adam7[ps][0] : 0, y0 = interlace ? adam7[ps][1] : 0;
            const int dx = interlace ? adam7[ps][2] : 1, dy = interlace ? adam7[ps][3] : 1;
            const size_t pw = w > (uint32_t)x0 ? (w - x0 + dx - 1) / dx : 0;
            const size_t ph = h > (uint32_t)y0 ? (h - y0 + dy - 1) / dy : 0;
            if (pw && ph) raw_size += ph * (1 + pw * bpp);
        }
        std::vector<unsigned char> raw(raw_size);
        uLongf got = (uLongf)raw_size;
        if (uncompress(raw.data(), &got, idat.data(), (uLong)idat.size()) != Z_OK || got != raw_size)
            throw Error("corrupt or short image data (IDAT)");
        std::vector<unsigned char> px((size_t)w * h * bpp);
        size_t at = 0;
        for (int ps = 0; ps < npass; ++ps) {
            const int x0 = interlace ? adam7[ps][0] : 0, y0 = interlace ? adam7[ps][1] : 0;
            const int dx = interlace ? adam7[ps][2] : 1, dy = interlace ? adam7[ps][3] : 1;
            const size_t pw = w > (uint32_t)x0 ? (w - x0 + dx - 1) / dx : 0;
            const size_t ph = h > (uint32_t)y0 ? (h - y0 + dy - 1) / dy : 0;
            if (!pw || !ph) continue;
            std::vector<unsigned char> rows = unfilter(&raw[at], ph, pw * bpp, bpp);
            at += ph * (1 + pw * bpp);
            for (size_t y = 0; y < ph; ++y)
                for (size_t x = 0; x < pw; ++x)
                    memcpy(&px[((y0 + y * dy) * (size_t)w + x0 + x * dx) * bpp], &rows[(y * pw + x) * bpp], bpp);
        }
        Image img;
        img.w = w;
        img.h = h;
        img.data.assign(3 * (size_t)w * h, 0.f);
        const size_t hw = (size_t)w * h;
        const float sc = depth == 16 ? 1.0f / 65535.0f : 1.0f / 255.0f;
        auto sample = [&](size_t p, int c) -> float {
            const size_t i = p * channels + c;
            return depth == 16 ? (float)((px[2 * i] << 8) | px[2 * i + 1]) * sc : (float)px[i] * sc;
        };
        for (size_t p = 0; p < hw; ++p) {
            if (channels <= 2) {
                const float v = sample(p, 0);
                img.data[p] = img.data[hw + p] = img.data[2 * hw + p] = v;
            } else {
                img.data[p] = sample(p, 0);
                img.data[hw + p] = sample(p, 1);
                img.data[2 * hw + p] = sample(p, 2);
            }
        }
        return img;
    } catch (const Error& e) {
        throw Error(path + ": " + e.msg);
    }
}

std::vector<unsigned char> to_rgb8(size_t w, size_t h, const float* planes)
{
    const size_t hw = w * h;
    std::vector<unsigned char> out(hw * 3);
    for (size_t i = 0; i < hw; ++i)
        for (int c = 0; c < 3; ++c) {
            float v = planes[c * hw + i];
            v = (v < 0.f ? 0.f : v > 1.f ? 1.f : v) * 255.0f;
            const float r = std::floor(v + 0.5f);
            // `(v + 0.5).floor().min(255.0) as u8`: min() of a NaN gives 255
            out[i * 3 + c] = (unsigned char)(std::isnan(r) || r >= 255.f ? 255 : (int)r);
        }
    return out;
}

void save_png(const std::string& path, size_t w, size_t h, const float* planes)
{
    if (w == 0 || h == 0 || w > (1u << 24) || h > (1u << 24)) throw Error(path + ": image size out of range");
    std::vector<unsigned char> rgb = to_rgb8(w, h, planes);
    std::vector<unsigned char> raw(h * (1 + 3 * w));
    for (size_t y = 0; y < h; ++y) {
        raw[y * (1 + 3 * w)] = 0;  // filter: none
        memcpy(&raw[y * (1 + 3 * w) + 1], &rgb[y * 3 * w], 3 * w);
    }
    uLongf zlen = compressBound((uLong)raw.size());
    std::vector<unsigned char> z(zlen);
    if (compress2(z.data(), &zlen, raw.data(), (uLong)raw.size(), 6) != Z_OK) throw Error(path + ": deflate failed");
    z.resize(zlen);
    std::vector<unsigned char> o(kSig, kSig + 8);
    auto chunk = [&](const char* type, const unsigned char* data, size_t len) {
        put32(o, (uint32_t)len);
        const size_t start = o.size();
        o.insert(o.end(), type, type + 4);
        o.insert(o.end(), data, data + len);
        put32(o, (uint32_t)crc32(crc32(0L, Z_NULL, 0), &o[start], (uInt)(len + 4)));
    };
    std::vector<unsigned char> ihdr;
    put32(ihdr, (uint32_t)w);
    put32(ihdr, (uint32_t)h);
    ihdr.insert(ihdr.end(), {8, 2, 0, 0, 0});  // 8-bit RGB, deflate, adaptive filters, no interlace
    chunk("IHDR", ihdr.data(), ihdr.size());
    chunk("IDAT", z.data(), z.size());
    chunk("IEND", nullptr, 0);
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) throw Error("create " + path + ": " + strerror(errno));
    const size_t n = fwrite(o.data(), 1, o.size(), f);
    const int rc = fclose(f);
    if (n != o.size() || rc != 0) throw Error(path + ": write failed");
}

}  // namespace hat
