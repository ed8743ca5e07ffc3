// The `hat` binary: one image in, one image out (src/main.rs of the reference).
//
// Argument parsing, file I/O and reporting over the C ABI of libhat.so
// (include/hat.h) - the same flags, printed lines and exit codes as the
// reference's CLI, so a command line written for it works here:
//   0 success; 1 a run error, printed as `hat: <message>` (main.rs:189-195);
//   2 a command-line error (main.rs:182-187).
// The device is the MI355X: `--device gpu` or nothing; there is no CPU path,
// and `--device cpu` is refused rather than silently run elsewhere.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/hat.h"

namespace {

const char* kUsage =
    "hat - HAT super-resolution (S/M/L, x2/x3/x4) on an AMD MI355X\n"
    "\n"
    "USAGE:\n"
    "    hat -m <model.safetensors> -i <in.png> -o <out.png> [--device gpu]\n"
    "    hat -m <model.safetensors> --verify <fixture.bin>\n"
    "    hat -m <model.safetensors> --list-weights\n"
    "    hat --cuda-selftest\n"
    "\n"
    "OPTIONS:\n"
    "    -m, --model <path>    a checkpoint converted by tools/convert.py\n"
    "    -i, --input <path>    the image to upscale (PNG)\n"
    "    -o, --output <path>   where to write the result (PNG)\n"
    "        --verify <path>   compare the backend against a golden fixture and report the\n"
    "                          worst and mean absolute difference; exits 1 if it is over\n"
    "                          the tolerance, so it can be used as a test\n"
    "        --device <name>   gpu (the only device of this build; left out, the GPU is\n"
    "                          used when the HIP runtime can be brought up)\n"
    "        --list-weights    print every tensor the checkpoint holds, with its shape\n"
    "        --cuda-selftest   check every gfx950 kernel against a host implementation of\n"
    "                          the same operator, on seeded inputs (no -m needed); also\n"
    "                          accepted as --selftest\n"
    "        --tile <px>       run the image in <px>-wide tiles (rounded up to a window\n"
    "                          multiple) instead of one pass; the tile is approximate near\n"
    "                          its edges, since a window attention reaches across the whole\n"
    "                          window and each 3x3 conv widens the field by a pixel\n"
    "        --mem <MiB>       a working-set budget; chooses the largest window-multiple\n"
    "                          tile that fits it, and caps `--tile` if both are given\n"
    "    -h, --help            this text";

struct Args {
    std::string model, input, output, verify, device;
    bool list_weights = false, selftest = false;
    bool have_tile = false, have_mem = false;
    size_t tile = 0;
    double mem = 0.0;
};

struct CliError {
    std::string msg;
};
struct UsageError {
    std::string msg;
};

std::string last_error() { return hat_last_error(); }

Args parse(int argc, char** argv)
{
    Args a;
    for (int i = 1; i < argc; ++i) {
        const std::string flag = argv[i];
        auto next = [&]() -> std::string {
            if (i + 1 >= argc) throw UsageError{flag + " needs a value"};
            return argv[++i];
        };
        if (flag == "-m" || flag == "--model") a.model = next();
        else if (flag == "-i" || flag == "--input") a.input = next();
        else if (flag == "-o" || flag == "--output") a.output = next();
        else if (flag == "--verify") a.verify = next();
        else if (flag == "--device") a.device = next();
        else if (flag == "--list-weights") a.list_weights = true;
        else if (flag == "--cuda-selftest" || flag == "--selftest") a.selftest = true;
        else if (flag == "--tile") {
            const std::string v = next();
            char* end = nullptr;
            const unsigned long long t = strtoull(v.c_str(), &end, 10);
            if (v.empty() || *end != '\0' || v[0] == '-') throw UsageError{"--tile: invalid digit found in string"};
            a.tile = (size_t)t;
            a.have_tile = true;
        } else if (flag == "--mem") {
            const std::string v = next();
            char* end = nullptr;
            const double m = strtod(v.c_str(), &end);
            if (v.empty() || *end != '\0') throw UsageError{"--mem: invalid float literal"};
            a.mem = m;
            a.have_mem = true;
        } else if (flag == "-h" || flag == "--help") {
            printf("%s\n", kUsage);
            exit(0);
        } else {
            throw UsageError{"unknown argument `" + flag + "`\n\n" + kUsage};
        }
    }
    // --cuda-selftest runs on synthetic inputs, so it needs no checkpoint.
    if (a.model.empty() && !a.selftest) throw UsageError{std::string("no model: -m is required\n\n") + kUsage};
    return a;
}

// main.rs:148-174 resolve_device: the unspecified case uses the GPU when the
// runtime comes up; a CPU path does not exist in this build.
void resolve_device(const std::string& requested)
{
    if (requested == "cpu")
        throw CliError{"device `cpu`: this build is the MI355X backend and has only `gpu` "
                       "(the reference's CPU path is not part of it)"};
    if (!requested.empty() && requested != "gpu")
        throw CliError{"device `" + requested + "`: expected `gpu`"};
    if (!hat_gpu_available())
        throw CliError{"no HIP device could be brought up, and this build has no CPU path"};
}

std::string shape_str(const hat_weights* w, const char* name)
{
    size_t d[16];
    const int n = hat_weights_shape(w, name, d, 16);
    std::string s = "[";
    for (int i = 0; i < n && i < 16; ++i) s += (i ? ", " : "") + std::to_string(d[i]);
    return s + "]";
}

void run(const Args& a)
{
    if (a.selftest) {
        printf("cuda selftest - every gfx950 kernel against a host twin\n");
        fflush(stdout);
        if (hat_gpu_selftest() < 0) throw CliError{last_error()};
        return;
    }
    hat_weights* wt = hat_weights_open(a.model.c_str());
    if (!wt) throw CliError{last_error()};
    struct Closer {
        hat_weights* w;
        ~Closer() { hat_weights_close(w); }
    } closer{wt};
    hat_model_info info;
    if (hat_weights_info(wt, &info) != 0) throw CliError{last_error()};
    printf("hat %s - %s (x%d), %llu bytes\n", hat_version(), hat_weights_variant(wt), info.scale,
           (unsigned long long)hat_weights_file_bytes(wt));
    if (a.list_weights) {
        const int n = hat_weights_count(wt);
        for (int i = 0; i < n; ++i) {
            const char* name = hat_weights_name(wt, i);
            printf("  %s  %s\n", name, shape_str(wt, name).c_str());
        }
        return;
    }
    resolve_device(a.device);
    if (!a.verify.empty()) {
        const int rc = hat_verify(wt, "gpu", a.verify.c_str());
        if (rc != 0) throw CliError{last_error()};
        return;
    }
    if (a.input.empty() || a.output.empty()) throw CliError{"nothing to do: give -i and -o, or --verify"};
    size_t w = 0, h = 0;
    if (hat_png_load(a.input.c_str(), &w, &h, nullptr, 0) != 0) throw CliError{last_error()};
    std::vector<float> img(3 * w * h);
    if (hat_png_load(a.input.c_str(), &w, &h, img.data(), img.size()) != 0) throw CliError{last_error()};
    const size_t s = (size_t)info.scale;
    printf("  input  %zux%zu -> %zux%zu\n", w, h, w * s, h * s);
    fflush(stdout);
    const auto t0 = std::chrono::steady_clock::now();
    hat_backend* be = hat_backend_new(wt, "gpu");
    if (!be) throw CliError{last_error()};
    struct Freer {
        hat_backend* b;
        ~Freer() { hat_backend_free(b); }
    } freer{be};
    // main.rs:226-278: with neither --tile nor --mem the tile comes from the
    // device's free memory (one tile when the whole image fits); --mem picks it
    // from the per-pixel cost; an explicit --tile is capped by --mem.
    const size_t win = (size_t)info.window, margin = 2 * win;
    size_t tile = 0;
    if (!a.have_tile && !a.have_mem) {
        const long t = hat_gpu_auto_tile(wt, h, w);
        if (t < 0) throw CliError{last_error()};
        tile = (size_t)t;
        if (tile >= std::max(w, h)) printf("  whole-image pass fits in free VRAM\n");
        else printf("  free VRAM -> tile %zupx (margin %zu)\n", tile, margin);
    } else if (a.have_mem) {
        // The per-pixel cost is this backend's own per-plan device bytes at the
        // image's padded size. The reference divides Cpu::footprint_floats by the
        // plan's tokens for either device (main.rs:244-245); this build has no CPU
        // backend, and its device buffers are what a tile must fit.
        hat_mem_plan mp;
        if (hat_gpu_plan(wt, h, w, &mp) != 0) throw CliError{last_error()};
        const size_t hp = (h + win - 1) / win * win, wp = (w + win - 1) / win * win;
        const unsigned long long per_pixel = mp.activations / 4 / std::max<size_t>(1, hp * wp);
        // (mib * 1024 * 1024) as u64 (main.rs:270), Rust's saturating cast:
        // NaN and negatives give 0, values past the range u64::MAX (a plain C++
        // cast of those is undefined)
        const double bytes = a.mem * 1024.0 * 1024.0;
        const unsigned long long budget = !(bytes > 0.0)                ? 0ull
                                          : bytes >= 18446744073709551616.0 ? ~0ull
                                                                            : (unsigned long long)bytes;
        const size_t t = hat_auto_tile(h, w, win, budget, per_pixel, 0, margin);
        if (t == 0) {
            char m[160];
            snprintf(m, sizeof m, "--mem %g MiB is too small even for one window", a.mem);
            throw CliError{m};
        }
        printf("  --mem %g MiB -> tile %zupx (margin %zu)\n", a.mem, t, margin);
        tile = a.have_tile ? std::min(a.tile, t) : t;
    } else {
        tile = a.tile;
    }
    std::vector<float> out(3 * w * s * h * s);
    hat_tiling ti;
    if (hat_tile_forward(be, h, w, img.data(), out.data(), tile, margin, &ti) != 0) throw CliError{last_error()};
    // "largest" is the biggest sub-image as height x width (main.rs:278-280 prints
    // tile.rs's `largest`, which is (sh, sw))
    printf("  tiled %zux%zu into %zu tiles (%zupx cores, %zupx margin, largest %zux%zu)\n", w, h, ti.tiles,
           ti.tile, ti.margin, ti.largest_h, ti.largest_w);
    const double sec = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    printf("  gpu forward in %.1f ms (%.2f MP/s)\n", sec * 1e3, (double)(w * h) / 1e6 / sec);
    if (hat_png_save(a.output.c_str(), w * s, h * s, out.data()) != 0) throw CliError{last_error()};
    printf("  wrote %s\n", a.output.c_str());
}

}  // namespace

int main(int argc, char** argv)
{
    Args a;
    try {
        a = parse(argc, argv);
    } catch (const UsageError& e) {
        fprintf(stderr, "%s\n", e.msg.c_str());
        return 2;
    }
    try {
        run(a);
    } catch (const CliError& e) {
        fflush(stdout);
        fprintf(stderr, "hat: %s\n", e.msg.c_str());
        return 1;
    }
    return 0;
}
