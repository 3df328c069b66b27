// maxim_hip: the enhancement run on one MI355X, the reference CLI's `run`
// (src/main.rs:173-458) with the HIP backend, and its argument handling
// (src/main.rs:59-158) as a release build has it:
//
//   maxim_hip -m MODEL.safetensors [-i IN.png] [-o OUT.png] [-q]
//
// reads the PNG (from stdin when -i is `-` or absent, src/main.rs:205-214),
// runs mxh_enhance (checkpoint -> padded plan -> device pass -> crop) and
// writes the PNG (to stdout when -o is `-` or absent, src/main.rs:439-448).
// As in the reference, a pass that fails is reported, not retried elsewhere.
// There is no CPU backend in this binary: `--device gpu|hip` and `--gpu`
// select the one it has, `--device cpu` and `--cpu` are refused by name.
// The development flags (--dump, --profile, --factor) live in the Python
// package's entry point (python -m maxim_amd); like the reference's release
// build, this binary refuses them by name rather than ignoring them.

#include <cerrno>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "maxim_hip.h"

static const char *kVersion = "0.3.0";

static int usage() {
    std::fprintf(stderr,
                 "usage: maxim_hip -m MODEL.safetensors [-i IN.png] [-o OUT.png] [options]\n"
                 "    -m, --model <path>    converted .safetensors checkpoint\n"
                 "    -i, --input <path>    input PNG, or - for stdin (default: stdin)\n"
                 "    -o, --output <path>   output PNG, or - for stdout (default: stdout)\n"
                 "        --device <dev>    gpu (or hip): the MI355X; this binary has no CPU backend\n"
                 "        --gpu             same as --device gpu\n"
                 "    -q, --quiet           no progress output\n"
                 "    -h, --help            this text\n"
                 "    -V, --version         print the version\n");
    return 2;
}

static int fail() {
    std::fprintf(stderr, "maxim: %s\n", mx_last_error());
    return 1;
}

int main(int argc, char **argv) {
    std::string model, in = "-", out = "-";
    bool quiet = false;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&](std::string &v) {
            if (i + 1 >= argc) return false;
            v = argv[++i];
            return true;
        };
        std::string dev;
        if (a == "-m" || a == "--model") {
            if (!next(model)) return usage();
        } else if (a == "-i" || a == "--input") {
            if (!next(in)) return usage();
        } else if (a == "-o" || a == "--output") {
            if (!next(out)) return usage();
        } else if (a == "-q" || a == "--quiet") {
            quiet = true;
        } else if (a == "--device" || a == "--gpu" || a == "--cpu") {
            if (a == "--device" && !next(dev)) return usage();
            if (a == "--cpu" || (a == "--device" && dev != "gpu" && dev != "hip")) {
                std::fprintf(stderr, "maxim: `%s%s%s`: this binary runs on the MI355X only (no CPU backend)\n",
                             a.c_str(), dev.empty() ? "" : " ", dev.c_str());
                return 2;
            }
        } else if (a == "--dump" || a == "--profile" || a == "--timeline" || a == "--verify-gpu" ||
                   a == "--factor") {
            std::fprintf(stderr,
                         "maxim: `%s` is a development flag and this is the release command\n"
                         "maxim: python -m maxim_amd takes --dump, --profile and --factor\n",
                         a.c_str());
            return 2;
        } else if (a == "-h" || a == "--help") {
            return usage();
        } else if (a == "-V" || a == "--version") {
            std::printf("maxim_hip %s\n", kVersion);
            return 0;
        } else {
            std::fprintf(stderr, "maxim: unknown argument `%s`\n", a.c_str());
            return usage();
        }
    }
    if (model.empty()) {
        std::fprintf(stderr, "maxim: --model is required\n");
        return usage();
    }
    if (mxh_driver_ready() != 0) {
        std::fprintf(stderr, "maxim: hip: %s\n", mx_last_error());
        return 1;
    }
    // The image: decoded once, from the file or from everything on stdin.
    mx_png *png = nullptr;
    int64_t h = 0, w = 0;
    if (in == "-") {
        std::vector<unsigned char> buf;
        unsigned char chunk[1 << 16];
        size_t k;
        while ((k = std::fread(chunk, 1, sizeof chunk, stdin)) > 0) buf.insert(buf.end(), chunk, chunk + k);
        if (std::ferror(stdin)) {
            std::fprintf(stderr, "maxim: read stdin: %s\n", std::strerror(errno));
            return 1;
        }
        if (mx_png_open(nullptr, buf.data(), buf.size(), &png, &h, &w) != 0) return fail();
    } else if (mx_png_open(in.c_str(), nullptr, 0, &png, &h, &w) != 0) {
        return fail();
    }
    std::vector<float> img((size_t)(3 * h * w)), res(img.size());
    const int got = mx_png_pixels(png, img.data(), img.size());
    mx_png_close(png);
    if (got != 0) return fail();
    const auto t0 = std::chrono::steady_clock::now();
    if (mxh_enhance(model.c_str(), img.data(), h, w, res.data()) != 0) return fail();
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (!quiet) std::fprintf(stderr, "maxim: %lldx%lld enhanced in %.2fs on the GPU\n", (long long)w, (long long)h, secs);
    if (out == "-") {
        size_t n = 0;
        if (mx_png_encode(res.data(), h, w, nullptr, 0, &n) != 0) return fail();
        std::vector<unsigned char> bytes(n);
        if (mx_png_encode(res.data(), h, w, bytes.data(), bytes.size(), &n) != 0) return fail();
        if (std::fwrite(bytes.data(), 1, n, stdout) != n || std::fflush(stdout) != 0) {
            std::fprintf(stderr, "maxim: stdout: %s\n", std::strerror(errno));
            return 1;
        }
    } else {
        if (mx_png_write(out.c_str(), res.data(), h, w) != 0) return fail();
        if (!quiet) std::fprintf(stderr, "maxim: wrote %s\n", out.c_str());
    }
    return 0;
}
