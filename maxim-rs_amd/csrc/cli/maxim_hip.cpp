// maxim_hip: the enhancement run on one MI355X, the reference CLI's `run`
// (src/main.rs:173-458) with the HIP backend:
//
//   maxim_hip -m MODEL.safetensors [-i IN.png] [-o OUT.png] [-q]
//
// reads the PNG, runs mxh_enhance (checkpoint -> padded plan -> device pass
// -> crop) and writes the PNG. As in the reference, a pass that fails is
// reported, not retried elsewhere; there is no CPU backend in this binary.

#include <chrono>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "maxim_hip.h"

static int usage() {
    std::fprintf(stderr, "usage: maxim_hip -m MODEL.safetensors -i IN.png -o OUT.png [-q]\n");
    return 2;
}

int main(int argc, char **argv) {
    std::string model, in, out;
    bool quiet = false;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&](std::string &v) {
            if (i + 1 >= argc) return false;
            v = argv[++i];
            return true;
        };
        if ((a == "-m" || a == "--model") && next(model)) continue;
        if ((a == "-i" || a == "--input") && next(in)) continue;
        if ((a == "-o" || a == "--output") && next(out)) continue;
        if (a == "-q" || a == "--quiet") {
            quiet = true;
            continue;
        }
        return usage();
    }
    if (model.empty() || in.empty() || out.empty()) return usage();
    if (mxh_driver_ready() != 0) {
        std::fprintf(stderr, "maxim: hip: %s\n", mx_last_error());
        return 1;
    }
    int64_t h = 0, w = 0;
    if (mx_png_read(in.c_str(), nullptr, &h, &w) != 0) {
        std::fprintf(stderr, "maxim: %s\n", mx_last_error());
        return 1;
    }
    std::vector<float> img((size_t)(3 * h * w)), res(img.size());
    if (mx_png_read(in.c_str(), img.data(), &h, &w) != 0) {
        std::fprintf(stderr, "maxim: %s\n", mx_last_error());
        return 1;
    }
    const auto t0 = std::chrono::steady_clock::now();
    if (mxh_enhance(model.c_str(), img.data(), h, w, res.data()) != 0) {
        std::fprintf(stderr, "maxim: %s\n", mx_last_error());
        return 1;
    }
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (mx_png_write(out.c_str(), res.data(), h, w) != 0) {
        std::fprintf(stderr, "maxim: %s\n", mx_last_error());
        return 1;
    }
    if (!quiet) std::fprintf(stderr, "maxim: %lldx%lld enhanced in %.2fs on the GPU, wrote %s\n", (long long)w, (long long)h, secs, out.c_str());
    return 0;
}
