// The reference pipeline's padding and crop (src/image.rs:106-246), and the
// CPU memory guard (src/memguard.rs:35-172).

#include <cstdio>
#include <fstream>
#include <sstream>
#include <string>

#include "host.hpp"

namespace mx {

namespace {

// jnp.pad(mode='reflect'): mirror about the edge without repeating it.
int64_t reflect_index(int64_t i, int64_t n) {
    if (i < 0) return -i;
    if (i >= n) return 2 * n - 2 - i;
    return i;
}

void reflect_pad2(const float *img, int64_t c, int64_t h, int64_t w, int64_t top, int64_t bottom,
                  int64_t left, int64_t right, float *out) {
    int64_t nh = h + top + bottom, nw = w + left + right;
    for (int64_t y = 0; y < nh; ++y) {
        int64_t sy = reflect_index(y - top, h);
        for (int64_t x = 0; x < nw; ++x) {
            int64_t sx = reflect_index(x - left, w);
            for (int64_t ch = 0; ch < c; ++ch)
                out[ch * nh * nw + y * nw + x] = img[ch * h * w + sy * w + sx];
        }
    }
}

// The first even d below `factor` whose centred pad is smaller than d.
int64_t min_dimension(int64_t factor) {
    for (int64_t d = 2; d < factor; d += 2) {
        int64_t up = ((d + factor) / factor) * factor;
        if ((up - d) / 2 < d) return d;
    }
    return factor;
}

}  // namespace

}  // namespace mx

using namespace mx;

extern "C" {

void mx_same_pad(int64_t size, int64_t stride, int64_t k, int64_t *before, int64_t *after) {
    int64_t b, a;
    same_pad(size, stride, k, b, a);
    if (before) *before = b;
    if (after) *after = a;
}

int mx_preprocess(const float *img, int64_t c, int64_t h, int64_t w, int64_t factor, float *out,
                  int64_t *ph, int64_t *pw, int64_t *even_h, int64_t *even_w) {
    if (c <= 0 || h <= 0 || w <= 0 || factor <= 0) {
        set_error("preprocess: empty image or factor");
        return -1;
    }
    int64_t eh = h + h % 2, ew = w + w % 2;
    int64_t hp = eh % factor ? ((eh + factor) / factor) * factor : eh;
    int64_t wp = ew % factor ? ((ew + factor) / factor) * factor : ew;
    int64_t padh = hp - eh, padw = wp - ew;
    struct { const char *axis; int64_t dim, pad; } axes[2] = {{"height", eh, padh / 2},
                                                             {"width", ew, padw / 2}};
    for (auto &a : axes) {
        if (a.pad != 0 && a.pad >= a.dim) {
            std::ostringstream m;
            m << "this image is too small for MAXIM's " << factor << "-multiple padding: the "
              << a.axis << " is " << a.dim << " pixels and the pipeline reflects it out to the next "
              << "multiple of " << factor << ", which is " << a.pad
              << " pixels of padding a side - a reflection needs less padding than the dimension "
                 "it mirrors. The reference pipeline refuses this input for the same reason "
                 "(torch's reflect pad: `Padding size should be less than the corresponding input "
                 "dimension`). Give it an image at least "
              << min_dimension(factor) << " pixels on its " << a.axis << ".";
            set_error(m.str());
            return -1;
        }
    }
    // The even-ize pad must itself be a legal reflection (a 1-pixel axis is not).
    if ((h % 2 && h < 2) || (w % 2 && w < 2)) {
        set_error("preprocess: a 1-pixel axis cannot be reflected to an even size");
        return -1;
    }
    if (ph) *ph = hp;
    if (pw) *pw = wp;
    if (even_h) *even_h = eh;
    if (even_w) *even_w = ew;
    if (!out) return 0;
    std::vector<float> even((size_t)(c * eh * ew));
    reflect_pad2(img, c, h, w, 0, h % 2, 0, w % 2, even.data());
    reflect_pad2(even.data(), c, eh, ew, padh / 2, padh / 2, padw / 2, padw / 2, out);
    return 0;
}

int mx_crop_out(const float *img, int64_t c, int64_t ph, int64_t pw, int64_t even_h,
                int64_t even_w, int64_t orig_h, int64_t orig_w, float *out) {
    int64_t hs = ph / 2 - even_h / 2, ws = pw / 2 - even_w / 2;
    if (hs < 0 || ws < 0 || hs + orig_h > ph || ws + orig_w > pw) {
        set_error("crop_out: the crop does not fit the padded image");
        return -1;
    }
    for (int64_t ch = 0; ch < c; ++ch)
        for (int64_t y = 0; y < orig_h; ++y)
            for (int64_t x = 0; x < orig_w; ++x)
                out[ch * orig_h * orig_w + y * orig_w + x] = img[ch * ph * pw + (hs + y) * pw + (ws + x)];
    return 0;
}

// memguard: (arena + 2 * weights + conv1x1 scratch) * 1.05 + 64 MiB against
// MemAvailable. The scratch term is the CPU conv1x1's per-task tile: at most
// 12 * threads tasks, each PB x c_in + PB + c_out floats, PB = 256.
int mx_memguard_check(const mx_plan *pp, int threads, int64_t avail_override, uint64_t *peak_bytes) {
    const Plan *p = reinterpret_cast<const Plan *>(pp);
    const uint64_t PB = 256, BASE = 64ull << 20;
    const double SLACK = 1.05;
    uint64_t arena = p->arena_len * 4, weights = p->weight_bytes() * 2;
    int64_t ci = 1, co = 1;
    bool any = false;
    for (auto &op : p->ops)
        if (op.kind == MX_OP_CONV1X1) {
            // (c_in, c_out) tuples compared lexicographically, as the reference's max().
            if (!any || op.c_in > ci || (op.c_in == ci && op.c_out > co)) { ci = op.c_in; co = op.c_out; }
            any = true;
        }
    uint64_t tasks = 12ull * (threads > 0 ? threads : 1);
    uint64_t scratch = tasks * (PB * ci * 4 + PB * 4 + co * 4);
    uint64_t peak = (uint64_t)((double)(arena + weights + scratch) * SLACK) + BASE;
    if (peak_bytes) *peak_bytes = peak;
    int64_t avail = avail_override;
    if (avail < 0) {
        std::ifstream f("/proc/meminfo");
        std::string line;
        while (std::getline(f, line)) {
            if (line.rfind("MemAvailable:", 0) != 0) continue;
            avail = std::stoll(line.substr(13)) * 1024;
            break;
        }
    }
    if (avail < 0 || peak <= (uint64_t)avail) return 0;
    std::ostringstream m;
    m << "not enough memory for a " << p->shape.w << "x" << p->shape.h << " pass on the CPU\n"
      << "maxim: it needs about " << (peak >> 20) << " MiB (" << (arena >> 20) << " of arena + "
      << (weights >> 20) << " of weights, twice + " << (scratch >> 20)
      << " of per-task scratch, plus 5% for allocator slack); " << ((uint64_t)avail >> 20)
      << " MiB is available";
    set_error(m.str());
    return -1;
}

}  // extern "C"
