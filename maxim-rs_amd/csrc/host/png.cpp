// PNG in and out for the enhancement run (the reference's image::read_png /
// read_png_stream / write_png / write_png_stream, src/image.rs:33-104, which
// use the `png` crate).
//
// Reading: 8-bit grayscale, gray + alpha, RGB and RGBA, plain or Adam7
// interlaced, from a file or from bytes in memory (the CLI's `-i -`), as
// [3][h][w] floats in 0..1 (grayscale expanded to RGB, alpha dropped, like
// the reference's `Image.convert('RGB')` match arms); indexed images are
// refused with the reference's message, and so are bit depths other than 8.
// The zlib stream is decoded by the inflate below (RFC 1951: stored,
// fixed-Huffman and dynamic-Huffman blocks), then the five PNG row filters
// are undone, per pass for an interlaced image (PNG 1.2, 8.2: seven passes,
// each a sub-image filtered on its own), whose pixels are then put in place.
// A decoded image is held by an mx_png handle, so the file is read and
// decoded once and the caller copies it out into a buffer of stated size.
//
// Writing: [3][h][w] clamped to 0..1 as 8-bit RGB, rounding half up
// (v * 255 + 0.5), every row unfiltered, the zlib stream in stored deflate
// blocks (a valid PNG that any decoder reads; compression is not the
// point of an enhancement run's output), to a file or into memory (`-o -`).

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "host.hpp"

namespace mx {
namespace {

// The CRC-32 table, built once by the first caller (a function-local static:
// its initialisation is thread-safe).
struct CrcTable {
    uint32_t t[256];
    CrcTable() {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t v = i;
            for (int k = 0; k < 8; ++k) v = (v & 1) ? 0xedb88320u ^ (v >> 1) : v >> 1;
            t[i] = v;
        }
    }
};

uint32_t crc32(const unsigned char *p, size_t n, uint32_t c = 0xffffffffu) {
    static const CrcTable table;
    for (size_t i = 0; i < n; ++i) c = table.t[(c ^ p[i]) & 0xff] ^ (c >> 8);
    return c;
}

uint32_t adler32(const unsigned char *p, size_t n) {
    uint32_t a = 1, b = 0;
    for (size_t i = 0; i < n; ++i) {
        a = (a + p[i]) % 65521u;
        b = (b + a) % 65521u;
    }
    return (b << 16) | a;
}

uint32_t be32(const unsigned char *p) {
    return ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | p[3];
}

// ---------------------------------------------------------------- inflate

struct Bits {
    const unsigned char *p;
    size_t n, pos = 0;  // bit position
    uint32_t get(int k) {
        uint32_t v = 0;
        for (int i = 0; i < k; ++i, ++pos) {
            if ((pos >> 3) >= n) throw Error("png: the compressed image data ends early");
            v |= (uint32_t)((p[pos >> 3] >> (pos & 7)) & 1) << i;
        }
        return v;
    }
};

// A canonical Huffman code (RFC 1951 3.2.2): counts per length and the
// symbols in code order; decoded bit by bit, most significant first.
struct Huff {
    int count[16] = {0};
    std::vector<int> sym;
    void build(const int *len, int n) {
        std::memset(count, 0, sizeof count);
        for (int i = 0; i < n; ++i) ++count[len[i]];
        count[0] = 0;
        int offs[16] = {0};
        for (int l = 1; l < 16; ++l) offs[l] = offs[l - 1] + count[l - 1];
        sym.assign(n, 0);
        for (int i = 0; i < n; ++i)
            if (len[i]) sym[offs[len[i]]++] = i;
    }
    int decode(Bits &b) const {
        int code = 0, first = 0, index = 0;
        for (int l = 1; l < 16; ++l) {
            code |= (int)b.get(1);
            const int c = count[l];
            if (code - first < c) return sym[index + code - first];
            index += c;
            first = (first + c) << 1;
            code <<= 1;
        }
        throw Error("png: an invalid Huffman code in the image data");
    }
};

// The fixed Huffman codes of RFC 1951 3.2.6.
struct FixedCodes {
    Huff lit, dist;
    FixedCodes() {
        int l[288];
        for (int i = 0; i < 288; ++i) l[i] = i < 144 ? 8 : i < 256 ? 9 : i < 280 ? 7 : 8;
        lit.build(l, 288);
        int d[30];
        for (int i = 0; i < 30; ++i) d[i] = 5;
        dist.build(d, 30);
    }
};

const int kLenBase[29] = {3, 4, 5, 6, 7, 8, 9, 10, 11, 13, 15, 17, 19, 23, 27, 31, 35, 43, 51, 59, 67, 83, 99, 115, 131, 163, 195, 227, 258};
const int kLenExtra[29] = {0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3, 4, 4, 4, 4, 5, 5, 5, 5, 0};
const int kDistBase[30] = {1, 2, 3, 4, 5, 7, 9, 13, 17, 25, 33, 49, 65, 97, 129, 193, 257, 385, 513, 769, 1025, 1537, 2049, 3073, 4097, 6145, 8193, 12289, 16385, 24577};
const int kDistExtra[30] = {0, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 6, 6, 7, 7, 8, 8, 9, 9, 10, 10, 11, 11, 12, 12, 13, 13};

void inflate_block(Bits &b, const Huff &lit, const Huff &dist, std::vector<unsigned char> &out, size_t limit) {
    for (;;) {
        const int s = lit.decode(b);
        if (s < 256) {
            out.push_back((unsigned char)s);
        } else if (s == 256) {
            return;
        } else {
            const int li = s - 257;
            if (li >= 29) throw Error("png: an invalid length code in the image data");
            const size_t len = (size_t)kLenBase[li] + b.get(kLenExtra[li]);
            const int di = dist.decode(b);
            if (di >= 30) throw Error("png: an invalid distance code in the image data");
            const size_t d = (size_t)kDistBase[di] + b.get(kDistExtra[di]);
            if (d > out.size()) throw Error("png: a back reference before the start of the image data");
            const size_t from = out.size() - d;
            for (size_t k = 0; k < len; ++k) out.push_back(out[from + k]);
        }
        if (out.size() > limit) throw Error("png: the image data inflates past the image size");
    }
}

std::vector<unsigned char> inflate(const unsigned char *p, size_t n, size_t limit) {
    Bits b{p, n};
    std::vector<unsigned char> out;
    out.reserve(limit);
    int last = 0;
    do {
        last = (int)b.get(1);
        const int type = (int)b.get(2);
        if (type == 0) {
            b.pos = (b.pos + 7) & ~(size_t)7;
            const size_t at = b.pos >> 3;
            if (at + 4 > n) throw Error("png: a stored block runs past the image data");
            const unsigned len = p[at] | (p[at + 1] << 8), nlen = p[at + 2] | (p[at + 3] << 8);
            if ((len ^ 0xffffu) != nlen) throw Error("png: a stored block with a bad length");
            if (at + 4 + len > n) throw Error("png: a stored block runs past the image data");
            out.insert(out.end(), p + at + 4, p + at + 4 + len);
            b.pos = (at + 4 + len) << 3;
            if (out.size() > limit) throw Error("png: the image data inflates past the image size");
        } else if (type == 1) {
            static const FixedCodes fixed;  // built once, thread-safe
            inflate_block(b, fixed.lit, fixed.dist, out, limit);
        } else if (type == 2) {
            const int hlit = (int)b.get(5) + 257, hdist = (int)b.get(5) + 1, hclen = (int)b.get(4) + 4;
            static const int order[19] = {16, 17, 18, 0, 8, 7, 9, 6, 10, 5, 11, 4, 12, 3, 13, 2, 14, 1, 15};
            int cl[19] = {0};
            for (int i = 0; i < hclen; ++i) cl[order[i]] = (int)b.get(3);
            Huff clh;
            clh.build(cl, 19);
            int lens[320] = {0};
            for (int i = 0; i < hlit + hdist;) {
                const int s = clh.decode(b);
                if (s < 16) {
                    lens[i++] = s;
                } else {
                    int rep = 0, val = 0;
                    if (s == 16) {
                        if (i == 0) throw Error("png: a repeat with no previous code length");
                        val = lens[i - 1];
                        rep = 3 + (int)b.get(2);
                    } else if (s == 17) {
                        rep = 3 + (int)b.get(3);
                    } else {
                        rep = 11 + (int)b.get(7);
                    }
                    if (i + rep > hlit + hdist) throw Error("png: too many code lengths");
                    while (rep--) lens[i++] = val;
                }
            }
            Huff lit, dist;
            lit.build(lens, hlit);
            dist.build(lens + hlit, hdist);
            inflate_block(b, lit, dist, out, limit);
        } else {
            throw Error("png: an invalid deflate block type");
        }
    } while (!last);
    return out;
}

int paeth(int a, int b, int c) {
    const int p = a + b - c, pa = p > a ? p - a : a - p, pb = p > b ? p - b : b - p, pc = p > c ? p - c : c - p;
    return (pa <= pb && pa <= pc) ? a : pb <= pc ? b : c;
}

struct Png {
    int64_t w = 0, h = 0;
    std::vector<float> rgb;  // [3][h][w]
};

// Undoes the row filters of one (sub-)image of `rows` rows of `stride`
// bytes, `ch` bytes per pixel, from raw[at..]: each row is a filter byte and
// the filtered bytes (PNG 1.2, 6.3). Returns the bytes consumed.
size_t unfilter(const std::vector<unsigned char> &raw, size_t at, size_t rows, size_t stride, int ch,
                unsigned char *px, const std::string &what) {
    for (size_t y = 0; y < rows; ++y) {
        const unsigned char ft = raw[at + y * (stride + 1)];
        const unsigned char *src = &raw[at + y * (stride + 1) + 1];
        unsigned char *row = px + y * stride;
        const unsigned char *up = y ? row - stride : nullptr;
        for (size_t x = 0; x < stride; ++x) {
            const int a = x >= (size_t)ch ? row[x - ch] : 0, b = up ? up[x] : 0;
            const int c = (up && x >= (size_t)ch) ? up[x - ch] : 0;
            int v = src[x];
            switch (ft) {
                case 0: break;
                case 1: v += a; break;
                case 2: v += b; break;
                case 3: v += (a + b) >> 1; break;
                case 4: v += paeth(a, b, c); break;
                default: throw Error(what + ": unknown PNG row filter " + std::to_string(ft));
            }
            row[x] = (unsigned char)v;
        }
    }
    return rows * (stride + 1);
}

// Adam7 (PNG 1.2, 8.2): pass p covers rows r0 + k * dr and columns
// c0 + k * dc of the image.
const int kA7r0[7] = {0, 0, 4, 0, 2, 0, 1}, kA7c0[7] = {0, 4, 0, 2, 0, 1, 0};
const int kA7dr[7] = {8, 8, 8, 4, 4, 2, 2}, kA7dc[7] = {8, 8, 4, 4, 2, 2, 1};

Png decode_png(const unsigned char *d, size_t size, const std::string &what) {
    static const unsigned char sig[8] = {137, 80, 78, 71, 13, 10, 26, 10};
    if (size < 8 || std::memcmp(d, sig, 8)) throw Error(what + ": not a PNG file");
    size_t at = 8;
    int depth = 0, ctype = -1, interlace = 0;
    bool have_ihdr = false;
    Png img;
    std::vector<unsigned char> z;
    bool end = false;
    while (!end) {
        if (at + 12 > size) throw Error(what + ": the PNG ends before IEND");
        const uint32_t n = be32(&d[at]);
        if ((size_t)n > size - at - 12) throw Error(what + ": a PNG chunk runs past the file");
        const unsigned char *type = &d[at + 4], *data = &d[at + 8];
        if (crc32(type, 4 + (size_t)n) ^ 0xffffffffu ^ be32(data + n))
            throw Error(what + ": a PNG chunk fails its CRC");
        if (!std::memcmp(type, "IHDR", 4)) {
            if (n < 13) throw Error(what + ": a short IHDR");
            img.w = be32(data);
            img.h = be32(data + 4);
            depth = data[8];
            ctype = data[9];
            interlace = data[12];
            have_ihdr = true;
        } else if (!std::memcmp(type, "IDAT", 4)) {
            z.insert(z.end(), data, data + n);
        } else if (!std::memcmp(type, "IEND", 4)) {
            end = true;
        }
        at += 12 + (size_t)n;
    }
    if (!have_ihdr) throw Error(what + ": no IHDR");
    if (ctype == 3) throw Error(what + ": indexed PNG; re-save it as RGB");
    const int ch = ctype == 0 ? 1 : ctype == 4 ? 2 : ctype == 2 ? 3 : ctype == 6 ? 4 : 0;
    if (!ch) throw Error(what + ": unknown PNG colour type " + std::to_string(ctype));
    if (depth != 8) throw Error(what + ": " + std::to_string(depth) + "-bit PNG; re-save it with 8 bits per channel");
    if (interlace > 1) throw Error(what + ": unknown PNG interlace method " + std::to_string(interlace));
    if (img.w <= 0 || img.h <= 0 || img.w > (1 << 20) || img.h > (1 << 20)) throw Error(what + ": bad PNG size");
    if (z.size() < 6 || (z[0] & 0x0f) != 8 || ((z[0] << 8) | z[1]) % 31) throw Error(what + ": bad zlib header");
    const size_t W = (size_t)img.w, H = (size_t)img.h, stride = W * ch;
    // the filtered data's size: every (non-empty) pass's rows, each with its filter byte
    size_t need = 0;
    if (!interlace) {
        need = (stride + 1) * H;
    } else {
        for (int p = 0; p < 7; ++p) {
            const size_t pw = W > (size_t)kA7c0[p] ? (W - kA7c0[p] + kA7dc[p] - 1) / kA7dc[p] : 0;
            const size_t ph = H > (size_t)kA7r0[p] ? (H - kA7r0[p] + kA7dr[p] - 1) / kA7dr[p] : 0;
            if (pw && ph) need += (pw * ch + 1) * ph;
        }
    }
    std::vector<unsigned char> raw = inflate(z.data() + 2, z.size() - 2, need);
    if (raw.size() != need) throw Error(what + ": the image data has the wrong size");
    std::vector<unsigned char> px(stride * H);
    if (!interlace) {
        unfilter(raw, 0, H, stride, ch, px.data(), what);
    } else {
        size_t pos = 0;
        std::vector<unsigned char> sub;
        for (int p = 0; p < 7; ++p) {
            const size_t pw = W > (size_t)kA7c0[p] ? (W - kA7c0[p] + kA7dc[p] - 1) / kA7dc[p] : 0;
            const size_t ph = H > (size_t)kA7r0[p] ? (H - kA7r0[p] + kA7dr[p] - 1) / kA7dr[p] : 0;
            if (!pw || !ph) continue;  // an empty pass has no rows (and no filter bytes)
            sub.assign(pw * ch * ph, 0);
            pos += unfilter(raw, pos, ph, pw * ch, ch, sub.data(), what);
            for (size_t y = 0; y < ph; ++y)
                for (size_t x = 0; x < pw; ++x)
                    std::memcpy(&px[((kA7r0[p] + y * kA7dr[p]) * W + kA7c0[p] + x * kA7dc[p]) * ch],
                                &sub[(y * pw + x) * ch], (size_t)ch);
        }
    }
    const size_t plane = W * H;
    img.rgb.assign(3 * plane, 0.0f);
    for (size_t p = 0; p < plane; ++p) {
        const unsigned char *s = &px[p * ch];
        const unsigned char r = s[0], g = ch >= 3 ? s[1] : s[0], bl = ch >= 3 ? s[2] : s[0];
        img.rgb[p] = (float)r / 255.0f;
        img.rgb[plane + p] = (float)g / 255.0f;
        img.rgb[2 * plane + p] = (float)bl / 255.0f;
    }
    return img;
}

std::vector<unsigned char> read_file(const std::string &path) {
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) throw Error(path + ": cannot open");
    std::vector<unsigned char> d;
    unsigned char buf[1 << 16];
    size_t k;
    while ((k = std::fread(buf, 1, sizeof buf, f)) > 0) d.insert(d.end(), buf, buf + k);
    std::fclose(f);
    return d;
}

void put32(std::vector<unsigned char> &v, uint32_t x) {
    for (int s = 24; s >= 0; s -= 8) v.push_back((unsigned char)(x >> s));
}

void chunk(std::vector<unsigned char> &out, const char *type, const std::vector<unsigned char> &data) {
    put32(out, (uint32_t)data.size());
    const size_t at = out.size();
    out.insert(out.end(), type, type + 4);
    out.insert(out.end(), data.begin(), data.end());
    put32(out, crc32(&out[at], 4 + data.size()) ^ 0xffffffffu);
}

// Stored-deflate PNG bytes of [3][h][w] in 0..1 (the size depends on h and w only).
std::vector<unsigned char> encode_png(const float *img, int64_t h, int64_t w, const std::string &what) {
    if (h <= 0 || w <= 0 || h > (1 << 20) || w > (1 << 20)) throw Error(what + ": bad image size");
    const size_t plane = (size_t)h * (size_t)w, stride = (size_t)w * 3;
    std::vector<unsigned char> raw((stride + 1) * (size_t)h);
    for (int64_t y = 0; y < h; ++y) {
        unsigned char *row = &raw[(size_t)y * (stride + 1)];
        row[0] = 0;
        for (int64_t x = 0; x < w; ++x)
            for (int c = 0; c < 3; ++c) {
                float v = img[c * plane + (size_t)y * w + x];
                // clamp to 0..1; NaN becomes 0 (the reference's saturating
                // `as u8` of a NaN)
                v = v >= 0.0f ? (v > 1.0f ? 1.0f : v) : 0.0f;
                row[1 + x * 3 + c] = (unsigned char)(v * 255.0f + 0.5f);
            }
    }
    std::vector<unsigned char> z = {0x78, 0x01};
    for (size_t at = 0; at < raw.size();) {
        const size_t n = std::min<size_t>(65535, raw.size() - at);
        z.push_back(at + n == raw.size() ? 1 : 0);
        z.push_back((unsigned char)(n & 0xff));
        z.push_back((unsigned char)(n >> 8));
        z.push_back((unsigned char)(~n & 0xff));
        z.push_back((unsigned char)((~n >> 8) & 0xff));
        z.insert(z.end(), raw.begin() + at, raw.begin() + at + n);
        at += n;
    }
    put32(z, adler32(raw.data(), raw.size()));
    std::vector<unsigned char> out = {137, 80, 78, 71, 13, 10, 26, 10}, ihdr;
    put32(ihdr, (uint32_t)w);
    put32(ihdr, (uint32_t)h);
    ihdr.insert(ihdr.end(), {8, 2, 0, 0, 0});
    chunk(out, "IHDR", ihdr);
    chunk(out, "IDAT", z);
    chunk(out, "IEND", {});
    return out;
}

void write_png(const std::string &path, const float *img, int64_t h, int64_t w) {
    const std::vector<unsigned char> out = encode_png(img, h, w, path);
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) throw Error(path + ": cannot create");
    const bool ok = std::fwrite(out.data(), 1, out.size(), f) == out.size();
    if (std::fclose(f) != 0 || !ok) throw Error(path + ": write failed");
}

}  // namespace
}  // namespace mx

using namespace mx;

// A decoded image (mx_png_open .. mx_png_close).
struct mx_png {
    mx::Png img;
};

extern "C" {

int mx_png_open(const char *path, const unsigned char *data, size_t n, mx_png **img, int64_t *h, int64_t *w) {
    try {
        if (!img) throw Error("mx_png_open: no handle to fill");
        *img = nullptr;
        std::unique_ptr<mx_png> p(new mx_png);
        if (path) {
            const std::vector<unsigned char> d = read_file(path);
            p->img = decode_png(d.data(), d.size(), path);
        } else {
            if (!data && n) throw Error("mx_png_open: no path and no bytes");
            p->img = decode_png(data, n, "stdin");
        }
        if (h) *h = p->img.h;
        if (w) *w = p->img.w;
        *img = p.release();
        return 0;
    } catch (const std::exception &e) {
        set_error(e.what());
        return -1;
    }
}

int mx_png_pixels(const mx_png *img, float *out, size_t cap) {
    try {
        if (!img || !out) throw Error("mx_png_pixels: no image or no buffer");
        const size_t n = img->img.rgb.size();
        if (cap < n)
            throw Error("mx_png_pixels: the buffer holds " + std::to_string(cap) + " floats, the image needs " +
                        std::to_string(n));
        std::memcpy(out, img->img.rgb.data(), n * sizeof(float));
        return 0;
    } catch (const std::exception &e) {
        set_error(e.what());
        return -1;
    }
}

void mx_png_close(mx_png *img) { delete img; }

int mx_png_encode(const float *img, int64_t h, int64_t w, unsigned char *out, size_t cap, size_t *n) {
    try {
        if (!img) throw Error("mx_png_encode: no image");
        const std::vector<unsigned char> d = encode_png(img, h, w, "mx_png_encode");
        if (n) *n = d.size();
        if (!out) return 0;
        if (cap < d.size())
            throw Error("mx_png_encode: the buffer holds " + std::to_string(cap) + " bytes, the PNG needs " +
                        std::to_string(d.size()));
        std::memcpy(out, d.data(), d.size());
        return 0;
    } catch (const std::exception &e) {
        set_error(e.what());
        return -1;
    }
}

int mx_png_write(const char *path, const float *img, int64_t h, int64_t w) {
    try {
        if (!img) throw Error("mx_png_write: no image");
        write_png(path ? path : "", img, h, w);
        return 0;
    } catch (const std::exception &e) {
        set_error(e.what());
        return -1;
    }
}

}  // extern "C"
