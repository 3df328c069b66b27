// Checkpoint access: the safetensors container, the variant table, the
// seeded random-init generator and the kernel layout transforms.
//
// Layout transforms follow src/weights.rs:57-211; the container follows the
// writer in tools/convert.py:88-137; the variant table follows
// src/config.rs:33-116.

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>

#include "host.hpp"

namespace mx {

// ------------------------------------------------------------------ config

Config Config::variant(const std::string &v) {
    int features, stages;
    if (v == "S-1") { features = 32; stages = 1; }
    else if (v == "S-2") { features = 32; stages = 2; }
    else if (v == "S-3") { features = 32; stages = 3; }
    else if (v == "M-1") { features = 64; stages = 1; }
    else if (v == "M-2") { features = 64; stages = 2; }
    else if (v == "M-3") { features = 64; stages = 3; }
    else throw Error("unknown variant " + v + " (expected S-1..S-3, M-1..M-3)");
    Config c;
    c.features = features;
    c.num_stages = stages;
    return c;
}

Config Config::for_task(const std::string &task) {
    std::string t = task;
    std::transform(t.begin(), t.end(), t.begin(), ::tolower);
    if (t == "denoising" || t == "deblurring") return variant("S-3");
    if (t == "deraining" || t == "dehazing" || t == "enhancement") return variant("S-2");
    throw Error("unknown task " + t +
                " (expected denoising, deblurring, deraining, dehazing, enhancement)");
}

mx_config Config::to_c() const {
    mx_config c;
    c.features = features; c.depth = depth; c.num_stages = num_stages; c.num_groups = num_groups;
    c.num_supervision_scales = num_supervision_scales; c.num_outputs = num_outputs;
    c.use_cross_gating = use_cross_gating; c.high_res_stages = high_res_stages;
    c.block_size_hr = block_size_hr; c.block_size_lr = block_size_lr;
    c.grid_size_hr = grid_size_hr; c.grid_size_lr = grid_size_lr;
    c.channels_reduction = channels_reduction; c.num_bottleneck_blocks = num_bottleneck_blocks;
    return c;
}

// --------------------------------------------------------- a tiny JSON reader
//
// The safetensors header is one JSON object of objects, strings, integer
// arrays and integers; nothing else is needed.

namespace {

struct JVal {
    enum Kind { Null, Num, Str, Arr, Obj } kind = Null;
    double num = 0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal *find(const std::string &k) const {
        for (auto &kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char *p, *e;
    int depth = 0;  // nesting, bounded so a hostile header cannot exhaust the stack
    void ws() { while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p; }
    [[noreturn]] void fail(const char *what) {
        throw Error(std::string("safetensors header: ") + what);
    }
    std::string string() {
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
                        unsigned v = std::stoul(std::string(p, p + 4), nullptr, 16);
                        p += 4;
                        if (v < 0x80) s += char(v);
                        else if (v < 0x800) { s += char(0xC0 | (v >> 6)); s += char(0x80 | (v & 63)); }
                        else { s += char(0xE0 | (v >> 12)); s += char(0x80 | ((v >> 6) & 63)); s += char(0x80 | (v & 63)); }
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
        return s;
    }
    JVal value() {
        if (++depth > 64) fail("nested too deeply");
        JVal v = item();
        --depth;
        return v;
    }
    JVal item() {
        ws();
        if (p >= e) fail("unexpected end");
        JVal v;
        if (*p == '{') {
            v.kind = JVal::Obj;
            ++p; ws();
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
            v.kind = JVal::Arr;
            ++p; ws();
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
        } else if (*p == 'n' && e - p >= 4 && !strncmp(p, "null", 4)) {
            p += 4;
        } else {
            char *end = nullptr;
            std::string tmp(p, std::min<ptrdiff_t>(e - p, 64));
            v.num = strtod(tmp.c_str(), &end);
            if (end == tmp.c_str()) fail("bad number");
            v.kind = JVal::Num;
            p += end - tmp.c_str();
        }
        return v;
    }
};

std::string jstr(const std::string &s) {
    std::string o = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') { o += '\\'; o += c; }
        else if ((unsigned char)c < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", c); o += b; }
        else o += c;
    }
    return o + "\"";
}

// fp16 / bf16 -> fp32, so a checkpoint stored at reduced width still loads.
float half_to_float(uint16_t h) {
    uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
    float f;
    if (e == 0) f = std::ldexp((float)m, -24);
    else if (e == 31) f = m ? NAN : INFINITY;
    else f = std::ldexp((float)(m | 1024), (int)e - 25);
    return s ? -f : f;
}

// ------------------------------------------------------ the seeded generator

uint64_t splitmix64(uint64_t &x) {
    uint64_t z = (x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t fnv1a(const std::string &s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) { h ^= c; h *= 0x100000001b3ull; }
    return h;
}

// xoshiro256** seeded from splitmix64; N(0,1) by Box-Muller in double.
struct Rng {
    uint64_t s[4];
    explicit Rng(uint64_t seed) {
        uint64_t x = seed;
        for (auto &v : s) v = splitmix64(x);
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3]; s[2] ^= t; s[3] = rotl(s[3], 45);
        return r;
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    bool have = false;
    double spare = 0;
    double normal() {
        if (have) { have = false; return spare; }
        double u = uniform(), v = uniform();
        double r = std::sqrt(-2.0 * std::log(u)), t = 6.283185307179586 * v;
        spare = r * std::sin(t);
        have = true;
        return r * std::cos(t);
    }
};

bool ends_with(const std::string &s, const std::string &suf) {
    return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

}  // namespace

// ------------------------------------------------------------------ weights

Weights *Weights::open(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error(path + ": cannot open");
    uint64_t hlen = 0;
    f.read(reinterpret_cast<char *>(&hlen), 8);
    if (!f || hlen > (1ull << 30)) throw Error(path + ": not a safetensors file");
    std::string hdr(hlen, '\0');
    f.read(&hdr[0], hlen);
    if (!f) throw Error(path + ": truncated header");
    JParser jp{hdr.data(), hdr.data() + hdr.size()};
    JVal root = jp.value();
    if (root.kind != JVal::Obj) throw Error(path + ": header is not an object");
    f.seekg(0, std::ios::end);
    uint64_t fsize = (uint64_t)f.tellg();
    uint64_t base = 8 + hlen;
    auto *w = new Weights();
    try {
        for (auto &kv : root.obj) {
            if (kv.first == "__metadata__") continue;
            const JVal &t = kv.second;
            const JVal *dt = t.find("dtype"), *sh = t.find("shape"), *off = t.find("data_offsets");
            if (!dt || !sh || !off || off->arr.size() != 2)
                throw Error(path + ": tensor " + kv.first + " has an incomplete entry");
            // Sizes and offsets are whole non-negative numbers, the element
            // count does not overflow, and the byte count is checked before
            // anything is allocated: a header cannot make the reader allocate
            // more than the file holds.
            auto whole = [&](const JVal &v, const char *what) -> uint64_t {
                if (v.kind != JVal::Num || !(v.num >= 0.0) || v.num > 9.0e15 || v.num != (double)(uint64_t)v.num)
                    throw Error(path + ": tensor " + kv.first + " has a bad " + what);
                return (uint64_t)v.num;
            };
            if (sh->kind != JVal::Arr || off->kind != JVal::Arr)
                throw Error(path + ": tensor " + kv.first + " has an incomplete entry");
            Tensor ten;
            uint64_t n = 1;
            for (auto &d : sh->arr) {
                const uint64_t k = whole(d, "shape");
                ten.shape.push_back((int64_t)k);
                if (__builtin_mul_overflow(n, k, &n)) throw Error(path + ": tensor " + kv.first + " is too large");
            }
            const uint64_t a = whole(off->arr[0], "data offset"), b = whole(off->arr[1], "data offset");
            if (b < a || base + b > fsize) throw Error(path + ": tensor " + kv.first + " runs past the file");
            const uint64_t esz = dt->str == "F32" ? 4 : dt->str == "F16" || dt->str == "BF16" ? 2 : dt->str == "F64" ? 8 : 0;
            if (!esz) throw Error(path + ": " + kv.first + " has unsupported dtype " + dt->str);
            if (n > (b - a) / esz || b - a != n * esz) throw Error(path + ": " + kv.first + " has the wrong byte count");
            std::vector<char> raw(b - a);
            f.seekg(base + a);
            f.read(raw.data(), b - a);
            if (!f) throw Error(path + ": tensor " + kv.first + " could not be read");
            ten.data.resize(n);
            if (dt->str == "F32") {
                memcpy(ten.data.data(), raw.data(), n * 4);
            } else if (dt->str == "F16" || dt->str == "BF16") {
                for (uint64_t i = 0; i < n; ++i) {
                    uint16_t h;
                    memcpy(&h, raw.data() + 2 * i, 2);
                    if (dt->str == "F16") ten.data[i] = half_to_float(h);
                    else { uint32_t u = (uint32_t)h << 16; memcpy(&ten.data[i], &u, 4); }
                }
            } else {
                for (uint64_t i = 0; i < n; ++i) {
                    double d;
                    memcpy(&d, raw.data() + 8 * i, 8);
                    ten.data[i] = (float)d;
                }
            }
            w->tensors.emplace(kv.first, std::move(ten));
        }
        // Config::of_checkpoint (src/config.rs:71-100): the width is c_out of the
        // first encoder conv, the stage count is the last stage with an output conv.
        const std::string first = "stage_0_encoder_block_0/Conv_0/kernel";
        auto it = w->tensors.find(first);
        if (it == w->tensors.end())
            throw Error(first + " is missing (not a converted MAXIM checkpoint?)");
        int features = it->second.shape.empty() ? 0 : (int)it->second.shape.back();
        int stages = 1;
        for (int n = 1; n < 3; ++n)
            if (w->tensors.count("stage_" + std::to_string(n) + "_output_conv_1/kernel")) stages = n + 1;
        std::string v;
        if (features == 32) v = "S-"; else if (features == 64) v = "M-";
        if (v.empty())
            throw Error("checkpoint has " + std::to_string(features) + " features and " +
                        std::to_string(stages) +
                        " stage(s), which is not one of the six published MAXIM variants");
        w->config = Config::variant(v + std::to_string(stages));
    } catch (...) {
        delete w;
        throw;
    }
    return w;
}

Weights *Weights::make_synthetic(const std::string &variant, uint64_t seed, float gain,
                                 float bias_std, float ln_std) {
    auto *w = new Weights();
    w->config = Config::variant(variant);
    w->synthetic = true;
    w->seed = seed;
    w->kernel_gain = gain;
    w->bias_std = bias_std;
    w->ln_std = ln_std;
    // Materialise every tensor the graph reads by building the smallest plan the
    // model accepts: the parameter set does not depend on the image size (the
    // gating Dense is sized by the fixed cell/block counts), so this is the
    // checkpoint.
    try {
        int64_t side = 8LL << w->config.depth;
        Plan *p = build_plan(*w, side, side, false, false, false);
        delete p;
    } catch (...) {
        delete w;
        throw;
    }
    w->synthetic = false;  // frozen: from here on it behaves like a file
    return w;
}

bool Weights::has(const std::string &name) const {
    return synthetic || tensors.count(name) != 0;
}

Tensor &Weights::generate(const std::string &name, const std::vector<int64_t> &shape) const {
    auto &m = const_cast<std::map<std::string, Tensor> &>(tensors);
    Tensor t;
    t.shape = shape;
    int64_t n = 1;
    for (auto d : shape) n *= d;
    t.data.resize(n);
    Rng rng(seed ^ fnv1a(name));
    if (ends_with(name, "/kernel")) {
        int64_t fan_in = 1;
        for (size_t i = 0; i + 1 < shape.size(); ++i) fan_in *= shape[i];
        double sd = kernel_gain * std::sqrt(2.0 / (double)std::max<int64_t>(fan_in, 1));
        for (auto &v : t.data) v = (float)(rng.normal() * sd);
    } else if (ends_with(name, "/scale")) {
        for (auto &v : t.data) v = (float)(1.0 + rng.normal() * ln_std);
    } else {
        for (auto &v : t.data) v = (float)(rng.normal() * bias_std);
    }
    return m.emplace(name, std::move(t)).first->second;
}

const Tensor &Weights::get(const std::string &name, const std::vector<int64_t> &expect) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) {
        if (synthetic) return generate(name, expect);
        throw Error(name + " is missing from the checkpoint");
    }
    const Tensor &t = it->second;
    // A 1x1 kernel may be stored as a Dense [ci][co] or as a conv [1][1][ci][co]
    // (src/weights.rs:57-85); everything else must match exactly.
    auto squeeze = [](std::vector<int64_t> s) {
        while (s.size() > 2 && s[0] == 1) s.erase(s.begin());
        return s;
    };
    if (t.shape != expect && squeeze(t.shape) != squeeze(expect)) {
        std::ostringstream m;
        m << name << ": expected shape [";
        for (size_t i = 0; i < expect.size(); ++i) m << (i ? "," : "") << expect[i];
        m << "], the checkpoint has [";
        for (size_t i = 0; i < t.shape.size(); ++i) m << (i ? "," : "") << t.shape[i];
        m << "]";
        throw Error(m.str());
    }
    return t;
}

// Flax names 1x1 convs `Conv_N` / `input_proj` and stores them 4-D; the
// projections and the MLP layers are Dense and stored 2-D.
static std::vector<int64_t> pointwise_shape(const std::string &name, int64_t ci, int64_t co) {
    std::string stem = name.substr(0, name.rfind('/'));
    std::string leaf = stem.substr(stem.rfind('/') + 1);
    if (leaf.rfind("Conv_", 0) == 0 || leaf == "input_proj") return {1, 1, ci, co};
    return {ci, co};
}

std::vector<float> Weights::conv1x1(const std::string &name, int64_t ci, int64_t co) const {
    const Tensor &t = get(name, pointwise_shape(name, ci, co));
    std::vector<float> out(ci * co);
    for (int64_t o = 0; o < co; ++o)
        for (int64_t i = 0; i < ci; ++i) out[o * ci + i] = t.data[i * co + o];
    return out;
}

std::vector<float> Weights::conv1x1_t(const std::string &name, int64_t ci, int64_t co) const {
    return get(name, pointwise_shape(name, ci, co)).data;
}

std::vector<float> Weights::convkxk(const std::string &name, int64_t k, int64_t ci, int64_t co) const {
    const Tensor &t = get(name, {k, k, ci, co});
    std::vector<float> out(t.data.size());
    for (int64_t o = 0; o < co; ++o)
        for (int64_t i = 0; i < ci; ++i)
            for (int64_t y = 0; y < k; ++y)
                for (int64_t x = 0; x < k; ++x)
                    out[((o * ci + i) * k + y) * k + x] = t.data[((y * k + x) * ci + i) * co + o];
    return out;
}

std::vector<float> Weights::conv3x3_t(const std::string &name, int64_t ci, int64_t co) const {
    // Flax's own [kh][kw][ci][co] order is already [tap][ci][co].
    return get(name, {3, 3, ci, co}).data;
}

std::vector<float> Weights::convt2x2(const std::string &name, int64_t ci, int64_t co) const {
    // flax's ConvTranspose is the adjoint of its Conv, so a scatter needs the
    // kernel spatially reversed (src/weights.rs:170-191).
    const Tensor &t = get(name, {2, 2, ci, co});
    std::vector<float> out(t.data.size());
    for (int64_t i = 0; i < ci; ++i)
        for (int64_t o = 0; o < co; ++o)
            for (int64_t y = 0; y < 2; ++y)
                for (int64_t x = 0; x < 2; ++x)
                    out[((i * co + o) * 2 + y) * 2 + x] =
                        t.data[((1 - y) * 2 + (1 - x)) * ci * co + i * co + o];
    return out;
}

std::vector<float> Weights::dense(const std::string &name, int64_t k) const {
    const Tensor &t = get(name, {k, k});
    std::vector<float> out(k * k);
    for (int64_t o = 0; o < k; ++o)
        for (int64_t i = 0; i < k; ++i) out[o * k + i] = t.data[i * k + o];
    return out;
}

std::vector<float> Weights::owned(const std::string &name, int64_t n) const {
    return get(name, {n}).data;
}

uint64_t Weights::params() const {
    uint64_t n = 0;
    for (auto &kv : tensors) n += kv.second.data.size();
    return n;
}

void Weights::save(const std::string &path, const std::string &task) const {
    // std::map iterates in sorted key order, which is the order the reference
    // converter lays the data out in (tools/convert.py:90-137).
    std::string hdr = "{";
    const char *cfg_variant = config.features == 32 ? "S-" : "M-";
    std::string meta = "\"__metadata__\":{\"format\":\"maxim\",\"source\":\"seeded random init\","
                       "\"task\":" + jstr(task) + ",\"tensor_count\":\"" +
                       std::to_string(tensors.size()) + "\",\"variant\":\"" + cfg_variant +
                       std::to_string(config.num_stages) + "\"}";
    // JSON keys are sorted: "__metadata__" sorts after upper-case names and
    // before lower-case ones ('_' is 0x5F), exactly as json.dumps(sort_keys) does.
    std::vector<std::pair<std::string, std::string>> entries;
    entries.emplace_back("__metadata__", meta);
    uint64_t off = 0;
    for (auto &kv : tensors) {
        std::string e = jstr(kv.first) + ":{\"data_offsets\":[" + std::to_string(off) + "," +
                        std::to_string(off + kv.second.data.size() * 4) + "],\"dtype\":\"F32\",\"shape\":[";
        for (size_t i = 0; i < kv.second.shape.size(); ++i)
            e += (i ? "," : "") + std::to_string(kv.second.shape[i]);
        e += "]}";
        entries.emplace_back(kv.first, e);
        off += kv.second.data.size() * 4;
    }
    std::sort(entries.begin(), entries.end(),
              [](const std::pair<std::string, std::string> &a, const std::pair<std::string, std::string> &b) {
                  return a.first < b.first;
              });
    for (size_t i = 0; i < entries.size(); ++i) hdr += (i ? "," : "") + entries[i].second;
    hdr += "}";
    while ((8 + hdr.size()) % 8) hdr += ' ';
    std::ofstream f(path, std::ios::binary);
    if (!f) throw Error(path + ": cannot write");
    uint64_t hl = hdr.size();
    f.write(reinterpret_cast<const char *>(&hl), 8);
    f.write(hdr.data(), hdr.size());
    for (auto &kv : tensors)
        f.write(reinterpret_cast<const char *>(kv.second.data.data()), kv.second.data.size() * 4);
    if (!f) throw Error(path + ": write failed");
}

}  // namespace mx
