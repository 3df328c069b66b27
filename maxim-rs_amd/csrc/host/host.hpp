// Internal C++ side of the plan contract. The C ABI over it is in
// include/maxim_plan.h; this header is shared by the host library's own files.
#pragma once

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "maxim_plan.h"

namespace mx {

// The reference's `Error(String)` (src/lib.rs:29): every failure here is a bad
// file, a missing parameter or an unsupported shape, so a message is enough.
struct Error : std::runtime_error {
    explicit Error(const std::string &m) : std::runtime_error(m) {}
};

void set_error(const std::string &m);

// LayerNorm epsilon, flax's default (src/model.rs:35).
constexpr float kEps = 1e-6f;

struct Config {
    int features = 32, depth = 3, num_stages = 2, num_groups = 2;
    int num_supervision_scales = 3, num_outputs = 3;
    bool use_cross_gating = true;
    int high_res_stages = 2, block_size_hr = 16, block_size_lr = 8;
    int grid_size_hr = 16, grid_size_lr = 8;
    int channels_reduction = 4, num_bottleneck_blocks = 2;

    static Config variant(const std::string &v);
    static Config for_task(const std::string &task);
    mx_config to_c() const;
};

struct Tensor {
    std::vector<int64_t> shape;
    std::vector<float> data;
};

// A checkpoint: named tensors plus the architecture the file implies.
// `synthetic` weights create a missing tensor on first request, with the shape
// the builder asks for, from a stream keyed by (seed, name).
class Weights {
public:
    std::map<std::string, Tensor> tensors;
    Config config;
    bool synthetic = false;
    uint64_t seed = 0;
    float kernel_gain = 1.0f, bias_std = 0.0f, ln_std = 0.0f;

    static Weights *open(const std::string &path);
    static Weights *make_synthetic(const std::string &variant, uint64_t seed, float gain,
                                   float bias_std, float ln_std);
    void save(const std::string &path, const std::string &task) const;

    // `expect` is the shape the graph needs; a file-backed tensor must match it
    // (kernels may be stored either as a Dense [ci][co] or as a 1x1 conv).
    bool has(const std::string &name) const;
    const Tensor &get(const std::string &name, const std::vector<int64_t> &expect) const;

    // Layout transforms (src/weights.rs:57-211).
    std::vector<float> conv1x1(const std::string &name, int64_t ci, int64_t co) const;
    std::vector<float> conv1x1_t(const std::string &name, int64_t ci, int64_t co) const;
    std::vector<float> convkxk(const std::string &name, int64_t k, int64_t ci, int64_t co) const;
    std::vector<float> conv3x3_t(const std::string &name, int64_t ci, int64_t co) const;
    std::vector<float> convt2x2(const std::string &name, int64_t ci, int64_t co) const;
    std::vector<float> dense(const std::string &name, int64_t k) const;
    std::vector<float> owned(const std::string &name, int64_t n) const;

    uint64_t params() const;

private:
    Tensor &generate(const std::string &name, const std::vector<int64_t> &shape) const;
};

struct BufShape {
    int64_t c, h, w;
    int64_t len() const { return c * h * w; }
};

struct Plan {
    std::vector<BufShape> bufs;
    std::vector<uint64_t> offs;
    std::vector<mx_op> ops;
    std::vector<std::vector<float>> weights;
    uint64_t arena_len = 0;
    int64_t input = -1, output = -1;
    std::vector<std::pair<std::string, int64_t>> dumps;
    BufShape shape{0, 0, 0};
    std::vector<std::string> labels;
    std::vector<int64_t> alias_parent;   // -1 = owns its bytes
    std::vector<uint64_t> alias_delta;   // elements into the parent

    // Views for mx_plan_describe.
    std::vector<const float *> wptr;
    std::vector<uint64_t> wlen;
    std::vector<uint8_t> keep;
    void index_weights();
    uint64_t weight_bytes() const;
};

Plan *build_plan(const Weights &w, int64_t h, int64_t wd, bool named, bool gpu_twins, bool deep);

// The buffers an op reads or writes, dst first (src/model.rs:114-139).
void op_operands(const mx_op &op, std::vector<int64_t> &out);

// image.rs helpers.
void same_pad(int64_t size, int64_t stride, int64_t k, int64_t &before, int64_t &after);

}  // namespace mx
