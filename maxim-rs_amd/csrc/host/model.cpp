// The MAXIM graph as a flat list of ops over one packed arena.
//
// The block structure follows the reference builder block for block
// (src/model.rs:400-1076): the op sequence, the buffer creation order, the
// weight order and the parameter names must all be the reference's, because
// the packed arena, the op counts and the checkpoint names are the contract.
// The packer follows src/model.rs:1091-1234 (largest first, first use as the
// tie-break, first fit over the candidate offsets {0} u {off + size}).

#include <algorithm>
#include <cstdlib>
#include <numeric>

#include "host.hpp"

namespace mx {

void same_pad(int64_t size, int64_t stride, int64_t k, int64_t &before, int64_t &after) {
    int64_t out = (size + stride - 1) / stride;
    int64_t need = (out - 1) * stride + k;
    int64_t total = need > size ? need - size : 0;
    before = total / 2;
    after = total - total / 2;
}

void op_operands(const mx_op &op, std::vector<int64_t> &out) {
    switch (op.kind) {
        case MX_OP_ADD:
        case MX_OP_MUL:
        case MX_OP_GATE_APPLY:
        case MX_OP_CHAN_SCALE:
        case MX_OP_RESIZE:
            out.push_back(op.dst);
            out.push_back(op.src);
            out.push_back(op.src2);
            break;
        default:
            out.push_back(op.dst);
            out.push_back(op.src);
            break;
    }
}

uint64_t Plan::weight_bytes() const {
    uint64_t b = 0;
    for (auto &w : weights) b += w.size() * 4;
    return b;
}

void Plan::index_weights() {
    wptr.clear();
    wlen.clear();
    for (auto &w : weights) {
        wptr.push_back(w.data());
        wlen.push_back(w.size());
    }
}

namespace {

mx_op blank(int kind) {
    mx_op o{};
    o.kind = kind;
    o.dst = o.src = o.src2 = -1;
    o.w = o.wt = o.bias = o.scale = -1;
    return o;
}

std::string S(int64_t v) { return std::to_string(v); }

class Builder {
public:
    Builder(const Weights &w, bool record, bool gpu_twins, bool deep)
        : w_(w), cfg_(w.config), record_(record), twins_(gpu_twins), deep_(deep) {}

    Plan *build(int64_t h, int64_t wd);

private:
    const Weights &w_;
    Config cfg_;
    bool record_, twins_, deep_;
    std::vector<std::vector<float>> weights_;
    std::vector<BufShape> bufs_;
    std::vector<std::string> labels_;
    std::vector<int64_t> alias_parent_;
    std::vector<uint64_t> alias_delta_;
    std::vector<mx_op> ops_;
    std::vector<std::pair<std::string, int64_t>> named_;
    int up_index_ = 0;

    int64_t buf(int64_t c, int64_t h, int64_t w, const char *label) {
        bufs_.push_back({c, h, w});
        labels_.push_back(label);
        alias_parent_.push_back(-1);
        alias_delta_.push_back(0);
        return (int64_t)bufs_.size() - 1;
    }
    // A channel range of another buffer: no storage of its own.
    int64_t view(int64_t base, int64_t ch, int64_t c, const char *label) {
        BufShape s = bufs_[base];
        bufs_.push_back({c, s.h, s.w});
        labels_.push_back(label);
        alias_parent_.push_back(base);
        alias_delta_.push_back((uint64_t)(ch * s.h * s.w));
        return (int64_t)bufs_.size() - 1;
    }
    void rec(const std::string &name, int64_t id) {
        if (record_) named_.emplace_back(name, id);
    }
    void deep_rec(const std::string &name, int64_t id) {
        if (deep_) rec(name, id);
    }
    int64_t weight(std::vector<float> v) {
        weights_.push_back(std::move(v));
        return (int64_t)weights_.size() - 1;
    }
    int64_t own(const std::string &name, int64_t n) { return weight(w_.owned(name, n)); }
    int64_t own_or_zeros(const std::string &name, int64_t n) {
        if (w_.has(name)) return own(name, n);
        return weight(std::vector<float>(n, 0.0f));
    }
    int64_t opt_bias(const std::string &prefix, int64_t n) {
        std::string b = prefix + "/bias";
        return w_.has(b) ? own(b, n) : -1;
    }
    void push(const mx_op &o) { ops_.push_back(o); }

    // -- op emitters ----------------------------------------------------
    void chan_ln(int64_t dst, int64_t src, const std::string &prefix, int64_t c, int64_t hw) {
        int64_t s = own(prefix + "/scale", c);
        int64_t b = own_or_zeros(prefix + "/bias", c);
        mx_op o = blank(MX_OP_CHAN_LN);
        o.dst = dst; o.src = src; o.scale = s; o.bias = b; o.c = c; o.hw = hw;
        push(o);
    }
    void conv1x1(int64_t dst, int64_t src, const std::string &prefix, int64_t ci, int64_t co,
                 int64_t h, int64_t wd) {
        std::string k = prefix + "/kernel";
        mx_op o = blank(MX_OP_CONV1X1);
        o.w = weight(w_.conv1x1(k, ci, co));
        if (twins_) o.wt = weight(w_.conv1x1_t(k, ci, co));
        o.bias = opt_bias(prefix, co);
        o.dst = dst; o.src = src; o.c_in = ci; o.c_out = co; o.h = h; o.wd = wd;
        push(o);
    }
    void conv3x3(int64_t dst, int64_t src, const std::string &prefix, int64_t ci, int64_t co,
                 int64_t h, int64_t wd) {
        std::string k = prefix + "/kernel";
        mx_op o = blank(MX_OP_CONV3X3);
        o.w = weight(w_.convkxk(k, 3, ci, co));
        if (twins_) o.wt = weight(w_.conv3x3_t(k, ci, co));
        o.bias = opt_bias(prefix, co);
        o.dst = dst; o.src = src; o.c_in = ci; o.c_out = co; o.h = h; o.wd = wd;
        push(o);
    }
    // Conv_down: 4x4 stride 2, flax SAME padding (ceil(h/2) out).
    void conv_down(int64_t dst, int64_t src, const std::string &prefix, int64_t ci, int64_t co,
                   int64_t h, int64_t wd) {
        mx_op o = blank(MX_OP_CONV4X4S2);
        o.w = weight(w_.convkxk(prefix + "/kernel", 4, ci, co));
        o.bias = opt_bias(prefix, co);
        int64_t pt, pb, pl, pr;
        same_pad(h, 2, 4, pt, pb);
        same_pad(wd, 2, 4, pl, pr);
        o.dst = dst; o.src = src; o.c_in = ci; o.c_out = co; o.h = h; o.wd = wd;
        o.oh = (h + 1) / 2; o.ow = (wd + 1) / 2; o.p[0] = pt; o.p[1] = pl;
        push(o);
    }
    // ConvT_up: 2x2 stride 2 transposed, doubling the resolution.
    void convt_up(int64_t dst, int64_t src, const std::string &prefix, int64_t ci, int64_t co,
                  int64_t h, int64_t wd) {
        mx_op o = blank(MX_OP_CONVT2X2);
        o.w = weight(w_.convt2x2(prefix + "/kernel", ci, co));
        o.bias = opt_bias(prefix, co);
        o.dst = dst; o.src = src; o.c_in = ci; o.c_out = co; o.h = h; o.wd = wd;
        push(o);
    }
    void flat(int kind, int64_t dst, int64_t a, int64_t b, int64_t n) {
        mx_op o = blank(kind);
        o.dst = dst; o.src = a; o.src2 = b; o.n = n;
        push(o);
    }
    void gelu(int64_t dst, int64_t src, int64_t n) { flat(MX_OP_GELU, dst, src, -1, n); }
    void add(int64_t dst, int64_t a, int64_t b, int64_t n) { flat(MX_OP_ADD, dst, a, b, n); }
    void mul(int64_t dst, int64_t a, int64_t b, int64_t n) { flat(MX_OP_MUL, dst, a, b, n); }
    void copy(int64_t dst, int64_t src, int64_t n) { flat(MX_OP_COPY, dst, src, -1, n); }
    void lrelu(int64_t dst, int64_t src, int64_t n, float slope) {
        mx_op o = blank(MX_OP_LRELU);
        o.dst = dst; o.src = src; o.n = n; o.slope = slope;
        push(o);
    }
    void block_perm(int64_t dst, int64_t src, int64_t c, int64_t h, int64_t wd, int64_t gh,
                    int64_t gw, int64_t fh, int64_t fw, bool forward) {
        mx_op o = blank(MX_OP_BLOCK_PERM);
        o.dst = dst; o.src = src; o.c = c; o.h = h; o.wd = wd;
        o.p[0] = gh; o.p[1] = gw; o.p[2] = fh; o.p[3] = fw;
        o.mode = forward ? MX_PERM_FORWARD : 0;
        push(o);
    }
    void gate_mm(int64_t dst, int64_t src, int64_t w, int64_t bias, int64_t c, int64_t outer,
                 int64_t inner, int mode) {
        mx_op o = blank(MX_OP_GATE_MM);
        o.dst = dst; o.src = src; o.w = w; o.bias = bias; o.c = c;
        o.p[0] = outer; o.p[1] = inner; o.mode = mode;
        push(o);
    }
    // jax's `nearest` for an integer downsample: stride `factor`, offset factor/2.
    void nearest_down(int64_t dst, int64_t src, int64_t c, int64_t h, int64_t w, int64_t factor) {
        mx_op o = blank(MX_OP_DOWN_S);
        o.dst = dst; o.src = src; o.c = c; o.h = h; o.wd = w;
        o.p[0] = factor; o.p[1] = factor / 2; o.oh = h / factor; o.ow = w / factor;
        push(o);
    }
    // Bilinear resize, or a Copy when the shape does not change.
    void resize(int64_t dst, int64_t src, int64_t c, int64_t hin, int64_t win, int64_t hout,
                int64_t wout) {
        if (hin == hout && win == wout) {
            copy(dst, src, c * hin * win);
            return;
        }
        int64_t tmp = buf(c, hin, wout, "resize_tmp");
        mx_op o = blank(MX_OP_RESIZE);
        o.dst = dst; o.src = src; o.src2 = tmp; o.c = c;
        o.h = hin; o.wd = win; o.oh = hout; o.ow = wout;
        push(o);
    }

    // -- blocks ------------------------------------------------------------
    int64_t calayer(const std::string &prefix, int64_t x, int64_t c, int64_t h, int64_t wd, int64_t red);
    int64_t rcab(const std::string &prefix, int64_t x, int64_t c, int64_t h, int64_t wd, int64_t red);
    int64_t rdcab(const std::string &prefix, int64_t x, int64_t c, int64_t h, int64_t wd, int64_t red);
    void gating(const std::string &prefix, int64_t u, int64_t v, int64_t dst, int64_t c,
                int64_t gg, int64_t pp, bool over_grid);
    void gmlp_axis(const std::string &prefix, int64_t x, int64_t dst, int64_t c, int64_t h,
                   int64_t wd, int64_t size, bool over_grid);
    int64_t split_head_gmlp(const std::string &prefix, int64_t x, int64_t c, int64_t h, int64_t wd,
                            int64_t block_size, int64_t grid_size);
    int64_t spatial_gating_weights(const std::string &prefix, int64_t x, int64_t c, int64_t h,
                                   int64_t wd, int64_t block_size, int64_t grid_size);
    std::pair<int64_t, int64_t> cross_gating(const std::string &prefix, int64_t x, int64_t cx,
                                             int64_t y, int64_t cy, int64_t h, int64_t wd,
                                             int64_t features, int64_t block_size,
                                             int64_t grid_size, bool upsample_y);
    std::pair<int64_t, int64_t> block_grid(int level) const {
        if (level < cfg_.high_res_stages) return {cfg_.block_size_hr, cfg_.grid_size_hr};
        return {cfg_.block_size_lr, cfg_.grid_size_lr};
    }
    int64_t upsampled(int64_t enc, int64_t c_in, int from, int to, int64_t h, int64_t wd,
                      int64_t features_i);
    int64_t multiscale_signal(const std::vector<int64_t> &encs, int i, int64_t features_i,
                              int64_t h, int64_t wd);
    int64_t decoder_signal(const std::vector<int64_t> &skips, int i, int64_t features_i,
                           int64_t h, int64_t wd, int depth);
    std::pair<int64_t, int64_t> unet_encoder_block(const std::string &prefix, int64_t x,
                                                   int64_t features, int64_t block_size,
                                                   int64_t grid_size, int num_groups, int64_t red,
                                                   bool downsample, int64_t skip, int64_t enc,
                                                   int64_t dec, int64_t h, int64_t wd);
    int64_t unet_decoder_block(const std::string &prefix, int64_t x, int64_t bridge,
                               int64_t features, int64_t block_size, int64_t grid_size,
                               int num_groups, int64_t red, int64_t h, int64_t wd);
    std::pair<int64_t, int64_t> sam(const std::string &prefix, int64_t x, int64_t x_image,
                                    int64_t features, int64_t h, int64_t wd);
    int64_t bottleneck(const std::string &prefix, int64_t x, int64_t features, int64_t h,
                       int64_t wd, int64_t block_size, int num_groups, int64_t red);
    Plan *finish(int64_t input, int64_t output, BufShape shape);
};

// CALayer: squeeze-and-excitation, x * sigmoid(conv(relu(conv(mean(x))))).
int64_t Builder::calayer(const std::string &prefix, int64_t x, int64_t c, int64_t h, int64_t wd,
                         int64_t red) {
    int64_t hw = h * wd;
    int64_t mean = buf(c, 1, 1, "ca_mean");
    mx_op o = blank(MX_OP_CHAN_MEAN);
    o.dst = mean; o.src = x; o.c = c; o.hw = hw;
    push(o);
    deep_rec(prefix + "_mean", mean);
    int64_t sq = buf(c / red, 1, 1, "ca_squeeze");
    conv1x1(sq, mean, prefix + "/Conv_0", c, c / red, 1, 1);
    deep_rec(prefix + "_sq", sq);
    int64_t rl = buf(c / red, 1, 1, "ca_relu");
    lrelu(rl, sq, c / red, 0.0f);
    deep_rec(prefix + "_relu", rl);
    int64_t ex = buf(c, 1, 1, "ca_excite");
    conv1x1(ex, rl, prefix + "/Conv_1", c / red, c, 1, 1);
    deep_rec(prefix + "_excite", ex);
    int64_t sg = buf(c, 1, 1, "ca_sigmoid");
    flat(MX_OP_SIGMOID, sg, ex, -1, c);
    deep_rec(prefix + "_sigmoid", sg);
    int64_t out = buf(c, h, wd, "ca_out");
    mx_op s = blank(MX_OP_CHAN_SCALE);
    s.dst = out; s.src = x; s.src2 = sg; s.c = c; s.hw = hw;
    push(s);
    return out;
}

// RCAB: LayerNorm, 3x3, leaky relu, 3x3, channel attention, residual.
int64_t Builder::rcab(const std::string &prefix, int64_t x, int64_t c, int64_t h, int64_t wd,
                      int64_t red) {
    int64_t n = c * h * wd;
    int64_t y = buf(c, h, wd, "rcab_ln");
    chan_ln(y, x, prefix + "/LayerNorm", c, h * wd);
    deep_rec(prefix + "_ln", y);
    int64_t t = buf(c, h, wd, "rcab_conv1");
    conv3x3(t, y, prefix + "/conv1", c, c, h, wd);
    deep_rec(prefix + "_conv1", t);
    int64_t r = buf(c, h, wd, "rcab_lrelu");
    lrelu(r, t, n, 0.2f);
    deep_rec(prefix + "_lrelu", r);
    int64_t t2 = buf(c, h, wd, "rcab_conv2");
    conv3x3(t2, r, prefix + "/conv2", c, c, h, wd);
    deep_rec(prefix + "_conv2", t2);
    int64_t ca = calayer(prefix + "/channel_attention", t2, c, h, wd, red);
    deep_rec(prefix + "_ca", ca);
    int64_t out = buf(c, h, wd, "rcab_out");
    add(out, ca, x, n);
    return out;
}

// RDCAB: the bottleneck's residual dense channel-attention block.
int64_t Builder::rdcab(const std::string &prefix, int64_t x, int64_t c, int64_t h, int64_t wd,
                       int64_t red) {
    int64_t n = c * h * wd;
    int64_t y = buf(c, h, wd, "rdcab_ln");
    chan_ln(y, x, prefix + "/LayerNorm", c, h * wd);
    int64_t c1 = buf(c, h, wd, "rdcab_dense0");
    conv1x1(c1, y, prefix + "/channel_mixing/Dense_0", c, c, h, wd);
    int64_t g = buf(c, h, wd, "rdcab_gelu");
    gelu(g, c1, n);
    int64_t c2 = buf(c, h, wd, "rdcab_dense1");
    conv1x1(c2, g, prefix + "/channel_mixing/Dense_1", c, c, h, wd);
    int64_t ca = calayer(prefix + "/channel_attention", c2, c, h, wd, red);
    int64_t out = buf(c, h, wd, "rdcab_out");
    add(out, ca, x, n);
    return out;
}

// Grid/Block gating unit: u * (Dense(LN(v)) over one axis + 1), into `dst`.
void Builder::gating(const std::string &prefix, int64_t u, int64_t v, int64_t dst, int64_t c,
                     int64_t gg, int64_t pp, bool over_grid) {
    int64_t n = c * gg * pp;
    int64_t ln = buf(c, gg, pp, "gmlp_gate_ln");
    chan_ln(ln, v, prefix + "/intermediate_layernorm", c, gg * pp);
    int64_t g = buf(c, gg, pp, "gmlp_gate");
    int64_t k = over_grid ? gg : pp;
    int64_t wi = weight(w_.dense(prefix + "/Dense_0/kernel", k));
    int64_t b = own_or_zeros(prefix + "/Dense_0/bias", k);
    gate_mm(g, ln, wi, b, c, gg, pp, over_grid ? 0 : 1);
    flat(MX_OP_GATE_APPLY, dst, u, g, n);
}

// One half of a multi-axis gMLP: block, LN, project, gate, project, residual,
// unblock. Grid: `size` is a cell count; block: `size` is a pixel count.
void Builder::gmlp_axis(const std::string &prefix, int64_t x, int64_t dst, int64_t c, int64_t h,
                        int64_t wd, int64_t size, bool over_grid) {
    int64_t gh, gw, fh, fw;
    if (over_grid) { gh = size; gw = size; fh = h / size; fw = wd / size; }
    else { gh = h / size; gw = wd / size; fh = size; fw = size; }
    if (gh == 0 || gw == 0 || fh == 0 || fw == 0)
        throw Error(prefix + ": a " + S(size) + "-" + (over_grid ? "cell grid" : "pixel block") +
                    " does not fit a " + S(h) + "x" + S(wd) + " feature map (cells " + S(gh) + "x" +
                    S(gw) + ", " + S(fh) + "x" + S(fw) +
                    " pixels) - the input is too small for this model");
    int64_t gg = gh * gw, pp = fh * fw;
    int64_t xb = buf(c, gg, pp, "gmlp_blocked");
    block_perm(xb, x, c, h, wd, gh, gw, fh, fw, true);
    deep_rec(prefix + "_blocked", xb);
    int64_t ln = buf(c, gg, pp, "gmlp_ln");
    chan_ln(ln, xb, prefix + "/LayerNorm", c, gg * pp);
    deep_rec(prefix + "_ln", ln);
    int64_t t = buf(2 * c, gg, pp, "gmlp_inproject");
    conv1x1(t, ln, prefix + "/in_project", c, 2 * c, gg, pp);
    deep_rec(prefix + "_inproject", t);
    int64_t tg = buf(2 * c, gg, pp, "gmlp_gelu");
    gelu(tg, t, 2 * c * gg * pp);
    deep_rec(prefix + "_gelu", tg);
    int64_t u = view(tg, 0, c, "gmlp_u");
    int64_t v = view(tg, c, c, "gmlp_v");
    int64_t gated = buf(c, gg, pp, "gmlp_gated");
    gating(prefix + (over_grid ? "/GridGatingUnit" : "/BlockGatingUnit"), u, v, gated, c, gg, pp,
           over_grid);
    deep_rec(prefix + "_gated", gated);
    int64_t proj = buf(c, gg, pp, "gmlp_outproject");
    conv1x1(proj, gated, prefix + "/out_project", c, c, gg, pp);
    deep_rec(prefix + "_proj", proj);
    int64_t mixed = buf(c, gg, pp, "gmlp_residual");
    add(mixed, proj, xb, c * gg * pp);
    block_perm(dst, mixed, c, h, wd, gh, gw, fh, fw, false);
}

// ResidualSplitHeadMultiAxisGmlpLayer: grid and block gMLPs on the two halves.
int64_t Builder::split_head_gmlp(const std::string &prefix, int64_t x, int64_t c, int64_t h,
                                 int64_t wd, int64_t block_size, int64_t grid_size) {
    int64_t ln = buf(c, h, wd, "shg_ln");
    chan_ln(ln, x, prefix + "/LayerNorm_in", c, h * wd);
    int64_t t = buf(2 * c, h, wd, "shg_inproject");
    conv1x1(t, ln, prefix + "/in_project", c, 2 * c, h, wd);
    int64_t g = buf(2 * c, h, wd, "shg_gelu");
    gelu(g, t, 2 * c * h * wd);
    int64_t u = view(g, 0, c, "shg_u");
    int64_t v = view(g, c, c, "shg_v");
    gmlp_axis(prefix + "/GridGmlpLayer", u, u, c, h, wd, grid_size, true);
    gmlp_axis(prefix + "/BlockGmlpLayer", v, v, c, h, wd, block_size, false);
    int64_t proj = buf(c, h, wd, "shg_outproject");
    conv1x1(proj, g, prefix + "/out_project", 2 * c, c, h, wd);
    int64_t out = buf(c, h, wd, "shg_out");
    add(out, proj, x, c * h * wd);
    return out;
}

// GetSpatialGatingWeights: the cross-gating block's weight branch.
int64_t Builder::spatial_gating_weights(const std::string &prefix, int64_t x, int64_t c, int64_t h,
                                        int64_t wd, int64_t block_size, int64_t grid_size) {
    int64_t ln = buf(c, h, wd, "sgw_ln");
    chan_ln(ln, x, prefix + "/LayerNorm_in", c, h * wd);
    int64_t t = buf(2 * c, h, wd, "sgw_inproject");
    conv1x1(t, ln, prefix + "/in_project", c, 2 * c, h, wd);
    int64_t g = buf(2 * c, h, wd, "sgw_gelu");
    gelu(g, t, 2 * c * h * wd);
    int64_t u = view(g, 0, c, "sgw_u");
    int64_t v = view(g, c, c, "sgw_v");

    int64_t gh = grid_size, gw = grid_size, fh = h / gh, fw = wd / gw;
    int64_t gg = gh * gw, pp = fh * fw;
    int64_t ub = buf(c, gg, pp, "sgw_u_blocked");
    block_perm(ub, u, c, h, wd, gh, gw, fh, fw, true);
    int64_t um = buf(c, gg, pp, "sgw_u_mixed");
    int64_t uw = weight(w_.dense(prefix + "/Dense_0/kernel", gg));
    int64_t ubias = own_or_zeros(prefix + "/Dense_0/bias", gg);
    gate_mm(um, ub, uw, ubias, c, gg, pp, 0);
    int64_t uu = buf(c, h, wd, "sgw_u_out");
    block_perm(uu, um, c, h, wd, gh, gw, fh, fw, false);

    int64_t fh2 = block_size, fw2 = block_size, gh2 = h / fh2, gw2 = wd / fw2;
    int64_t gg2 = gh2 * gw2, pp2 = fh2 * fw2;
    int64_t vb = buf(c, gg2, pp2, "sgw_v_blocked");
    block_perm(vb, v, c, h, wd, gh2, gw2, fh2, fw2, true);
    int64_t vm = buf(c, gg2, pp2, "sgw_v_mixed");
    int64_t vw = weight(w_.dense(prefix + "/Dense_1/kernel", pp2));
    int64_t vbias = own_or_zeros(prefix + "/Dense_1/bias", pp2);
    gate_mm(vm, vb, vw, vbias, c, gg2, pp2, 1);
    int64_t vv = buf(c, h, wd, "sgw_v_out");
    block_perm(vv, vm, c, h, wd, gh2, gw2, fh2, fw2, false);

    int64_t cat = buf(2 * c, h, wd, "sgw_cat");
    int64_t lo = view(cat, 0, c, "sgw_cat_lo");
    int64_t hi = view(cat, c, c, "sgw_cat_hi");
    copy(lo, uu, c * h * wd);
    copy(hi, vv, c * h * wd);
    int64_t out = buf(c, h, wd, "sgw_out");
    conv1x1(out, cat, prefix + "/out_project", 2 * c, c, h, wd);
    return out;
}

// CrossGatingBlock, returning (x, y).
std::pair<int64_t, int64_t> Builder::cross_gating(const std::string &prefix, int64_t x, int64_t cx,
                                                  int64_t y, int64_t cy, int64_t h, int64_t wd,
                                                  int64_t features, int64_t block_size,
                                                  int64_t grid_size, bool upsample_y) {
    int64_t n = features * h * wd;
    int64_t y_up = y;
    if (upsample_y) {
        y_up = buf(features, h, wd, "cg_y_up");
        convt_up(y_up, y, prefix + "/ConvTranspose_0", cy, features, h / 2, wd / 2);
    }
    int64_t x0 = buf(features, h, wd, "cg_x0");
    conv1x1(x0, x, prefix + "/Conv_0", cx, features, h, wd);
    int64_t y0 = buf(features, h, wd, "cg_y0");
    conv1x1(y0, y_up, prefix + "/Conv_1", features, features, h, wd);

    int64_t xl = buf(features, h, wd, "cg_xln");
    chan_ln(xl, x0, prefix + "/LayerNorm_x", features, h * wd);
    int64_t xd = buf(features, h, wd, "cg_xdense");
    conv1x1(xd, xl, prefix + "/in_project_x", features, features, h, wd);
    int64_t xg = buf(features, h, wd, "cg_xgelu");
    gelu(xg, xd, n);
    int64_t gx = spatial_gating_weights(prefix + "/SplitHeadMultiAxisGating_x", xg, features, h,
                                        wd, block_size, grid_size);

    int64_t yl = buf(features, h, wd, "cg_yln");
    chan_ln(yl, y0, prefix + "/LayerNorm_y", features, h * wd);
    int64_t yd = buf(features, h, wd, "cg_ydense");
    conv1x1(yd, yl, prefix + "/in_project_y", features, features, h, wd);
    int64_t yg = buf(features, h, wd, "cg_ygelu");
    gelu(yg, yd, n);
    int64_t gy = spatial_gating_weights(prefix + "/SplitHeadMultiAxisGating_y", yg, features, h,
                                        wd, block_size, grid_size);

    int64_t ym = buf(features, h, wd, "cg_y_mul");
    mul(ym, yg, gx, n);
    int64_t yp = buf(features, h, wd, "cg_y_proj");
    conv1x1(yp, ym, prefix + "/out_project_y", features, features, h, wd);
    int64_t yo = buf(features, h, wd, "cg_y_out");
    add(yo, yp, y0, n);

    int64_t xm = buf(features, h, wd, "cg_x_mul");
    mul(xm, xg, gy, n);
    int64_t xp = buf(features, h, wd, "cg_x_proj");
    conv1x1(xp, xm, prefix + "/out_project_x", features, features, h, wd);
    int64_t xs = buf(features, h, wd, "cg_x_sum");
    add(xs, xp, yo, n);
    int64_t xo = buf(features, h, wd, "cg_x_out");
    add(xo, xs, x0, n);
    return {xo, yo};
}

// UpSampleRatio: bilinear resize to level `to`, then a 1x1 to features_i. The
// parameter names come from one counter over the whole graph, in call order.
int64_t Builder::upsampled(int64_t enc, int64_t c_in, int from, int to, int64_t h, int64_t wd,
                           int64_t features_i) {
    std::string name = "UpSampleRatio_" + std::to_string(up_index_++);
    int64_t r = buf(c_in, h >> to, wd >> to, "up_resize");
    resize(r, enc, c_in, h >> from, wd >> from, h >> to, wd >> to);
    int64_t o = buf(features_i, h >> to, wd >> to, "up_conv");
    conv1x1(o, r, name + "/Conv_0", c_in, features_i, h >> to, wd >> to);
    return o;
}

int64_t Builder::multiscale_signal(const std::vector<int64_t> &encs, int i, int64_t features_i,
                                   int64_t h, int64_t wd) {
    int64_t ch = h >> i, cw = wd >> i;
    int64_t cat = buf(3 * features_i, ch, cw, "cg_signal");
    for (size_t j = 0; j < encs.size(); ++j) {
        int64_t e = encs[j];
        int64_t p = upsampled(e, bufs_[e].c, (int)j, i, h, wd, features_i);
        int64_t dst = view(cat, (int64_t)j * features_i, features_i, "cg_signal_part");
        copy(dst, p, features_i * ch * cw);
    }
    return cat;
}

int64_t Builder::decoder_signal(const std::vector<int64_t> &skips, int i, int64_t features_i,
                                int64_t h, int64_t wd, int depth) {
    int64_t ch = h >> i, cw = wd >> i;
    int64_t cat = buf(3 * features_i, ch, cw, "dec_signal");
    for (size_t j = 0; j < skips.size(); ++j) {
        int64_t sk = skips[j];
        int from = depth - 1 - (int)j;
        int64_t p = upsampled(sk, bufs_[sk].c, from, i, h, wd, features_i);
        int64_t dst = view(cat, (int64_t)j * features_i, features_i, "dec_signal_part");
        copy(dst, p, features_i * ch * cw);
    }
    return cat;
}

// UNetEncoderBlock, returning (downsampled, bridge).
std::pair<int64_t, int64_t> Builder::unet_encoder_block(
    const std::string &prefix, int64_t x, int64_t features, int64_t block_size, int64_t grid_size,
    int num_groups, int64_t red, bool downsample, int64_t skip, int64_t enc, int64_t dec,
    int64_t h, int64_t wd) {
    int64_t cx = bufs_[x].c;
    int64_t c_in = cx + (skip >= 0 ? bufs_[skip].c : 0);
    int64_t xin = x;
    if (skip >= 0) {
        // flax concatenates along channels in the order (x, skip).
        int64_t cat = buf(c_in, h, wd, "enc_skip_cat");
        int64_t a = view(cat, 0, cx, "enc_skip_x");
        int64_t b = view(cat, cx, bufs_[skip].c, "enc_skip_skip");
        copy(a, x, bufs_[x].len());
        copy(b, skip, bufs_[skip].len());
        xin = cat;
    }
    deep_rec(prefix + "_mid_cat", xin);
    int64_t t = buf(features, h, wd, "enc_conv");
    conv1x1(t, xin, prefix + "/Conv_0", c_in, features, h, wd);
    deep_rec(prefix + "_mid_conv", t);
    int64_t y = t;
    for (int g = 0; g < num_groups; ++g) {
        y = split_head_gmlp(prefix + "/SplitHeadMultiAxisGmlpLayer_" + std::to_string(g), y,
                            features, h, wd, block_size, grid_size);
        deep_rec(prefix + "_mid_g" + std::to_string(g) + "_gmlp", y);
        // flax's own name: "channel_attention_block_1" followed by the index.
        y = rcab(prefix + "/channel_attention_block_1" + std::to_string(g), y, features, h, wd, red);
        deep_rec(prefix + "_mid_g" + std::to_string(g) + "_rcab", y);
    }
    int64_t summed = buf(features, h, wd, "enc_residual");
    add(summed, y, t, features * h * wd);
    deep_rec(prefix + "_mid_sum", summed);
    int64_t out = summed;
    if (enc >= 0 && dec >= 0) {
        int64_t yd = buf(features, h, wd, "enc_encdec");
        add(yd, enc, dec, features * h * wd);
        out = cross_gating(prefix + "/cross_gating_block", summed, features, yd, features, h, wd,
                           features, block_size, grid_size, false)
                  .first;
    }
    if (downsample) {
        int64_t down = buf(features, (h + 1) / 2, (wd + 1) / 2, "enc_down");
        conv_down(down, out, prefix + "/Conv_1", features, features, h, wd);
        return {down, out};
    }
    return {out, out};
}

int64_t Builder::unet_decoder_block(const std::string &prefix, int64_t x, int64_t bridge,
                                    int64_t features, int64_t block_size, int64_t grid_size,
                                    int num_groups, int64_t red, int64_t h, int64_t wd) {
    int64_t up = buf(features, h, wd, "dec_up");
    convt_up(up, x, prefix + "/ConvTranspose_0", bufs_[x].c, features, h / 2, wd / 2);
    return unet_encoder_block(prefix + "/UNetEncoderBlock_0", up, features, block_size, grid_size,
                              num_groups, red, false, bridge, -1, -1, h, wd)
        .first;
}

// Supervised attention module, returning (sam feature, image).
std::pair<int64_t, int64_t> Builder::sam(const std::string &prefix, int64_t x, int64_t x_image,
                                         int64_t features, int64_t h, int64_t wd) {
    int64_t n = features * h * wd;
    int64_t x1 = buf(features, h, wd, "sam_x1");
    conv3x3(x1, x, prefix + "/Conv_0", features, features, h, wd);
    int64_t t = buf(3, h, wd, "sam_img_conv");
    conv3x3(t, x, prefix + "/Conv_1", features, 3, h, wd);
    int64_t image = buf(3, h, wd, "sam_image");
    add(image, t, x_image, 3 * h * wd);
    int64_t s = buf(features, h, wd, "sam_img_pre_sigmoid");
    conv3x3(s, image, prefix + "/Conv_2", 3, features, h, wd);
    int64_t gate = buf(features, h, wd, "sam_sigmoid");
    flat(MX_OP_SIGMOID, gate, s, -1, n);
    int64_t g = buf(features, h, wd, "sam_gated");
    mul(g, x1, gate, n);
    int64_t out = buf(features, h, wd, "sam_out");
    add(out, g, x, n);
    return {out, image};
}

int64_t Builder::bottleneck(const std::string &prefix, int64_t x, int64_t features, int64_t h,
                            int64_t wd, int64_t block_size, int num_groups, int64_t red) {
    int64_t t = buf(features, h, wd, "bn_inputproj");
    conv1x1(t, x, prefix + "/input_proj", bufs_[x].c, features, h, wd);
    int64_t y = t;
    for (int g = 0; g < num_groups; ++g) {
        y = split_head_gmlp(prefix + "/SplitHeadMultiAxisGmlpLayer_" + std::to_string(g), y,
                            features, h, wd, block_size, block_size);
        y = rdcab(prefix + "/channel_attention_block_1_" + std::to_string(g), y, features, h, wd,
                  red);
    }
    int64_t out = buf(features, h, wd, "bn_out");
    add(out, y, t, features * h * wd);
    return out;
}

Plan *Builder::build(int64_t h, int64_t wd) {
    const int depth = cfg_.depth, stages = cfg_.num_stages, nss = cfg_.num_supervision_scales;
    const int64_t features = cfg_.features;
    if (h <= 0 || wd <= 0) throw Error("the plan needs a positive input size");
    // Every buffer's element count (at most 16 x features channels times the
    // input plane) and every offset of the packed arena must stay far inside
    // 64 bits; 2^24 per side is 256 TB per full-resolution tensor, far beyond
    // any device or host, which refuse long before.
    if (h > (int64_t)1 << 24 || wd > (int64_t)1 << 24)
        throw Error("the plan's input is " + std::to_string(wd) + "x" + std::to_string(h) +
                    "; each side is limited to 16777216 pixels");

    int64_t input = buf(3, h, wd, "input");
    rec("input", input);
    // The input pyramid, jax `nearest`: shortcuts[i] samples the INPUT directly.
    std::vector<int64_t> shortcuts{input};
    for (int i = 1; i < nss; ++i) {
        int64_t f = 1LL << i;
        int64_t d = buf(3, h / f, wd / f, "shortcut");
        nearest_down(d, input, 3, h, wd, f);
        shortcuts.push_back(d);
    }

    std::vector<std::vector<int64_t>> outputs_all;
    std::vector<int64_t> sam_prev, encs_prev, decs_prev;
    auto pop = [](std::vector<int64_t> &v, const char *what) {
        if (v.empty()) throw Error(what);
        int64_t x = v.back();
        v.pop_back();
        return x;
    };

    for (int s = 0; s < stages; ++s) {
        std::string st = "stage_" + std::to_string(s);
        std::vector<int64_t> x_scales;
        for (int i = 0; i < nss; ++i) {
            int64_t c = (1LL << i) * features;
            int64_t xs = buf(c, h >> i, wd >> i, "input_conv");
            conv3x3(xs, shortcuts[i], st + "_input_conv_" + std::to_string(i), 3, c, h >> i, wd >> i);
            if (s > 0) {
                auto bg = block_grid(i);
                int64_t sm = pop(sam_prev, "stage input fuse: no SAM feature left");
                x_scales.push_back(cross_gating(st + "_input_fuse_sam_" + std::to_string(i), xs, c,
                                                sm, c, h >> i, wd >> i, c, bg.first, bg.second,
                                                false)
                                       .first);
            } else {
                x_scales.push_back(xs);
            }
            rec("stage" + std::to_string(s) + "_input_conv" + std::to_string(i), x_scales.back());
        }

        std::vector<int64_t> encs;
        int64_t x = x_scales[0];
        for (int i = 0; i < depth; ++i) {
            auto bg = block_grid(i);
            int64_t fi = (1LL << i) * features;
            int64_t skip = i < nss ? x_scales[i] : -1;
            int64_t ep = s > 0 ? pop(encs_prev, "encoder: no enc feature left") : -1;
            int64_t dp = s > 0 ? pop(decs_prev, "encoder: no dec feature left") : -1;
            auto r = unet_encoder_block(st + "_encoder_block_" + std::to_string(i), x, fi, bg.first,
                                        bg.second, cfg_.num_groups, cfg_.channels_reduction, true,
                                        skip, ep, dp, h >> i, wd >> i);
            rec("stage" + std::to_string(s) + "_enc" + std::to_string(i) + "_bridge", r.second);
            rec("stage" + std::to_string(s) + "_enc" + std::to_string(i) + "_out", r.first);
            x = r.first;
            encs.push_back(r.second);
        }

        int64_t global_c = (1LL << (depth - 1)) * features;
        for (int i = 0; i < cfg_.num_bottleneck_blocks; ++i)
            x = bottleneck(st + "_global_block_" + std::to_string(i), x, global_c, h >> depth,
                           wd >> depth, cfg_.block_size_lr, cfg_.num_groups, cfg_.channels_reduction);
        rec("stage" + std::to_string(s) + "_global", x);
        int64_t global_feature = x;

        std::vector<int64_t> skip_features;
        for (int i = depth - 1; i >= 0; --i) {
            auto bg = block_grid(i);
            int64_t fi = (1LL << i) * features;
            int64_t signal = multiscale_signal(encs, i, fi, h, wd);
            auto r = cross_gating(st + "_cross_gating_block_" + std::to_string(i), signal, 3 * fi,
                                  global_feature, global_c, h >> i, wd >> i, fi, bg.first,
                                  bg.second, true);
            global_feature = r.second;
            global_c = fi;
            rec("stage" + std::to_string(s) + "_skip" + std::to_string(i), r.first);
            skip_features.push_back(r.first);
        }

        std::vector<int64_t> outputs, decs, sam_new;
        for (int i = depth - 1; i >= 0; --i) {
            auto bg = block_grid(i);
            int64_t fi = (1LL << i) * features;
            int64_t ch = h >> i, cw = wd >> i;
            int64_t signal = decoder_signal(skip_features, i, fi, h, wd, depth);
            x = unet_decoder_block(st + "_decoder_block_" + std::to_string(i), x, signal, fi,
                                   bg.first, bg.second, cfg_.num_groups, cfg_.channels_reduction,
                                   ch, cw);
            rec("stage" + std::to_string(s) + "_dec" + std::to_string(i), x);
            decs.push_back(x);
            if (i < nss) {
                if (s + 1 < stages) {
                    auto r = sam(st + "_supervised_attention_module_" + std::to_string(i), x,
                                 shortcuts[i], fi, ch, cw);
                    outputs.push_back(r.second);
                    sam_new.push_back(r.first);
                    rec("stage" + std::to_string(s) + "_sam" + std::to_string(i), r.first);
                } else {
                    int64_t o = buf(3, ch, cw, "output");
                    conv3x3(o, x, st + "_output_conv_" + std::to_string(i), fi, 3, ch, cw);
                    int64_t out = buf(3, ch, cw, "stage_out");
                    add(out, o, shortcuts[i], 3 * ch * cw);
                    outputs.push_back(out);
                }
                rec("stage" + std::to_string(s) + "_out" + std::to_string(i), outputs.back());
            }
        }
        encs_prev.assign(encs.rbegin(), encs.rend());
        decs_prev = decs;
        sam_prev = sam_new;
        outputs_all.push_back(outputs);
    }
    if (outputs_all.empty() || outputs_all.back().empty()) throw Error("the model produced no output");
    int64_t output = outputs_all.back().back();
    rec("final", output);
    return finish(input, output, BufShape{3, h, wd});
}

// Live ranges per owning buffer, then largest-first first-fit offsets.
Plan *Builder::finish(int64_t input, int64_t output, BufShape shape) {
    const size_t n = bufs_.size();
    const uint64_t DEAD = UINT64_MAX - 1;
    std::vector<int64_t> base(n);
    std::vector<uint64_t> delta(n);
    for (size_t i = 0; i < n; ++i) {
        if (alias_parent_[i] < 0) { base[i] = (int64_t)i; delta[i] = 0; }
        else { base[i] = base[alias_parent_[i]]; delta[i] = delta[alias_parent_[i]] + alias_delta_[i]; }
    }
    std::vector<uint64_t> first(n, UINT64_MAX), last(n, 0);
    std::vector<int64_t> touch, seen;
    for (size_t oi = 0; oi < ops_.size(); ++oi) {
        touch.clear();
        seen.clear();
        op_operands(ops_[oi], touch);
        for (int64_t t : touch) {
            int64_t b = base[t];
            if (std::find(seen.begin(), seen.end(), b) != seen.end()) continue;
            seen.push_back(b);
            if (first[b] == UINT64_MAX) first[b] = oi;
            last[b] = oi;
        }
    }
    for (size_t i = 0; i < n; ++i)
        if (first[i] == UINT64_MAX) { first[i] = DEAD; last[i] = 0; }
    // Named buffers live to the end so a dump taken after the run sees them.
    for (auto &nm : named_) {
        int64_t b = base[nm.second];
        if (first[b] != DEAD) last[b] = ops_.empty() ? 0 : ops_.size() - 1;
    }

    std::vector<int64_t> order;
    for (size_t i = 0; i < n; ++i)
        if (base[i] == (int64_t)i && first[i] != DEAD) order.push_back((int64_t)i);
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
        if (bufs_[a].len() != bufs_[b].len()) return bufs_[a].len() > bufs_[b].len();
        return first[a] < first[b];
    });

    struct Block { uint64_t start, end, off, size; };
    std::vector<Block> placed;
    std::vector<uint64_t> off(n, 0);
    uint64_t arena_len = 0;
    std::vector<uint64_t> cands;
    std::vector<const Block *> live;
    for (int64_t i : order) {
        uint64_t size = (uint64_t)bufs_[i].len();
        uint64_t start = first[i], end = last[i];
        // Candidates come from every placed block; only the blocks whose live
        // range overlaps this one's can clash, so those are filtered once.
        cands.assign(1, 0);
        live.clear();
        for (auto &b : placed) {
            cands.push_back(b.off + b.size);
            if (start <= b.end && b.start <= end) live.push_back(&b);
        }
        std::sort(cands.begin(), cands.end());
        cands.erase(std::unique(cands.begin(), cands.end()), cands.end());
        uint64_t chosen = arena_len;
        for (uint64_t c : cands) {
            bool clash = false;
            for (const Block *b : live)
                if (c < b->off + b->size && b->off < c + size) { clash = true; break; }
            if (!clash) { chosen = c; break; }
        }
        off[i] = chosen;
        arena_len = std::max(arena_len, chosen + size);
        placed.push_back({start, end, chosen, size});
    }

    auto *p = new Plan();
    p->offs.resize(n);
    for (size_t i = 0; i < n; ++i) p->offs[i] = off[base[i]] + delta[i];
    p->bufs = std::move(bufs_);
    p->ops = std::move(ops_);
    p->weights = std::move(weights_);
    p->arena_len = arena_len;
    p->input = input;
    p->output = output;
    p->dumps = std::move(named_);
    p->shape = shape;
    p->labels = std::move(labels_);
    p->alias_parent = std::move(alias_parent_);
    p->alias_delta = std::move(alias_delta_);
    p->keep.assign(n, 0);
    for (auto &nm : p->dumps) p->keep[base[nm.second]] = 1;
    p->index_weights();
    return p;
}

}  // namespace

Plan *build_plan(const Weights &w, int64_t h, int64_t wd, bool named, bool gpu_twins, bool deep) {
    Builder b(w, named, gpu_twins, deep);
    return b.build(h, wd);
}

}  // namespace mx
