// The C ABI over the plan contract (include/maxim_plan.h).

#include <cstring>
#include <iterator>
#include <string>

#include "host.hpp"

namespace mx {

static thread_local std::string g_err;

void set_error(const std::string &m) { g_err = m; }

}  // namespace mx

using namespace mx;

namespace {

template <typename F>
int guard(F &&f) {
    try {
        f();
        return 0;
    } catch (const std::exception &e) {
        set_error(e.what());
        return -1;
    }
}

}  // namespace

extern "C" {

const char *mx_last_error(void) { return g_err.c_str(); }

int mx_config_variant(const char *variant, mx_config *out) {
    return guard([&] { *out = Config::variant(variant ? variant : "").to_c(); });
}

int mx_config_for_task(const char *task, mx_config *out) {
    return guard([&] { *out = Config::for_task(task ? task : "").to_c(); });
}

mx_weights *mx_weights_open(const char *path) {
    Weights *w = nullptr;
    guard([&] { w = Weights::open(path ? path : ""); });
    return reinterpret_cast<mx_weights *>(w);
}

mx_weights *mx_weights_synthetic(const char *variant, uint64_t seed, float kernel_gain,
                                 float bias_std, float ln_std) {
    Weights *w = nullptr;
    guard([&] { w = Weights::make_synthetic(variant ? variant : "", seed, kernel_gain, bias_std, ln_std); });
    return reinterpret_cast<mx_weights *>(w);
}

int mx_weights_save(const mx_weights *w, const char *path, const char *task) {
    return guard([&] {
        reinterpret_cast<const Weights *>(w)->save(path ? path : "", task ? task : "enhancement");
    });
}

int mx_weights_config(const mx_weights *w, mx_config *out) {
    *out = reinterpret_cast<const Weights *>(w)->config.to_c();
    return 0;
}

uint64_t mx_weights_count(const mx_weights *w) {
    return reinterpret_cast<const Weights *>(w)->tensors.size();
}

uint64_t mx_weights_params(const mx_weights *w) {
    return reinterpret_cast<const Weights *>(w)->params();
}

const char *mx_weights_name(const mx_weights *w, uint64_t i) {
    auto &t = reinterpret_cast<const Weights *>(w)->tensors;
    if (i >= t.size()) return nullptr;
    auto it = t.begin();
    std::advance(it, (long)i);
    return it->first.c_str();
}

uint64_t mx_weights_tensor(const mx_weights *w, const char *name, const float **data,
                           int64_t shape[4], int32_t *ndim) {
    auto &t = reinterpret_cast<const Weights *>(w)->tensors;
    auto it = t.find(name ? name : "");
    if (it == t.end()) return 0;
    if (data) *data = it->second.data.data();
    if (ndim) *ndim = (int32_t)it->second.shape.size();
    if (shape)
        for (size_t i = 0; i < 4; ++i) shape[i] = i < it->second.shape.size() ? it->second.shape[i] : 0;
    return it->second.data.size();
}

void mx_weights_free(mx_weights *w) { delete reinterpret_cast<Weights *>(w); }

mx_plan *mx_plan_build(const mx_weights *w, int64_t h, int64_t wd, int named, int gpu_twins, int deep) {
    Plan *p = nullptr;
    guard([&] {
        if (!w) throw Error("mx_plan_build: no weights");
        p = build_plan(*reinterpret_cast<const Weights *>(w), h, wd, named != 0, gpu_twins != 0,
                       deep != 0);
    });
    return reinterpret_cast<mx_plan *>(p);
}

void mx_plan_free(mx_plan *p) { delete reinterpret_cast<Plan *>(p); }

void mx_plan_describe(const mx_plan *pp, mx_plan_desc *d) {
    const Plan *p = reinterpret_cast<const Plan *>(pp);
    static_assert(sizeof(BufShape) == sizeof(mx_bufshape), "BufShape layout");
    d->n_ops = p->ops.size();
    d->ops = p->ops.data();
    d->n_bufs = p->bufs.size();
    d->bufs = reinterpret_cast<const mx_bufshape *>(p->bufs.data());
    d->offs = p->offs.data();
    d->n_weights = p->weights.size();
    d->weights = p->wptr.data();
    d->weight_lens = p->wlen.data();
    d->arena_len = p->arena_len;
    d->input = (uint64_t)p->input;
    d->output = (uint64_t)p->output;
    d->alias_parent = p->alias_parent.data();
    d->alias_delta = p->alias_delta.data();
    d->keep = p->keep.data();
}

uint64_t mx_plan_n_dumps(const mx_plan *p) { return reinterpret_cast<const Plan *>(p)->dumps.size(); }

const char *mx_plan_dump_name(const mx_plan *p, uint64_t i) {
    auto &d = reinterpret_cast<const Plan *>(p)->dumps;
    return i < d.size() ? d[i].first.c_str() : nullptr;
}

int64_t mx_plan_dump_buf(const mx_plan *p, uint64_t i) {
    auto &d = reinterpret_cast<const Plan *>(p)->dumps;
    return i < d.size() ? d[i].second : -1;
}

const char *mx_plan_label(const mx_plan *p, uint64_t buf) {
    auto &l = reinterpret_cast<const Plan *>(p)->labels;
    return buf < l.size() ? l[buf].c_str() : nullptr;
}

int64_t mx_plan_alias_parent(const mx_plan *p, uint64_t buf) {
    auto &a = reinterpret_cast<const Plan *>(p)->alias_parent;
    return buf < a.size() ? a[buf] : -1;
}

uint64_t mx_plan_alias_delta(const mx_plan *p, uint64_t buf) {
    auto &a = reinterpret_cast<const Plan *>(p)->alias_delta;
    return buf < a.size() ? a[buf] : 0;
}

uint64_t mx_plan_weight_bytes(const mx_plan *p) {
    return reinterpret_cast<const Plan *>(p)->weight_bytes();
}

}  // extern "C"
