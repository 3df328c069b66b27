/*
 * maxim_plan.h - the plan contract: the op list, the buffer table, the packed
 * arena and the weight blobs that every executor walks.
 *
 * This is the C-ABI form of the reference's `model::Plan` / `Op` / `BufShape`
 * (src/model.rs:37-140, 1237-1272), of `Weights` (src/weights.rs:17-217), of
 * `Config` (src/config.rs:8-135), of the image padding helpers
 * (src/image.rs:106-246) and of the CPU memory guard (src/memguard.rs:35-172).
 *
 * A host that already owns a plan (the reference's Rust `Plan`) does not need
 * the builder in here: it fills an `mx_plan_desc` from its own vectors and hands
 * that to the HIP executor (maxim_hip.h). The builder exists so that this repo
 * can produce the same plan without a Rust toolchain, and it reproduces the
 * reference's op counts, buffer counts and arena sizes exactly.
 *
 * Conventions: every function returns 0 / a non-NULL handle on success; on
 * failure it returns a negative status / NULL and `mx_last_error()` holds the
 * message (thread-local), the C form of `maxim::Error(String)` (src/lib.rs:29).
 * All tensors are fp32, planar `[c][h][w]`.
 */
#ifndef MAXIM_PLAN_H
#define MAXIM_PLAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The 18 ops, in the order of the reference's `Op` enum (src/model.rs:65-112). */
enum mx_op_kind {
    MX_OP_COPY = 0,
    MX_OP_ADD = 1,
    MX_OP_MUL = 2,
    MX_OP_GATE_APPLY = 3,
    MX_OP_GELU = 4,
    MX_OP_LRELU = 5,
    MX_OP_SIGMOID = 6,
    MX_OP_CHAN_LN = 7,
    MX_OP_CHAN_MEAN = 8,
    MX_OP_CHAN_SCALE = 9,
    MX_OP_CONV1X1 = 10,
    MX_OP_CONV3X3 = 11,
    MX_OP_CONV4X4S2 = 12,
    MX_OP_CONVT2X2 = 13,
    MX_OP_GATE_MM = 14,
    MX_OP_BLOCK_PERM = 15,
    MX_OP_RESIZE = 16,
    MX_OP_DOWN_S = 17,
    MX_OP_KINDS = 18
};

/* BlockPerm flag bits in `mx_op.mode`. */
#define MX_PERM_SWAP 1
#define MX_PERM_FORWARD 2

/*
 * One op. Buffer and weight fields are indices (-1 = absent), never offsets;
 * the arena offset of a buffer is `offs[id]`. Field use per kind:
 *
 *   Copy         dst, src, n
 *   Add / Mul    dst, src (= a), src2 (= b), n
 *   GateApply    dst, src (= u), src2 (= v), n          y = u * (v + 1)
 *   Gelu/Sigmoid dst, src, n
 *   Lrelu        dst, src, n, slope
 *   ChanLn       dst, src, scale, bias, c, hw
 *   ChanMean     dst, src, c, hw
 *   ChanScale    dst, src, src2 (= s, a [c] buffer), c, hw
 *   Conv1x1      dst, src, w ([co][ci]), wt ([ci][co]), bias, c_in, c_out, h, wd
 *   Conv3x3      dst, src, w ([co][ci][3][3]), wt ([tap][ci][co]), bias, c_in, c_out, h, wd
 *   Conv4x4s2    dst, src, w ([co][ci][4][4]), bias, c_in, c_out, h, wd, oh, ow,
 *                p[0] = pad_top, p[1] = pad_left
 *   ConvT2x2     dst, src, w ([ci][co][2][2], spatially flipped), bias, c_in, c_out, h, wd
 *   GateMm       dst, src, w ([a][t]), bias, c, mode, p[0] = outer, p[1] = inner
 *   BlockPerm    dst, src, c, h, wd, mode (MX_PERM_*), p[0..3] = gh, gw, fh, fw
 *   Resize       dst, src, src2 (= tmp [c][hin][wout]), c, h = hin, wd = win,
 *                oh = hout, ow = wout
 *   DownS        dst, src, c, h, wd, oh, ow, p[0] = stride, p[1] = off
 */
typedef struct mx_op {
    int32_t kind;
    int32_t mode;
    float slope;
    int32_t reserved;
    int64_t dst, src, src2;
    int64_t w, wt, bias, scale;
    int64_t n, c, hw;
    int64_t c_in, c_out, h, wd, oh, ow;
    int64_t p[4];
} mx_op;

/* A `[c][h][w]` plane triple (src/model.rs:37-59). */
typedef struct mx_bufshape {
    int64_t c, h, w;
} mx_bufshape;

/*
 * A plan as plain arrays: what any host (the reference's Rust `Plan`, or the
 * builder below) hands to an executor. Nothing here is owned by the struct.
 */
typedef struct mx_plan_desc {
    uint64_t n_ops;
    const mx_op *ops;
    uint64_t n_bufs;
    const mx_bufshape *bufs;
    const uint64_t *offs;          /* absolute element offset of every buffer */
    uint64_t n_weights;
    const float *const *weights;   /* host blobs, indexed the way ops index them */
    const uint64_t *weight_lens;   /* elements per blob */
    uint64_t arena_len;            /* elements */
    uint64_t input, output;        /* buffer ids */
    /* Optional (NULL when the host does not have them): the view table -
     * alias_parent[b] is the buffer whose channels `b` is a range of, or -1,
     * and alias_delta[b] the element offset into it (Plan::alias,
     * src/model.rs:1265-1271) - and keep[b] != 0 for buffers that must stay
     * intact to the end of a pass (the named dumps). With them, an executor
     * may lay its device arena out itself; without them it uses `offs`. */
    const int64_t *alias_parent;
    const uint64_t *alias_delta;
    const uint8_t *keep;
} mx_plan_desc;

/* The model geometry (src/config.rs:8-59). */
typedef struct mx_config {
    int32_t features, depth, num_stages, num_groups;
    int32_t num_supervision_scales, num_outputs, use_cross_gating, high_res_stages;
    int32_t block_size_hr, block_size_lr, grid_size_hr, grid_size_lr;
    int32_t channels_reduction, num_bottleneck_blocks;
} mx_config;

typedef struct mx_weights mx_weights;
typedef struct mx_plan mx_plan;

/* The thread's last error message ("" when none). */
const char *mx_last_error(void);

/* Config::variant (src/config.rs:33-60): "S-1".."S-3", "M-1".."M-3". */
int mx_config_variant(const char *variant, mx_config *out);
/* Config::for_task (src/config.rs:101-116). */
int mx_config_for_task(const char *task, mx_config *out);

/* Weights::open (src/weights.rs:37-41) + Config::of_checkpoint (src/config.rs:71-100):
 * a safetensors checkpoint in the tools/convert.py layout, variant derived from the file. */
mx_weights *mx_weights_open(const char *path);
/*
 * Seeded random-init weights for a variant, with the checkpoint's Flax names and
 * shapes: every Conv/Dense kernel ~ N(0, 2/fan_in) (He-normal, fan_in = kh*kw*c_in),
 * every bias ~ N(0, bias_std), every LayerNorm scale ~ 1 + N(0, ln_std) and its
 * bias ~ N(0, bias_std). Each tensor has its own stream, keyed by (seed, name).
 * `kernel_gain` multiplies every kernel's standard deviation (1 = He-normal).
 */
mx_weights *mx_weights_synthetic(const char *variant, uint64_t seed, float kernel_gain,
                                 float bias_std, float ln_std);
/* Write the tensors in the tools/convert.py:88-137 layout (sorted JSON header,
 * __metadata__, 8-byte aligned data). */
int mx_weights_save(const mx_weights *w, const char *path, const char *task);
int mx_weights_config(const mx_weights *w, mx_config *out);
uint64_t mx_weights_count(const mx_weights *w);
uint64_t mx_weights_params(const mx_weights *w);
/* The i-th tensor name in sorted order (the file's order), NULL past the end. */
const char *mx_weights_name(const mx_weights *w, uint64_t i);
/* One tensor by name: returns its element count (0 if absent); `shape` gets up to 4 dims. */
uint64_t mx_weights_tensor(const mx_weights *w, const char *name, const float **data,
                           int64_t shape[4], int32_t *ndim);
void mx_weights_free(mx_weights *w);

/*
 * Builder::new(&w, cfg)[.without_dumps()].build(h, wd) (src/model.rs:200-251,743-891).
 * `h`/`wd` are the PADDED dimensions. `named` = 1 keeps the named activations live
 * to the end (the `--dump` plan), 0 is the release plan. `gpu_twins` = 1 adds the
 * conv1x1 `[ci][co]` and conv3x3 `[tap][ci][co]` weight twins the reference adds
 * for its GPU build (src/model.rs:296-324); `deep` = 1 also names the
 * per-block-internal activations (MAXIM_DEEP_DUMPS).
 */
mx_plan *mx_plan_build(const mx_weights *w, int64_t h, int64_t wd, int named, int gpu_twins,
                       int deep);
void mx_plan_free(mx_plan *p);
/* Fill a descriptor that points into the plan (valid while the plan lives). */
void mx_plan_describe(const mx_plan *p, mx_plan_desc *out);
uint64_t mx_plan_n_dumps(const mx_plan *p);
const char *mx_plan_dump_name(const mx_plan *p, uint64_t i);
int64_t mx_plan_dump_buf(const mx_plan *p, uint64_t i);
const char *mx_plan_label(const mx_plan *p, uint64_t buf);
/* Views: parent id (-1 when the buffer owns its bytes) and element delta. */
int64_t mx_plan_alias_parent(const mx_plan *p, uint64_t buf);
uint64_t mx_plan_alias_delta(const mx_plan *p, uint64_t buf);
uint64_t mx_plan_weight_bytes(const mx_plan *p);

/* image::same_pad (src/image.rs:106-111). */
void mx_same_pad(int64_t size, int64_t stride, int64_t k, int64_t *before, int64_t *after);
/*
 * image::preprocess (src/image.rs:171-207): even-ize by reflecting the bottom/right
 * edge, then centred reflect pad to the next multiple of `factor`. Two calls: with
 * out == NULL it only reports the padded shape and the even shape (or refuses with
 * the reference's message); then with a buffer of c*ph*pw floats it fills it.
 */
int mx_preprocess(const float *img, int64_t c, int64_t h, int64_t w, int64_t factor,
                  float *out, int64_t *ph, int64_t *pw, int64_t *even_h, int64_t *even_w);
/* image::crop_out (src/image.rs:232-246). */
int mx_crop_out(const float *img, int64_t c, int64_t ph, int64_t pw, int64_t even_h,
                int64_t even_w, int64_t orig_h, int64_t orig_w, float *out);

/* image::read_png / read_png_stream (src/image.rs:33-72): an 8-bit grayscale,
 * gray + alpha, RGB or RGBA PNG, plain or Adam7-interlaced, decoded once
 * into a handle: from the file `path`, or, with path NULL, from the n bytes
 * at data (the CLI's `-i -`, src/main.rs:205-214). Reports h and w. */
typedef struct mx_png mx_png;
int mx_png_open(const char *path, const unsigned char *data, size_t n, mx_png **img, int64_t *h, int64_t *w);
/* The decoded image as [3][h][w] floats in 0..1 (gray expanded, alpha
 * dropped) into out, which holds cap floats; refused when cap < 3*h*w. */
int mx_png_pixels(const mx_png *img, float *out, size_t cap);
void mx_png_close(mx_png *img);
/* image::write_png_stream (src/image.rs:84-104) into memory (the CLI's
 * `-o -`, src/main.rs:439-448): sets *n to the PNG's size; with out != NULL
 * also writes the bytes, refused when cap < *n. */
int mx_png_encode(const float *img, int64_t h, int64_t w, unsigned char *out, size_t cap, size_t *n);
/* image::write_png (src/image.rs:74-104): [3][h][w] in 0..1 as an 8-bit RGB
 * PNG, each value clamped and rounded half up. */
int mx_png_write(const char *path, const float *img, int64_t h, int64_t w);

/* memguard::CpuPlan::of / check (src/memguard.rs:61-172), for `threads` workers.
 * `avail_override` >= 0 replaces /proc/meminfo's MemAvailable (for tests).
 * Returns 0 when the CPU pass fits, -1 (with the reference's message) when not. */
int mx_memguard_check(const mx_plan *p, int threads, int64_t avail_override, uint64_t *peak_bytes);

#ifdef __cplusplus
}
#endif

#endif /* MAXIM_PLAN_H */
