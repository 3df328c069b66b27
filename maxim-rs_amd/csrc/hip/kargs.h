// Kernel argument blocks, shared by the host executor (g++) and the gfx950
// kernels (hipcc). Each kernel takes exactly one of these by value, so the
// launch passes one parameter and both sides agree on the layout by
// construction: only 8-byte fields, then 4-byte fields in pairs.
#pragma once

#include <stdint.h>

#define MXK_BLOCK 256

// Floats in the code object's `scratch` array (32 MiB): the most scratch a
// plan run through mxh_run_noalloc may need.
#define MXK_NOALLOC_SCRATCH_FLOATS (8u << 20)

// Flat elementwise ops over n elements.
enum { MXK_COPY = 0, MXK_ADD, MXK_MUL, MXK_GATE_APPLY, MXK_GELU, MXK_LRELU, MXK_SIGMOID };

struct EwArgs {
    const float *a;
    const float *b;
    float *y;
    int64_t n;
    int32_t op;
    float slope;
};

// y[ch][p] = x[ch][p] * s[ch] (+ r[ch][p] when r is set: a residual add
// fused into the scale; then + r2[ch][p] when r2 is set: a second add)
struct ChanScaleArgs {
    const float *x;
    const float *s;
    float *y;
    int64_t hw;
    int64_t c;
    const float *r;
    const float *r2;
};

// The channel-attention MLP on a [c] vector, one block:
// h = lrelu(b1 + W1 . x) ([r]), y = sigmoid(b2 + W2 . h) ([c]).
struct CaArgs {
    const float *x, *w1, *b1, *w2, *b2;
    float *y;
    int32_t c, r;
    float slope;
    int32_t pad;
};

// The CALayer's global average pool finished in the MLP's block: the
// channel means from mx_chan_mean_part's partial sums (mx_chan_mean_final's
// order), kept in LDS for the MLP and also written to `mean`.
struct CaMeanArgs {
    CaArgs mlp;        // mlp.x unused: the means are computed here
    const float *part;
    float *mean;
    int64_t hw;
    int32_t nchunk, pad;
};

// ChanScale -> Add [-> Add] as mx_chan_scale_add computes it (y = x * s[ch]
// + r (+ r2)), with the per-pixel LayerNorm statistics of y ([2][hw]: mean,
// then 1 / std) for a LayerNorm folded into a later GEMM.
struct ScaleAddLnArgs {
    const float *x, *s, *r, *r2;
    float *y, *stats;
    int64_t hw;
    int32_t c;
    float eps;
};

// Channel LayerNorm over [c][hw].
struct ChanLnArgs {
    const float *x;
    const float *scale;
    const float *bias;
    float *y;
    int64_t hw;
    int32_t c;
    float eps;
};

// Channel mean: partial sums per (channel, chunk) into `part`, then one
// value per channel.
struct ChanMeanArgs {
    const float *x;
    float *part;
    float *y;
    int64_t hw;
    int64_t chunk;     // elements per partial
    int32_t c;
    int32_t nchunk;
};

// Space <-> block permutation.
struct PermArgs {
    const float *x;
    float *y;
    int64_t c;
    int32_t h, wd, gh, gw, fh, fw, swap, forward;
};

// One axis of the jax bilinear resize. axis 2 = horizontal (rows of `n_in`
// elements -> rows of `n_out`), axis 1 = vertical (planes of n_in rows of
// `width` -> n_out rows).
struct ResizeArgs {
    const float *x;
    float *y;
    int64_t rows;      // horizontal: c * hin; vertical: c
    int32_t n_in, n_out, width, axis;
};

// Both resize axes in one pass (mx_resize_hv[4]): tap tables as for the
// two-pass kernels, `rows` output rows x 64 (256) output columns per block.
struct Resize2Args {
    const float *x;
    float *y;
    const float *th, *tv;   // tap tables: horizontal (per output column), vertical (per output row)
    int32_t h, wd, oh, ow;  // input and output plane
    int32_t mth, mtv;       // taps per table row
    int32_t rows, tiles_x;  // output rows per block, column tiles per row band
    int32_t band, span;     // LDS input rows and columns (the most any block reads)
    int32_t vec, pad;       // 1: input rows staged with 128-bit loads (wd % 4 == 0, 16-byte aligned x)
};

// Nearest subsample.
struct DownArgs {
    const float *x;
    float *y;
    int64_t c;
    int32_t h, wd, stride, off, oh, ow;
};

// C[b] = A[b] . B[b] (+ bias), A [M][K] and B [K][N] row-major, C [M][N].
// Epilogue modes: plain (bias by row or column) or the transposed-conv scatter.
enum { MXK_BIAS_NONE = 0, MXK_BIAS_ROW = 1, MXK_BIAS_COL = 2 };
enum { MXK_EPI_PLAIN = 0, MXK_EPI_CONVT = 1 };

// A fused epilogue, applied per output element after the bias and in the
// order of the ops it replaces, so the result is the unfused kernels' to the
// bit: v = bias + acc; [gate] v = u * (v + 1); [act] v = gelu(v), lrelu(v)
// or sigmoid(v); [mul] v = v * m; [res1] v = v + r1; [res2] v = v + r2.
// u, m, r1, r2 are indexed like C. (The streaming GEMM kernels take gate,
// GELU and the residuals; the convolutions every field.)
enum { MXK_ACT_NONE = 0, MXK_ACT_GELU = 1, MXK_ACT_LRELU = 2, MXK_ACT_SIGMOID = 3 };

struct Epilogue {
    const float *u;
    const float *r1;
    const float *r2;
    const float *m;
    int32_t act;
    float slope;
};

// A channel LayerNorm folded into a GEMM's X operand (channel-major layout):
// X[k][n] is used as (X[k][n] - mean[n]) * rstd[n] * scale[k] + bias[k], the
// LayerNorm kernels' own expression, with mean/rstd from mx_chan_ln_stats
// (or, in the split-reduction kernels' _ln2 form, from the X tile the block
// holds: mean/rstd unused, eps the LayerNorm's).
struct LnIn {
    const float *mean, *rstd, *scale, *bias;
    float eps;  // mode 2 (the statistics computed by the GEMM itself)
    int32_t pad;
};

// A block permutation folded into a GEMM (BlockPerm, no swap,
// src/model.rs:104-106). map takes the blocked index g * fh * fw + fy * fw + fx
// (g = gy * gw + gx) to the image index (gy * fh + fy) * wd + gx * fw + fx;
// fw % 4 == 0 keeps four consecutive elements contiguous.
//   ymap (backward permutation of the output): output element e (counted
//       from C) is written at (e / plane) * plane + map(e % plane); with
//       r1map the epilogue's r1 is read at that same position, i.e. r1 is the
//       image-ordered tensor whose blocked view the output is added to.
//   xmap (forward permutation of the input, channel-major GEMMs with a
//       folded LayerNorm): X column n is read at map(n) of the image-ordered
//       tensor, and so are the LayerNorm statistics.
struct BlockMap {
    int64_t plane;
    int32_t on, fh, fw, gw, wd, r1map;
    // The map's divisions (by plane, fh * fw, gw and fw) as multiplies:
    // n / d = umulhi(2 n, m) >> s for every n < 2^31, with s = ceil(log2 d)
    // and m = ceil(2^(31 + s) / d), set by the host (mx_block_map).
    uint32_t mpl, mpp, mgw, mfw;
    int32_t spl, spp, sgw, sfw;
};

// A channel LayerNorm of a channel-major GEMM's output (the streaming
// kernels' _lo form, one batch): bands of C output rows from row0 on, C
// being the tile width of `group` consecutive waves of a block.
//   mode 0: one band, normalised per pixel with the LayerNorm kernels' order
//       and expression and written to y as [C][N]; keep = 0 leaves the
//       band's raw values unstored (nothing else reads them).
//   mode 1: `nband` bands, each pixel's statistics only (mean, then 1/std,
//       the LayerNorm statistics kernels' values) written to y as
//       [nband][2][N] at the pixel's image position (through ymap), for the
//       GEMMs that fold those LayerNorms later; the output is stored as usual.
//   order (group > 1): 0 sums each pixel's band in ascending channel order
//       in one wave, the LayerNorm kernels' order; 1 has every wave of the
//       group sum its own channels, the group's partial sums then added in
//       wave order (other bits: rounding differs).
struct LnOut {
    const float *scale, *bias;
    float *y;
    float eps;
    int32_t row0, keep, group, mode, nband, order;
};

struct GemmArgs {
    const float *A;
    const float *B;
    const float *bias;
    float *C;
    int64_t sA, sB, sC;   // batch strides (elements)
    int32_t M, N, K, batch;
    int32_t bias_mode, epi;
    int32_t co, wd;       // convT: output channels and input width
    int32_t cvec, pad;    // 1: C, u, r1, r2 are 16-byte aligned (128-bit stores)
    Epilogue e;
    LnIn ln;
    BlockMap ymap, xmap;
    const float *B2;      // _mul: X is B * B2 elementwise (a folded Mul), same layout
    LnOut lo;
    // Channel-major with batch > 1: fold > 0 tiles the batch's columns as
    // one axis of batch * N columns (N = fold, a multiple of 4, so four
    // consecutive columns lie in one batch); column n is column n % fold of
    // batch n / fold (n / fold = umulhi(2 n, fmul) >> fsh, as BlockMap's).
    // The grid is then one-dimensional.
    int32_t fold, fsh;
    uint32_t fmul, pad2;
};

// Two independent streaming-GEMM launches of one kernel in one grid: blocks
// [0, na) run a, blocks [na, grid) run b (each with one batch).
struct DualGemmArgs {
    GemmArgs a, b;
    uint32_t na, pad[3];
};

// Two LayerNorm launches in one grid, likewise.
struct DualLnArgs {
    ChanLnArgs a, b;
    uint32_t na, pad[3];
};

// Small GEMV for the plane-1 CALayer convs: y[o] = b[o] + sum_i w[o][i] x[i].
struct GemvArgs {
    const float *w;
    const float *x;
    const float *bias;
    float *y;
    int32_t ci, co;
};

// Implicit-GEMM convolution (3x3 pad 1, or 4x4 stride 2 SAME).
// Weights are re-laid out at upload as [co][tap][ci] (K index = tap*ci + c).
struct ConvArgs {
    const float *x;
    const float *w;
    const float *bias;
    float *y;
    int32_t ci, co, h, wd;
    int32_t oh, ow, pad_top, pad_left;
    int32_t cvec;         // 1: y, u, r1, r2 are 16-byte aligned and ow % 4 == 0
    int32_t ksplit;       // split reduction (_s kernels): input-channel chunks per z-slice
    Epilogue e;
};

// The sum of a split-reduction conv's partial outputs, in z order, plus the
// bias: y[m][p] = b[m] + (((part[0] + part[1]) + ...) + part[S - 1]).
struct ConvSumArgs {
    const float *part;  // [nsplit][n]
    const float *bias;
    float *y;
    int64_t n;          // co * oh * ow, a multiple of 4
    int64_t plane;      // oh * ow, a multiple of 4
    int32_t nsplit, pad;
};
