/*
 * TEST INFRASTRUCTURE ONLY: the CPU oracle. Not part of the product; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may load it.
 *
 * A restatement of the reference's CPU executor, src/exec_cpu.rs, one function
 * per `Ctx::op` arm (src/exec_cpu.rs:530-1180), each keeping the reference's
 * order of operations for every output element. Compiled with
 * -ffp-contract=off and without -ffast-math: the reference is Rust, which never
 * contracts a*b+c into an FMA, so neither may this.
 *
 * Parity status of each arm (how it is pinned is in tests/test_oracle.py):
 *   copy/add/mul/gate_apply/lrelu/chan_scale  closed forms, exact
 *   gelu        0.5*x*(1+erf(x/sqrt2)) with libm erff. The reference calls
 *               lightgpu's `ops::cpu::erf`, an un-vendored, unpinned git
 *               dependency: erff agreement is "parity unpinned" beyond the
 *               few-ulp error bound both implementations must meet.
 *   sigmoid     1/(1+expf(-x)); the reference uses Rust's f32::exp (libm).
 *   chan_ln     one-pass s1/s2 in ascending channel order, var = s2/c - m^2
 *   chan_mean   serial left-to-right sum / hw
 *   conv1x1 / conv3x3 / conv4x4s2 / gate_mm   bias first, then the reduction
 *               in the reference's order: ic; (ky, kx, ic); (ky, kx, ic); t
 *   convt2x2    four tap sums from zero over ascending ic, bias added last
 *   block_perm / down_s   index maps, exact
 *   resize      jax bilinear with antialias, ResizeTaps, two passes, exact
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define EPS 1e-6f
#define PB 256
#define MAX_TAPS 64

static int g_threads_used = 1;

int oracle_threads_used(void) { return g_threads_used; }

/* ----------------------------------------------------------- elementwise */

void oracle_add(const float *a, const float *b, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}

void oracle_mul(const float *a, const float *b, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = a[i] * b[i];
}

/* u * (v + 1), src/exec_cpu.rs:553-560. */
void oracle_gate_apply(const float *u, const float *v, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = u[i] * (v[i] + 1.0f);
}

/* 0.5 * x * (1 + erf(x * FRAC_1_SQRT_2)), src/exec_cpu.rs:565-571. */
void oracle_gelu(const float *x, float *y, int64_t n) {
    const float k = 0.70710678118654752440f;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float v = x[i];
        y[i] = 0.5f * v * (1.0f + erff(v * k));
    }
}

/* src/exec_cpu.rs:572-575: slope 0.2 for RCAB, 0 for the CALayer relu. */
void oracle_lrelu(const float *x, float *y, int64_t n, float slope) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] >= 0.0f ? x[i] : slope * x[i];
}

/* src/exec_cpu.rs:576-579. */
void oracle_sigmoid(const float *x, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* ------------------------------------------------------- channel axis */

/* chan_ln, src/exec_cpu.rs:377-434: per pixel a left-to-right pass over the
 * channels for s1 and s2, then y = (x - m) * rstd * w + b. */
void oracle_chan_ln(const float *x, const float *scale, const float *bias, float *y, int64_t c, int64_t hw) {
    float *table = (float *)malloc(sizeof(float) * 2 * (size_t)(hw > 0 ? hw : 1));
    const float nf = (float)c;
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < hw; ++p) {
        float s1 = 0.0f, s2 = 0.0f;
        for (int64_t ic = 0; ic < c; ++ic) {
            float v = x[ic * hw + p];
            s1 += v;
            s2 += v * v;
        }
        float m = s1 / nf;
        float var = s2 / nf - m * m;
        table[2 * p] = m;
        table[2 * p + 1] = 1.0f / sqrtf(fmaxf(var, 0.0f) + EPS);
    }
#pragma omp parallel for schedule(static)
    for (int64_t ch = 0; ch < c; ++ch) {
        const float w = scale[ch], b = bias[ch];
        const float *s = x + ch * hw;
        float *d = y + ch * hw;
        for (int64_t p = 0; p < hw; ++p) d[p] = (s[p] - table[2 * p]) * table[2 * p + 1] * w + b;
    }
    free(table);
}

/* src/exec_cpu.rs:1124-1142: a serial left-to-right sum per channel. Rust's
 * float `sum()` folds from -0.0. */
void oracle_chan_mean(const float *x, float *y, int64_t c, int64_t hw) {
    for (int64_t ch = 0; ch < c; ++ch) {
        const float *p = x + ch * hw;
        float s = -0.0f;
        for (int64_t i = 0; i < hw; ++i) s += p[i];
        y[ch] = s / (float)hw;
    }
}

/* src/exec_cpu.rs:580-598. */
void oracle_chan_scale(const float *x, const float *s, float *y, int64_t c, int64_t hw) {
#pragma omp parallel for schedule(static)
    for (int64_t ch = 0; ch < c; ++ch) {
        const float sc = s[ch];
        for (int64_t p = 0; p < hw; ++p) y[ch * hw + p] = x[ch * hw + p] * sc;
    }
}

/* --------------------------------------------------------------- convs */

/* Conv1x1 / Dense, src/exec_cpu.rs:602-690: a PB-pixel tile of every input
 * channel staged once, every output channel from it; each output starts at its
 * bias and adds ic ascending. w is [co][ci]. */
void oracle_conv1x1(const float *x, const float *w, const float *bias, float *y, int64_t ci, int64_t co, int64_t plane) {
    int64_t ntile = (plane + PB - 1) / PB;
#pragma omp parallel
    {
        float *tile = (float *)malloc(sizeof(float) * PB * (size_t)(ci > 0 ? ci : 1));
        float acc[PB];
#pragma omp for schedule(static)
        for (int64_t t = 0; t < ntile; ++t) {
            int64_t p0 = t * PB;
            int64_t np = plane - p0 < PB ? plane - p0 : PB;
            for (int64_t ic = 0; ic < ci; ++ic) memcpy(tile + ic * PB, x + ic * plane + p0, sizeof(float) * np);
            for (int64_t oc = 0; oc < co; ++oc) {
                const float *wp = w + oc * ci;
                float bv = bias ? bias[oc] : 0.0f;
                for (int64_t p = 0; p < np; ++p) acc[p] = bv;
                for (int64_t ic = 0; ic < ci; ++ic) {
                    const float wv = wp[ic];
                    const float *ti = tile + ic * PB;
                    for (int64_t p = 0; p < np; ++p) acc[p] += wv * ti[p];
                }
                memcpy(y + oc * plane + p0, acc, sizeof(float) * np);
            }
        }
        free(tile);
    }
}

/* Conv3x3 pad 1, src/exec_cpu.rs:694-771: one output row at a time in a
 * (wd + 2) buffer seeded with the bias, taps added in (ky, kx, ic) order and
 * out-of-range rows skipped. w is [co][ci][3][3]. */
void oracle_conv3x3(const float *x, const float *w, const float *bias, float *y, int64_t ci, int64_t co, int64_t h, int64_t wd) {
    const int64_t plane = h * wd;
#pragma omp parallel
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)(wd + 2));
#pragma omp for schedule(static) collapse(2)
        for (int64_t oc = 0; oc < co; ++oc) {
            for (int64_t yy = 0; yy < h; ++yy) {
                const float bv = bias ? bias[oc] : 0.0f;
                const float *wp = w + oc * ci * 9;
                for (int64_t i = 0; i < wd + 2; ++i) row[i] = bv;
                for (int ky = 0; ky < 3; ++ky) {
                    int64_t iy = yy + ky - 1;
                    if (iy < 0 || iy >= h) continue;
                    for (int kx = 0; kx < 3; ++kx) {
                        const int shift = 2 - kx;
                        for (int64_t ic = 0; ic < ci; ++ic) {
                            const float wv = wp[ic * 9 + ky * 3 + kx];
                            const float *srow = x + ic * plane + iy * wd;
                            float *r = row + shift;
                            for (int64_t i = 0; i < wd; ++i) r[i] += wv * srow[i];
                        }
                    }
                }
                memcpy(y + oc * plane + yy * wd, row + 1, sizeof(float) * wd);
            }
        }
        free(row);
    }
}

/* floor division for the conv4x4s2 column bounds (Rust's div_euclid by 2). */
static int64_t div_floor2(int64_t a) { return a >= 0 ? a / 2 : -((-a + 1) / 2); }

/* Conv4x4 stride 2 SAME, src/exec_cpu.rs:772-845: output row accumulator from
 * the bias, (ky, kx, ic) order, the sweep clamped to columns whose input is in
 * range. w is [co][ci][4][4]. */
void oracle_conv4x4s2(const float *x, const float *w, const float *bias, float *y, int64_t ci, int64_t co,
                      int64_t h, int64_t wd, int64_t pad_top, int64_t pad_left, int64_t oh, int64_t ow) {
    const int64_t plane = h * wd, oplane = oh * ow;
#pragma omp parallel
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)(ow > 0 ? ow : 1));
#pragma omp for schedule(static) collapse(2)
        for (int64_t oc = 0; oc < co; ++oc) {
            for (int64_t oy = 0; oy < oh; ++oy) {
                const float bv = bias ? bias[oc] : 0.0f;
                const float *wp = w + oc * ci * 16;
                for (int64_t i = 0; i < ow; ++i) acc[i] = bv;
                for (int64_t ky = 0; ky < 4; ++ky) {
                    int64_t iy = oy * 2 + ky;
                    if (iy < pad_top || iy - pad_top >= h) continue;
                    iy -= pad_top;
                    for (int64_t kx = 0; kx < 4; ++kx) {
                        int64_t lo = div_floor2(pad_left - kx + 1);
                        if (lo < 0) lo = 0;
                        int64_t hi = div_floor2(wd - 1 + pad_left - kx) + 1;
                        if (hi < 0) hi = 0;
                        if (hi > ow) hi = ow;
                        for (int64_t ic = 0; ic < ci; ++ic) {
                            const float wv = wp[ic * 16 + ky * 4 + kx];
                            const float *srow = x + ic * plane + iy * wd;
                            for (int64_t ox = lo; ox < hi; ++ox) acc[ox] += wv * srow[ox * 2 + kx - pad_left];
                        }
                    }
                }
                memcpy(y + oc * oplane + oy * ow, acc, sizeof(float) * ow);
            }
        }
        free(acc);
    }
}

/* ConvT 2x2 stride 2, src/exec_cpu.rs:846-914: four tap accumulators from zero
 * over ascending ic, then bias + tap. w is [ci][co][2][2], spatially flipped. */
void oracle_convt2x2(const float *x, const float *w, const float *bias, float *y, int64_t ci, int64_t co, int64_t h, int64_t wd) {
    const int64_t plane = h * wd, ow = 2 * wd, oplane = 4 * plane;
#pragma omp parallel
    {
        float *a = (float *)malloc(sizeof(float) * 4 * (size_t)(wd > 0 ? wd : 1));
        float *a0 = a, *a1 = a + wd, *a2 = a + 2 * wd, *a3 = a + 3 * wd;
#pragma omp for schedule(static) collapse(2)
        for (int64_t oc = 0; oc < co; ++oc) {
            for (int64_t yy = 0; yy < h; ++yy) {
                const float bv = bias ? bias[oc] : 0.0f;
                memset(a, 0, sizeof(float) * 4 * wd);
                for (int64_t ic = 0; ic < ci; ++ic) {
                    const float *srow = x + ic * plane + yy * wd;
                    const float *wb = w + (ic * co + oc) * 4;
                    for (int64_t i = 0; i < wd; ++i) {
                        float v = srow[i];
                        a0[i] += wb[0] * v;
                        a1[i] += wb[1] * v;
                        a2[i] += wb[2] * v;
                        a3[i] += wb[3] * v;
                    }
                }
                float *r0 = y + oc * oplane + 2 * yy * ow, *r1 = r0 + ow;
                for (int64_t i = 0; i < wd; ++i) {
                    r0[2 * i] = bv + a0[i];
                    r0[2 * i + 1] = bv + a1[i];
                    r1[2 * i] = bv + a2[i];
                    r1[2 * i + 1] = bv + a3[i];
                }
            }
        }
        free(a);
    }
}

/* The gating matmul, src/exec_cpu.rs:915-1074. mode 0 reduces over `outer`:
 * out[c][r][b] = bias[r] + sum_t w[r][t] x[c][t][b]; mode 1 over `inner`:
 * out[c][b][a] = bias[a] + sum_t w[a][t] x[c][b][t]; t ascending. */
void oracle_gate_mm(const float *x, const float *w, const float *bias, float *y, int64_t c, int64_t outer, int64_t inner, int mode) {
    const int64_t pl = outer * inner;
    if (mode == 0) {
#pragma omp parallel for schedule(static) collapse(2)
        for (int64_t ch = 0; ch < c; ++ch) {
            for (int64_t r = 0; r < outer; ++r) {
                const float *xc = x + ch * pl;
                float *row = y + ch * pl + r * inner;
                const float bv = bias ? bias[r] : 0.0f;
                for (int64_t b = 0; b < inner; ++b) row[b] = bv;
                for (int64_t t = 0; t < outer; ++t) {
                    const float wv = w[r * outer + t];
                    const float *xr = xc + t * inner;
                    for (int64_t b = 0; b < inner; ++b) row[b] += wv * xr[b];
                }
            }
        }
    } else {
#pragma omp parallel for schedule(static) collapse(2)
        for (int64_t ch = 0; ch < c; ++ch) {
            for (int64_t b = 0; b < outer; ++b) {
                const float *xb = x + ch * pl + b * inner;
                float *yb = y + ch * pl + b * inner;
                for (int64_t a = 0; a < inner; ++a) {
                    const float *wa = w + a * inner;
                    float acc = bias ? bias[a] : 0.0f;
                    for (int64_t t = 0; t < inner; ++t) acc += wa[t] * xb[t];
                    yb[a] = acc;
                }
            }
        }
    }
}

/* ---------------------------------------------------------- index maps */

/* src/exec_cpu.rs:1075-1101: g = gy*gw + gx, p = fy*fw + fx, pixel
 * (gy*fh + fy, gx*fw + fx); forward gathers into the blocked layout. */
void oracle_block_perm(const float *x, float *y, int64_t c, int64_t h, int64_t wd, int64_t gh, int64_t gw,
                       int64_t fh, int64_t fw, int swap, int forward) {
    const int64_t gsz = gh * gw, psz = fh * fw, plane = h * wd;
#pragma omp parallel for schedule(static)
    for (int64_t ch = 0; ch < c; ++ch) {
        const float *pl = x + ch * plane;
        float *dl = y + ch * plane;
        for (int64_t gy = 0; gy < gh; ++gy)
            for (int64_t gx = 0; gx < gw; ++gx) {
                int64_t g = gy * gw + gx;
                for (int64_t fy = 0; fy < fh; ++fy)
                    for (int64_t fx = 0; fx < fw; ++fx) {
                        int64_t p = fy * fw + fx;
                        int64_t pix = (gy * fh + fy) * wd + gx * fw + fx;
                        int64_t blk = swap ? p * gsz + g : g * psz + p;
                        if (forward) dl[blk] = pl[pix];
                        else dl[pix] = pl[blk];
                    }
            }
    }
}

/* src/exec_cpu.rs:1102-1116: out[y][x] = in[y*stride + off][x*stride + off]. */
void oracle_down_s(const float *x, float *y, int64_t c, int64_t h, int64_t wd, int64_t stride, int64_t off, int64_t oh, int64_t ow) {
    for (int64_t ch = 0; ch < c; ++ch)
        for (int64_t yy = 0; yy < oh; ++yy)
            for (int64_t xx = 0; xx < ow; ++xx)
                y[ch * oh * ow + yy * ow + xx] = x[ch * h * wd + (yy * stride + off) * wd + xx * stride + off];
}

/* ------------------------------------------------------------- resize */

/* ResizeTaps::new, src/exec_cpu.rs:1195-1216, in fp32 exactly as written:
 * sample = (o + 0.5) * inv - 0.5, taps j in [ceil(s - k), floor(s + k)] clamped
 * to [0, n_in - 1], kept while |s - j| / k < 1 with weight 1 - d. */
int64_t oracle_resize_taps(int64_t n_in, int64_t n_out, int32_t *j0s, int32_t *ntap, float *wsum, float *wts) {
    const float inv = (float)n_in / (float)n_out;
    const float kscale = inv > 1.0f ? inv : 1.0f;
    int64_t total = 0;
    for (int64_t o = 0; o < n_out; ++o) {
        const float sample = ((float)o + 0.5f) * inv - 0.5f;
        int64_t j0 = (int64_t)ceilf(sample - kscale);
        int64_t j1 = (int64_t)floorf(sample + kscale);
        if (j0 < 0) j0 = 0;
        if (j1 > n_in - 1) j1 = n_in - 1;
        float s = 0.0f;
        int32_t k = 0;
        for (int64_t j = j0; j <= j1; ++j) {
            float d = fabsf(sample - (float)j) / kscale;
            if (d < 1.0f) {
                float wv = 1.0f - d;
                if (k < MAX_TAPS) wts[o * MAX_TAPS + k] = wv;
                ++k;
                s += wv;
            }
        }
        j0s[o] = (int32_t)j0;
        ntap[o] = k < MAX_TAPS ? k : MAX_TAPS;
        wsum[o] = s;
        total += k;
    }
    return total;
}

/* Two passes, horizontal into tmp [c][hin][wout], then vertical; each output
 * is sum_k w_k * src_{j0 + k} in ascending k, divided by the weight sum when
 * that is positive (src/exec_cpu.rs:1143-1178, 1230-1292). */
void oracle_resize(const float *x, float *tmp, float *y, int64_t c, int64_t hin, int64_t win, int64_t hout, int64_t wout) {
    int32_t *xj = (int32_t *)malloc(sizeof(int32_t) * 2 * (size_t)wout);
    float *xs = (float *)malloc(sizeof(float) * (size_t)wout);
    float *xw = (float *)malloc(sizeof(float) * MAX_TAPS * (size_t)wout);
    int32_t *yj = (int32_t *)malloc(sizeof(int32_t) * 2 * (size_t)hout);
    float *ys = (float *)malloc(sizeof(float) * (size_t)hout);
    float *yw = (float *)malloc(sizeof(float) * MAX_TAPS * (size_t)hout);
    oracle_resize_taps(win, wout, xj, xj + wout, xs, xw);
    oracle_resize_taps(hin, hout, yj, yj + hout, ys, yw);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < c * hin; ++r) {
        const float *sr = x + r * win;
        float *dr = tmp + r * wout;
        for (int64_t o = 0; o < wout; ++o) {
            const float *wv = xw + o * MAX_TAPS;
            const float *s = sr + xj[o];
            float acc = 0.0f;
            for (int32_t k = 0; k < xj[wout + o]; ++k) acc += wv[k] * s[k];
            dr[o] = xs[o] > 0.0f ? acc / xs[o] : acc;
        }
    }
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < c * hout; ++r) {
        int64_t ch = r / hout, o = r % hout;
        const float *pl = tmp + ch * hin * wout;
        float *dr = y + r * wout;
        const float *wv = yw + o * MAX_TAPS;
        const int32_t n = yj[hout + o], j0 = yj[o];
        const float s = ys[o];
        for (int64_t xx = 0; xx < wout; ++xx) {
            float acc = 0.0f;
            for (int32_t k = 0; k < n; ++k) acc += wv[k] * pl[(j0 + k) * wout + xx];
            dr[xx] = s > 0.0f ? acc / s : acc;
        }
    }
    free(xj); free(xs); free(xw); free(yj); free(ys); free(yw);
}

/* ------------------------------------------------------------ the loop */

static int step_op(const mx_plan_desc *P, float *A, const mx_op *op) {
#define BUF(id) (A + P->offs[(id)])
#define WT(id) ((id) >= 0 ? P->weights[(id)] : (const float *)0)
    switch (op->kind) {
        case MX_OP_COPY:
            memmove(BUF(op->dst), BUF(op->src), sizeof(float) * (size_t)op->n);
            break;
        case MX_OP_ADD: oracle_add(BUF(op->src), BUF(op->src2), BUF(op->dst), op->n); break;
        case MX_OP_MUL: oracle_mul(BUF(op->src), BUF(op->src2), BUF(op->dst), op->n); break;
        case MX_OP_GATE_APPLY: oracle_gate_apply(BUF(op->src), BUF(op->src2), BUF(op->dst), op->n); break;
        case MX_OP_GELU: oracle_gelu(BUF(op->src), BUF(op->dst), op->n); break;
        case MX_OP_LRELU: oracle_lrelu(BUF(op->src), BUF(op->dst), op->n, op->slope); break;
        case MX_OP_SIGMOID: oracle_sigmoid(BUF(op->src), BUF(op->dst), op->n); break;
        case MX_OP_CHAN_LN:
            oracle_chan_ln(BUF(op->src), WT(op->scale), WT(op->bias), BUF(op->dst), op->c, op->hw);
            break;
        case MX_OP_CHAN_MEAN: oracle_chan_mean(BUF(op->src), BUF(op->dst), op->c, op->hw); break;
        case MX_OP_CHAN_SCALE: oracle_chan_scale(BUF(op->src), BUF(op->src2), BUF(op->dst), op->c, op->hw); break;
        case MX_OP_CONV1X1:
            oracle_conv1x1(BUF(op->src), WT(op->w), WT(op->bias), BUF(op->dst), op->c_in, op->c_out, op->h * op->wd);
            break;
        case MX_OP_CONV3X3:
            oracle_conv3x3(BUF(op->src), WT(op->w), WT(op->bias), BUF(op->dst), op->c_in, op->c_out, op->h, op->wd);
            break;
        case MX_OP_CONV4X4S2:
            oracle_conv4x4s2(BUF(op->src), WT(op->w), WT(op->bias), BUF(op->dst), op->c_in, op->c_out, op->h, op->wd,
                             op->p[0], op->p[1], op->oh, op->ow);
            break;
        case MX_OP_CONVT2X2:
            oracle_convt2x2(BUF(op->src), WT(op->w), WT(op->bias), BUF(op->dst), op->c_in, op->c_out, op->h, op->wd);
            break;
        case MX_OP_GATE_MM:
            oracle_gate_mm(BUF(op->src), WT(op->w), WT(op->bias), BUF(op->dst), op->c, op->p[0], op->p[1], op->mode);
            break;
        case MX_OP_BLOCK_PERM:
            oracle_block_perm(BUF(op->src), BUF(op->dst), op->c, op->h, op->wd, op->p[0], op->p[1], op->p[2], op->p[3],
                              (op->mode & MX_PERM_SWAP) != 0, (op->mode & MX_PERM_FORWARD) != 0);
            break;
        case MX_OP_RESIZE:
            oracle_resize(BUF(op->src), BUF(op->src2), BUF(op->dst), op->c, op->h, op->wd, op->oh, op->ow);
            break;
        case MX_OP_DOWN_S:
            oracle_down_s(BUF(op->src), BUF(op->dst), op->c, op->h, op->wd, op->p[0], op->p[1], op->oh, op->ow);
            break;
        default:
            return -1;
    }
    return 0;
#undef BUF
#undef WT
}

int oracle_run_range(const mx_plan_desc *plan, float *arena, uint64_t first, uint64_t last, int threads) {
    int saved = omp_get_max_threads();
    if (threads > 0) omp_set_num_threads(threads);
    g_threads_used = omp_get_max_threads();
    int rc = 0;
    for (uint64_t i = first; i < last && i < plan->n_ops && rc == 0; ++i) rc = step_op(plan, arena, &plan->ops[i]);
    omp_set_num_threads(saved);
    return rc;
}

int oracle_run(const mx_plan_desc *plan, float *arena, int threads) {
    return oracle_run_range(plan, arena, 0, plan->n_ops, threads);
}

int oracle_step(const mx_plan_desc *plan, float *arena, uint64_t i, int threads) {
    return oracle_run_range(plan, arena, i, i + 1, threads);
}
