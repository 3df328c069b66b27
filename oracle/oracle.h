/*
 * oracle.h - TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU executor (src/exec_cpu.rs),
 * used as the checker for the HIP executor and as the reported CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product library never links it and never falls back to it.
 *
 * Every arm keeps the reference's order of operations per output element (no
 * FMA contraction, ascending reductions, bias first except where the reference
 * adds it last), so its results are the reference CPU path's results to the
 * bit, up to the two functions it takes from libm (erff, expf) - see the
 * parity notes in oracle/exec_cpu.c.
 */
#ifndef MAXIM_ORACLE_H
#define MAXIM_ORACLE_H

#include <stdint.h>

#include "../include/maxim_plan.h"

#ifdef __cplusplus
extern "C" {
#endif

/* exec_cpu::run (src/exec_cpu.rs:60-102): every op in order; `threads` <= 0 = all cores. */
int oracle_run(const mx_plan_desc *plan, float *arena, int threads);
/* exec_cpu::step (src/exec_cpu.rs:48-51): op `i` only. */
int oracle_step(const mx_plan_desc *plan, float *arena, uint64_t i, int threads);
/* Ops [first, last) in order. */
int oracle_run_range(const mx_plan_desc *plan, float *arena, uint64_t first, uint64_t last, int threads);
/* The number of threads the last call used. */
int oracle_threads_used(void);

/* The arms, on plain pointers (for the per-op tests). */
void oracle_add(const float *a, const float *b, float *y, int64_t n);
void oracle_mul(const float *a, const float *b, float *y, int64_t n);
void oracle_gate_apply(const float *u, const float *v, float *y, int64_t n);
void oracle_gelu(const float *x, float *y, int64_t n);
void oracle_lrelu(const float *x, float *y, int64_t n, float slope);
void oracle_sigmoid(const float *x, float *y, int64_t n);
void oracle_chan_ln(const float *x, const float *scale, const float *bias, float *y, int64_t c, int64_t hw);
void oracle_chan_mean(const float *x, float *y, int64_t c, int64_t hw);
void oracle_chan_scale(const float *x, const float *s, float *y, int64_t c, int64_t hw);
void oracle_conv1x1(const float *x, const float *w, const float *bias, float *y, int64_t ci, int64_t co, int64_t plane);
void oracle_conv3x3(const float *x, const float *w, const float *bias, float *y, int64_t ci, int64_t co, int64_t h, int64_t wd);
void oracle_conv4x4s2(const float *x, const float *w, const float *bias, float *y, int64_t ci, int64_t co,
                      int64_t h, int64_t wd, int64_t pad_top, int64_t pad_left, int64_t oh, int64_t ow);
void oracle_convt2x2(const float *x, const float *w, const float *bias, float *y, int64_t ci, int64_t co, int64_t h, int64_t wd);
void oracle_gate_mm(const float *x, const float *w, const float *bias, float *y, int64_t c, int64_t outer, int64_t inner, int mode);
void oracle_block_perm(const float *x, float *y, int64_t c, int64_t h, int64_t wd, int64_t gh, int64_t gw,
                       int64_t fh, int64_t fw, int swap, int forward);
void oracle_resize(const float *x, float *tmp, float *y, int64_t c, int64_t hin, int64_t win, int64_t hout, int64_t wout);
void oracle_down_s(const float *x, float *y, int64_t c, int64_t h, int64_t wd, int64_t stride, int64_t off, int64_t oh, int64_t ow);
/* The resize tap table of one axis (ResizeTaps::new, src/exec_cpu.rs:1195-1216):
 * per output, first input index, tap count and weight sum, weights in `wts`
 * (room for n_out * 64). Returns the total number of weights. */
int64_t oracle_resize_taps(int64_t n_in, int64_t n_out, int32_t *j0, int32_t *ntap, float *wsum, float *wts);

#ifdef __cplusplus
}
#endif

#endif
