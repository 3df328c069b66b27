/*
 * maxim_hip.h - the MI355X (gfx950) executor for a MAXIM plan.
 *
 * The C-ABI form of the reference's GPU executor, `exec_gpu::Gpu`
 * (src/exec_gpu.rs:48-357), standing beside it as a third executor behind the
 * same plan/arena/weights interface (maxim_plan.h's `mx_plan_desc`). The HIP
 * runtime is dlopen'd (`libamdhip64.so`), the way src/cuda.rs reaches
 * libcuda through lightgpu; the gfx950 code object is embedded in this
 * library and loaded with hipModuleLoadData.
 *
 * Ownership: the executor owns exactly one device arena of `arena_len` floats
 * and a device copy of the weights (uploaded eagerly by mxh_new, in the
 * layouts its kernels read). Plans and host buffers are borrowed per call.
 * The arena is NOT zeroed: every buffer is written before it is read.
 * Errors: negative status / NULL, message in mx_last_error() (thread-local).
 * Threading: one executor per thread; launches are asynchronous on the
 * executor's own stream and every call that returns host data synchronises.
 */
#ifndef MAXIM_HIP_H
#define MAXIM_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "maxim_plan.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mxh_gpu mxh_gpu;

/* exec_gpu::driver_ready (src/exec_gpu.rs:81-83): dlopen the HIP runtime and
 * bring device 0 up. The only failure that lets a caller choose another
 * backend; anything after this is reported, never retried elsewhere. */
int mxh_driver_ready(void);

/* Gpu::new (src/exec_gpu.rs:96-160): load the kernels, size the pass against
 * free device memory and REFUSE (with the numbers) if arena + weights do not
 * fit, then allocate the arena and upload the weights. */
mxh_gpu *mxh_new(const mx_plan_desc *plan);
void mxh_free(mxh_gpu *g);

/* Gpu::run (src/exec_gpu.rs:196-229): input in, every op, output out. */
int mxh_run(mxh_gpu *g, const mx_plan_desc *plan, const float *input, uint64_t n_in, float *output,
            uint64_t n_out);
/* Gpu::begin (src/exec_gpu.rs:329-344): place the input image in the arena. */
int mxh_begin(mxh_gpu *g, const mx_plan_desc *plan, const float *input, uint64_t n_in);
/* Gpu::step_op (src/exec_gpu.rs:348-352): execute exactly op `i`. */
int mxh_step_op(mxh_gpu *g, const mx_plan_desc *plan, uint64_t i);
/* No counterpart in the reference (one image per run): `n_images` images
 * through the same plan for a serving loop, each image's pass exactly
 * mxh_run's (so each output is mxh_run's to the bit), with the host's work
 * off the device's path: image k's input is staged into pinned memory while
 * pass k - 1 runs and image k - 1's output handed back while pass k runs, so
 * the device only adds the two DMA copies per image. inputs[k] (n_in floats)
 * and outputs[k] (n_out floats) are host arrays; every output is written
 * when the call returns. The staging (two pinned buffers each way and their
 * events) is allocated on the first call and kept with the executor. Not
 * with the timeline on. */
int mxh_run_batch(mxh_gpu *g, const mx_plan_desc *plan, const float *const *inputs, uint64_t n_in,
                  float *const *outputs, uint64_t n_out, uint64_t n_images);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). mxh_run's pass with device-resident input and output
 * (d_input, d_output: device pointers of n_in / n_out floats) that allocates
 * nothing: the executor's arena and weights (allocated once by mxh_new) hold
 * the pass, and the kernels' scratch (channel-mean partial sums, LayerNorm
 * statistics) is the code object's static array of 32 MiB per device, in
 * place of the per-executor scratch mxh_run uses. A plan whose scratch needs
 * more (e.g. 4096x4096) is refused with the numbers. Asynchronous, in stream
 * order on `stream` (a hipStream_t; NULL: the executor's own stream, which
 * mxh_sync waits for): the input copy, every kernel and the output copy are
 * queued there after whatever the caller queued before, so d_input must be
 * complete by then in that stream's order, d_output holds the result once
 * the stream has passed the call, and a caller capturing `stream` into a HIP
 * graph captures the whole pass (two device-to-device copies and kernel
 * nodes; no memsets). Every call on a device shares that device's array:
 * calls that overlap on one device (on different streams, or executors on
 * their own streams) race, so let one finish before another starts. Every
 * pass writes the scratch before reading it, so nothing needs clearing. */
int mxh_run_noalloc(mxh_gpu *g, const mx_plan_desc *plan, const float *d_input, uint64_t n_in, float *d_output,
                    uint64_t n_out, void *stream);
/* Every op over the image already in the arena as ONE captured HIP graph
 * (captured on the first call, replayed after), asynchronously. The graph
 * launches exactly the kernels mxh_run_ops would, in the same order. */
int mxh_run_graph(mxh_gpu *g, const mx_plan_desc *plan);
/* Make mxh_run replay the captured graph instead of launching op by op. */
void mxh_set_graph(mxh_gpu *g, int on);
/* Fusion (on by default) runs mxh_run / mxh_run_ops / mxh_run_graph through
 * the fused program: a producer whose output has one reader applies that
 * reader in its epilogue (GEMM + GELU, GEMM + residual add(s), gate Dense +
 * gate multiply, GEMM into a concatenation slot, 3x3 conv + leaky ReLU). The
 * fused epilogue performs the same float operations in the same order, so
 * results are bitwise those of the unfused launches. mxh_step_op never fuses. */
void mxh_set_fusion(mxh_gpu *g, int on);
/* The same decisions without a device: how many ops fuse away, the device
 * arena length and every buffer's device offset (n_bufs entries), and the
 * steps' op ranges (room for n_ops entries each). `repack` = 0 keeps the
 * plan's own layout. */
int mxh_plan_program(const mx_plan_desc *plan, int repack, uint64_t *fused_ops, uint64_t *arena_len,
                     uint64_t *offs, uint64_t *step_first, uint64_t *step_last, uint64_t *n_steps);
/* Which buffer owns each buffer's storage in that device layout (n_bufs
 * entries): a view's base, the buffer itself, or - for the source of a copy
 * the executor elides - the copy destination's owner. */
int mxh_plan_storage(const mx_plan_desc *plan, int repack, int64_t *owner);
uint64_t mxh_fused_ops(mxh_gpu *g);
uint64_t mxh_steps(mxh_gpu *g);
int mxh_step_info(mxh_gpu *g, uint64_t i, uint64_t *first, uint64_t *last, const char **kernel);
/* All ops [first, last) in order, asynchronously (no host synchronisation). */
int mxh_run_ops(mxh_gpu *g, const mx_plan_desc *plan, uint64_t first, uint64_t last);
/* Gpu::read_buf (src/exec_gpu.rs:354-357): one buffer back to the host. */
int mxh_read_buf(mxh_gpu *g, const mx_plan_desc *plan, uint64_t buf, float *out, uint64_t n);
/* One buffer from the host (Gpu::write_at, src/exec_gpu.rs:275-282, by
 * buffer id): the per-op parity walk uses it to give an op exactly the CPU
 * path's inputs. */
int mxh_write_buf(mxh_gpu *g, const mx_plan_desc *plan, uint64_t buf, const float *in, uint64_t n);
/* The device arena: where buffer `buf` lives in it (elements). This is the
 * plan's own offset unless the executor laid the arena out by fused steps
 * (the plan supplied its view table); mxh_arena_bytes is its size. */
uint64_t mxh_buf_offset(mxh_gpu *g, uint64_t buf);
/* Gpu::read_into / read_arena (src/exec_gpu.rs:295-305): `n` floats from
 * device-arena element `off` (mxh_buf_offset), and the whole device arena. */
int mxh_read_into(mxh_gpu *g, uint64_t off, float *out, uint64_t n);
int mxh_read_arena(mxh_gpu *g, float *out, uint64_t n);
/* `n` floats to device-arena element `off`. */
int mxh_write_into(mxh_gpu *g, uint64_t off, const float *in, uint64_t n);
/* MAXIM_POISON (src/exec_gpu.rs:320-340): fill the whole arena, and the
 * executor's scratch (partial sums, LayerNorm statistics), with 0xCD bytes. */
int mxh_poison(mxh_gpu *g);
/* Wait for all queued work. */
int mxh_sync(mxh_gpu *g);

/* Gpu::set_timeline / timeline (src/exec_gpu.rs:185-194, 241-265): with the
 * timeline on, mxh_run records one HIP event per step and reports per-step
 * device milliseconds, synchronising once at the end. A step is one op, or -
 * with fusion on - one fused launch standing for several ops (mxh_step_info);
 * with fusion off there is one step per op. */
void mxh_set_timeline(mxh_gpu *g, int on);
int mxh_timeline(mxh_gpu *g, float *per_step_ms, uint64_t n, float *total_ms);
/* Gpu::run_timed (src/exec_gpu.rs:241-265) without the copies: every op over
 * the image already in the arena, every launch timed by its dispatch, one
 * synchronisation. */
int mxh_run_timed(mxh_gpu *g, const mx_plan_desc *plan);

/* The launches of the current program (fused steps with fusion on, ops
 * with it off), in order: how many, each one's step (or op) and kernel, and -
 * after mxh_run_timed - each one's device milliseconds, from the start/stop
 * events the dispatch itself records (hipExtModuleLaunchKernel: the kernel's
 * execution, not the gap before it). A step's entry in mxh_timeline is the
 * sum over its launches. */
uint64_t mxh_launches(mxh_gpu *g);
int mxh_launch_info(mxh_gpu *g, uint64_t i, uint64_t *step, const char **kernel);
/* The ops launch i computes: ops[0..1] the first range [first, last), and
 * for a launch that runs two steps' work side by side (a step pairing the
 * grid and block branches of a multi-axis gMLP block) ops[2..3] the second,
 * else 0, 0. No counterpart in the reference (one launch per op there); it
 * lets a profile charge each launch its own ops. */
int mxh_launch_span(mxh_gpu *g, uint64_t i, uint64_t ops[4]);
int mxh_launch_timeline(mxh_gpu *g, float *ms, uint64_t n);

/* Time `iters` passes of ops [first, last) back to back with HIP events on
 * the executor's stream; `ms` gets the total device time. */
int mxh_time_ops(mxh_gpu *g, const mx_plan_desc *plan, uint64_t first, uint64_t last, int iters,
                 float *ms);

/* `n` passes over the image already in the arena, each one replay of the
 * captured graph (mxh_run_graph) bracketed by its own pair of HIP events on
 * the executor's stream, back to back, one synchronisation at the end;
 * ms[k] gets pass k's device milliseconds. No counterpart in the reference:
 * the per-pass times a median is taken over. */
int mxh_time_graph(mxh_gpu *g, const mx_plan_desc *plan, int n, float *ms);

/* Gpu::device_name / arena_bytes / weight_bytes / pool_bytes / ops_launched
 * (src/exec_gpu.rs:165-183). kernels_launched counts launches (one op may be
 * several, e.g. the two resize passes). */
const char *mxh_device_name(mxh_gpu *g);
uint64_t mxh_arena_bytes(mxh_gpu *g);
uint64_t mxh_weight_bytes(mxh_gpu *g);
uint64_t mxh_pool_bytes(mxh_gpu *g);
uint64_t mxh_ops_launched(mxh_gpu *g);
uint64_t mxh_kernels_launched(mxh_gpu *g);
/* The name of the first kernel op `i` launches (for per-kernel reports). */
const char *mxh_op_kernel(mxh_gpu *g, uint64_t i);
/* Device facts for the roofline: compute units and peak engine clock (kHz). */
int mxh_device_info(mxh_gpu *g, int *cus, int *clock_khz);
/* The enhancement run with the HIP backend, what a `--device hip` arm of the
 * reference's CLI calls between reading and writing the PNG (src/main.rs
 * 173-458): open the safetensors checkpoint (variant from the file), pad the
 * [3][h][w] image (0..1) by the reference pipeline to a multiple of 64, build
 * the release plan, run it on the device (refusing up front if it does not
 * fit), and crop the prediction back to [3][h][w] in `out`. */
int mxh_enhance(const char *checkpoint, const float *image, int64_t h, int64_t w, float *out);
/* Free and total device memory (bytes) of device 0, what Gpu::new sizes its
 * refusal against (lightgpu `free_vram`, src/exec_gpu.rs:86-146). */
int mxh_device_memory(uint64_t *free_bytes, uint64_t *total_bytes);

#ifdef __cplusplus
}
#endif

#endif /* MAXIM_HIP_H */
