// Bandwidth-bound kernels: the flat elementwise family, the channel-axis ops
// (LayerNorm, mean, scale) and the index maps (block permutation, nearest
// subsample, bilinear resize).
//
// Arithmetic follows the reference's CPU arms term for term (src/exec_cpu.rs
// 537-598, 377-434, 1075-1178) and this file is compiled without FP
// contraction, so add / mul / gate / lrelu / chan_scale / chan_ln /
// block_perm / down_s / resize reproduce the CPU path bit for bit; sigmoid
// differs from it through its hardware exp2 and reciprocal, gelu through its
// fitted exponent (common.h: within 1.3e-7 and 6.3e-8 * (1 + |x|) of the
// exact functions).
#pragma once

#include "common.h"

// ------------------------------------------------------------ elementwise

template <int OP>
__device__ __forceinline__ float ew1(float a, float b, float slope) {
    if (OP == MXK_COPY) return a;
    if (OP == MXK_ADD) return a + b;
    if (OP == MXK_MUL) return a * b;
    if (OP == MXK_GATE_APPLY) return a * (b + 1.0f);
    if (OP == MXK_GELU) return gelu(a);
    if (OP == MXK_LRELU) return a >= 0.0f ? a : slope * a;
    return sigmoid(a);  // MXK_SIGMOID
}

// Each thread moves UNROLL float4s spaced one block apart, so every load of a
// wave is one contiguous 1 KiB run.
template <int OP, int UNROLL>
__device__ void ew_vec4(const EwArgs &a) {
    const int64_t nv = a.n >> 2;
    int64_t i = (int64_t)blockIdx.x * (MXK_BLOCK * UNROLL) + threadIdx.x;
    float4 va[UNROLL], vb[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
        int64_t j = i + u * MXK_BLOCK;
        if (j < nv) {
            va[u] = ld4(a.a + 4 * j);
            if (OP == MXK_ADD || OP == MXK_MUL || OP == MXK_GATE_APPLY) vb[u] = ld4(a.b + 4 * j);
        }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
        int64_t j = i + u * MXK_BLOCK;
        if (j < nv) {
            float4 r;
            r.x = ew1<OP>(va[u].x, vb[u].x, a.slope);
            r.y = ew1<OP>(va[u].y, vb[u].y, a.slope);
            r.z = ew1<OP>(va[u].z, vb[u].z, a.slope);
            r.w = ew1<OP>(va[u].w, vb[u].w, a.slope);
            st4(a.y + 4 * j, r);
        }
    }
}

template <int OP>
__device__ void ew_scalar(const EwArgs &a) {
    int64_t i = (int64_t)blockIdx.x * MXK_BLOCK + threadIdx.x;
    if (i < a.n) a.y[i] = ew1<OP>(a.a[i], (OP == MXK_ADD || OP == MXK_MUL || OP == MXK_GATE_APPLY) ? a.b[i] : 0.0f, a.slope);
}

#define MXK_EW(NAME, OP)                                                                     \
    extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_##NAME##_v4(EwArgs a) {      \
        ew_vec4<OP, 4>(a);                                                                   \
    }                                                                                        \
    extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_##NAME##_s(EwArgs a) { ew_scalar<OP>(a); }

MXK_EW(copy, MXK_COPY)
MXK_EW(add, MXK_ADD)
MXK_EW(mul, MXK_MUL)
MXK_EW(gate_apply, MXK_GATE_APPLY)
MXK_EW(gelu, MXK_GELU)
MXK_EW(lrelu, MXK_LRELU)
MXK_EW(sigmoid, MXK_SIGMOID)

// y[ch][p] = x[ch][p] * s[ch]; grid (ceil(hw / (256 * 4 * V)), c).
extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_scale_v4(ChanScaleArgs a) {
    const int64_t ch = blockIdx.y;
    const float s = a.s[ch];
    const float *x = a.x + ch * a.hw;
    float *y = a.y + ch * a.hw;
    const int64_t nv = a.hw >> 2;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        int64_t j = (int64_t)blockIdx.x * (MXK_BLOCK * 4) + u * MXK_BLOCK + threadIdx.x;
        if (j < nv) {
            float4 v = ld4(x + 4 * j);
            v.x = v.x * s; v.y = v.y * s; v.z = v.z * s; v.w = v.w * s;
            st4(y + 4 * j, v);
        }
    }
}

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_scale_s(ChanScaleArgs a) {
    const int64_t ch = blockIdx.y;
    int64_t p = (int64_t)blockIdx.x * MXK_BLOCK + threadIdx.x;
    if (p < a.hw) a.y[ch * a.hw + p] = a.x[ch * a.hw + p] * a.s[ch];
}

// The CALayer's excitation and the residual add as one pass:
// y = x * s[ch] + r (+ r2), the unfused kernels' operations in their order.
extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_scale_add_v4(ChanScaleArgs a) {
    const int64_t ch = blockIdx.y;
    const float s = a.s[ch];
    const float *x = a.x + ch * a.hw;
    const float *r = a.r + ch * a.hw;
    const float *r2 = a.r2 ? a.r2 + ch * a.hw : nullptr;
    float *y = a.y + ch * a.hw;
    const int64_t nv = a.hw >> 2;
    float4 v[4], w[4], w2[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t j = (int64_t)blockIdx.x * (MXK_BLOCK * 4) + u * MXK_BLOCK + threadIdx.x;
        if (j < nv) {
            v[u] = ld4(x + 4 * j);
            w[u] = ld4(r + 4 * j);
            if (r2) w2[u] = ld4(r2 + 4 * j);
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t j = (int64_t)blockIdx.x * (MXK_BLOCK * 4) + u * MXK_BLOCK + threadIdx.x;
        if (j < nv) {
            float4 t = v[u];
            t.x = t.x * s + w[u].x;
            t.y = t.y * s + w[u].y;
            t.z = t.z * s + w[u].z;
            t.w = t.w * s + w[u].w;
            if (r2) {
                t.x = t.x + w2[u].x;
                t.y = t.y + w2[u].y;
                t.z = t.z + w2[u].z;
                t.w = t.w + w2[u].w;
            }
            st4(y + 4 * j, t);
        }
    }
}

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_scale_add_s(ChanScaleArgs a) {
    const int64_t ch = blockIdx.y;
    int64_t p = (int64_t)blockIdx.x * MXK_BLOCK + threadIdx.x;
    if (p < a.hw) {
        const int64_t i = ch * a.hw + p;
        float v = a.x[i] * a.s[ch] + a.r[i];
        if (a.r2) v = v + a.r2[i];
        a.y[i] = v;
    }
}

// The channel-attention MLP (CALayer, two plane-1 1x1 convs around a leaky
// ReLU, then the sigmoid) in one block, with mx_gemv's summation order (bias
// first, inputs ascending) and the elementwise kernels' expressions, so the
// result is that of the four unfused launches to the bit.
__device__ __forceinline__ void ca_mlp_body(const CaArgs &a, const float *x) {
    __shared__ float h[1024];
    for (int j = threadIdx.x; j < a.r; j += MXK_BLOCK) {
        const float *w = a.w1 + (int64_t)j * a.c;
        float acc = a.b1 ? a.b1[j] : 0.0f;
#pragma unroll 16
        for (int i = 0; i < a.c; ++i) acc += w[i] * x[i];
        h[j] = acc >= 0.0f ? acc : a.slope * acc;
    }
    __syncthreads();
    for (int o = threadIdx.x; o < a.c; o += MXK_BLOCK) {
        const float *w = a.w2 + (int64_t)o * a.r;
        float acc = a.b2 ? a.b2[o] : 0.0f;
#pragma unroll 16
        for (int j = 0; j < a.r; ++j) acc += w[j] * h[j];
        a.y[o] = sigmoid(acc);
    }
}

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_ca_mlp(CaArgs a) { ca_mlp_body(a, a.x); }

// Channel means (mx_chan_mean_final's ordered sum of the partials and its
// division) straight into the MLP: one launch fewer, and the means never
// leave the block before the MLP reads them (c <= 1024, checked by the host).
extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_ca_mean_mlp(CaMeanArgs a) {
    __shared__ float xm[1024];
    for (int ch = threadIdx.x; ch < a.mlp.c; ch += MXK_BLOCK) {
        const float *p = a.part + (int64_t)ch * a.nchunk;
        float s = 0.0f;
#pragma unroll 8
        for (int k = 0; k < a.nchunk; ++k) s += p[k];
        const float m = s / (float)a.hw;
        xm[ch] = m;
        a.mean[ch] = m;
    }
    __syncthreads();
    ca_mlp_body(a.mlp, xm);
}

// ------------------------------------------------------------ LayerNorm
//
// Per pixel: s1, s2 in ascending channel order, m = s1/c, var = s2/c - m*m,
// r = 1/sqrt(max(var, 0) + eps), y = (x - m) * r * w + b
// (src/exec_cpu.rs:392-432) - the same operations in the same order, so the
// result is the CPU path's to the bit.
//
// A block owns P adjacent pixels: all 256 threads stage the [C][P] tile in
// LDS with 128-bit loads (every channel row is P contiguous floats), then P
// threads run the serial channel sums out of LDS, then all 256 threads
// normalise and store. The staging is what keeps many loads in flight; the
// serial part runs at LDS latency, not memory latency.

// STATS: write only the statistics (mean into y[0 .. hw), 1 / std into
// y[hw .. 2 hw)), for a LayerNorm folded into the next op's GEMM.
// bx: the block's index among the launch's blocks (a kernel pairing two
// launches in one grid passes each part its own).
template <int C, int P, bool STATS = false>
__device__ void chan_ln_tile(const ChanLnArgs &a, int bx) {
    static_assert(C * P <= 8192 && P % 4 == 0 && P <= MXK_BLOCK, "a tile of at most 32 KiB");
    __shared__ float t[C][P];
    __shared__ float st[2][P];
    const int tid = threadIdx.x;
    const int64_t p0 = (int64_t)bx * P;
    const bool full = p0 + P <= a.hw;
    constexpr int Q = P / 4;  // float4s per channel row
    for (int i = tid; i < C * Q; i += MXK_BLOCK) {
        const int c = i / Q, q = (i % Q) * 4;
        const float *src = a.x + (int64_t)c * a.hw + p0 + q;
        float4 v;
        if (full) {
            v = ld4(src);
        } else {
            v.x = p0 + q < a.hw ? src[0] : 0.0f;
            v.y = p0 + q + 1 < a.hw ? src[1] : 0.0f;
            v.z = p0 + q + 2 < a.hw ? src[2] : 0.0f;
            v.w = p0 + q + 3 < a.hw ? src[3] : 0.0f;
        }
        st4(&t[c][q], v);
    }
    __syncthreads();
    if (tid < P) {
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll 8
        for (int c = 0; c < C; ++c) {
            const float v = t[c][tid];
            s1 += v;
            s2 += v * v;
        }
        const float nf = (float)C;
        const float m = s1 / nf;
        const float var = s2 / nf - m * m;
        const float r = 1.0f / sqrtf(fmaxf(var, 0.0f) + a.eps);
        if (STATS) {
            if (p0 + tid < a.hw) {
                a.y[p0 + tid] = m;
                a.y[a.hw + p0 + tid] = r;
            }
            return;
        }
        st[0][tid] = m;
        st[1][tid] = r;
    }
    if (STATS) return;
    __syncthreads();
    for (int i = tid; i < C * Q; i += MXK_BLOCK) {
        const int c = i / Q, q = (i % Q) * 4;
        const float w = a.scale[c], b = a.bias[c];
        float4 v = ld4(&t[c][q]);
        v.x = (v.x - st[0][q]) * st[1][q] * w + b;
        v.y = (v.y - st[0][q + 1]) * st[1][q + 1] * w + b;
        v.z = (v.z - st[0][q + 2]) * st[1][q + 2] * w + b;
        v.w = (v.w - st[0][q + 3]) * st[1][q + 3] * w + b;
        float *dst = a.y + (int64_t)c * a.hw + p0 + q;
        if (full) {
            st4(dst, v);
        } else {
            if (p0 + q < a.hw) dst[0] = v.x;
            if (p0 + q + 1 < a.hw) dst[1] = v.y;
            if (p0 + q + 2 < a.hw) dst[2] = v.z;
            if (p0 + q + 3 < a.hw) dst[3] = v.w;
        }
    }
}

// The CALayer's excitation and residual add(s), as mx_chan_scale_add_v4
// computes them, with the LayerNorm statistics of the result in
// chan_ln_tile's order and expression: the same LDS tile, filled with the
// sums it stores.
template <int C, int P>
__device__ void scale_add_stats_tile(const ScaleAddLnArgs &a) {
    static_assert(C * P <= 8192 && P % 4 == 0 && P <= MXK_BLOCK, "a tile of at most 32 KiB");
    __shared__ float t[C][P];
    const int tid = threadIdx.x;
    const int64_t p0 = (int64_t)blockIdx.x * P;
    const bool full = p0 + P <= a.hw;
    constexpr int Q = P / 4;
    for (int i = tid; i < C * Q; i += MXK_BLOCK) {
        const int c = i / Q, q = (i % Q) * 4;
        const int64_t off = (int64_t)c * a.hw + p0 + q;
        const float s = a.s[c];
        float4 v;
        if (full) {
            v = ld4(a.x + off);
            const float4 w = ld4(a.r + off);
            v.x = v.x * s + w.x;
            v.y = v.y * s + w.y;
            v.z = v.z * s + w.z;
            v.w = v.w * s + w.w;
            if (a.r2) {
                const float4 w2 = ld4(a.r2 + off);
                v.x = v.x + w2.x;
                v.y = v.y + w2.y;
                v.z = v.z + w2.z;
                v.w = v.w + w2.w;
            }
            st4(a.y + off, v);
        } else {
            float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (p0 + q + u < a.hw) {
                    float y = a.x[off + u] * s + a.r[off + u];
                    if (a.r2) y = y + a.r2[off + u];
                    a.y[off + u] = y;
                    e[u] = y;
                }
            v = make_float4(e[0], e[1], e[2], e[3]);
        }
        st4(&t[c][q], v);
    }
    __syncthreads();
    if (tid < P && p0 + tid < a.hw) {
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll 8
        for (int c = 0; c < C; ++c) {
            const float v = t[c][tid];
            s1 += v;
            s2 += v * v;
        }
        const float nf = (float)C;
        const float m = s1 / nf;
        const float var = s2 / nf - m * m;
        a.stats[p0 + tid] = m;
        a.stats[a.hw + p0 + tid] = 1.0f / sqrtf(fmaxf(var, 0.0f) + a.eps);
    }
}

// 128-bit paths need hw % 4 == 0 and 16-byte aligned x and y.
// mx_chan_ln_c<C>[_p<P>] and mx_chan_ln_stats_c<C>[_p<P>]: C channels x P
// pixels per block (P = 8192 / C without the suffix); the smaller tiles give
// small planes more blocks, since each block's serial channel pass is
// latency-bound.
// mx_chan_ln_c<C>[_p<P>]_x2: two independent LayerNorms of one shape as one
// grid (the first d.na blocks run d.a, the rest d.b).
#define MXK_LN(C, P, SUF)                                                                           \
    extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_ln_c##C##SUF(ChanLnArgs a) {    \
        chan_ln_tile<C, P>(a, blockIdx.x);                                                          \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_ln_c##C##SUF##_x2(DualLnArgs d) { \
        if (blockIdx.x < d.na)                                                                      \
            chan_ln_tile<C, P>(d.a, blockIdx.x);                                                    \
        else                                                                                        \
            chan_ln_tile<C, P>(d.b, blockIdx.x - d.na);                                             \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_ln_stats_c##C##SUF(ChanLnArgs a) { \
        chan_ln_tile<C, P, true>(a, blockIdx.x);                                                    \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_scale_add_stats_c##C##SUF(ScaleAddLnArgs a) { \
        scale_add_stats_tile<C, P>(a);                                                              \
    }
MXK_LN(32, 256, )
MXK_LN(32, 128, _p128)
MXK_LN(32, 64, _p64)
MXK_LN(64, 128, )
MXK_LN(64, 64, _p64)
MXK_LN(64, 32, _p32)
MXK_LN(128, 64, )
MXK_LN(128, 32, _p32)
MXK_LN(128, 16, _p16)

// Any channel count, any alignment: reads x twice.
extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_ln_any(ChanLnArgs a) {
    const int64_t p = (int64_t)blockIdx.x * MXK_BLOCK + threadIdx.x;
    if (p >= a.hw) return;
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = 0; c < a.c; ++c) {
        float v = a.x[(int64_t)c * a.hw + p];
        s1 += v;
        s2 += v * v;
    }
    const float nf = (float)a.c;
    const float m = s1 / nf;
    const float var = s2 / nf - m * m;
    const float r = 1.0f / sqrtf(fmaxf(var, 0.0f) + a.eps);
    for (int c = 0; c < a.c; ++c) {
        int64_t i = (int64_t)c * a.hw + p;
        a.y[i] = (a.x[i] - m) * r * a.scale[c] + a.bias[c];
    }
}

// The per-pixel statistics alone, for a LayerNorm folded into the following
// 1x1 conv (the mx_chan_ln_stats_c* forms above use chan_ln_tile's staging,
// sums, order and expressions, so the normalised values the GEMM forms from
// them are that kernel's to the bit). This one takes any channel count: four
// pixels per thread, the channel loop in registers. Needs hw % 4 == 0 and
// 16-byte aligned x and y.
extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_ln_stats(ChanLnArgs a) {
    const int64_t p = ((int64_t)blockIdx.x * MXK_BLOCK + threadIdx.x) * 4;
    if (p >= a.hw) return;
    float s1[4] = {0.0f, 0.0f, 0.0f, 0.0f}, s2[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float *x = a.x + p;
#pragma unroll 4
    for (int c = 0; c < a.c; ++c) {
        const float4 v = ld4(x + (int64_t)c * a.hw);
        s1[0] += v.x;
        s2[0] += v.x * v.x;
        s1[1] += v.y;
        s2[1] += v.y * v.y;
        s1[2] += v.z;
        s2[2] += v.z * v.z;
        s1[3] += v.w;
        s2[3] += v.w * v.w;
    }
    const float nf = (float)a.c;
    float m[4], r[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        m[u] = s1[u] / nf;
        const float var = s2[u] / nf - m[u] * m[u];
        r[u] = 1.0f / sqrtf(fmaxf(var, 0.0f) + a.eps);
    }
    st4(a.y + p, make_float4(m[0], m[1], m[2], m[3]));
    st4(a.y + a.hw + p, make_float4(r[0], r[1], r[2], r[3]));
}

// ----------------------------------------------------------- channel mean
//
// Two fixed-order passes: partial sums of `chunk` elements per (channel,
// chunk), then one ordered sum of the partials per channel. Deterministic,
// but not the CPU's serial order, so it agrees with it to rounding only.

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_mean_part(ChanMeanArgs a) {
    __shared__ float red[MXK_BLOCK];
    const int ch = blockIdx.y, k = blockIdx.x;
    const float *x = a.x + (int64_t)ch * a.hw;
    int64_t lo = (int64_t)k * a.chunk, hi = lo + a.chunk < a.hw ? lo + a.chunk : a.hw;
    float s = 0.0f;
    for (int64_t i = lo + threadIdx.x; i < hi; i += MXK_BLOCK) s += x[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = MXK_BLOCK / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) a.part[(int64_t)ch * a.nchunk + k] = red[0];
}

// The same partial sums with 128-bit loads, for planes whose length is a
// multiple of 4 and chunks of a multiple of 1024 elements: each thread adds
// four consecutive elements, then every 1024th float4, and the block reduces
// by a fixed butterfly within each wave and an ordered sum of the four waves.
extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_mean_part4(ChanMeanArgs a) {
    __shared__ float red[MXK_BLOCK / 64];
    const int ch = blockIdx.y, k = blockIdx.x;
    const float *x = a.x + (int64_t)ch * a.hw;
    const int64_t lo = (int64_t)k * a.chunk, hi = lo + a.chunk < a.hw ? lo + a.chunk : a.hw;
    float s = 0.0f;
    for (int64_t i = lo + 4 * threadIdx.x; i < hi; i += 4 * MXK_BLOCK) {
        const float4 v = ld4(x + i);
        s += ((v.x + v.y) + v.z) + v.w;
    }
#pragma unroll
    for (int w = 32; w > 0; w >>= 1) s += __shfl_xor(s, w);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) a.part[(int64_t)ch * a.nchunk + k] = ((red[0] + red[1]) + red[2]) + red[3];
}

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_chan_mean_final(ChanMeanArgs a) {
    const int ch = blockIdx.x * MXK_BLOCK + threadIdx.x;
    if (ch >= a.c) return;
    float s = 0.0f;
#pragma unroll 8
    for (int k = 0; k < a.nchunk; ++k) s += a.part[(int64_t)ch * a.nchunk + k];
    a.y[ch] = s / (float)a.hw;
}

// ------------------------------------------------------ block permutation
//
// Block (ch, g) moves the psz = fh * fw pixels of one cell; threads sweep p in
// runs of V (V divides fw, so a run stays inside one pixel row). Forward
// gathers [c][h][w] -> [c][g][p]; backward scatters it back. Pure copies.

template <int V>
__device__ void perm_body(const PermArgs &a) {
    const int gsz = a.gh * a.gw, psz = a.fh * a.fw;
    const int64_t e = blockIdx.x;
    const int64_t ch = e / gsz;
    const int g = (int)(e - ch * gsz);
    const int gy = g / a.gw, gx = g - gy * a.gw;
    const int64_t plane = (int64_t)a.h * a.wd;
    const float *x = a.x + ch * plane;
    float *y = a.y + ch * plane;
    for (int p = threadIdx.x * V; p < psz; p += blockDim.x * V) {
        const int fy = p / a.fw, fx = p - fy * a.fw;
        const int64_t pix = (int64_t)(gy * a.fh + fy) * a.wd + gx * a.fw + fx;
        const int64_t blk = a.swap ? (int64_t)p * gsz + g : (int64_t)g * psz + p;
        if (V == 4) {
            if (a.forward) st4(y + blk, ld4(x + pix));
            else st4(y + pix, ld4(x + blk));
        } else if (V == 2) {
            if (a.forward) *reinterpret_cast<float2 *>(y + blk) = *reinterpret_cast<const float2 *>(x + pix);
            else *reinterpret_cast<float2 *>(y + pix) = *reinterpret_cast<const float2 *>(x + blk);
        } else {
            if (a.forward) y[blk] = x[pix];
            else y[pix] = x[blk];
        }
    }
}

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_block_perm_v4(PermArgs a) { perm_body<4>(a); }
extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_block_perm_v2(PermArgs a) { perm_body<2>(a); }
extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_block_perm_v1(PermArgs a) { perm_body<1>(a); }

// --------------------------------------------------------- nearest subsample

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_down_s(DownArgs a) {
    const int64_t n = a.c * a.oh * a.ow;
    const int64_t i = (int64_t)blockIdx.x * MXK_BLOCK + threadIdx.x;
    if (i >= n) return;
    const int64_t op = (int64_t)a.oh * a.ow;
    const int64_t ch = i / op;
    const int r = (int)(i - ch * op);
    const int oy = r / a.ow, ox = r - oy * a.ow;
    a.y[i] = a.x[ch * a.h * a.wd + (int64_t)(oy * a.stride + a.off) * a.wd + ox * a.stride + a.off];
}

// --------------------------------------------------------------- resize
//
// The tap table of each axis is built on the host by the same arithmetic as
// the CPU's ResizeTaps (src/exec_cpu.rs:1195-1216) and handed in as
// `x` rows of [j0, n, wsum, w0 .. w(maxt-1)] (j0 and n as floats, exact for
// any size this engine runs). Each output is sum_k w_k * src[j0 + k] in
// ascending k, then / wsum when wsum > 0.

struct ResizeTab {
    const float *t;
    int32_t maxt, pad;
};

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_resize_h(ResizeArgs a, ResizeTab tab) {
    const int64_t n = a.rows * a.n_out;
    const int64_t i = (int64_t)blockIdx.x * MXK_BLOCK + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / a.n_out;
    const int o = (int)(i - r * a.n_out);
    const float *e = tab.t + (int64_t)o * (3 + tab.maxt);
    const int j0 = (int)e[0], nt = (int)e[1];
    const float ws = e[2];
    const float *src = a.x + r * a.n_in + j0;
    float acc = 0.0f;
    for (int k = 0; k < nt; ++k) acc += e[3 + k] * src[k];
    a.y[i] = ws > 0.0f ? acc / ws : acc;
}

extern "C" __global__ __launch_bounds__(MXK_BLOCK) void mx_resize_v(ResizeArgs a, ResizeTab tab) {
    const int64_t n = a.rows * a.n_out * (int64_t)a.width;
    const int64_t i = (int64_t)blockIdx.x * MXK_BLOCK + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / a.width;            // channel * n_out + o
    const int x = (int)(i - r * a.width);
    const int64_t ch = r / a.n_out;
    const int o = (int)(r - ch * a.n_out);
    const float *e = tab.t + (int64_t)o * (3 + tab.maxt);
    const int j0 = (int)e[0], nt = (int)e[1];
    const float ws = e[2];
    const float *src = a.x + ch * a.n_in * (int64_t)a.width + (int64_t)j0 * a.width + x;
    float acc = 0.0f;
    for (int k = 0; k < nt; ++k) acc += e[3 + k] * src[(int64_t)k * a.width];
    a.y[i] = ws > 0.0f ? acc / ws : acc;
}

// Both axes in one pass, without the intermediate plane. A block owns TW
// output columns x `rows` output rows of one channel. It stages in LDS the
// input rows its outputs read (the vertical taps of its first row through
// those of its last: `band` rows at most) over the input columns they read
// (the horizontal taps of its first column through those of its last: `span`
// at most; the host sizes the dynamic LDS and checks both ranges; with
// 128-bit loads a row holds up to 6 more columns, from the 16-byte boundary
// before the first), with coalesced loads; runs the horizontal pass from
// there into LDS; and then the
// vertical pass from LDS to the output. Every intermediate value is computed
// by the same expression as in mx_resize_h, so the result is bit-identical to
// the two-pass kernels; rows and columns shared by two blocks are simply
// staged twice. Tables are at most RS_MAXT taps wide (checked by the host).
// TW = 64: one output column per lane; TW = 256 (ow % 4 == 0, 16-byte aligned
// y): four adjacent columns per lane in the vertical pass, 128-bit stores.
constexpr int RS_MAXT = 8;

// A value every lane of the wave holds alike, as the wave's scalar.
__device__ __forceinline__ float uniform(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// acc / wsum when wsum > 0 (the CPU path's normalisation). Upsampling tables
// mostly sum to exactly 1, and x / 1 is x in IEEE arithmetic, so those skip
// the division and the result is the same to the bit.
__device__ __forceinline__ float rs_norm(float acc, float ws) {
    return ws > 0.0f && ws != 1.0f ? acc / ws : acc;
}

// MT: taps per table row the loops are unrolled for (>= the tables' own,
// which the host picks it from: 2 for bilinear upsampling, 4 or 8 for the
// antialiased downsampling), so an upsampling kernel carries no predicated
// dead taps.
template <int TW, int MT>
__device__ void resize_hv(const Resize2Args &a) {
    static_assert(MT <= RS_MAXT, "taps");
    extern __shared__ float rs_lds[];
    float *in = rs_lds;                               // [band][span]
    float *tmp = rs_lds + a.band * a.span;            // [band][TW]
    float *vt = tmp + a.band * TW;                    // [rows][3 + mtv]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ch = blockIdx.y;
    const int tx = blockIdx.x % a.tiles_x, ty = blockIdx.x / a.tiles_x;
    const int ox0 = tx * TW, oy0 = ty * a.rows;
    const int nrow = min(a.rows, a.oh - oy0), ncol = min(TW, a.ow - ox0);
    const int sv = 3 + a.mtv, sh = 3 + a.mth;
    const float *vf = a.tv + (int64_t)oy0 * sv, *vl = vf + (int64_t)(nrow - 1) * sv;
    const float *hf = a.th + (int64_t)ox0 * sh, *hl = hf + (int64_t)(ncol - 1) * sh;
    const int jlo = (int)vf[0], nr = (int)vl[0] + (int)vl[1] - jlo;
    const int xlo = (int)hf[0], xn = (int)hl[0] + (int)hl[1] - xlo;
    for (int q = tid; q < nrow * sv; q += 256) vt[q] = vf[q];
    // the input rows and columns this block reads, eight loads in flight per
    // thread before any of them is written to LDS: 128-bit loads from the
    // 16-byte boundary at or before the first column (the LDS rows then
    // start `lead` <= 3 columns early), else one float at a time
    int lead = 0;
    if (a.vec) {
        const int x4 = xlo & ~3;
        lead = xlo - x4;
        const int n4 = (lead + xn + 3) >> 2;
        const float *src = a.x + ((int64_t)ch * a.h + jlo) * a.wd + x4;
        const int total = nr * n4;
        // (r, c) of element q, advanced by 256 elements a step without a
        // division: dr rows and dc columns, plus a carry
        int r = tid / n4, c = tid - (tid / n4) * n4;
        const int dr = 256 / n4, dc = 256 - dr * n4;
        for (int q0 = tid; q0 < total; q0 += 8 * 256) {
            float4 v[8];
            int at[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int q = q0 + u * 256;
                at[u] = -1;
                if (q < total) {
                    v[u] = ld4(src + (int64_t)r * a.wd + 4 * c);
                    at[u] = r * a.span + 4 * c;
                }
                r += dr;
                c += dc;
                if (c >= n4) {
                    c -= n4;
                    ++r;
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (at[u] >= 0) st4(in + at[u], v[u]);
        }
    } else {
        const float *src = a.x + ((int64_t)ch * a.h + jlo) * a.wd + xlo;
        const int total = nr * xn;
        int r = tid / xn, c = tid - (tid / xn) * xn;
        const int dr = 256 / xn, dc = 256 - dr * xn;
        for (int q0 = tid; q0 < total; q0 += 8 * 256) {
            float v[8];
            int at[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int q = q0 + u * 256;
                at[u] = -1;
                if (q < total) {
                    v[u] = src[(int64_t)r * a.wd + c];
                    at[u] = r * a.span + c;
                }
                r += dr;
                c += dc;
                if (c >= xn) {
                    c -= xn;
                    ++r;
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (at[u] >= 0) in[at[u]] = v[u];
        }
    }
    __syncthreads();

    // horizontal pass: TW = 256, thread t owns column t over every row;
    // TW = 64, lane l owns column l over the rows of its wave
    const int col = TW == 256 ? tid : lane;
    if (col < ncol) {
        const float *e = a.th + (int64_t)(ox0 + col) * sh;
        const int b = (int)e[0] - xlo, nt = (int)e[1];
        const float ws = e[2];
        float w[MT];
#pragma unroll
        for (int k = 0; k < MT; ++k) w[k] = k < a.mth ? e[3 + k] : 0.0f;
        const int r0 = TW == 256 ? 0 : wave, dr = TW == 256 ? 1 : 4;
        // rs_norm's test once per column: columns whose taps sum to 1 (most
        // of an upsampling) run the loop without the division
        auto hrows = [&](auto norm) {
            for (int r = r0; r < nr; r += dr) {
                const float *sr = in + r * a.span + lead + b;
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < MT; ++k)
                    if (k < nt) acc += w[k] * sr[k];
                tmp[r * TW + col] = norm(acc);
            }
        };
        if (ws > 0.0f && ws != 1.0f)
            hrows([&](float acc) { return acc / ws; });
        else
            hrows([](float acc) { return acc; });
    }
    __syncthreads();

    // vertical pass, wave w takes output rows w, w + 4, ...
    float *yrow = a.y + ((int64_t)ch * a.oh + oy0) * a.ow + ox0;
    if (TW == 256) {
        const int c0 = 4 * lane;
        if (c0 >= ncol) return;
        for (int r = wave; r < nrow; r += 4) {
            // (row r's table entry is the wave's own: scalar registers)
            const float *e = vt + r * sv;
            const int b = __builtin_amdgcn_readfirstlane((int)e[0]) - jlo;
            const int n = __builtin_amdgcn_readfirstlane((int)e[1]);
            const float vs = uniform(e[2]);
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < MT; ++k)
                if (k < n) {
                    const float wk = uniform(e[3 + k]);
                    const float4 t = ld4(tmp + (b + k) * TW + c0);
                    acc[0] += wk * t.x;
                    acc[1] += wk * t.y;
                    acc[2] += wk * t.z;
                    acc[3] += wk * t.w;
                }
            float o[4];
            if (vs > 0.0f && vs != 1.0f) {
#pragma unroll
                for (int u = 0; u < 4; ++u) o[u] = acc[u] / vs;
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) o[u] = acc[u];
            }
            float *yo = yrow + (int64_t)r * a.ow + c0;
            if (c0 + 3 < ncol) {
                st4(yo, make_float4(o[0], o[1], o[2], o[3]));
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (c0 + u < ncol) yo[u] = o[u];
            }
        }
    } else {
        if (lane >= ncol) return;
        for (int r = wave; r < nrow; r += 4) {
            const float *e = vt + r * sv;
            const int b = __builtin_amdgcn_readfirstlane((int)e[0]) - jlo;
            const int n = __builtin_amdgcn_readfirstlane((int)e[1]);
            const float vs = uniform(e[2]);
            const float *t = tmp + b * TW + lane;
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < MT; ++k)
                if (k < n) acc += uniform(e[3 + k]) * t[k * TW];
            yrow[(int64_t)r * a.ow + lane] = vs > 0.0f && vs != 1.0f ? acc / vs : acc;
        }
    }
}

// mx_resize_hv[4]_t<MT>: 64 (256) output columns per block, tables of at
// most MT taps.
#define MXK_RS(MT)                                                                                  \
    extern "C" __global__ __launch_bounds__(256) void mx_resize_hv_t##MT(Resize2Args a) { resize_hv<64, MT>(a); } \
    extern "C" __global__ __launch_bounds__(256) void mx_resize_hv4_t##MT(Resize2Args a) { resize_hv<256, MT>(a); }
MXK_RS(2)
MXK_RS(4)
MXK_RS(8)
