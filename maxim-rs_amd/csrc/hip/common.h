// Shared device helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "kargs.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One 16x16x4 fp32 MFMA: acc[16x16] += A[16x4] * B[4x16].
// Lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]; the accumulator
// holds D[4 * (l / 16) + r][l % 16] in element r.
__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Work-group placement. The dispatcher deals consecutive work-group ids to
// the 8 XCDs in turn, and each XCD has its own L2, so neighbouring tiles
// (which share halo rows, cache lines and operands) land in different L2s.
// xcd_tile() renumbers the (gridDim.x x gridDim.y) grid so that each XCD
// walks one contiguous run of the new ids, and splits the new id into a tile
// index and a band (e.g. the output-channel block) with the band fastest, so
// every band of a tile is computed under the same L2.
__device__ __forceinline__ void xcd_tile(int &tile, int &band) {
    const int gy = gridDim.y, n = gridDim.x * gy;
    const int id = blockIdx.x + blockIdx.y * gridDim.x;
    const int x = id & 7, q = n >> 3, r = n & 7;
    const int nid = x * q + min(x, r) + (id >> 3);
    tile = nid / gy;
    band = nid - tile * gy;
}

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }

// GELU, x Phi(x) = 0.5 x (1 + erf(x / sqrt 2)), branch-free: with
// R = Phi(-|x|), GELU is max(x, 0) - |x| R for either sign of x, and
// R = 2^q(t) at t = min(|x|, 6), q the degree-6 polynomial fitted by
// weighted least squares to log2 Phi(-t) over [0, 6] (each point weighted by
// how little error its GELU value allows, so the fit is tightest near 0),
// evaluated by Horner and raised on the transcendental unit (v_exp_f32, 1
// ulp): a min, six FMAs, one exp2, a max and an FMA (the |x| and the sign
// are source modifiers). Within 6.3e-8 * (1 + |x|) of the exact function
// (past |x| = 6 the clamped R is below 1e-9). The standalone GELU op and
// every fused epilogue use this one function, so fusing a GELU changes no
// bit.
__device__ __forceinline__ float gelu(float x) {
    const float ax = fabsf(x);
    const float t = fminf(ax, 6.0f);
    float q = __builtin_fmaf(3.3113869e-05f, t, -7.6996483e-04f);
    q = __builtin_fmaf(q, t, 8.0852984e-03f);
    q = __builtin_fmaf(q, t, -5.3423237e-02f);
    q = __builtin_fmaf(q, t, -4.5875868e-01f);
    q = __builtin_fmaf(q, t, -1.1512076e+00f);
    q = __builtin_fmaf(q, t, -9.9999213e-01f);
    const float r = __builtin_amdgcn_exp2f(q);  // Phi(-|x|)
    return __builtin_fmaf(-ax, r, fmaxf(x, 0.0f));
}

// 1 / (1 + e^-x) with e^-x = 2^(-x log2 e) on the transcendental unit and
// one hardware reciprocal (v_exp_f32, v_rcp_f32, 1 ulp each): within
// 1.3e-7 (1 + |x|) of the exact function, 0 and 1 in the tails where the
// power overflows or vanishes; held to the CPU path's 1 / (1 + expf(-x))
// within 4e-7 (1 + |x|). One function, so the standalone kernel, the CALayer
// block and the fused epilogue agree to the bit.
__device__ __forceinline__ float sigmoid(float x) {
    const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
    return __builtin_amdgcn_rcpf(1.0f + e);
}

// The fused epilogue (kargs.h, Epilogue) for output element `idx`, after bias.
__device__ __forceinline__ float epilogue(const Epilogue &e, float v, int64_t idx) {
    if (e.u) v = e.u[idx] * (v + 1.0f);
    if (e.act == MXK_ACT_GELU) v = gelu(v);
    else if (e.act == MXK_ACT_LRELU) v = v >= 0.0f ? v : e.slope * v;
    else if (e.act == MXK_ACT_SIGMOID) v = sigmoid(v);
    if (e.m) v = v * e.m[idx];
    if (e.r1) v = v + e.r1[idx];
    if (e.r2) v = v + e.r2[idx];
    return v;
}

// The same for the two elements idx, idx + 1, with 64-bit operand loads
// (idx even and every operand 8-byte aligned): each element's operations and
// their order are epilogue()'s.
__device__ __forceinline__ void epilogue2(const Epilogue &e, float &v0, float &v1, int64_t idx) {
    const float2 zero = make_float2(0.0f, 0.0f);
    const float2 u2 = e.u ? *reinterpret_cast<const float2 *>(e.u + idx) : zero;
    const float2 m2 = e.m ? *reinterpret_cast<const float2 *>(e.m + idx) : zero;
    const float2 a2 = e.r1 ? *reinterpret_cast<const float2 *>(e.r1 + idx) : zero;
    const float2 b2 = e.r2 ? *reinterpret_cast<const float2 *>(e.r2 + idx) : zero;
    const float uu[2] = {u2.x, u2.y}, mm[2] = {m2.x, m2.y}, aa[2] = {a2.x, a2.y}, bb[2] = {b2.x, b2.y};
    float v[2] = {v0, v1};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        float x = v[k];
        if (e.u) x = uu[k] * (x + 1.0f);
        if (e.act == MXK_ACT_GELU) x = gelu(x);
        else if (e.act == MXK_ACT_LRELU) x = x >= 0.0f ? x : e.slope * x;
        else if (e.act == MXK_ACT_SIGMOID) x = sigmoid(x);
        if (e.m) x = x * mm[k];
        if (e.r1) x = x + aa[k];
        if (e.r2) x = x + bb[k];
        v[k] = x;
    }
    v0 = v[0];
    v1 = v[1];
}

// The same for the four elements idx .. idx + 3, with 128-bit operand loads
// (idx % 4 == 0 and every operand 16-byte aligned): each element's operations
// and their order are epilogue()'s.
__device__ __forceinline__ void epilogue4(const Epilogue &e, float *v, int64_t idx) {
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 u4 = e.u ? *reinterpret_cast<const float4 *>(e.u + idx) : zero;
    const float4 m4 = e.m ? *reinterpret_cast<const float4 *>(e.m + idx) : zero;
    const float4 a4 = e.r1 ? *reinterpret_cast<const float4 *>(e.r1 + idx) : zero;
    const float4 b4 = e.r2 ? *reinterpret_cast<const float4 *>(e.r2 + idx) : zero;
    const float uu[4] = {u4.x, u4.y, u4.z, u4.w}, mm[4] = {m4.x, m4.y, m4.z, m4.w};
    const float aa[4] = {a4.x, a4.y, a4.z, a4.w}, bb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float x = v[k];
        if (e.u) x = uu[k] * (x + 1.0f);
        if (e.act == MXK_ACT_GELU) x = gelu(x);
        else if (e.act == MXK_ACT_LRELU) x = x >= 0.0f ? x : e.slope * x;
        else if (e.act == MXK_ACT_SIGMOID) x = sigmoid(x);
        if (e.m) x = x * mm[k];
        if (e.r1) x = x + aa[k];
        if (e.r2) x = x + bb[k];
        v[k] = x;
    }
}
