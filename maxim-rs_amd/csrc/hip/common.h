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

// GELU, 0.5 x (1 + erf(x / sqrt 2)), branch-free: erfc(z) for z = |x| / sqrt 2
// from Abramowitz & Stegun 7.1.28, erfc(z) = (1 + a1 z + ... + a6 z^6)^-16
// with |error| <= 3e-7, so 1 + erf(x / sqrt 2) is 2 - R for x >= 0 and R for
// x < 0. Within 2.2e-7 * (1 + |x|) of the exact function, and about a third
// of the instructions of the device erff (whose two divergent branches both
// run in a wave of mixed signs). The standalone GELU op and every fused
// epilogue use this one function, so fusing a GELU changes no bit.
__device__ __forceinline__ float gelu(float x) {
    const float z = fabsf(x) * 0.70710678118654752440f;
    float t = __builtin_fmaf(0.0000430638f, z, 0.0002765672f);
    t = __builtin_fmaf(t, z, 0.0001520143f);
    t = __builtin_fmaf(t, z, 0.0092705272f);
    t = __builtin_fmaf(t, z, 0.0422820123f);
    t = __builtin_fmaf(t, z, 0.0705230784f);
    t = __builtin_fmaf(t, z, 1.0f);
    t = t * t;
    t = t * t;
    t = t * t;
    t = t * t;
    const float r = __builtin_amdgcn_rcpf(t);  // erfc(z); 0 once t overflows
    const float h = 0.5f * x;
    return x >= 0.0f ? h * (2.0f - r) : h * r;
}

// The fused epilogue (kargs.h, Epilogue) for output element `idx`, after bias.
__device__ __forceinline__ float epilogue(const Epilogue &e, float v, int64_t idx) {
    if (e.u) v = e.u[idx] * (v + 1.0f);
    if (e.act == MXK_ACT_GELU) v = gelu(v);
    else if (e.act == MXK_ACT_LRELU) v = v >= 0.0f ? v : e.slope * v;
    if (e.r1) v = v + e.r1[idx];
    if (e.r2) v = v + e.r2[idx];
    return v;
}
