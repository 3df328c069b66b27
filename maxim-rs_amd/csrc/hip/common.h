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

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }

__device__ __forceinline__ float gelu_erf(float a) {
    return 0.5f * a * (1.0f + erff(a * 0.70710678118654752440f));
}

// The fused epilogue (kargs.h, Epilogue) for output element `idx`, after bias.
__device__ __forceinline__ float epilogue(const Epilogue &e, float v, int64_t idx) {
    if (e.u) v = e.u[idx] * (v + 1.0f);
    if (e.act == MXK_ACT_GELU) v = gelu_erf(v);
    else if (e.act == MXK_ACT_LRELU) v = v >= 0.0f ? v : e.slope * v;
    if (e.r1) v = v + e.r1[idx];
    if (e.r2) v = v + e.r2[idx];
    return v;
}
