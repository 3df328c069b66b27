// fp32 GEMM on the gfx950 matrix cores: C[b][M][N] = A[b][M][K] . B[b][K][N]
// (+ bias), A and B row-major, fp32 in and fp32 accumulate
// (v_mfma_f32_16x16x4_f32), no reduced-precision inputs.
//
// One kernel serves every Dense-shaped op of the plan:
//   Conv1x1 / Dense  A = W [co][ci], B = X [ci][plane], bias by row
//   GateMm mode 0    batched over channels: A = W [r][t] (shared),
//                    B = X[c] [t][b], bias by row
//   GateMm mode 1    A = X [c*outer][t], B = W^T [t][a], bias by column
//   ConvT 2x2 s2     A = W [tap*co + oc][ci], B = X [ci][plane]; the epilogue
//                    scatters row (tap, oc), column (y, x) to
//                    out[oc][2y + ky][2x + kx] and adds the bias last
// The reduction order is the matrix core's, not the CPU's, so results agree
// with the CPU path to rounding.
//
// Block: 256 threads = 4 waves on a WAVES_M x WAVES_N grid, block tile
// BM x BN, K staged through LDS in steps of BK (A stored k-major so a lane's
// fragment element is one conflict-free LDS word).
#pragma once

#include "common.h"

template <int BM, int BN, int WAVES_M, int WAVES_N, bool VEC_B>
__device__ void gemm_body(const GemmArgs &a) {
    constexpr int BK = 16;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 16, TN = WTN / 16;
    static_assert(WAVES_M * WAVES_N == 4, "4 waves");
    static_assert(TM >= 1 && TN >= 1, "wave tile");
    __shared__ float As[BK][BM + 4];
    __shared__ float Bs[BK][BN + 4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM, b = blockIdx.z;
    const float *A = a.A + (int64_t)b * a.sA;
    const float *B = a.B + (int64_t)b * a.sB;
    const int M = a.M, N = a.N, K = a.K;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int lr = lane & 15, lk = lane >> 4;
    for (int k0 = 0; k0 < K; k0 += BK) {
        // A tile BM x BK, k fastest in the read, stored k-major.
        for (int i = tid; i < BM * BK; i += 256) {
            const int m = i / BK, k = i % BK;
            const int gm = m0 + m, gk = k0 + k;
            As[k][m] = (gm < M && gk < K) ? A[(int64_t)gm * K + gk] : 0.0f;
        }
        // B tile BK x BN, n fastest.
        if (VEC_B) {
            for (int i = tid; i < BK * BN / 4; i += 256) {
                const int k = i / (BN / 4), n = (i % (BN / 4)) * 4;
                const int gk = k0 + k, gn = n0 + n;
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (gk < K && gn < N) v = ld4(B + (int64_t)gk * N + gn);  // N % 4 == 0
                Bs[k][n] = v.x; Bs[k][n + 1] = v.y; Bs[k][n + 2] = v.z; Bs[k][n + 3] = v.w;
            }
        } else {
            for (int i = tid; i < BK * BN; i += 256) {
                const int k = i / BN, n = i % BN;
                const int gk = k0 + k, gn = n0 + n;
                Bs[k][n] = (gk < K && gn < N) ? B[(int64_t)gk * N + gn] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            float af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = As[kk + lk][wm * WTM + i * 16 + lr];
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = Bs[kk + lk][wn * WTN + j * 16 + lr];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
        }
        __syncthreads();
    }

    // Epilogue: element r of acc[i][j] is row 4*(lane/16) + r, column lane%16.
    float *C = a.C + (int64_t)b * a.sC;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn * WTN + j * 16 + lr;
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * WTM + i * 16 + 4 * lk + r;
                if (m >= M) continue;
                float v = acc[i][j][r];
                if (a.epi == MXK_EPI_CONVT) {
                    const int tap = m / a.co, oc = m - tap * a.co;
                    const int ky = tap >> 1, kx = tap & 1;
                    const int y = n / a.wd, x = n - y * a.wd;
                    const int64_t ow = 2 * (int64_t)a.wd;
                    if (a.bias) v = a.bias[oc] + v;
                    C[(int64_t)oc * (4 * (int64_t)N) + (2 * y + ky) * ow + 2 * x + kx] = v;
                } else {
                    if (a.bias_mode == MXK_BIAS_ROW) v = a.bias[m] + v;
                    else if (a.bias_mode == MXK_BIAS_COL) v = a.bias[n] + v;
                    C[(int64_t)m * N + n] = v;
                }
            }
        }
    }
}

#define MXK_GEMM(NAME, BM, BN, WM, WN)                                                          \
    extern "C" __global__ __launch_bounds__(256) void mx_gemm_##NAME(GemmArgs a) {              \
        gemm_body<BM, BN, WM, WN, false>(a);                                                    \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(256) void mx_gemm_##NAME##_v4(GemmArgs a) {         \
        gemm_body<BM, BN, WM, WN, true>(a);                                                     \
    }

MXK_GEMM(32x128, 32, 128, 1, 4)
MXK_GEMM(64x128, 64, 128, 2, 2)
MXK_GEMM(128x128, 128, 128, 2, 2)
MXK_GEMM(128x64, 128, 64, 4, 1)

// The CALayer's plane-1 convs: y[o] = b[o] + sum_i w[o][i] x[i], i ascending,
// exactly the CPU arm's order (bias first), so this one is bit-exact.
extern "C" __global__ __launch_bounds__(256) void mx_gemv(GemvArgs a) {
    const int o = blockIdx.x * 256 + threadIdx.x;
    if (o >= a.co) return;
    const float *w = a.w + (int64_t)o * a.ci;
    float acc = a.bias ? a.bias[o] : 0.0f;
    for (int i = 0; i < a.ci; ++i) acc += w[i] * a.x[i];
    a.y[o] = acc;
}
