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
// BM x BN, K in steps of 32. Both operands are staged k-contiguous in LDS
// ([m][k] and [n][k], rows padded to 36 floats so 128-bit reads of eight
// consecutive rows cover all 32 banks once), and every lane reads its
// fragments for four MFMA steps with one 128-bit load: lane group g supplies
// k = 4g + j at step j, which covers each k of the 16 exactly once. The next
// K tile is fetched into registers while the current one is multiplied.
#pragma once

#include "common.h"

namespace gemm {

constexpr int BK = 32;
constexpr int LDK = BK + 4;

template <int BM, int BN, bool VEC>
struct Stage {
    // Per thread: A as float4 along k, B as 4 k-rows of one column.
    static constexpr int NA = BM * BK / 4 / 256;
    static constexpr int NB = BN * BK / 4 / 256;
    static_assert(NA >= 1 && NB >= 1, "tile too small for 256 threads");
    float4 a[NA];
    float4 b[NB];

    __device__ void load(const float *A, const float *B, int M, int N, int K, int m0, int n0, int k0,
                         int tid) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int idx = tid + i * 256;
            const int m = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
            const int gm = m0 + m, gk = k0 + k;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (gm < M) {
                const float *p = A + (int64_t)gm * K + gk;
                if (VEC && gk + 3 < K) {
                    v = ld4(p);
                } else {
                    if (gk < K) v.x = p[0];
                    if (gk + 1 < K) v.y = p[1];
                    if (gk + 2 < K) v.z = p[2];
                    if (gk + 3 < K) v.w = p[3];
                }
            }
            a[i] = v;
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int idx = tid + i * 256;
            const int n = idx % BN, k = (idx / BN) * 4;
            const int gn = n0 + n, gk = k0 + k;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (gn < N) {
                const float *p = B + (int64_t)gk * N + gn;
                if (gk < K) v.x = p[0];
                if (gk + 1 < K) v.y = p[N];
                if (gk + 2 < K) v.z = p[2 * (int64_t)N];
                if (gk + 3 < K) v.w = p[3 * (int64_t)N];
            }
            b[i] = v;
        }
    }

    __device__ void store(float (*As)[LDK], float (*Bs)[LDK], int tid) const {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int idx = tid + i * 256;
            st4(&As[idx / (BK / 4)][(idx % (BK / 4)) * 4], a[i]);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int idx = tid + i * 256;
            st4(&Bs[idx % BN][(idx / BN) * 4], b[i]);
        }
    }
};

template <int BM, int BN, int WAVES_M, int WAVES_N, bool VEC>
__device__ void body(const GemmArgs &a) {
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 16, TN = WTN / 16;
    static_assert(WAVES_M * WAVES_N == 4, "4 waves");
    static_assert(TM >= 1 && TN >= 1, "wave tile");
    __shared__ float As[BM][LDK];
    __shared__ float Bs[BN][LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int lr = lane & 15, lg = lane >> 4;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM, b = blockIdx.z;
    const float *A = a.A + (int64_t)b * a.sA;
    const float *B = a.B + (int64_t)b * a.sB;
    const int M = a.M, N = a.N, K = a.K;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    Stage<BM, BN, VEC> st;
    st.load(A, B, M, N, K, m0, n0, 0, tid);
    for (int k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();
        st.store(As, Bs, tid);
        __syncthreads();
        if (k0 + BK < K) st.load(A, B, M, N, K, m0, n0, k0 + BK, tid);
#pragma unroll
        for (int kq = 0; kq < BK; kq += 16) {
            float4 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = ld4(&As[wm * WTM + i * 16 + lr][kq + 4 * lg]);
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = ld4(&Bs[wn * WTN + j * 16 + lr][kq + 4 * lg]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    acc[i][j] = mfma16(af[i].x, bf[j].x, acc[i][j]);
                    acc[i][j] = mfma16(af[i].y, bf[j].y, acc[i][j]);
                    acc[i][j] = mfma16(af[i].z, bf[j].z, acc[i][j]);
                    acc[i][j] = mfma16(af[i].w, bf[j].w, acc[i][j]);
                }
        }
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
                const int m = m0 + wm * WTM + i * 16 + 4 * lg + r;
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

}  // namespace gemm

// Entry points: mx_gemm_<BM>x<BN>[_v4]. _v4 reads A with 128-bit loads and
// needs K % 4 == 0 and A 16-byte aligned; the plain form has no requirement.
#define MXK_GEMM(BM, BN, WM, WN)                                                                   \
    extern "C" __global__ __launch_bounds__(256) void mx_gemm_##BM##x##BN(GemmArgs a) {            \
        gemm::body<BM, BN, WM, WN, false>(a);                                                      \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(256) void mx_gemm_##BM##x##BN##_v4(GemmArgs a) {       \
        gemm::body<BM, BN, WM, WN, true>(a);                                                       \
    }

MXK_GEMM(128, 128, 2, 2)
MXK_GEMM(64, 128, 2, 2)
MXK_GEMM(128, 64, 2, 2)
MXK_GEMM(64, 64, 2, 2)
MXK_GEMM(32, 128, 1, 4)
MXK_GEMM(32, 64, 2, 2)

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
