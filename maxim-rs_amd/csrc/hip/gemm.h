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

// Output modes: plain (bias by row or column), fused (bias then the
// Epilogue), and the transposed-conv scatter.
enum { PLAIN = 0, FUSED = 1, CONVT = 2 };

template <int BM, int BN, int WAVES_M, int WAVES_N, bool VEC, int MODE>
__device__ void body(const GemmArgs &a) {
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 16, TN = WTN / 16;
    constexpr int LDS = WTN + 4;  // row pitch of a wave's output staging tile
    static_assert(WAVES_M * WAVES_N == 4, "4 waves");
    static_assert(TM >= 1 && TN >= 1, "wave tile");
    static_assert(4 * 16 * LDS <= (BM + BN) * LDK, "output staging must fit the operand tiles");
    __shared__ float smem[(BM + BN) * LDK];
    float (*As)[LDK] = reinterpret_cast<float (*)[LDK]>(smem);
    float (*Bs)[LDK] = reinterpret_cast<float (*)[LDK]>(smem + BM * LDK);

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

    float *C = a.C + (int64_t)b * a.sC;
    if (MODE == CONVT) {
        // Element r of acc[i][j] is row 4*(lane/16) + r, column lane%16; row
        // (tap, oc) and column (y, x) scatter to out[oc][2y + ky][2x + kx].
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = n0 + wn * WTN + j * 16 + lr;
                if (n >= N) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + wm * WTM + i * 16 + 4 * lg + r;
                    if (m >= M) continue;
                    const int tap = m / a.co, oc = m - tap * a.co;
                    const int y = n / a.wd, x = n - y * a.wd;
                    float v = acc[i][j][r];
                    if (a.bias) v = a.bias[oc] + v;
                    C[(int64_t)oc * (4 * (int64_t)N) + (2 * y + (tap >> 1)) * (2 * (int64_t)a.wd) + 2 * x + (tap & 1)] = v;
                }
            }
        return;
    }

    // Stage each 16-row slab of the wave's tile in LDS (the operand tiles are
    // free now) and write it out row-contiguous, four columns per lane.
    __syncthreads();
    float *sw = smem + wave * (16 * LDS);
    const bool vec = (N % 4) == 0 && a.cvec;
    constexpr int PER = 16 * WTN / 4 / 64;  // float4s per lane per slab
    static_assert(PER * 64 * 4 == 16 * WTN, "slab split");
    // One float4 at a time through the fused epilogue keeps its registers
    // (erf and three operand loads per element) from multiplying.
    constexpr int QU = MODE == FUSED ? 1 : PER;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) sw[(4 * lg + r) * LDS + j * 16 + lr] = acc[i][j][r];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll QU
        for (int q = 0; q < PER; ++q) {
            const int e = lane + q * 64;
            const int row = e / (WTN / 4), c4 = (e % (WTN / 4)) * 4;
            const int m = m0 + wm * WTM + i * 16 + row;
            const int n = n0 + wn * WTN + c4;
            if (m >= M || n >= N) continue;
            float v[4];
            {
                const float4 t = ld4(&sw[row * LDS + c4]);
                v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
            }
            const int64_t row_off = (int64_t)m * N;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (a.bias_mode == MXK_BIAS_ROW) v[t] = a.bias[m] + v[t];
                else if (a.bias_mode == MXK_BIAS_COL && n + t < N) v[t] = a.bias[n + t] + v[t];
            }
            if (MODE == FUSED) {
                const int64_t base = (int64_t)b * a.sC + row_off + n;
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (n + t < N) v[t] = epilogue(a.e, v[t], base + t);
            }
            if (vec && n + 3 < N) {
                st4(C + row_off + n, make_float4(v[0], v[1], v[2], v[3]));
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (n + t < N) C[row_off + n + t] = v[t];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

}  // namespace gemm

// Entry points: mx_gemm_<BM>x<BN>[_v4][_f|_t]. _v4 reads A with 128-bit loads
// and needs K % 4 == 0 and A 16-byte aligned; _f applies the fused epilogue,
// _t is the transposed-conv scatter.
#define MXK_GEMM1(BM, BN, WM, WN, VEC, MODE, SUF)                                                 \
    extern "C" __global__ __launch_bounds__(256) void mx_gemm_##BM##x##BN##SUF(GemmArgs a) {      \
        gemm::body<BM, BN, WM, WN, VEC, gemm::MODE>(a);                                           \
    }
#define MXK_GEMM(BM, BN, WM, WN)                          \
    MXK_GEMM1(BM, BN, WM, WN, false, PLAIN, )             \
    MXK_GEMM1(BM, BN, WM, WN, true, PLAIN, _v4)           \
    MXK_GEMM1(BM, BN, WM, WN, false, FUSED, _f)           \
    MXK_GEMM1(BM, BN, WM, WN, true, FUSED, _v4_f)         \
    MXK_GEMM1(BM, BN, WM, WN, false, CONVT, _t)           \
    MXK_GEMM1(BM, BN, WM, WN, true, CONVT, _v4_t)

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
