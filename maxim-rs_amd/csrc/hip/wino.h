// 3x3 convolution (pad 1) by Winograd's minimal filtering F(2x2, 3x3) on the
// fp32 matrix cores (Lavin and Gray, "Fast Algorithms for Convolutional
// Neural Networks", 2016): each 2x2 output tile is
//     Y = A^T [ sum_c U[c] (.) V[c] ] A,   U = G g G^T,   V = B^T d B,
// with d the tile's 4x4 input patch (rows y - 1 .. y + 2) and g a 3x3
// filter, so the 9 multiplies per output of the direct form become 16 per
// four outputs. The sum over input channels is, for each of the 16 positions
// p of the 4x4 transform, a GEMM M_p[m][t] = sum_c U_p[m][c] V_p[c][t] over
// the output channels m and the block's tiles t, which is what the MFMAs do.
//
//   B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1]
//   G   = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1]
//   A^T = [1 1 1 0; 0 1 -1 -1]
//
// A block owns 32 output channels x a TR x TC grid of tiles (2TR x 2TC output
// pixels: 8 x 8, 8 x 16 or 4 x 32) and walks the input channels in chunks of
// 8. Per chunk the input halo ((2TR + 2) x (2TC + 2) per channel) is staged
// in LDS (128-bit loads of the tile's columns stored as words, the two edge
// columns as scalars; two buffers, so one block barrier per chunk). Wave w owns the transform row xi = w (positions
// p = 4w + nu, nu = 0..3), and each of its lanes transforms exactly the
// patches whose V its MFMA B operand needs - channel 4 ks + (lane / 16) of
// tile 16 ni + (lane % 16) - for that row only (B^T d needs two rows of the
// patch: d0 - d2, d1 + d2, d2 - d1 or d1 - d3), so V never goes through
// LDS. The A operand, U_p[m][c], comes straight from memory into registers
// (the host lays each (m-block, chunk) out lane by lane), fetched a chunk
// ahead. The output transform A^T . A runs in two halves: the column half
// (over nu) in registers, the row half (over xi, across the waves) after one
// exchange through LDS. The filter transform is the host's (weights are
// uploaded in the transformed domain, in double precision rounded once).
#pragma once

#include "common.h"

namespace wino {

constexpr int BM = 32;  // output channels per block
constexpr int CK = 8;   // input channels per chunk

// EP: -1 the generic fused epilogue, 16 a LeakyReLU only (the residual
// blocks' first conv; the same expression as the generic one).
template <int TC, bool FUSED, int EP = -1>
__device__ void body(const ConvArgs &a) {
    constexpr int TR = TC == 16 ? 2 : 4;  // tile rows per block
    constexpr int NT = TR * TC;          // tiles per block
    constexpr int OW = 2 * TC;           // output columns per block
    constexpr int HH = 2 * TR + 2;       // halo rows
    constexpr int HP = OW + 8;           // halo LDS pitch: columns at 3 .. OW + 4
    constexpr int MP = NT == 32 ? 36 : 20;  // M pitch: the 4-row steps of a half-wave's stores on distinct banks
    constexpr int NQ = CK * HH * (OW / 4);  // 128-bit halo loads per chunk
    constexpr int NQT = (NQ + 255) / 256;
    constexpr int NE = CK * HH * 2;         // halo edge columns per chunk
    constexpr int NI = NT / 16;             // MFMA column tiles (tiles of 16)
    // channel pitch odd: the four channels of a wave's patch reads (tiles 2
    // columns apart) fall on both bank parities
    constexpr int CS = HH * HP + 1;
    constexpr int HALO = CK * CS;
    constexpr int MS = 4 * 2 * BM * MP;
    constexpr int POOL = 2 * HALO > MS ? 2 * HALO : MS;
    static_assert(TC == 16 || TC == 8 || TC == 4, "2 x 16, 4 x 8 or 4 x 4 tiles");
    static_assert(NE <= 256, "one edge per thread");
    __shared__ float smem[POOL];
    float *Ms = smem;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lk = lane >> 4;
    const int tiles_x = (a.ow + OW - 1) / OW;
    int tile, mb;
    xcd_tile(tile, mb);
    const int oy0 = (tile / tiles_x) * (2 * TR), ox0 = (tile % tiles_x) * OW;
    const int m0 = mb * BM;
    // the bias of this thread's (output channel, tile) pairs of the
    // epilogue, fetched now so its latency hides behind the main loop
    constexpr int PAIRS = BM * NT / 256;
    float bsv[PAIRS];
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) {
        const int m = m0 + (tid + q * 256) / NT;
        bsv[q] = a.bias && m < a.co ? a.bias[m] : 0.0f;
    }
    const int plane = a.h * a.wd;  // 8 planes < 2^31, checked by the host
    const int nchunk = (a.ci + CK - 1) / CK;
    // this block's transformed filters, [chunk][wave][lane][16]
    const float *ublk = a.w + ((int64_t)mb * nchunk) * (4 * 64 * 16);

    // the halo loads of this thread: offsets from the chunk's first channel
    // plane (-1: outside the image, zeros) and LDS offsets
    int qoff[NQT], qlds[NQT], eoff = -1, elds = 0;
#pragma unroll
    for (int i = 0; i < NQT; ++i) {
        const int q = tid + i * 256, c = q / (HH * (OW / 4)), r = (q / (OW / 4)) % HH, k = q % (OW / 4);
        const int iy = oy0 - 1 + r;
        qoff[i] = (q < NQ && iy >= 0 && iy < a.h) ? c * plane + iy * a.wd + ox0 + 4 * k : -1;
        qlds[i] = q < NQ ? c * CS + r * HP + 4 + 4 * k : -1;
    }
    if (tid < NE) {
        const int c = tid / (HH * 2), r = (tid / 2) % HH, side = tid % 2, iy = oy0 - 1 + r;
        const int ix = side ? ox0 + OW : ox0 - 1;
        eoff = (iy >= 0 && iy < a.h && ix >= 0 && ix < a.wd) ? c * plane + iy * a.wd + ix : -1;
        elds = c * CS + r * HP + (side ? OW + 4 : 3);
    }
    float4 qr[NQT], ur[4];
    float er = 0.0f;
    auto fetch_halo = [&](int chunk) {
        const int cmax = a.ci - chunk * CK;
        const float *xc = a.x + (int64_t)chunk * CK * plane;
#pragma unroll
        for (int i = 0; i < NQT; ++i) {
            const int c = (tid + i * 256) / (HH * (OW / 4));
            qr[i] = (qoff[i] >= 0 && c < cmax) ? ld4(xc + qoff[i]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        er = (eoff >= 0 && tid / (HH * 2) < cmax) ? xc[eoff] : 0.0f;
    };
    auto fetch_u = [&](int chunk) {
        const float *u = ublk + ((int64_t)chunk * 4 * 64 + wave * 64 + lane) * 16;
#pragma unroll
        for (int k = 0; k < 4; ++k) ur[k] = ld4(u + 4 * k);
    };

    // This wave's row of B^T d: T = d[r0] + sgn d[r1] (d0 - d2, d1 + d2,
    // d2 - d1, d1 - d3 for xi = 0..3), and this lane's patches: channel
    // 4 ks + lk of tile 16 ni + lr.
    const int r0 = wave == 0 ? 0 : wave == 3 ? 1 : wave == 1 ? 1 : 2;
    const int r1 = wave == 0 ? 2 : wave == 3 ? 3 : wave == 1 ? 2 : 1;
    const float sgn = wave == 1 ? 1.0f : -1.0f;
    int pofs[2][NI];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
            const int c = 4 * ks + lk, t = 16 * ni + lr;
            pofs[ks][ni] = c * CS + (t / TC) * 2 * HP + (t % TC) * 2 + 3;
        }

    f32x4 acc[4][2][NI];  // set by the first chunk

    fetch_halo(0);
    fetch_u(0);
    // first: chunk 0, whose multiplies start from an inline zero
    auto chunk_step = [&](int chunk, bool first) {
        float *Hs = smem + (chunk & 1) * HALO;
        // (every wave finished reading this buffer two chunks ago, before
        // the previous chunk's barrier)
#pragma unroll
        for (int i = 0; i < NQT; ++i)
            if (qlds[i] >= 0) {
                float *d = Hs + qlds[i];  // 4-byte aligned only
                d[0] = qr[i].x;
                d[1] = qr[i].y;
                d[2] = qr[i].z;
                d[3] = qr[i].w;
            }
        if (tid < NE) Hs[elds] = er;
        __syncthreads();
        if (chunk + 1 < nchunk) fetch_halo(chunk + 1);
        // V[xi][nu] of this lane's patches
        float v[2][NI][4];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) {
                const float *h0 = Hs + pofs[ks][ni] + r0 * HP, *h1 = Hs + pofs[ks][ni] + r1 * HP;
                float t[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) t[j] = __builtin_fmaf(sgn, h1[j], h0[j]);
                v[ks][ni][0] = t[0] - t[2];
                v[ks][ni][1] = t[1] + t[2];
                v[ks][ni][2] = t[2] - t[1];
                v[ks][ni][3] = t[1] - t[3];
            }
        const float uv[16] = {ur[0].x, ur[0].y, ur[0].z, ur[0].w, ur[1].x, ur[1].y, ur[1].z, ur[1].w,
                              ur[2].x, ur[2].y, ur[2].z, ur[2].w, ur[3].x, ur[3].y, ur[3].z, ur[3].w};
#pragma unroll
        for (int nu = 0; nu < 4; ++nu)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                    for (int ni = 0; ni < NI; ++ni) {
                        const f32x4 c = first && ks == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : acc[nu][mi][ni];
                        acc[nu][mi][ni] = mfma16(uv[(nu * 2 + ks) * 2 + mi], v[ks][ni][nu], c);
                    }
        if (chunk + 1 < nchunk) fetch_u(chunk + 1);
    };
    chunk_step(0, true);
    for (int chunk = 1; chunk < nchunk; ++chunk) chunk_step(chunk, false);

    // (.) A over nu in registers: u[dx] for this wave's transform row xi;
    // then the rows of all four waves meet in LDS as Ms[xi][dx][m][t].
    __syncthreads();
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float a0 = acc[0][mi][ni][r], a1 = acc[1][mi][ni][r], a2 = acc[2][mi][ni][r],
                            a3 = acc[3][mi][ni][r];
                const int m = mi * 16 + 4 * lk + r, t = ni * 16 + lr;
                Ms[((wave * 2 + 0) * BM + m) * MP + t] = a0 + a1 + a2;
                Ms[((wave * 2 + 1) * BM + m) * MP + t] = a1 - a2 - a3;
            }
    __syncthreads();
    // A^T . over xi, bias, epilogue, stores: thread -> (m, tile), tiles fastest
    // The host launches whole tiles along x (ow % 2 TC == 0), so each
    // pair's second column is inside the image; rows may be ragged.
    const int64_t oplane = (int64_t)a.oh * a.ow;
    const bool vec = a.cvec != 0;
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) {
        const int e = tid + q * 256, m = e / NT, t = e % NT;
        if (m0 + m >= a.co) continue;
        float u[4][2];
#pragma unroll
        for (int xi = 0; xi < 4; ++xi)
#pragma unroll
            for (int dx = 0; dx < 2; ++dx) u[xi][dx] = Ms[((xi * 2 + dx) * BM + m) * MP + t];
        float y[2][2];
#pragma unroll
        for (int dx = 0; dx < 2; ++dx) {
            y[0][dx] = u[0][dx] + u[1][dx] + u[2][dx];
            y[1][dx] = u[1][dx] - u[2][dx] - u[3][dx];
        }
        const int oy = oy0 + 2 * (t / TC), ox = ox0 + 2 * (t % TC);
        const int64_t ib = (int64_t)(m0 + m) * oplane + ox;
        const float bb = bsv[q];
#pragma unroll
        for (int dy = 0; dy < 2; ++dy) {
            if (oy + dy >= a.oh) continue;
            const int64_t idx = ib + (int64_t)(oy + dy) * a.ow;
            float v0 = bb + y[dy][0], v1 = bb + y[dy][1];
            if (EP == 16) {
                v0 = v0 >= 0.0f ? v0 : a.e.slope * v0;
                v1 = v1 >= 0.0f ? v1 : a.e.slope * v1;
            }
            if (vec) {
                if (FUSED && EP < 0) epilogue2(a.e, v0, v1, idx);
                *reinterpret_cast<float2 *>(a.y + idx) = make_float2(v0, v1);
            } else {
                if (FUSED && EP < 0) {
                    v0 = epilogue(a.e, v0, idx);
                    v1 = epilogue(a.e, v1, idx + 1);
                }
                a.y[idx] = v0;
                a.y[idx + 1] = v1;
            }
        }
    }
}

}  // namespace wino

// mx_wino3_t<TC>[_f]: 3x3 pad 1 by F(2x2, 3x3), 32 output channels x TR x TC
// tiles (TR = 2 for TC = 16, else 4) per block; _f applies the fused epilogue. The host
// guarantees: input rows 16-byte aligned (width % 4 == 0, aligned base) and
// output width a multiple of 2 TC; cvec: the output and every epilogue
// operand 8-byte aligned (paired loads and stores). _f_e16: the fused
// epilogue when it is a LeakyReLU alone.
#define MXK_WINO(TC)                                                                               \
    extern "C" __global__ __launch_bounds__(256) void mx_wino3_t##TC(ConvArgs a) {                  \
        wino::body<TC, false>(a);                                                                  \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(256) void mx_wino3_t##TC##_f(ConvArgs a) {              \
        wino::body<TC, true>(a);                                                                   \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(256) void mx_wino3_t##TC##_f_e16(ConvArgs a) {          \
        wino::body<TC, true, 16>(a);                                                               \
    }
MXK_WINO(16)
MXK_WINO(8)
MXK_WINO(4)
