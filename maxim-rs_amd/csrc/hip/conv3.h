// 3x3 convolution (pad 1) on the fp32 matrix cores, for input-channel counts
// that are a multiple of 16: out[m][y][x] = b[m] + sum_{tap, c} W[m][c][tap] *
// x[c][y + dy][x + dx], zero outside the image.
//
// A block owns BM output channels x TH rows x 16 columns and walks the input
// channels in chunks of 16. Per chunk it stages in LDS
//   - the input halo, channel-last: [TH + 2][18][16 (+4 pad)], so a lane's
//     four consecutive channels of one pixel are one 128-bit read;
//   - the weights, which the host has laid out per (m-block, chunk) as
//     [BM][9 taps][16 channels], m-major with the channels contiguous, rows
//     padded to 148 floats;
// both paddings put the 128-bit reads of 16 lanes on distinct banks. The
// next chunk is fetched into registers while the current one multiplies.
//
// MFMA 16x16x4: rows are 16 adjacent pixels of one output row (lane i <->
// column x0 + i), columns are 16 output channels, and lane group g supplies
// channels 4g .. 4g + 3 of the chunk at steps t = 0..3 of each tap - so the
// accumulator of lane (g, i) holds pixels x0 + 4g .. + 3 of channel i, one
// 128-bit store per (row, channel tile), 64-byte runs per channel row.
#pragma once

#include "common.h"

namespace c3 {

constexpr int CK = 16;            // input channels per chunk
constexpr int CKP = CK + 4;       // channel-last pixel pitch in LDS
constexpr int KP = 9 * CK + 4;    // weight row pitch in LDS
constexpr int HWD = 18;           // halo width (16 + 2)

__device__ __forceinline__ float comp(const float4 &v, int t) {
    return t == 0 ? v.x : t == 1 ? v.y : t == 2 ? v.z : v.w;
}

template <int BM, int TH, int WAVES_M, int WAVES_N, bool FUSED>
__device__ void body(const ConvArgs &a) {
    constexpr int HH = TH + 2;
    constexpr int WTM = BM / WAVES_M, TM = WTM / 16;
    constexpr int TN = TH / WAVES_N;            // output rows (pixel tiles) per wave
    static_assert(WAVES_M * WAVES_N == 4 && TM >= 1 && TN >= 1 && TH % WAVES_N == 0, "wave grid");
    // global -> register staging: the halo as (channel, row) segments of 16
    // interior floats (four 128-bit loads) and two edge floats; the weights
    // as 128-bit pieces
    constexpr int HITEMS = CK * HH * 6;
    constexpr int NH = (HITEMS + 255) / 256;
    constexpr int W4 = BM * 9 * CK / 4;
    constexpr int NW = (W4 + 255) / 256;
    __shared__ float halo[HH * HWD * CKP];
    __shared__ float wts[BM * KP];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int i = lane & 15, g = lane >> 4;
    const int tiles_x = (a.wd + 15) / 16;
    int tile, mb;
    xcd_tile(tile, mb);
    const int ty0 = (tile / tiles_x) * TH, tx0 = (tile % tiles_x) * 16;
    const int m0 = mb * BM;
    const int64_t plane = (int64_t)a.h * a.wd;
    const int nchunk = a.ci / CK;
    const float *wblk = a.w + (int64_t)mb * nchunk * (BM * 9 * CK);

    float4 hr[NH];
    float4 wr[NW];
    auto fetch = [&](int chunk) {
        const int c0 = chunk * CK;
#pragma unroll
        for (int k = 0; k < NH; ++k) {
            const int q = tid + k * 256;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (q < HITEMS) {
                const int seg = q / 6, part = q % 6;
                const int c = seg / HH, row = seg % HH;
                const int y = ty0 - 1 + row;
                if (y >= 0 && y < a.h) {
                    const float *src = a.x + (c0 + c) * plane + (int64_t)y * a.wd;
                    if (part < 4) {
                        const int x = tx0 + 4 * part;
                        if (x < a.wd) v = ld4(src + x);
                    } else {
                        const int x = part == 4 ? tx0 - 1 : tx0 + 16;
                        if (x >= 0 && x < a.wd) v.x = src[x];
                    }
                }
            }
            hr[k] = v;
        }
        const float4 *ws = reinterpret_cast<const float4 *>(wblk + (int64_t)chunk * (BM * 9 * CK));
#pragma unroll
        for (int k = 0; k < NW; ++k)
            if (tid + k * 256 < W4) wr[k] = ws[tid + k * 256];
    };
    auto stage = [&]() {
#pragma unroll
        for (int k = 0; k < NH; ++k) {
            const int q = tid + k * 256;
            if (q >= HITEMS) continue;
            const int seg = q / 6, part = q % 6;
            const int c = seg / HH, row = seg % HH;
            float *d = &halo[(row * HWD) * CKP + c];
            if (part < 4) {
                const int col = 1 + 4 * part;
                d[(col + 0) * CKP] = hr[k].x;
                d[(col + 1) * CKP] = hr[k].y;
                d[(col + 2) * CKP] = hr[k].z;
                d[(col + 3) * CKP] = hr[k].w;
            } else {
                d[(part == 4 ? 0 : 17) * CKP] = hr[k].x;
            }
        }
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            const int e = (tid + k * 256) * 4;  // [m][tap][c] element index
            if (e < BM * 9 * CK) st4(&wts[(e / (9 * CK)) * KP + e % (9 * CK)], wr[k]);
        }
    };

    f32x4 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int mt = 0; mt < TM; ++mt) acc[j][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    fetch(0);
    for (int chunk = 0; chunk < nchunk; ++chunk) {
        __syncthreads();
        stage();
        __syncthreads();
        if (chunk + 1 < nchunk) fetch(chunk + 1);
#pragma unroll 3
        for (int tap = 0; tap < 9; ++tap) {
            const int dy = tap / 3, dx = tap % 3;
            float4 av[TN], bv[TM];
#pragma unroll
            for (int j = 0; j < TN; ++j)
                av[j] = ld4(&halo[((wn * TN + j + dy) * HWD + i + dx) * CKP + 4 * g]);
#pragma unroll
            for (int mt = 0; mt < TM; ++mt)
                bv[mt] = ld4(&wts[(wm * WTM + mt * 16 + i) * KP + tap * CK + 4 * g]);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int mt = 0; mt < TM; ++mt)
                        acc[j][mt] = mfma16(comp(av[j], t), comp(bv[mt], t), acc[j][mt]);
        }
    }

    // acc[j][mt][r] = out[m0 + wm * WTM + mt * 16 + i][ty0 + wn * TN + j][tx0 + 4 g + r]
    const int x = tx0 + 4 * g;
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) {
        const int m = m0 + wm * WTM + mt * 16 + i;
        if (m >= a.co || x >= a.ow) continue;
        const float bb = a.bias ? a.bias[m] : 0.0f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int y = ty0 + wn * TN + j;
            if (y >= a.oh) continue;
            float v[4] = {acc[j][mt][0], acc[j][mt][1], acc[j][mt][2], acc[j][mt][3]};
            if (a.bias) {
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = bb + v[u];
            }
            const int64_t idx = m * plane + (int64_t)y * a.ow + x;
            if (FUSED) {
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = epilogue(a.e, v[u], idx + u);
            }
            st4(a.y + idx, make_float4(v[0], v[1], v[2], v[3]));
        }
    }
}

}  // namespace c3

// mx_c3_m<BM>_t<TH>[_f]: BM output channels x TH rows x 16 columns per block;
// needs c_in % 16 == 0, width % 4 == 0 and 16-byte aligned x and y.
#define MXK_C3(BM, TH, WM, WN)                                                                    \
    extern "C" __global__ __launch_bounds__(256) void mx_c3_m##BM##_t##TH(ConvArgs a) {          \
        c3::body<BM, TH, WM, WN, false>(a);                                                       \
    }                                                                                             \
    extern "C" __global__ __launch_bounds__(256) void mx_c3_m##BM##_t##TH##_f(ConvArgs a) {      \
        c3::body<BM, TH, WM, WN, true>(a);                                                        \
    }
MXK_C3(32, 8, 1, 4)
MXK_C3(64, 4, 1, 4)
MXK_C3(64, 2, 2, 2)
