// Implicit-GEMM convolutions on the fp32 matrix cores: 3x3 pad 1 and 4x4
// stride 2 (flax SAME). out[m][p] = b[m] + sum_{tap, c} W[m][tap][c] * x[c][p + tap]
// with zero padding. Weights arrive re-laid out as [co][tap][ci].
//
// A block owns BM output channels x a TH x TW output tile. Per chunk of CK
// input channels it stages the weight slice (k-major) and the input halo of
// the tile (planar [c][rows][cols], zero outside the image) in LDS; the B
// operand of every MFMA is read straight from the halo, so each input
// element is fetched from memory once per (tile, m-block) instead of
// once per tap.
#pragma once

#include "common.h"

template <int BM, int TH, int TW, int CK, int KS, int STRIDE, int WAVES_M, int WAVES_N>
__device__ void conv_body(const ConvArgs &a) {
    constexpr int TAPS = KS * KS;
    constexpr int KC = TAPS * CK;
    constexpr int BN = TH * TW;
    constexpr int HH = (TH - 1) * STRIDE + KS, HW = (TW - 1) * STRIDE + KS;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 16, TN = WTN / 16;
    static_assert(KC % 4 == 0, "K chunk must be a multiple of the MFMA K");
    static_assert(WAVES_M * WAVES_N == 4, "4 waves");
    __shared__ float Ws[KC][BM + 4];
    __shared__ float Hs[CK][HH][HW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int lr = lane & 15, lk = lane >> 4;
    const int tiles_x = (a.ow + TW - 1) / TW;
    const int ty0 = (blockIdx.x / tiles_x) * TH, tx0 = (blockIdx.x % tiles_x) * TW;
    const int m0 = blockIdx.y * BM;
    const int iy0 = ty0 * STRIDE - a.pad_top, ix0 = tx0 * STRIDE - a.pad_left;
    const int64_t plane = (int64_t)a.h * a.wd;

    // The halo offset of each B column this lane reads, fixed for the block.
    int nofs[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = wn * WTN + j * 16 + lr;
        const int ty = n / TW, tx = n % TW;
        nofs[j] = ty * STRIDE * HW + tx * STRIDE;
    }

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int c0 = 0; c0 < a.ci; c0 += CK) {
        for (int i = tid; i < KC * BM; i += 256) {
            const int m = i / KC, k = i % KC;
            const int tap = k / CK, c = k % CK;
            const int gm = m0 + m, gc = c0 + c;
            Ws[k][m] = (gm < a.co && gc < a.ci) ? a.w[((int64_t)gm * TAPS + tap) * a.ci + gc] : 0.0f;
        }
        for (int i = tid; i < CK * HH * HW; i += 256) {
            const int c = i / (HH * HW), r = i % (HH * HW);
            const int hy = r / HW, hx = r % HW;
            const int gc = c0 + c, iy = iy0 + hy, ix = ix0 + hx;
            float v = 0.0f;
            if (gc < a.ci && iy >= 0 && iy < a.h && ix >= 0 && ix < a.wd) v = a.x[gc * plane + (int64_t)iy * a.wd + ix];
            Hs[c][hy][hx] = v;
        }
        __syncthreads();
#pragma unroll 4
        for (int kk = 0; kk < KC; kk += 4) {
            const int k = kk + lk;
            const int tap = k / CK, c = k % CK;
            const int ky = tap / KS, kx = tap % KS;
            const float *hb = &Hs[c][ky][kx];
            float af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = Ws[k][wm * WTM + i * 16 + lr];
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = hb[nofs[j]];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
        }
        __syncthreads();
    }

    const int64_t oplane = (int64_t)a.oh * a.ow;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = wn * WTN + j * 16 + lr;
        const int oy = ty0 + n / TW, ox = tx0 + n % TW;
        if (oy >= a.oh || ox >= a.ow) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * WTM + i * 16 + 4 * lk + r;
                if (m >= a.co) continue;
                float v = acc[i][j][r];
                if (a.bias) v = a.bias[m] + v;
                a.y[m * oplane + (int64_t)oy * a.ow + ox] = v;
            }
        }
    }
}

// 3x3 pad 1: tile 8 x 16 outputs.
extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_m32(ConvArgs a) {
    conv_body<32, 8, 16, 8, 3, 1, 1, 4>(a);
}
extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_m64(ConvArgs a) {
    conv_body<64, 8, 16, 8, 3, 1, 2, 2>(a);
}
extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_m128(ConvArgs a) {
    conv_body<128, 8, 16, 8, 3, 1, 2, 2>(a);
}
// Few input channels (the RGB input convs): CK = 4.
extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_m32_c4(ConvArgs a) {
    conv_body<32, 8, 16, 4, 3, 1, 1, 4>(a);
}
extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_m64_c4(ConvArgs a) {
    conv_body<64, 8, 16, 4, 3, 1, 2, 2>(a);
}
extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_m128_c4(ConvArgs a) {
    conv_body<128, 8, 16, 4, 3, 1, 2, 2>(a);
}

// 4x4 stride 2 SAME: tile 8 x 16 outputs over an 18 x 34 input halo.
extern "C" __global__ __launch_bounds__(256) void mx_conv4x4_m32(ConvArgs a) {
    conv_body<32, 8, 16, 4, 4, 2, 1, 4>(a);
}
extern "C" __global__ __launch_bounds__(256) void mx_conv4x4_m64(ConvArgs a) {
    conv_body<64, 8, 16, 4, 4, 2, 2, 2>(a);
}
extern "C" __global__ __launch_bounds__(256) void mx_conv4x4_m128(ConvArgs a) {
    conv_body<128, 8, 16, 4, 4, 2, 2, 2>(a);
}
