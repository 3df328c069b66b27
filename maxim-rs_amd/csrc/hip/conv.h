// Implicit-GEMM convolutions on the fp32 matrix cores: 3x3 pad 1 and 4x4
// stride 2 (flax SAME). out[m][p] = b[m] + sum_{tap, c} W[m][tap][c] * x[c][p + tap]
// with zero padding.
//
// A block owns BM output channels x a TH x TW output tile, and walks the
// input channels in chunks of CK. Per chunk it stages in LDS
//   - the weight slice, which the host has already laid out as the exact
//     [KC][BM] tile (KC = taps * CK, k = tap * CK + c) of each (m-block,
//     chunk), so the fill is a straight 128-bit copy;
//   - the input halo of the tile, planar [c][rows][cols], zero outside the
//     image;
// and the B operand of every MFMA is read straight from the halo, so an input
// element is fetched from memory once per (tile, m-block), not once per tap.
// The next chunk is fetched into registers while the current one is multiplied.
#pragma once

#include "common.h"

namespace conv {

// XV (3x3, stride 1, 16-wide tiles, input rows 16-byte aligned and the
// output a whole number of tiles wide): the halo is fetched as four 128-bit
// loads per row (the tile's 16 columns) plus the two edge columns, each
// thread's row, column and channel offsets fixed for the block, and stored
// in LDS rows of HP = 24 floats with the tile's columns at 4..19 (16-byte
// aligned), the left edge at 3 and the right edge at 20.
// SPLIT: the reduction over input channels is split along the grid's z
// (a.ksplit chunks per slice); each slice writes its raw partial sums, no
// bias, to slice z of a.y ([z][co][oh][ow]), for mx_conv_split_sum.
template <int BM, int TH, int TW, int CK, int KS, int STRIDE, int WAVES_M, int WAVES_N, bool FUSED, bool XV = false,
          bool SPLIT = false>
__device__ void body(const ConvArgs &a) {
    constexpr int TAPS = KS * KS;
    constexpr int KC = TAPS * CK;
    constexpr int BN = TH * TW;
    constexpr int HH = (TH - 1) * STRIDE + KS, HW = (TW - 1) * STRIDE + KS;
    static_assert(!XV || (KS == 3 && STRIDE == 1 && TW == 16), "vector halo: 3x3, stride 1, 16 columns");
    constexpr int HP = XV ? 24 : HW;   // LDS row pitch of the halo
    constexpr int HC = XV ? 3 : 0;     // LDS column of halo column 0
    constexpr int HALO = CK * HH * HP;
    constexpr int NQ = CK * HH * 4;    // XV: 128-bit loads per chunk (four per row)
    constexpr int NE = CK * HH * 2;    // XV: edge columns per chunk
    constexpr int NQT = (NQ + 255) / 256;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int TM = WTM / 16, TN = WTN / 16;
    constexpr int LDM = BM + 4;
    constexpr int NW4 = KC * BM / 4;                // float4s in the weight tile
    constexpr int NW = (NW4 + 255) / 256;           // ... per thread
    constexpr int NH = (HALO + 255) / 256;          // halo elements per thread
    constexpr int LDS = WTN + 4;  // row pitch of a wave's output staging tile
    constexpr int POOL = KC * LDM + HALO > 4 * 16 * LDS ? KC * LDM + HALO : 4 * 16 * LDS;
    static_assert(KC % 4 == 0 && CK % 4 == 0 && BM % 16 == 0 && TW % 4 == 0, "tile");
    static_assert(WAVES_M * WAVES_N == 4 && TM >= 1 && TN >= 1, "wave grid");
    __shared__ float smem[POOL];
    float (*Ws)[LDM] = reinterpret_cast<float (*)[LDM]>(smem);
    float *Hs = smem + KC * LDM;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int lr = lane & 15, lk = lane >> 4;
    const int tiles_x = (a.ow + TW - 1) / TW;
    int tile, mb;
    xcd_tile(tile, mb);
    const int ty0 = (tile / tiles_x) * TH, tx0 = (tile % tiles_x) * TW;
    const int m0 = mb * BM;
    const int iy0 = ty0 * STRIDE - a.pad_top, ix0 = tx0 * STRIDE - a.pad_left;
    const int64_t plane = (int64_t)a.h * a.wd;
    const int nchunk = (a.ci + CK - 1) / CK;
    const float *wblk = a.w + (int64_t)mb * nchunk * (KC * BM);

    // The halo offset of each B column this lane reads, fixed for the block.
    int nofs[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = wn * WTN + j * 16 + lr;
        nofs[j] = (n / TW) * STRIDE * HP + (n % TW) * STRIDE + HC;
    }

    float4 wr[NW];
    float hr[XV ? 1 : NH];
    // Generic halo: this thread's elements e = tid + 256 i as (channel within
    // the chunk, offset c * plane + iy * wd + ix from the chunk's first plane;
    // -1 outside the image or the halo), fixed for the block, so a chunk's
    // fetch is unconditional loads from clamped addresses and selects (no
    // per-element branches, whose exec masks would crowd the scalar registers).
    int hc[XV ? 1 : NH], ho[XV ? 1 : NH];
    if (!XV) {
#pragma unroll
        for (int i = 0; i < NH; ++i) {
            const int e = tid + i * 256, c = e / (HH * HW), r = e % (HH * HW);
            const int iy = iy0 + r / HW, ix = ix0 + r % HW;
            hc[i] = c;
            ho[i] = (e < HALO && iy >= 0 && iy < a.h && ix >= 0 && ix < a.wd) ? c * (int)plane + iy * a.wd + ix : -1;
        }
    }
    // XV: this thread's 128-bit loads (channel c, halo row r, quarter k) and
    // edge column, as element offsets from the chunk's first channel plane
    // (-1: outside the image, stored as zeros) and LDS offsets.
    float4 qr[XV ? NQT : 1];
    float er = 0.0f;
    int qoff[XV ? NQT : 1], qlds[XV ? NQT : 1], eoff = -1, elds = 0;
    if (XV) {
#pragma unroll
        for (int i = 0; i < NQT; ++i) {
            const int q = tid + i * 256, c = q / (HH * 4), r = (q / 4) % HH, k = q % 4, iy = iy0 + r;
            qoff[i] = (q < NQ && iy >= 0 && iy < a.h) ? c * (int)plane + iy * a.wd + tx0 + 4 * k : -1;
            qlds[i] = q < NQ ? (c * HH + r) * HP + 4 + 4 * k : -1;
        }
        if (tid < NE) {
            const int c = tid / (HH * 2), r = (tid / 2) % HH, side = tid % 2, iy = iy0 + r;
            const int ix = side ? tx0 + 16 : tx0 - 1;
            eoff = (iy >= 0 && iy < a.h && ix >= 0 && ix < a.wd) ? c * (int)plane + iy * a.wd + ix : -1;
            elds = (c * HH + r) * HP + (side ? 20 : 3);
        }
    }
    auto fetch = [&](int chunk) {
        const float4 *src = reinterpret_cast<const float4 *>(wblk + (int64_t)chunk * (KC * BM));
#pragma unroll
        for (int i = 0; i < NW; ++i)
            if (tid + i * 256 < NW4) wr[i] = src[tid + i * 256];
        const int c0 = chunk * CK;
        if constexpr (XV) {
            // CK channels at a time; a chunk past the last channel reads zeros
            const int cmax = a.ci - c0;
            const float *xc = a.x + (int64_t)c0 * plane;
#pragma unroll
            for (int i = 0; i < NQT; ++i) {
                const int c = (tid + i * 256) / (HH * 4);
                qr[i] = (qoff[i] >= 0 && c < cmax) ? ld4(xc + qoff[i]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            er = (eoff >= 0 && tid / (HH * 2) < cmax) ? xc[eoff] : 0.0f;
        } else {
            const float *xc = a.x + (int64_t)c0 * plane;  // chunk < nchunk: c0 < ci
            const int cmax = a.ci - c0;
#pragma unroll
            for (int i = 0; i < NH; ++i) {
                const bool ok = ho[i] >= 0 && hc[i] < cmax;
                const float v = xc[ok ? ho[i] : 0];
                hr[i] = ok ? v : 0.0f;
            }
        }
    };

    // This lane's LDS read bases: its k row of the weight tile (k = kk + lk)
    // and its channel plane of the halo at each of its B columns; every step
    // of the reduction adds a constant to them, so the fully unrolled loop
    // below addresses LDS through instruction offsets alone.
    const float *wl = &Ws[lk][wm * WTM + lr];
    const float *hl[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) hl[j] = Hs + lk * (HH * HP) + nofs[j];

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int cbeg = SPLIT ? (int)blockIdx.z * a.ksplit : 0;
    const int cend = SPLIT ? min(nchunk, cbeg + a.ksplit) : nchunk;
    fetch(cbeg);
    for (int chunk = cbeg; chunk < cend; ++chunk) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const int e = (tid + i * 256) * 4;
            if (e < KC * BM) st4(&Ws[e / BM][e % BM], wr[i]);
        }
        if constexpr (XV) {
#pragma unroll
            for (int i = 0; i < NQT; ++i)
                if (qlds[i] >= 0) st4(Hs + qlds[i], qr[i]);
            if (tid < NE) Hs[elds] = er;
        } else {
#pragma unroll
            for (int i = 0; i < NH; ++i) {
                const int e = tid + i * 256;
                if (e < HALO) Hs[e] = hr[i];
            }
        }
        __syncthreads();
        if (chunk + 1 < cend) fetch(chunk + 1);
        // k = kk + lk: tap kk / CK (CK % 4 == 0), channel kk % CK + lk
#pragma unroll
        for (int kk = 0; kk < KC; kk += 4) {
            const int tap = kk / CK, hofs = (kk % CK) * (HH * HP) + (tap / KS) * HP + (tap % KS);
            float af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = wl[kk * LDM + i * 16];
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = hl[j][hofs];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
        }
    }

    // Stage each 16-channel slab of the wave's tile in LDS and write it out as
    // rows of four adjacent output pixels per lane.
    const int64_t oplane = (int64_t)a.oh * a.ow;
    float *yout = SPLIT ? a.y + (int64_t)blockIdx.z * a.co * oplane : a.y;
    __syncthreads();
    float *sw = smem + wave * (16 * LDS);
    constexpr int PER = 16 * WTN / 4 / 64;
    static_assert(PER * 64 * 4 == 16 * WTN, "slab split");
    // One float4 at a time through the fused epilogue keeps its registers
    // (erf and three operand loads per element) from multiplying.
    constexpr int QU = FUSED ? 1 : PER;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) sw[(4 * lk + r) * LDS + j * 16 + lr] = acc[i][j][r];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll QU
        for (int q = 0; q < PER; ++q) {
            const int e = lane + q * 64;
            const int row = e / (WTN / 4), c4 = (e % (WTN / 4)) * 4;
            const int m = m0 + wm * WTM + i * 16 + row;
            const int n = wn * WTN + c4;
            const int oy = ty0 + n / TW, ox = tx0 + n % TW;
            if (m >= a.co || oy >= a.oh || ox >= a.ow) continue;
            const float4 t = ld4(&sw[row * LDS + c4]);
            float v[4] = {t.x, t.y, t.z, t.w};
            const int64_t idx = m * oplane + (int64_t)oy * a.ow + ox;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (a.bias && !SPLIT) v[u] = a.bias[m] + v[u];
            if (FUSED) {
                // (past the row's end there is nothing to read: the lanes
                // of a ragged last column group skip those elements)
                if (a.cvec && ox + 3 < a.ow) {
                    epilogue4(a.e, v, idx);
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (ox + u < a.ow) v[u] = epilogue(a.e, v[u], idx + u);
                }
            }
            if (a.cvec && ox + 3 < a.ow) {
                st4(yout + idx, make_float4(v[0], v[1], v[2], v[3]));
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (ox + u < a.ow) yout[idx + u] = v[u];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

}  // namespace conv

// mx_conv3x3_m<BM>_t<TH>[_c4][_f]: BM output channels x a TH x 16 output
// tile, CK = 8 input channels per chunk (4 for the _c4 RGB-input forms); _f
// applies the fused epilogue.
#define MXK_CONV3(BM, TH, CK, WM, WN, SUF)                                                        \
    extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_m##BM##_t##TH##SUF(ConvArgs a) {   \
        conv::body<BM, TH, 16, CK, 3, 1, WM, WN, false>(a);                                       \
    }                                                                                             \
    extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_m##BM##_t##TH##SUF##_f(ConvArgs a) { \
        conv::body<BM, TH, 16, CK, 3, 1, WM, WN, true>(a);                                        \
    }
// mx_conv3x3v_m<BM>_t<TH>[_f]: the same with the vector halo fetch (XV).
#define MXK_CONV3V(BM, TH, WM, WN)                                                                 \
    extern "C" __global__ __launch_bounds__(256) void mx_conv3x3v_m##BM##_t##TH(ConvArgs a) {       \
        conv::body<BM, TH, 16, 8, 3, 1, WM, WN, false, true>(a);                                   \
    }                                                                                             \
    extern "C" __global__ __launch_bounds__(256) void mx_conv3x3v_m##BM##_t##TH##_f(ConvArgs a) {   \
        conv::body<BM, TH, 16, 8, 3, 1, WM, WN, true, true>(a);                                    \
    }
MXK_CONV3V(16, 8, 1, 4)
MXK_CONV3V(32, 8, 1, 4)
MXK_CONV3V(64, 8, 2, 2)
MXK_CONV3V(128, 8, 2, 2)
MXK_CONV3V(32, 4, 2, 2)
MXK_CONV3V(64, 4, 2, 2)
MXK_CONV3V(128, 4, 4, 1)
MXK_CONV3(16, 8, 8, 1, 4, )
MXK_CONV3(32, 8, 8, 1, 4, )
MXK_CONV3(64, 8, 8, 2, 2, )
MXK_CONV3(128, 8, 8, 2, 2, )
MXK_CONV3(32, 4, 8, 2, 2, )
MXK_CONV3(64, 4, 8, 2, 2, )
MXK_CONV3(128, 4, 8, 4, 1, )
MXK_CONV3(32, 8, 4, 1, 4, _c4)
MXK_CONV3(64, 8, 4, 2, 2, _c4)
MXK_CONV3(128, 8, 4, 2, 2, _c4)
MXK_CONV3(32, 4, 4, 2, 2, _c4)
MXK_CONV3(64, 4, 4, 2, 2, _c4)
MXK_CONV3(128, 4, 4, 4, 1, _c4)

// mx_conv4x4_m<BM>_t<TH>[_s]: 4x4 stride 2 SAME, CK = 4, TH x 16 outputs
// over a (2 TH + 2) x 34 input halo; _s: the reduction split along z.
#define MXK_CONV4(BM, TH, WM, WN)                                                               \
    extern "C" __global__ __launch_bounds__(256) void mx_conv4x4_m##BM##_t##TH(ConvArgs a) {    \
        conv::body<BM, TH, 16, 4, 4, 2, WM, WN, false>(a);                                      \
    }                                                                                           \
    extern "C" __global__ __launch_bounds__(256) void mx_conv4x4_m##BM##_t##TH##_s(ConvArgs a) { \
        conv::body<BM, TH, 16, 4, 4, 2, WM, WN, false, false, true>(a);                         \
    }
MXK_CONV4(32, 8, 1, 4)
MXK_CONV4(64, 8, 2, 2)
MXK_CONV4(128, 8, 2, 2)
MXK_CONV4(32, 4, 2, 2)
MXK_CONV4(64, 4, 2, 2)
MXK_CONV4(128, 4, 4, 1)

// 3x3 pad 1 with at most four output channels (the stage outputs to RGB): on
// the vector ALUs, where an MFMA tile would be 3/16 useful. A block owns an
// 8 x 8 output tile; its four waves split the input channels (wave w takes
// c = w, w + 4, ...), each staging a group of its channels' 10 x 10 halos in
// its own LDS rows (no block barrier) with the next group's halos already in
// flight, and each lane accumulates its pixel's outputs (weights are
// wave-uniform, read through the scalar cache) in ascending channel order;
// the four partial sums are added in LDS in a fixed order (wave 0 + 1 + 2 +
// 3), then bias and the epilogue. The grid is one-dimensional (gridDim.y = 1).
namespace conv {

template <bool FUSED>
__device__ void co4(const ConvArgs &a) {
    // A wave takes its channels CG at a time (channels w, w + 4, ... in
    // groups of CG consecutive ones of its own), the next group's halos in
    // flight while the current group is multiplied.
    constexpr int CG = 4;
    __shared__ float halo[4][CG][100];
    __shared__ float part[4][4][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tiles_x = (a.wd + 7) / 8;
    // each XCD walks one contiguous run of tiles (row-major), so the tiles
    // whose halos share cache lines (left-right neighbours share a 128-byte
    // line four tiles wide, rows above and below share halo rows) are
    // fetched into the same L2
    int tile, band;
    xcd_tile(tile, band);
    const int ty0 = (tile / tiles_x) * 8, tx0 = (tile % tiles_x) * 8;
    const int py = lane / 8, px = lane % 8;
    const int64_t plane = (int64_t)a.h * a.wd;
    // the halo elements this lane stages: e = lane and lane + 64 (< 100)
    int hoff[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int e = lane + 64 * k, iy = ty0 - 1 + e / 10, ix = tx0 - 1 + e % 10;
        hoff[k] = (e < 100 && iy >= 0 && iy < a.h && ix >= 0 && ix < a.wd) ? iy * a.wd + ix : -1;
    }
    // group g of this wave: channels (4 g + wave) ... in steps of 4 (the
    // wave's g-th run of CG of its own channels)
    auto chan = [&](int g, int j) { return 4 * (CG * g + j) + wave; };
    auto fetch = [&](int g, float *r) {
#pragma unroll
        for (int j = 0; j < CG; ++j) {
            const int c = chan(g, j);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const bool ok = c < a.ci && hoff[k] >= 0;
                const float v = a.x[(ok ? c : 0) * plane + (ok ? hoff[k] : 0)];
                r[2 * j + k] = ok ? v : 0.0f;
            }
        }
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float cur[2 * CG], nxt[2 * CG];
    const int ng = (a.ci + 4 * CG - 1) / (4 * CG);  // groups (every wave takes the same count)
    fetch(0, cur);
    for (int g = 0; g < ng; ++g) {
        if (g + 1 < ng) fetch(g + 1, nxt);
#pragma unroll
        for (int j = 0; j < CG; ++j) {
            halo[wave][j][lane] = cur[2 * j];
            if (lane < 36) halo[wave][j][lane + 64] = cur[2 * j + 1];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < CG; ++j) {
            const int c = chan(g, j);
            if (c >= a.ci) break;  // wave-uniform
            const float *w = a.w + (int64_t)c * 36;  // [c][tap][4]: wave-uniform
#pragma unroll
            for (int tap = 0; tap < 9; ++tap) {
                const float xv = halo[wave][j][(py + tap / 3) * 10 + px + tap % 3];
#pragma unroll
                for (int o = 0; o < 4; ++o) acc[o] = __builtin_fmaf(w[tap * 4 + o], xv, acc[o]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int k = 0; k < 2 * CG; ++k) cur[k] = nxt[k];
    }
#pragma unroll
    for (int o = 0; o < 4; ++o) part[o][wave][lane] = acc[o];
    __syncthreads();
    if (wave != 0) return;
    const int oy = ty0 + py, ox = tx0 + px;
    if (oy >= a.oh || ox >= a.ow) return;
    for (int o = 0; o < a.co; ++o) {
        float v = part[o][0][lane];
        v = v + part[o][1][lane];
        v = v + part[o][2][lane];
        v = v + part[o][3][lane];
        if (a.bias) v = a.bias[o] + v;
        const int64_t idx = o * (int64_t)a.oh * a.ow + (int64_t)oy * a.ow + ox;
        if (FUSED) v = epilogue(a.e, v, idx);
        a.y[idx] = v;
    }
}

}  // namespace conv

// mx_conv3x3_co4[_f]: 3x3 pad 1 to at most four output channels (weights
// [c_in][9][4], zero beyond c_out), one 8 x 8 output tile per block.
extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_co4(ConvArgs a) { conv::co4<false>(a); }
extern "C" __global__ __launch_bounds__(256) void mx_conv3x3_co4_f(ConvArgs a) { conv::co4<true>(a); }

// y = bias + the z-ordered sum of a split-reduction conv's partial outputs
// (ConvSumArgs), four elements per thread.
extern "C" __global__ __launch_bounds__(256) void mx_conv_split_sum(ConvSumArgs a) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (i >= a.n) return;
    float4 s = ld4(a.part + i);
    for (int z = 1; z < a.nsplit; ++z) {
        const float4 t = ld4(a.part + (int64_t)z * a.n + i);
        s.x = s.x + t.x;
        s.y = s.y + t.y;
        s.z = s.z + t.z;
        s.w = s.w + t.w;
    }
    if (a.bias) {
        const float b = a.bias[i / a.plane];
        s.x = b + s.x;
        s.y = b + s.y;
        s.z = b + s.z;
        s.w = b + s.w;
    }
    st4(a.y + i, s);
}
