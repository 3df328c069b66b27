// Streaming fp32 MFMA kernels for the Dense-shaped ops whose reduction is
// short next to their streamed axis: every 1x1 conv (K = c_in <= 512 over
// up to 286720 pixels) and both GateMm modes. Operands go straight from
// memory into the matrix cores with 128-bit loads (no LDS staging): each wave
// owns a 64 x (16 * TMW) output tile, or a quarter of its reduction, so a CU
// keeps many independent waves in flight and the epilogue of one overlaps
// the loads of another.
//
// Two layouts share one body (D = the 16x16 MFMA tile, lane l = 16g + i):
//
//   CH  Y[m][n] = bias[m] + sum_k W[m][k] X[k][n]       (conv1x1, GateMm mode 0)
//       A operand = X^T: lane i of tile j supplies pixel n0 + 16 (i % 4) +
//       4 (i / 4) + j, so one 128-bit load feeds four tiles (and the sixteen
//       lanes of a row still read 256 contiguous bytes), and the output
//       D_j[4g + r][i] = Y[m0 + i][n0 + 16r + 4g + j]: for each r the four
//       lanes of a channel hold 16 adjacent pixels, one 64-byte run per store.
//   RW  Y[n][a] = bias[a] + sum_k X[n][k] W[a][k]       (GateMm mode 1)
//       A operand = W, B operand = X^T, so a lane holds four consecutive
//       outputs of one row: D[4g + r][i] = Y[n0 + 16j + i][a0 + 4g + r].
//
// The reduction runs in supersteps of 16: within one, lane group g supplies
// k = 16 S + 4 g + t at MFMA step t, which covers the 16 k's exactly once and
// lets each lane fetch its four k's of a row with one 128-bit load.
#pragma once

#include "common.h"

namespace pw {

enum { CH = 0, RW = 1 };

__device__ __forceinline__ float comp(const float4 &v, int t) {
    return t == 0 ? v.x : t == 1 ? v.y : t == 2 ? v.z : v.w;
}

// GemmArgs as used here: A = W ([M][K] for CH, [N][K] for RW), B = X
// ([K][N] for CH, [M][K] for RW), C = Y; M is the weight-output dimension for
// CH and the row count for RW. Preconditions (checked by the host): K % 16 ==
// 0 (K % 64 == 0 when KS = 4), N % 4 == 0, every pointer 16-byte aligned,
// batch strides % 4 == 0.
//
// Work unit: one output tile of 64 streamed elements x TW weight outputs.
// KS = 1: every wave owns a tile; KS = 4: the four waves of a block split one
// tile's reduction into quarters and add the partial sums in LDS in a fixed
// order (wave 0 + 1 + 2 + 3), for the shapes with too few tiles to fill the
// chip.
//
// Operand loads are clamped into range instead of guarded: an X column or
// weight row past the edge only feeds output rows/columns of the MFMA tile
// that are never stored, so no branch or select sits between the loads and
// the matrix cores. The reduction ping-pongs between two register buffers,
// so the loads of superstep s + 1 are in flight while superstep s multiplies.
// The image index of blocked index e (0 <= e < plane) under map q (32-bit:
// the host enables a map only below 2^31 elements).
// n / d for n < 2^31, with the host's multiplier m and shift s for d.
__device__ __forceinline__ uint32_t mdiv(uint32_t n, uint32_t m, int32_t s) { return __umulhi(n + n, m) >> s; }
__device__ __forceinline__ uint32_t unblock(const BlockMap &q, uint32_t e) {
    const uint32_t pp = (uint32_t)(q.fh * q.fw);
    const uint32_t gi = mdiv(e, q.mpp, q.spp), p = e - gi * pp;
    const uint32_t gy = mdiv(gi, q.mgw, q.sgw), gx = gi - gy * (uint32_t)q.gw;
    const uint32_t fy = mdiv(p, q.mfw, q.sfw), fx = p - fy * (uint32_t)q.fw;
    return (gy * q.fh + fy) * q.wd + gx * q.fw + fx;
}

// The epilogue's operand set as a compile-time mask (EP >= 0), so that a
// kernel specialised for it has no per-slot tests of the argument block and
// its memory waits count exactly the loads each use needs; EP = -1 reads the
// set from the argument block at run time (every combination, one kernel).
enum { EP_U = 1, EP_R1 = 2, EP_R2 = 4, EP_GELU = 8, EP_LRELU = 16, EP_YMAP = 32, EP_BIAS = 64, EP_R1MAP = 128 };

// LN: 0 no folded LayerNorm; 1 the LayerNorm's expression on X,
// (x - m) r w + c with w and c per input channel, in the LayerNorm kernels'
// order (folding w and c into the weights changes the rounding), with m and r
// read from a statistics pass; 2 the same with m and r computed here, from
// the X tile the block's four waves hold between them (KS = 4 with two
// supersteps per wave: 128 channels), so no statistics pass runs. Mode 2
// sums each pixel's channels in another order than the LayerNorm kernels
// (a wave's 32 in its lanes' order, the four lane groups pairwise, then the
// waves in turn), so its normalised X differs from theirs by rounding.
// (ux, nx): this block's index and the block count along x, by: the batch;
// a kernel pairing two launches in one grid passes each part its own.
// XR: the split reduction's LDS buffer comes from the caller (xred, 4 x 16
// TMW x 64 floats), so two different instances in one kernel share one.
template <int LAYOUT, int TMW, int KS, bool FUSED, int LN, bool XM = false, bool XMUL = false, bool CT = false,
          bool LNO = false, int EP = -1, bool FOLD = false, bool XR = false>
__device__ void body(const GemmArgs &a, int ux, int nx, int by, float *xred = nullptr) {
    const bool has_u = EP < 0 ? a.e.u != nullptr : (EP & EP_U) != 0;
    const bool has_r1 = EP < 0 ? a.e.r1 != nullptr : (EP & EP_R1) != 0;
    const bool has_r2 = EP < 0 ? a.e.r2 != nullptr : (EP & EP_R2) != 0;
    const bool has_gelu = EP < 0 ? a.e.act == MXK_ACT_GELU : (EP & EP_GELU) != 0;
    const bool has_lrelu = EP < 0 ? a.e.act == MXK_ACT_LRELU : (EP & EP_LRELU) != 0;
    const bool has_ymap = EP < 0 ? a.ymap.on != 0 : (EP & EP_YMAP) != 0;
    const bool has_bias = EP < 0 ? a.bias != nullptr : (EP & EP_BIAS) != 0;
    const bool r1map = EP < 0 ? a.ymap.r1map != 0 : (EP & EP_R1MAP) != 0;
    constexpr int TW = 16 * TMW;    // weight outputs per tile
    constexpr int NACC = 16 * TMW;  // accumulator floats per lane
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;
    const int wout = LAYOUT == CH ? M : N;
    // CH with the batch folded into the columns: batch * N columns, batch
    // n / N holding column n (whole 4-column groups; the grid is 1-D)
    static_assert(!FOLD || (LAYOUT == CH && !LN && !CT && !LNO && !XMUL), "a folded batch: GateMm mode 0");
    constexpr bool fold = FOLD;
    const int slen = LAYOUT == CH ? (fold ? a.batch * N : N) : M;
    const int nib = (wout + TW - 1) / TW;
    const int ntiles = nib * ((slen + 63) / 64);  // < 2^31, checked by the host
    const int b = fold ? 0 : by;
    const float *W = a.A + (int64_t)b * a.sA;
    const float *X = a.B + (int64_t)b * a.sB;
    float *Y = a.C + (int64_t)b * a.sC;
    // X's advance per superstep (16 k's): 16 rows (CH) or 16 columns (RW);
    // through a token map, whole rows of cells or of cell pixels.
    const BlockMap &xm = a.xmap;
    int64_t xstep = LAYOUT == CH ? 16 * (int64_t)N : 16;
    if (XM) xstep = LAYOUT == CH ? (int64_t)(16 / xm.gw) * xm.fh * xm.wd : (int64_t)(16 / xm.fw) * xm.wd;

    // One XCD per contiguous range of blocks, so neighbouring tiles (which
    // share operands) meet in the same L2.
    int unit = ux;
    const int nb = nx;
    if ((nb & 7) == 0) unit = (unit & 7) * (nb >> 3) + (unit >> 3);
    const int tile = KS == 1 ? unit * 4 + wave : unit;
    if (tile >= ntiles) return;  // KS = 4: the whole block
    const int nS = K / 16;
    const int S0 = KS == 1 ? 0 : wave * (nS / 4);
    const int nSw = KS == 1 ? nS : nS / 4;  // supersteps of this wave

    const int w0 = (tile % nib) * TW;
    const int s0 = (tile / nib) * 64;
    // This lane's operand streams at the wave's first superstep.
    const float *wp[TMW];
#pragma unroll
    for (int mt = 0; mt < TMW; ++mt)
        wp[mt] = W + (int64_t)min(w0 + mt * 16 + i, wout - 1) * K + 4 * g + S0 * 16;
    // Input maps: X as the blocked view of an image-ordered tensor (an
    // elided forward permutation). With a folded LayerNorm (CH, xmap.on): X
    // is [channels][pixels] and only the pixel axis is blocked. XM (GateMm):
    // each batch's X is [cells][pixels of a cell] of one channel plane, so
    // element (r, c) sits at cell(r) + pixel(c); the host guarantees that 16
    // k's advance whole cell rows (CH: 16 % gw == 0) or whole pixel rows
    // (RW: 16 % fw == 0), and fw % 4 == 0 for the 128-bit reads.
    auto cell = [&](uint32_t r) -> int64_t {
        const uint32_t gy = mdiv(r, xm.mgw, xm.sgw), gx = r - gy * (uint32_t)xm.gw;
        return (int64_t)gy * xm.fh * xm.wd + (int64_t)gx * xm.fw;
    };
    auto pixel = [&](uint32_t c) -> int64_t {
        const uint32_t fy = mdiv(c, xm.mfw, xm.sfw), fx = c - fy * (uint32_t)xm.fw;
        return (int64_t)fy * xm.wd + fx;
    };
    // CH: this lane's four columns, s0 + 16 (i % 4) + 4 (i / 4) .. + 3 (with
    // a folded batch: column xcol of batch xb)
    int xcol = 0;
    int64_t xbo = 0;  // the folded batch's X offset
    if (LAYOUT == CH) {
        xcol = min(s0 + 16 * (i & 3) + 4 * (i >> 2), slen - 4);
        if (fold) {
            const uint32_t xb = mdiv((uint32_t)xcol, a.fmul, a.fsh);
            xcol -= (int)xb * N;
            xbo = (int64_t)xb * a.sB;
        }
        if (LN && xm.on) xcol = (int)unblock(xm, (uint32_t)xcol);
    }
    const float *xp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (LAYOUT == CH) {  // row k = 16 S + 4 g + q
            if (XM)
                xp[q] = X + xbo + cell(16 * S0 + 4 * g + q) + pixel(xcol);
            else
                xp[q] = X + xbo + (int64_t)(4 * g + q) * N + xcol + S0 * xstep;
        } else {  // row s0 + 16 q + i, k = 16 S + 4 g .. + 3
            const int row = min(s0 + 16 * q + i, M - 1);
            if (XM)
                xp[q] = X + cell(row) + pixel(16 * S0 + 4 * g);
            else
                xp[q] = X + (int64_t)row * K + 4 * g + S0 * xstep;
        }
    }

    f32x4 acc[4][TMW];  // set by the first superstep

    // A folded LayerNorm (CH only): this lane's four pixels' statistics for
    // the whole tile, and each superstep's scale/bias for k = 16 S + 4 g + q.
    float4 lmean, lrstd;
    const float *lsc = nullptr, *lbi = nullptr;
    if (LN == 1) {  // a single 1x1 conv (no batch): statistics indexed like X's columns
        lmean = ld4(a.ln.mean + xcol);
        lrstd = ld4(a.ln.rstd + xcol);
    }
    if (LN) {
        {
            lsc = a.ln.scale + 4 * g + S0 * 16;
            lbi = a.ln.bias + 4 * g + S0 * 16;
        }
    }
    // A folded Mul: X = B * B2 elementwise, B2 read at X's offsets.
    const float *xq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) xq[q] = XMUL ? a.B2 + (int64_t)b * a.sB + (xp[q] - X) : nullptr;
    auto load = [&](int s, float4 *xv, float4 *wv, float4 *lv, float4 *mv) {
#pragma unroll
        for (int q = 0; q < 4; ++q) xv[q] = ld4(xp[q] + s * xstep);
        if (XMUL) {
#pragma unroll
            for (int q = 0; q < 4; ++q) mv[q] = ld4(xq[q] + s * xstep);
        }
#pragma unroll
        for (int mt = 0; mt < TMW; ++mt) wv[mt] = ld4(wp[mt] + s * 16);
        if (LN) {
            lv[0] = ld4(lsc + s * 16);
            lv[1] = ld4(lbi + s * 16);
        }
    };
    auto norm = [&](float4 *xv, const float4 *lv) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float w = comp(lv[0], q), c = comp(lv[1], q);
            xv[q].x = (xv[q].x - lmean.x) * lrstd.x * w + c;
            xv[q].y = (xv[q].y - lmean.y) * lrstd.y * w + c;
            xv[q].z = (xv[q].z - lmean.z) * lrstd.z * w + c;
            xv[q].w = (xv[q].w - lmean.w) * lrstd.w * w + c;
        }
    };
    // first: the wave's first superstep, whose multiplies start from zero
    // (an inline-constant accumulator instead of 16 TMW register moves)
    auto mma = [&](float4 *xv, const float4 *wv, const float4 *lv, const float4 *mv, bool first) {
        if (LN) norm(xv, lv);
        if (XMUL) {  // mx_mul's a * b
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                xv[q].x = xv[q].x * mv[q].x;
                xv[q].y = xv[q].y * mv[q].y;
                xv[q].z = xv[q].z * mv[q].z;
                xv[q].w = xv[q].w * mv[q].w;
            }
        }
        const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int mt = 0; mt < TMW; ++mt) {
                    const f32x4 c = first && t == 0 ? zero : acc[j][mt];
                    if (LAYOUT == CH)
                        acc[j][mt] = mfma16(comp(xv[t], j), comp(wv[mt], t), c);
                    else
                        acc[j][mt] = mfma16(comp(wv[mt], t), comp(xv[j], t), c);
                }
    };
    // The bias of this lane's outputs, fetched before the reduction.
    float4 bias[TMW];
#pragma unroll
    for (int mt = 0; mt < TMW; ++mt) {
        if (!has_bias) continue;
        if (LAYOUT == CH) {
            const int m = min(w0 + mt * 16 + i, wout - 1);
            bias[mt].x = a.bias[CT ? (m % (2 * a.co)) >> 1 : m];  // CT: row (ky, oc, kx) has oc's bias
        }
        else bias[mt] = ld4(a.bias + min(w0 + mt * 16 + 4 * g, wout - 4));
    }

    float4 xa[4], wa[TMW], la[2], ma[4], xb[4], wb[TMW], lb[2], mb[4];
    // Loads are unconditional (past the wave's last superstep they re-read
    // it), so the wait before each multiply counts only the loads it needs.
    load(0, xa, wa, la, ma);
    load(min(1, nSw - 1), xb, wb, lb, mb);
    if constexpr (LN == 2) {
        static_assert(KS == 4 && LAYOUT == CH, "in-kernel statistics: the split-reduction channel-major form");
        // This lane's rows k = 16 S + 4 g + q of its two supersteps (xa, xb)
        // for pixels xcol .. xcol + 3; lanes i, i + 16, i + 32 and i + 48
        // hold the same pixels, the four waves the four quarters of k.
        __shared__ float4 lst[4][16][2];
        float4 p1 = xa[0], p2 = make_float4(xa[0].x * xa[0].x, xa[0].y * xa[0].y, xa[0].z * xa[0].z, xa[0].w * xa[0].w);
        auto add = [&](const float4 &v) {
            p1.x = p1.x + v.x;
            p1.y = p1.y + v.y;
            p1.z = p1.z + v.z;
            p1.w = p1.w + v.w;
            p2.x = p2.x + v.x * v.x;
            p2.y = p2.y + v.y * v.y;
            p2.z = p2.z + v.z * v.z;
            p2.w = p2.w + v.w * v.w;
        };
#pragma unroll
        for (int q = 1; q < 4; ++q) add(xa[q]);
#pragma unroll
        for (int q = 0; q < 4; ++q) add(xb[q]);
#pragma unroll
        for (int d = 16; d <= 32; d *= 2) {
            p1.x = p1.x + __shfl_xor(p1.x, d);
            p1.y = p1.y + __shfl_xor(p1.y, d);
            p1.z = p1.z + __shfl_xor(p1.z, d);
            p1.w = p1.w + __shfl_xor(p1.w, d);
            p2.x = p2.x + __shfl_xor(p2.x, d);
            p2.y = p2.y + __shfl_xor(p2.y, d);
            p2.z = p2.z + __shfl_xor(p2.z, d);
            p2.w = p2.w + __shfl_xor(p2.w, d);
        }
        if (g == 0) {
            lst[wave][i][0] = p1;
            lst[wave][i][1] = p2;
        }
        __syncthreads();
        float4 s1 = lst[0][i][0], s2 = lst[0][i][1];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const float4 t1 = lst[w][i][0], t2 = lst[w][i][1];
            s1.x = s1.x + t1.x;
            s1.y = s1.y + t1.y;
            s1.z = s1.z + t1.z;
            s1.w = s1.w + t1.w;
            s2.x = s2.x + t2.x;
            s2.y = s2.y + t2.y;
            s2.z = s2.z + t2.z;
            s2.w = s2.w + t2.w;
        }
        // mean, then 1 / std, as the LayerNorm statistics kernels form them
        // (K = 128: the product with 1 / K is the quotient to the bit; the
        // reciprocal square root on the transcendental unit, 1 ulp, where
        // those kernels divide by a correctly rounded square root)
        const float inv = 1.0f / (float)K;
        auto stat = [&](float a1, float a2, float &m, float &r) {
            m = a1 * inv;
            const float var = a2 * inv - m * m;
            r = __builtin_amdgcn_rsqf(fmaxf(var, 0.0f) + a.ln.eps);
        };
        stat(s1.x, s2.x, lmean.x, lrstd.x);
        stat(s1.y, s2.y, lmean.y, lrstd.y);
        stat(s1.z, s2.z, lmean.z, lrstd.z);
        stat(s1.w, s2.w, lmean.w, lrstd.w);
    }
    const int64_t cbase = (int64_t)b * a.sC;
    // Slot k of this lane: (mt, x) = (k / 4, k % 4) with KS = 1, and
    // (k, wave) with KS = 4 (the wave's share of the slots).
    constexpr int NK = KS == 1 ? 4 * TMW : TMW;
    // (the lane's first slot offset once; the others differ from it by a
    // wave-uniform amount)
    const int64_t obase = LAYOUT == CH ? (int64_t)(w0 + i) * N + s0 + 4 * g : (int64_t)(s0 + i) * N + w0 + 4 * g;
    auto where = [&](int k, int64_t &off) -> bool {
        const int mt = KS == 1 ? k / 4 : k, x = KS == 1 ? k % 4 : wave;
        if (LAYOUT == CH) {
            const int m = w0 + mt * 16 + i, n = s0 + 16 * x + 4 * g;
            if (fold) {  // batch nb, column n - nb N of it
                const uint32_t nb = mdiv((uint32_t)min(n, slen - 4), a.fmul, a.fsh);
                off = (int64_t)nb * a.sC + (int64_t)(w0 + i + mt * 16) * N + (n - (int)nb * N);
                return m < M && n < slen;
            }
            off = obase + (int64_t)(mt * 16) * N + 16 * x;
            return m < M && n < N;
        }
        const int row = s0 + 16 * x + i, c = w0 + mt * 16 + 4 * g;
        off = obase + (int64_t)(16 * x) * N + mt * 16;
        return row < M && c < N;
    };
    // The fused epilogue's operands are fetched one slot ahead, so their
    // latency overlaps the previous slot's arithmetic and store (the
    // compiler cannot move a load above a store that might alias it).
    // Where output element off (counted from this batch's Y) is stored: off
    // itself, or its image position under a folded backward permutation.
    auto placed = [&](int64_t off) -> int64_t {
        if (!has_ymap) return off;
        const uint32_t e = (uint32_t)(cbase + off), pl = (uint32_t)a.ymap.plane;
        const uint32_t base = mdiv(e, a.ymap.mpl, a.ymap.spl) * pl;
        return (int64_t)(base + unblock(a.ymap, e - base)) - cbase;
    };
    // Each slot's stored position is computed once, with its operands, and
    // serves both the residual read at that position and the store.
    float4 ou[2], o1[2], o2[2];
    int64_t pb[2] = {0, 0};
    auto operands = [&](int k, int buf) {
        int64_t off;
        const bool ok = where(k, off);
        const int64_t at = cbase + (ok ? off : 0);
        pb[buf] = placed(ok ? off : 0);
        if (has_u) ou[buf] = ld4(a.e.u + at);
        if (has_r1) o1[buf] = ld4(a.e.r1 + (r1map ? cbase + pb[buf] : at));
        if (has_r2) o2[buf] = ld4(a.e.r2 + at);
    };
    // A split reduction's wave takes both its slots' operands now, so their
    // latency hides behind the multiplies and the reduction (measured 2-5%
    // faster per launch; a whole-reduction wave keeps fetching one slot
    // ahead in its epilogue, which measured faster there).
    if (FUSED && KS == 4) {
        operands(0, 0);
        if (NK > 1) operands(1, 1);
    }
    mma(xa, wa, la, ma, true);
    int s = 1;
    for (; s + 2 <= nSw; s += 2) {
        load(s + 1, xa, wa, la, ma);
        mma(xb, wb, lb, mb, false);
        load(min(s + 2, nSw - 1), xb, wb, lb, mb);
        mma(xa, wa, la, ma, false);
    }
    if (s < nSw) mma(xb, wb, lb, mb, false);

    __shared__ float red_own[KS == 1 || XR ? 1 : 4 * NACC * 64];
    float *const red = XR ? xred : red_own;
    if (KS == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int mt = 0; mt < TMW; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    red[((wave * NACC) + (j * TMW + mt) * 4 + r) * 64 + lane] = acc[j][mt][r];
        __syncthreads();
    }
    // LNO: the wave whose tile is the output LayerNorm's channels keeps its
    // final values for it (and stores them raw only when asked to): with
    // KS = 1 in its own rows of LDS at once, with KS = 4 (where LDS still
    // holds the partial sums) in registers until every wave has read them.
    constexpr int PC = KS == 1 ? 64 : 16;  // pixel columns of a wave's tile
    constexpr int LDT = PC + 4;            // padded LDS row
    constexpr int PER = TW * LDT + 2 * PC;  // LDS floats per wave
    __shared__ float lt[LNO && KS == 1 ? 4 * PER : 1];
    const int lnspan = (KS == 1 ? a.lo.group : 1) * TW * a.lo.nband;  // rows with a LayerNorm
    const bool lnw = LNO && w0 >= a.lo.row0 && w0 < a.lo.row0 + lnspan;
    float4 vs[LNO && KS == 4 ? NK : 1];
    if (FUSED && KS == 1) operands(0, 0);
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        if (LNO && KS == 4) vs[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (FUSED && k + 1 < NK && (KS == 1 || k + 1 > 1)) operands(k + 1, (k + 1) & 1);
        const int mt = KS == 1 ? k / 4 : k, x = KS == 1 ? k % 4 : wave;
        // Out-of-range slots run the arithmetic on clamped operands and skip
        // only the global stores, so the uniform branches below stay
        // uniform (no lane-divergent region around them).
        int64_t off;
        const bool inside = where(k, off);
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // CH: v[u] = Y[m][n + u] is acc[u][mt][x]; RW: v[u] = Y[row][c + u] is acc[x][mt][u]
            const int j = LAYOUT == CH ? u : x, r = LAYOUT == CH ? x : u;
            if (KS == 1) {
                v[u] = acc[j][mt][r];
            } else {
                const int q = (j * TMW + mt) * 4 + r;
                float t = red[q * 64 + lane];
                t = t + red[(NACC + q) * 64 + lane];
                t = t + red[(2 * NACC + q) * 64 + lane];
                v[u] = t + red[(3 * NACC + q) * 64 + lane];
            }
        }
        if (has_bias) {
            if (LAYOUT == CH) {
                const float bb = bias[mt].x;
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = bb + v[u];
            } else {
                const float4 bb = bias[mt];
                v[0] = bb.x + v[0];
                v[1] = bb.y + v[1];
                v[2] = bb.z + v[2];
                v[3] = bb.w + v[3];
            }
        }
        if (FUSED) {
            const int bi = k & 1;
            if (has_u) {
                v[0] = ou[bi].x * (v[0] + 1.0f);
                v[1] = ou[bi].y * (v[1] + 1.0f);
                v[2] = ou[bi].z * (v[2] + 1.0f);
                v[3] = ou[bi].w * (v[3] + 1.0f);
            }
            if (has_gelu) {
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = gelu(v[u]);
            } else if (has_lrelu) {
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = v[u] >= 0.0f ? v[u] : a.e.slope * v[u];
            }
            if (has_r1) {
                v[0] = v[0] + o1[bi].x;
                v[1] = v[1] + o1[bi].y;
                v[2] = v[2] + o1[bi].z;
                v[3] = v[3] + o1[bi].w;
            }
            if (has_r2) {
                v[0] = v[0] + o2[bi].x;
                v[1] = v[1] + o2[bi].y;
                v[2] = v[2] + o2[bi].z;
                v[3] = v[3] + o2[bi].w;
            }
        }
        if (CT) {
            // Transposed 2x2 stride-2 conv: row m = (ky * co + oc) * 2 + kx, so
            // lanes i and i ^ 1 hold kx = 0 and 1 of one (ky, oc) for the same
            // four input pixels (x .. x + 3 of input row y): together the eight
            // contiguous outputs 2x .. 2x + 7 of output row 2y + ky, four each.
            float pv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) pv[u] = __shfl_xor(v[u], 1);
            if (!inside) continue;
            const int m = w0 + mt * 16 + i, two = 2 * a.co;
            const int ky = m / two, rem = m - ky * two, oc = rem >> 1, kx = rem & 1;
            const int n = (int)(off - (int64_t)m * N), y = n / a.wd, xx = n - y * a.wd;
            float *o = Y + (int64_t)oc * 4 * N + (int64_t)(2 * y + ky) * (2 * a.wd) + 2 * xx + 4 * kx;
            st4(o, kx == 0 ? make_float4(v[0], pv[0], v[1], pv[1]) : make_float4(pv[2], v[2], pv[3], v[3]));
            continue;
        }
        if (LNO && lnw) {
            if (KS == 1)
                st4(lt + wave * PER + (mt * 16 + i) * LDT + 16 * x + 4 * g, make_float4(v[0], v[1], v[2], v[3]));
            else
                vs[k] = make_float4(v[0], v[1], v[2], v[3]);
            if (!a.lo.keep) continue;
        }
        if (inside) st4(Y + (FUSED ? pb[k & 1] : placed(off)), make_float4(v[0], v[1], v[2], v[3]));
    }
    if constexpr (LNO) {
        // Per pixel, the LayerNorm's statistics in the LayerNorm kernels'
        // order (ascending channel, one pass for s1 and s2): the tiles go
        // through LDS so that one lane reads a pixel's channels in turn; then
        // every lane normalises the values it holds with the LayerNorm's
        // expression (mode 0), or writes the statistics (mode 1). A band's
        // G * TW channels are the tiles of G consecutive waves of one block
        // (G = lo.group; G = 1 with KS = 4).
        // With G = 1 the exchange stays within the wave (its own LDS rows)
        // and needs no block barrier; with G > 1 every wave of a block that
        // holds a group takes both barriers (block-uniform, and the host
        // launches whole blocks of tiles, so no wave has left early).
        const int G = KS == 1 ? a.lo.group : 1;
        bool any = lnw;
        if (KS == 1 && G > 1) {
            any = false;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int bw = ((unit * 4 + j) % nib) * TW;
                any = any || (bw >= a.lo.row0 && bw < a.lo.row0 + lnspan);
            }
        }
        if (any) {
            float *t;
            if constexpr (KS == 1) {
                t = lt + wave * PER;
            } else {
                static_assert(4 * PER <= 4 * NACC * 64, "the reduction buffer holds the exchange");
                __syncthreads();  // every wave has read its sums out of red
                t = red + wave * PER;
#pragma unroll
                for (int k = 0; k < NK; ++k) st4(t + (k * 16 + i) * LDT + 4 * g, vs[k]);
            }
            auto sync = [&]() {
                if (G > 1) {
                    __syncthreads();
                } else {
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                }
            };
            const int band = lnw ? (w0 - a.lo.row0) / (G * TW) : 0;
            const int lq = lnw ? (w0 - a.lo.row0) / TW - band * G : 0;  // place in the group
            // mode 0: this wave's values of the band, normalised with the
            // statistics at ts (mean row, then 1 / std row) and stored
            auto normalise = [&](const float *ts) {
                float lw[TMW], lb[TMW];
#pragma unroll
                for (int mt = 0; mt < TMW; ++mt) {
                    lw[mt] = a.lo.scale[lq * TW + mt * 16 + i];
                    lb[mt] = a.lo.bias[lq * TW + mt * 16 + i];
                }
                float *ly = a.lo.y - (int64_t)a.lo.row0 * N;  // indexed like Y (one batch)
#pragma unroll
                for (int k = 0; k < NK; ++k) {
                    const int mt = KS == 1 ? k / 4 : k, x = KS == 1 ? k % 4 : 0;
                    int64_t off;
                    if (!where(k, off)) continue;
                    const float4 m4 = ld4(ts + 16 * x + 4 * g);
                    const float4 r4 = ld4(ts + PC + 16 * x + 4 * g);
                    const float w = lw[mt], c = lb[mt];
                    float4 y = ld4(t + (mt * 16 + i) * LDT + 16 * x + 4 * g);
                    y.x = (y.x - m4.x) * r4.x * w + c;
                    y.y = (y.y - m4.y) * r4.y * w + c;
                    y.z = (y.z - m4.z) * r4.z * w + c;
                    y.w = (y.w - m4.w) * r4.w * w + c;
                    st4(ly + off, y);
                }
            };
            // (G TW is a power of two, so the product with its reciprocal is
            // the quotient to the bit; with the per-wave partial sums, whose
            // order already differs from the LayerNorm kernels', 1 / std is
            // the transcendental unit's reciprocal square root, 1 ulp)
            const float inv = 1.0f / (float)(G * TW);
            auto stats = [&](float s1, float s2, int n_at) {
                const float m = s1 * inv;
                const float var = s2 * inv - m * m;
                const float r = a.lo.order ? __builtin_amdgcn_rsqf(fmaxf(var, 0.0f) + a.lo.eps)
                                           : 1.0f / sqrtf(fmaxf(var, 0.0f) + a.lo.eps);
                if (a.lo.mode) {  // the statistics only, at the pixel's image position
                    const int n = s0 + n_at;
                    if (n < N) {
                        float *sy = a.lo.y + (int64_t)band * 2 * N;
                        const int64_t at = placed(n);
                        sy[at] = m;
                        sy[N + at] = r;
                    }
                } else {
                    t[TW * LDT + lane] = m;
                    t[TW * LDT + PC + lane] = r;
                }
            };
            if (KS == 1 && TW >= 32 && G > 1 && a.lo.order) {
                // Each wave of the group sums its own channels of a pixel
                // (its own LDS rows: a wave barrier), the partial sums meet
                // in LDS (one block barrier), and every wave adds the
                // group's partials in wave order and keeps the statistics
                // it needs (its own rows again). A wave's partial sums of
                // pixel p sit in its tile's row padding: s1 in rows 0..15,
                // s2 in rows 16..31, column PC + p % 4 of row p / 4 (the
                // padding holds 4 TW >= 2 PC floats and is read nowhere else).
                auto pad = [&](int which, int p) { return (which * 16 + (p >> 2)) * LDT + PC + (p & 3); };
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (lnw) {
                    float p1 = 0.0f, p2 = 0.0f;
#pragma unroll 8
                    for (int c = 0; c < TW; ++c) {
                        const float v = t[c * LDT + lane];
                        p1 += v;
                        p2 += v * v;
                    }
                    t[pad(0, lane)] = p1;
                    t[pad(1, lane)] = p2;
                }
                __syncthreads();
                if (lnw) {
                    const float *g0 = t - lq * PER;
                    float s1 = g0[pad(0, lane)], s2 = g0[pad(1, lane)];
                    for (int q = 1; q < G; ++q) {
                        s1 = s1 + g0[q * PER + pad(0, lane)];
                        s2 = s2 + g0[q * PER + pad(1, lane)];
                    }
                    if (!a.lo.mode || lq == 0) stats(s1, s2, KS == 1 ? lane : 16 * wave + lane);
                }
                if (!a.lo.mode) {
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                }
                if (lnw && !a.lo.mode) normalise(t + TW * LDT);
            } else {
                sync();
                if (lnw && lq == 0 && lane < PC) {
                    float s1 = 0.0f, s2 = 0.0f;
                    for (int q = 0; q < G; ++q) {
#pragma unroll 8
                        for (int c = 0; c < TW; ++c) {
                            const float v = t[q * PER + c * LDT + lane];
                            s1 += v;
                            s2 += v * v;
                        }
                    }
                    stats(s1, s2, KS == 1 ? lane : 16 * wave + lane);
                }
                if (!a.lo.mode) sync();
                if (lnw && !a.lo.mode) normalise(t - lq * PER + TW * LDT);  // the group's statistics
            }
        }
    }
}

}  // namespace pw

// mx_pw_{ch,rw}<TMW>[_k4][_ln|_xm|_mul][_f]: 256 threads; _k4 splits the
// reduction over the block's four waves, _ln folds a channel LayerNorm into X
// (CH only), _xm reads X through a token map (GateMm over an elided forward
// permutation), _mul forms X as the product of two tensors (a folded Mul, CH
// only), _f applies the fused epilogue. mx_pw_ch<TMW>[_k4]_t: the transposed
// 2x2 stride-2 conv (rows ordered (ky, oc, kx), co and the input width in
// GemmArgs co / wd, wd % 4 == 0).
#define MXK_PW2(LNAME, LAYOUT, TMW, KS, LN, XM, XMUL, SUF)                                         \
    extern "C" __global__ __launch_bounds__(256) void mx_pw_##LNAME##TMW##SUF(GemmArgs a) {        \
        pw::body<pw::LAYOUT, TMW, KS, false, LN, XM, XMUL>(a, blockIdx.x, gridDim.x, blockIdx.y);                                     \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(256) void mx_pw_##LNAME##TMW##SUF##_f(GemmArgs a) {    \
        pw::body<pw::LAYOUT, TMW, KS, true, LN, XM, XMUL>(a, blockIdx.x, gridDim.x, blockIdx.y);                                      \
    }
#define MXK_PW1(LNAME, LAYOUT, TMW, KS, LN, XM, SUF) MXK_PW2(LNAME, LAYOUT, TMW, KS, LN, XM, false, SUF)
#define MXK_PW(LNAME, LAYOUT, TMW)                                                                 \
    MXK_PW1(LNAME, LAYOUT, TMW, 1, false, false, ) MXK_PW1(LNAME, LAYOUT, TMW, 4, false, false, _k4) \
    MXK_PW1(LNAME, LAYOUT, TMW, 1, false, true, _xm) MXK_PW1(LNAME, LAYOUT, TMW, 4, false, true, _k4_xm)
#define MXK_PW_LN(TMW) MXK_PW1(ch, CH, TMW, 1, 1, false, _ln) MXK_PW1(ch, CH, TMW, 4, 1, false, _k4_ln)
// _k4_ln2: the LayerNorm statistics computed by the block itself (LN = 2)
MXK_PW1(ch, CH, 2, 4, 2, false, _k4_ln2)
#define MXK_PW_CT(TMW, KS, SUF)                                                                    \
    extern "C" __global__ __launch_bounds__(256) void mx_pw_ch##TMW##SUF##_t(GemmArgs a) {          \
        pw::body<pw::CH, TMW, KS, false, false, false, false, true>(a, blockIdx.x, gridDim.x, blockIdx.y);                             \
    }
// mx_pw_ch<TMW>[_k4][_ln]_f_lo: with a LayerNorm of one wave-wide band of
// the output rows (GemmArgs lo).
#define MXK_PW_LO(TMW, KS, LN, SUF)                                                               \
    extern "C" __global__ __launch_bounds__(256) void mx_pw_ch##TMW##SUF##_f_lo(GemmArgs a) {      \
        pw::body<pw::CH, TMW, KS, true, LN, false, false, false, true>(a, blockIdx.x, gridDim.x, blockIdx.y);                          \
    }
#define MXK_PW_MUL(TMW) \
    MXK_PW2(ch, CH, TMW, 1, false, false, true, _mul) MXK_PW2(ch, CH, TMW, 4, false, false, true, _k4_mul)
MXK_PW(ch, CH, 1)
MXK_PW(ch, CH, 2)
MXK_PW(ch, CH, 4)
// mx_pw_chb<TMW>[_k4][_xm][_f]: channel-major over a folded batch (GemmArgs
// fold; GateMm mode 0, whose channels are the batch)
#define MXK_PWB1(TMW, KS, XM, SUF)                                                                  \
    extern "C" __global__ __launch_bounds__(256) void mx_pw_chb##TMW##SUF(GemmArgs a) {             \
        pw::body<pw::CH, TMW, KS, false, 0, XM, false, false, false, -1, true>(a, blockIdx.x, gridDim.x, 0); \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(256) void mx_pw_chb##TMW##SUF##_f(GemmArgs a) {         \
        pw::body<pw::CH, TMW, KS, true, 0, XM, false, false, false, -1, true>(a, blockIdx.x, gridDim.x, 0); \
    }
#define MXK_PWB(TMW) \
    MXK_PWB1(TMW, 1, false, ) MXK_PWB1(TMW, 4, false, _k4) MXK_PWB1(TMW, 1, true, _xm) MXK_PWB1(TMW, 4, true, _k4_xm)
MXK_PWB(1)
MXK_PWB(2)
MXK_PWB(4)
MXK_PW(rw, RW, 1)
MXK_PW(rw, RW, 2)
MXK_PW(rw, RW, 4)
MXK_PW_LN(1)
MXK_PW_LN(2)
MXK_PW_LN(4)
MXK_PW_MUL(1)
MXK_PW_MUL(2)
MXK_PW_MUL(4)
MXK_PW_CT(1, 1, )
MXK_PW_CT(1, 4, _k4)
MXK_PW_CT(2, 1, )
MXK_PW_CT(2, 4, _k4)
MXK_PW_CT(4, 1, )
MXK_PW_CT(4, 4, _k4)
MXK_PW_LO(1, 1, 0, )
MXK_PW_LO(2, 1, 0, )
MXK_PW_LO(2, 4, 0, _k4)
MXK_PW_LO(2, 1, 1, _ln)
MXK_PW_LO(2, 4, 1, _k4_ln)
MXK_PW_LO(4, 1, 0, )
MXK_PW_LO(4, 4, 0, _k4)
MXK_PW_LO(4, 1, 1, _ln)
MXK_PW_LO(4, 4, 1, _k4_ln)

// mx_pw_..._f[_lo]_e<EP>: a fused streaming kernel specialised for one
// epilogue operand set (pw::EP_* mask), for the combinations the MAXIM
// program launches most; the host takes one when it exists and the generic
// _f kernel otherwise (the same arithmetic in the same order).
#define MXK_PW_E(NAME, LAYOUT, TMW, KS, LN, XM, XMUL, LNO, EP)                                     \
    extern "C" __global__ __launch_bounds__(256) void NAME##_e##EP(GemmArgs a) {                  \
        pw::body<pw::LAYOUT, TMW, KS, true, LN, XM, XMUL, false, LNO, EP>(a, blockIdx.x, gridDim.x, blockIdx.y); \
    }
// NAME_e<EP>_x2: two independent launches of that kernel as one grid (the
// first d.na blocks run d.a, the rest d.b; one batch each), so that two
// steps too small to fill the chip share its CUs and one launch's tail. Both
// parts run the same function, so they share its LDS.
#define MXK_PW_X2(NAME, LAYOUT, TMW, KS, LN, XM, XMUL, LNO, EP)                                    \
    extern "C" __global__ __launch_bounds__(256) void NAME##_e##EP##_x2(DualGemmArgs d) {         \
        if (blockIdx.x < d.na)                                                                     \
            pw::body<pw::LAYOUT, TMW, KS, true, LN, XM, XMUL, false, LNO, EP>(d.a, blockIdx.x, d.na, 0); \
        else                                                                                       \
            pw::body<pw::LAYOUT, TMW, KS, true, LN, XM, XMUL, false, LNO, EP>(d.b, blockIdx.x - d.na, \
                                                                            gridDim.x - d.na, 0);  \
    }
MXK_PW_E(mx_pw_ch2_ln_f_lo, CH, 2, 1, 1, false, false, true, 72)
MXK_PW_E(mx_pw_ch4_k4_ln_f_lo, CH, 4, 4, 1, false, false, true, 72)
MXK_PW_E(mx_pw_ch2_ln_f, CH, 2, 1, 1, false, false, false, 72)
MXK_PW_E(mx_pw_ch2_k4_ln_f, CH, 2, 4, 1, false, false, false, 72)
MXK_PW_E(mx_pw_ch2_k4_ln2_f, CH, 2, 4, 2, false, false, false, 72)
MXK_PW_E(mx_pw_ch2_f_lo, CH, 2, 1, 0, false, false, true, 64)
MXK_PW_E(mx_pw_ch2_f_lo, CH, 2, 1, 0, false, false, true, 66)
MXK_PW_E(mx_pw_ch1_f_lo, CH, 1, 1, 0, false, false, true, 66)
MXK_PW_E(mx_pw_ch2_k4_f_lo, CH, 2, 4, 0, false, false, true, 64)
MXK_PW_E(mx_pw_ch2_k4_f_lo, CH, 2, 4, 0, false, false, true, 66)
MXK_PW_E(mx_pw_ch4_k4_f_lo, CH, 4, 4, 0, false, false, true, 64)
MXK_PW_E(mx_pw_ch4_k4_f_lo, CH, 4, 4, 0, false, false, true, 66)
MXK_PW_E(mx_pw_ch1_f, CH, 1, 1, 0, false, false, false, 226)
MXK_PW_E(mx_pw_ch2_f, CH, 2, 1, 0, false, false, false, 64)
MXK_PW_E(mx_pw_ch2_f, CH, 2, 1, 0, false, false, false, 226)
MXK_PW_E(mx_pw_ch2_k4_f, CH, 2, 4, 0, false, false, false, 64)
MXK_PW_E(mx_pw_ch2_k4_f, CH, 2, 4, 0, false, false, false, 65)
MXK_PW_E(mx_pw_ch2_k4_f, CH, 2, 4, 0, false, false, false, 66)
MXK_PW_E(mx_pw_ch2_k4_f, CH, 2, 4, 0, false, false, false, 226)
MXK_PW_E(mx_pw_ch1_mul_f, CH, 1, 1, 0, false, true, false, 66)
MXK_PW_E(mx_pw_ch1_mul_f, CH, 1, 1, 0, false, true, false, 70)
MXK_PW_E(mx_pw_ch2_mul_f, CH, 2, 1, 0, false, true, false, 66)
MXK_PW_E(mx_pw_ch2_mul_f, CH, 2, 1, 0, false, true, false, 70)
MXK_PW_E(mx_pw_ch2_k4_mul_f, CH, 2, 4, 0, false, true, false, 66)
MXK_PW_E(mx_pw_ch2_k4_mul_f, CH, 2, 4, 0, false, true, false, 70)
MXK_PW_E(mx_pw_rw2_k4_f, RW, 2, 4, 0, false, false, false, 65)
extern "C" __global__ __launch_bounds__(256) void mx_pw_chb2_k4_f_e65(GemmArgs a) {
    pw::body<pw::CH, 2, 4, true, 0, false, false, false, false, 65, true>(a, blockIdx.x, gridDim.x, 0);
}
MXK_PW_E(mx_pw_rw4_k4_f, RW, 4, 4, 0, false, false, false, 65)
MXK_PW_X2(mx_pw_ch2_ln_f_lo, CH, 2, 1, 1, false, false, true, 72)
MXK_PW_X2(mx_pw_ch1_f, CH, 1, 1, 0, false, false, false, 226)
MXK_PW_X2(mx_pw_ch2_f, CH, 2, 1, 0, false, false, false, 226)
MXK_PW_X2(mx_pw_ch2_k4_f, CH, 2, 4, 0, false, false, false, 226)
MXK_PW_X2(mx_pw_ch2_k4_ln2_f, CH, 2, 4, 2, false, false, false, 72)
// A__B_x2: two different split-reduction GEMMs, independent of each other,
// side by side in one grid (the first d.na blocks run A, the rest B) with one
// reduction buffer for both (each instance would otherwise bring its own and
// halve the blocks per CU): the grid and block branches' GateMms of a
// multi-axis gMLP block, mode 0 over a folded batch and mode 1.
extern "C" __global__ __launch_bounds__(256) void mx_pw_chb2_k4_xm__rw2_k4_xm_x2(DualGemmArgs d) {
    __shared__ float red[4 * 32 * 64];
    if (blockIdx.x < d.na)
        pw::body<pw::CH, 2, 4, false, 0, true, false, false, false, -1, true, true>(d.a, blockIdx.x, d.na, 0, red);
    else
        pw::body<pw::RW, 2, 4, false, 0, true, false, false, false, -1, false, true>(d.b, blockIdx.x - d.na,
                                                                                      gridDim.x - d.na, 0, red);
}
extern "C" __global__ __launch_bounds__(256) void mx_pw_chb2_k4_f_e65__rw2_k4_f_e65_x2(DualGemmArgs d) {
    __shared__ float red[4 * 32 * 64];
    if (blockIdx.x < d.na)
        pw::body<pw::CH, 2, 4, true, 0, false, false, false, false, 65, true, true>(d.a, blockIdx.x, d.na, 0, red);
    else
        pw::body<pw::RW, 2, 4, true, 0, false, false, false, false, 65, false, true>(d.b, blockIdx.x - d.na,
                                                                                      gridDim.x - d.na, 0, red);
}
// the out-projections of the two branches at the smallest resolutions: a
// residual add (grid branch), and a residual add into a backward permutation
// (block branch)
extern "C" __global__ __launch_bounds__(256) void mx_pw_ch2_k4_f_e66__ch2_k4_f_e226_x2(DualGemmArgs d) {
    __shared__ float red[4 * 32 * 64];
    if (blockIdx.x < d.na)
        pw::body<pw::CH, 2, 4, true, 0, false, false, false, false, 66, false, true>(d.a, blockIdx.x, d.na, 0, red);
    else
        pw::body<pw::CH, 2, 4, true, 0, false, false, false, false, 226, false, true>(d.b, blockIdx.x - d.na,
                                                                                       gridDim.x - d.na, 0, red);
}
// the unfused split-reduction kernel (a GEMM with no epilogue), paired
extern "C" __global__ __launch_bounds__(256) void mx_pw_ch2_k4_x2(DualGemmArgs d) {
    if (blockIdx.x < d.na)
        pw::body<pw::CH, 2, 4, false, 0, false, false>(d.a, blockIdx.x, d.na, 0);
    else
        pw::body<pw::CH, 2, 4, false, 0, false, false>(d.b, blockIdx.x - d.na, gridDim.x - d.na, 0);
}
