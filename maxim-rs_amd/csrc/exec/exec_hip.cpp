// The gfx950 executor: one plan, one device arena, one stream.
//
// The per-op dispatch follows the reference's `Gpu::op` (src/exec_gpu.rs
// 359-739) in what it computes; the kernels, their launch geometry and the
// device weight layouts are this engine's own. Everything that can be decided
// before the first launch is: `Gpu::Gpu` validates every op against the
// buffer table (so no kernel is ever launched over a shape it was not written
// for), converts each weight to the layout its kernel reads, builds the resize
// tap tables, uploads all of it in one copy, and records every launch (kernel,
// grid, argument block) so that running the plan is a loop of launches.

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../hip/kargs.h"
#include "hip_api.hpp"
#include "host.hpp"
#include "maxim_hip.h"

extern "C" const unsigned char mx_kernels_hsaco[];
extern "C" const unsigned char mx_kernels_hsaco_end[];

namespace mxh {

using mx::Error;

namespace {

// The embedded code object, loaded once per device and kept until the
// process ends (every executor on the device launches from it), with the
// device address of its `scratch` array, the scratch of mxh_run_noalloc.
// The code object is loaded through the module API, so the array is found
// by name in the loaded module (hipModuleGetGlobal): the device address,
// looked up with the device current, never the host-side name.
struct DeviceCode {
    hipModule_t mod = nullptr;
    float *scratch = nullptr;
    size_t scratch_bytes = 0;
};

constexpr int kMaxDevices = 64;

DeviceCode &device_code(HipApi &H, int dev) {
    static std::mutex mu;
    static DeviceCode codes[kMaxDevices];
    if (dev < 0 || dev >= kMaxDevices) throw Error("device ordinal out of range");
    std::lock_guard<std::mutex> lock(mu);
    DeviceCode &dc = codes[dev];
    if (!dc.mod) {
        check(H.hipSetDevice(dev), "hipSetDevice");
        hipModule_t m = nullptr;
        check(H.hipModuleLoadData(&m, mx_kernels_hsaco), "hipModuleLoadData (embedded gfx950 code object)");
        void *p = nullptr;
        size_t n = 0;
        const hipError_t rc = H.hipModuleGetGlobal(&p, &n, m, "scratch");
        if (rc != 0) {
            H.hipModuleUnload(m);
            check(rc, "hipModuleGetGlobal(scratch)");
        }
        if (!p || n < (size_t)MXK_NOALLOC_SCRATCH_FLOATS * 4) {
            H.hipModuleUnload(m);
            throw Error("the code object's scratch array is missing or smaller than " +
                        std::to_string((size_t)MXK_NOALLOC_SCRATCH_FLOATS * 4) + " bytes");
        }
        dc.scratch = static_cast<float *>(p);
        dc.scratch_bytes = n;
        dc.mod = m;
    }
    return dc;
}

struct Launch {
    hipFunction_t f = nullptr;
    const char *name = "";
    unsigned g[3] = {1, 1, 1};
    unsigned b[3] = {MXK_BLOCK, 1, 1};
    unsigned shm = 0;  // dynamic LDS bytes
    alignas(16) unsigned char a0[1024] = {};
    alignas(16) unsigned char a1[32] = {};
    int nparams = 1;
    int kind = 0;  // 1: a0 holds GemmArgs (plain epilogue), 2: ConvArgs, 3: DualGemmArgs, 4: DualLnArgs
    // The ops this launch computes when its step pairs launches of several
    // former steps: [span[0], span[1]), and for a paired launch also
    // [span[2], span[3]); all zero: the whole step's ops.
    uint64_t span[4] = {0, 0, 0, 0};
};

// A run of ops [first, last) executed by `launches`: one op's own launches,
// or one fused launch standing for several ops.
struct Step {
    Step(uint64_t f, uint64_t l, std::vector<Launch> v = {}) : first(f), last(l), launches(std::move(v)) {}
    uint64_t first, last;
    std::vector<Launch> launches;
    size_t main = 0;  // the launch that names the step in reports
    // A folded LayerNorm whose statistics step so_from's epilogue writes:
    // when a run of ops starts after that step, `pre` (the statistics pass)
    // runs first.
    int64_t so_from = -1;
    std::vector<Launch> pre;
};

template <typename T>
void set_args(Launch &l, const T &v) {
    static_assert(sizeof(T) <= sizeof(l.a0), "argument block too large");
    memcpy(l.a0, &v, sizeof(T));
    l.nparams = 1;
}

template <typename T, typename U>
void set_args(Launch &l, const T &v, const U &w) {
    static_assert(sizeof(T) <= sizeof(l.a0) && sizeof(U) <= sizeof(l.a1), "argument block too large");
    memcpy(l.a0, &v, sizeof(T));
    memcpy(l.a1, &w, sizeof(U));
    l.nparams = 2;
}

unsigned cdiv(int64_t a, int64_t b) {
    int64_t q = (a + b - 1) / b;
    if (q < 1) q = 1;
    if (q > 0x7fffffff) throw Error("a launch needs more than 2^31 blocks");
    return (unsigned)q;
}

unsigned grid_yz(int64_t n) {
    if (n < 1) n = 1;
    if (n > 65535) throw Error("a launch needs more than 65535 blocks on a y/z grid axis");
    return (unsigned)n;
}

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// The resize tap table of one axis: per output [j0, n, wsum, w0 .. w(maxt-1)],
// built with the CPU path's arithmetic (src/exec_cpu.rs:1195-1216) in fp32,
// so the device sums the same weights in the same order.
std::vector<float> resize_table(int64_t n_in, int64_t n_out, int &maxt) {
    const float inv = (float)n_in / (float)n_out;
    const float kscale = inv > 1.0f ? inv : 1.0f;
    std::vector<std::vector<float>> taps(n_out);
    std::vector<int64_t> j0s(n_out);
    std::vector<float> sums(n_out);
    maxt = 1;
    for (int64_t o = 0; o < n_out; ++o) {
        const float sample = ((float)o + 0.5f) * inv - 0.5f;
        int64_t j0 = (int64_t)std::ceil(sample - kscale);
        int64_t j1 = (int64_t)std::floor(sample + kscale);
        if (j0 < 0) j0 = 0;
        if (j1 > n_in - 1) j1 = n_in - 1;
        float s = 0.0f;
        for (int64_t j = j0; j <= j1; ++j) {
            float d = std::fabs(sample - (float)j) / kscale;
            if (d < 1.0f) {
                float wv = 1.0f - d;
                taps[o].push_back(wv);
                s += wv;
            }
        }
        // The CPU applies the k-th kept weight to input j0 + k; a table whose
        // run would read past the row is refused rather than clamped.
        if (j0 + (int64_t)taps[o].size() > n_in) throw Error("resize: a tap run leaves the input row");
        j0s[o] = j0;
        sums[o] = s;
        maxt = std::max<int>(maxt, (int)taps[o].size());
    }
    std::vector<float> t((size_t)n_out * (3 + maxt), 0.0f);
    for (int64_t o = 0; o < n_out; ++o) {
        float *e = &t[(size_t)o * (3 + maxt)];
        e[0] = (float)j0s[o];
        e[1] = (float)taps[o].size();
        e[2] = sums[o];
        for (size_t k = 0; k < taps[o].size(); ++k) e[3 + k] = taps[o][k];
    }
    return t;
}

struct ResizeTab {
    const float *t;
    int32_t maxt, pad;
};

// The multiplier and shift that divide every n < 2^31 by d (1 <= d < 2^31)
// as umulhi(2 n, m) >> s: with s = ceil(log2 d) and m = ceil(2^(31+s) / d),
// m d - 2^(31+s) < d <= 2^s, so n (m d - 2^(31+s)) < 2^(31+s) and the
// quotient's floor is exact; m < 2^32 since d > 2^(s-1).
void div_magic(uint32_t d, uint32_t &m, int32_t &s) {
    int l = 0;
    while ((1ULL << l) < d) ++l;
    m = (uint32_t)(((1ULL << (31 + l)) + d - 1) / d);
    s = l;
}

// The block map of BlockPerm q (cells fh x fw in a gh x gw grid of a wd-wide
// plane), with its divisions as multiplies.
BlockMap mx_block_map(const mx_op &q, int32_t r1map) {
    BlockMap b{};
    b.plane = q.h * q.wd;
    b.on = 1;
    b.fh = (int32_t)q.p[2];
    b.fw = (int32_t)q.p[3];
    b.gw = (int32_t)q.p[1];
    b.wd = (int32_t)q.wd;
    b.r1map = r1map;
    div_magic((uint32_t)b.plane, b.mpl, b.spl);
    div_magic((uint32_t)(b.fh * b.fw), b.mpp, b.spp);
    div_magic((uint32_t)b.gw, b.mgw, b.sgw);
    div_magic((uint32_t)b.fw, b.mfw, b.sfw);
    return b;
}

// The LayerNorm tile kernel for c in {32, 64, 128}: c x P pixels per block,
// the widest P (up to 8192 / c) that still gives four blocks per CU (two at
// 128 channels, whose longer serial pass favours wider tiles), else the
// narrowest: the serial channel pass of a block is latency-bound, so small
// planes want more blocks (measured at C4). Returns the pixels per block and
// the name suffix.
std::pair<int64_t, std::string> ln_tile(int64_t c, int64_t hw, int cus) {
    const int64_t want = (c >= 128 ? 2LL : 4LL) * (cus > 0 ? cus : 256);
    const int64_t full = 8192 / c;
    for (int64_t pp : {full, full / 2, full / 4})
        if ((hw + pp - 1) / pp >= want || pp == full / 4)
            return {pp, pp == full ? std::string() : "_p" + std::to_string(pp)};
    return {full, std::string()};
}

// Channel-mean partial sums: chunks of a multiple of 1024 elements (the
// 128-bit kernel's stride), about 64 per channel, at least 2048 elements.
int64_t mean_chunk(int64_t hw) { return std::max<int64_t>(2048, ((hw + 63) / 64 + 1023) / 1024 * 1024); }

// The one-pass resize stages, per band of `rows` outputs of one axis, the
// inputs from the first output's first tap to the last output's last one.
// Returns the most any band needs, or -1 if some output of a band reaches
// outside that range (taps not monotone), in which case the two-pass kernels
// run. Used for output rows and for output columns alike.
constexpr int kResizeLdsMax = 64 * 1024, kResizeTapsMax = 8;
int resize_band(const std::vector<float> &tv, int mt, int64_t n_out, int64_t rows) {
    const size_t sv = 3 + (size_t)mt;
    int most = 0;
    for (int64_t o0 = 0; o0 < n_out; o0 += rows) {
        const int64_t o1 = std::min(o0 + rows, n_out);
        const int lo = (int)tv[o0 * sv], hi = (int)tv[(o1 - 1) * sv] + (int)tv[(o1 - 1) * sv + 1];
        for (int64_t o = o0; o < o1; ++o) {
            const int j0 = (int)tv[o * sv], n = (int)tv[o * sv + 1];
            if (j0 < lo || j0 + n > hi) return -1;
        }
        most = std::max(most, hi - lo);
    }
    return most;
}

// The GEMM tile for an M x N problem (times `batch`): estimated time is the
// number of rounds of resident blocks (two per CU) times the tile's cost,
// where bigger tiles do more work per byte staged. Every tile reduces K in the
// same order, so the choice never changes a bit of the result.
struct Tile {
    int bm, bn;
};

Tile pick_tile(int64_t M, int64_t N, int64_t batch, int cus) {
    static const struct {
        int bm, bn;
        double eff;
    } cand[] = {{128, 128, 1.00}, {64, 128, 0.85}, {128, 64, 0.85},
                {64, 64, 0.70},   {32, 128, 0.70}, {32, 64, 0.55}};
    const int64_t slots = 2LL * (cus > 0 ? cus : 256);
    double best = 1e300;
    Tile t{128, 128};
    for (auto &c : cand) {
        int64_t blocks = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * batch;
        double rounds = (double)((blocks + slots - 1) / slots);
        double cost = rounds * c.bm * c.bn / c.eff;
        if (cost < best * 0.999) {
            best = cost;
            t = Tile{c.bm, c.bn};
        }
    }
    return t;
}

std::string gemm_name(Tile t, bool vec) {
    return "mx_gemm_" + std::to_string(t.bm) + "x" + std::to_string(t.bn) + (vec ? "_v4" : "");
}

// The implicit-GEMM conv tile: BM output channels x TH x 16 outputs, CK input
// channels per LDS chunk (4 for the few-channel RGB convs and every 4x4).
// Same cost model as the GEMM tile.
struct ConvCfg {
    int bm = 0, th = 0, ck = 0;
    int c3bm = 0, c3th = 0;  // the mx_c3 tile, when the op qualifies for it
    int wtc = 0;             // the Winograd kernel's tile columns (4 or 8), 0: not eligible
    int nsplit = 1;          // 4x4: slices of the split reduction (mx_conv4x4_*_s)
};

// The Winograd F(2x2, 3x3) kernels (wino.h) take 3x3 convs of at least 8
// input channels (a multiple of 8) and 32 output channels, in blocks of 32
// output channels x TR x TC tiles: TC = 16 (4 x 32 pixels) where the width
// allows, else 8 (8 x 16), else 4 (8 x 8). A block reads its 32 channels'
// transformed filters once per tile grid, so the 32-tile grids halve that
// traffic against 8 x 8 (at 112x160, 128 channels, 48.3 -> 37.6 us per
// launch), and 32-pixel rows move 128-byte runs of each plane instead of
// 64-byte ones (37.6 -> 36.5 us).
int pick_wino(int64_t ci, int64_t co, int64_t h, int64_t w) {
    if (ci < 8 || ci % 8 || co < 32 || w % 4 || 8 * h * w >= (1LL << 31)) return 0;
    if (w % 32 == 0) return 16;
    if (w % 16 == 0) return 8;
    return w % 8 == 0 ? 4 : 0;
}

// F(2x2, 3x3)'s filter transform U = G g G^T (G = [1 0 0; 1/2 1/2 1/2;
// 1/2 -1/2 1/2; 0 0 1]) of every (output, input) channel pair, in double and
// rounded once, laid out per (32-channel output block, 8-channel input
// chunk) as [wave][lane][16]: wave w holds the transform row xi = w, and lane
// (k, r) = (lane / 16, lane % 16) its MFMA A operand, value (nu, ks, mi) =
// U[4 w + nu][channel 8 chunk + 4 ks + k][output 32 block + 16 mi + r].
std::vector<float> wino_weights(const float *w, int64_t co, int64_t ci) {
    static const double G[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
    const int64_t nmb = (co + 31) / 32, nch = (ci + 7) / 8;
    std::vector<float> out((size_t)(nmb * nch * 4 * 64 * 16), 0.0f);
    for (int64_t m = 0; m < co; ++m)
        for (int64_t c = 0; c < ci; ++c) {
            const float *g = w + (m * ci + c) * 9;
            double U[4][4];
            for (int xi = 0; xi < 4; ++xi)
                for (int nu = 0; nu < 4; ++nu) {
                    double v = 0.0;
                    for (int u = 0; u < 3; ++u)
                        for (int t = 0; t < 3; ++t) v += G[xi][u] * (double)g[u * 3 + t] * G[nu][t];
                    U[xi][nu] = v;
                }
            const int64_t mb = m / 32, mi = (m % 32) / 16, r = m % 16, ch = c / 8, ks = (c % 8) / 4, k = c % 4;
            for (int xi = 0; xi < 4; ++xi)
                for (int nu = 0; nu < 4; ++nu) {
                    const int64_t lane = k * 16 + r, val = (nu * 2 + ks) * 2 + mi;
                    out[(size_t)((((mb * nch + ch) * 4 + xi) * 64 + lane) * 16 + val)] = (float)U[xi][nu];
                }
        }
    return out;
}

// The mx_c3 tile (c_in % 16 == 0 and >= 128, width % 4 == 0; measured
// faster than the implicit-GEMM kernel there, slower below): 64 output
// channels x 2 rows from 128 output channels on (twice the blocks of 64 x 4
// at the MAXIM 112x160 shape, 6% faster there), 64 x 4, or 32 x 8 for
// narrow outputs.
void pick_c3(ConvCfg &c, int64_t co) {
    c.c3bm = co >= 64 ? 64 : 32;
    c.c3th = co >= 128 ? 2 : co >= 64 ? 4 : 8;
}

ConvCfg pick_conv(int64_t co, int64_t ci, int64_t oh, int64_t ow, bool k3, int cus) {
    static const struct {
        int bm, th;
        double eff;
    } cand[] = {{128, 8, 1.00}, {64, 8, 0.85}, {128, 4, 0.85}, {64, 4, 0.70}, {32, 8, 0.70}, {32, 4, 0.55}};
    const int64_t slots = 2LL * (cus > 0 ? cus : 256);
    double best = 1e300;
    ConvCfg r;
    for (auto &c : cand) {
        int64_t blocks = ((co + c.bm - 1) / c.bm) * ((oh + c.th - 1) / c.th) * ((ow + 15) / 16);
        double rounds = (double)((blocks + slots - 1) / slots);
        double cost = rounds * c.bm * c.th * 16 / c.eff;
        if (cost < best * 0.999) {
            best = cost;
            r.bm = c.bm;
            r.th = c.th;
        }
    }
    r.ck = (k3 && ci > 4) ? 8 : 4;
    if (!k3) {
        // A 4x4 whose blocks do not fill the chip twice splits its reduction
        // over 2 or 4 z-slices of at least four chunks each (partial outputs
        // in scratch, then mx_conv_split_sum): at 112x160 and 56x80 (64 and
        // 128 channels, 280 blocks) one slice per block leaves most CUs idle.
        const int64_t blocks = ((co + r.bm - 1) / r.bm) * ((oh + r.th - 1) / r.th) * ((ow + 15) / 16);
        const int64_t nchunk = (ci + 3) / 4;
        if (blocks < slots && (oh * ow) % 4 == 0)
            for (int s : {4, 2})
                if (nchunk % s == 0 && nchunk / s >= 4 && blocks * s <= 5 * slots / 2) {
                    r.nsplit = s;
                    break;
                }
    }
    if (k3 && ci > 4) {
        // measured on MI355X at the MAXIM shapes (c -> c, 32 to 128 channels):
        // 32-channel blocks of 8 rows for narrow outputs, 64 x 4 up to 64
        // channels, 32 x 4 beyond (the grid-filling shapes win)
        r.bm = co <= 16 ? 16 : co <= 32 ? 32 : co <= 64 ? 64 : 32;
        r.th = co <= 32 ? 8 : 4;
    }
    return r;
}

std::string conv_name(ConvCfg c, bool k3) {
    return std::string(k3 ? "mx_conv3x3_m" : "mx_conv4x4_m") + std::to_string(c.bm) + "_t" + std::to_string(c.th) +
           (k3 && c.ck == 4 ? "_c4" : "");
}

}  // namespace

// What the executor decides about a plan before touching the device: which
// ops fuse into which steps, and where every buffer lives in the device arena.
enum { RULE_NONE = 0, RULE_CA_MLP = 1, RULE_SCALE_ADD = 2, RULE_ELIDED = 3, RULE_PERM_IN = 4, RULE_RS_CONV = 5 };

struct StepSpec {
    uint64_t first = 0, last = 0;
    int rule = RULE_NONE;  // a fusion that is not a producer's epilogue
    int64_t ln = -1;  // a LayerNorm op folded into the next op's GEMM (== first)
    bool epi = false;  // the producer applies readers in its epilogue
    int64_t perm = -1, pout = -1;  // a BlockPerm folded into the stores, and its source
    int64_t out = -1, u = -1, r1 = -1, r2 = -1, m = -1;
    int act = MXK_ACT_NONE;
    float slope = 0.0f;
    // An elided forward BlockPerm (op xperm / rperm, RULE_PERM_IN): the folded
    // LayerNorm's GEMM reads its source xsrc through the block map, and the
    // residual step reads r1 (then the source) at its stores' image positions
    // (r1p: the permutation's output, read instead if a kernel cannot map).
    int64_t xperm = -1, xsrc = -1, rperm = -1, r1p = -1;
    int64_t xmul = -1;  // a Mul folded into the next op's GEMM operand (== first)
    // A LayerNorm of (a band of) the GEMM's output, op lno == last - 1,
    // computed in the streaming kernel's epilogue (_lo); lno_keep: the raw
    // band is read elsewhere too, so it is still stored.
    int64_t lno = -1;
    bool lno_keep = true;
    // LayerNorm statistics from the epilogue (_lo, mode 1). Producer:
    // so_nband bands of so_c channels from output row so_row0, written at
    // so_out of the statistics region as [band][2][so_hw]. Consumer (a step
    // with a folded LayerNorm): its statistics at so_in, from step so_from,
    // when that step's kernel took them.
    int64_t so_row0 = -1, so_c = 0, so_from = -1;
    int so_nband = 0;
    uint64_t so_hw = 0, so_out = 0, so_in = 0;
};

struct Program {
    std::vector<StepSpec> specs;
    std::vector<int64_t> elide_to;  // x -> the copy destination whose storage x takes, or -1
    std::vector<int64_t> dbase;     // the buffer that owns each buffer's device storage
    std::vector<uint64_t> doff;     // device element offset of every buffer
    uint64_t arena_len = 0;
    uint64_t fused_ops = 0;
    uint64_t so_len = 0;  // floats of the LayerNorm statistics region
    bool repacked = false;
    // Runs of steps (spec index ranges, inclusive) holding two steps of the
    // same shape that touch disjoint memory - the grid and block branches of a
    // multi-axis gMLP block - whose buffers the layout keeps apart for the
    // whole run, so that their launches may share one grid.
    std::vector<std::pair<uint64_t, uint64_t>> regions;
    void plan_fusion(const mx_plan_desc *p, bool require_clear);
    void storage(const mx_plan_desc *p, std::vector<int64_t> &base, std::vector<uint64_t> &delta) const;
    void plan_regions(const mx_plan_desc *p);
    void layout(const mx_plan_desc *p, bool repack);
};

class Gpu {
public:
    explicit Gpu(const mx_plan_desc *p);
    ~Gpu();
    void init(const mx_plan_desc *p);
    void release();

    HipApi &H;
    hipModule_t mod = nullptr;
    hipStream_t stream = nullptr;
    float *arena = nullptr;
    uint64_t arena_len = 0;
    unsigned char *wdev = nullptr;
    uint64_t wbytes = 0;
    float *scratch = nullptr;
    uint64_t scratch_len = 0, ln_off = 0, so_base = 0, rs_off = 0, cs_off = 0;
    uint64_t n_ops = 0, n_bufs = 0;
    std::vector<std::vector<Launch>> ops;
    uint64_t launched = 0, kernels = 0;
    bool want_timeline = false;
    std::vector<float> per_op_ms;
    float total_ms = 0.0f;
    bool have_timeline = false;
    std::string name;
    int cus = 0, clock_khz = 0;
    bool use_graph = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;

    // mxh_run_batch's staging, allocated on its first call: pinned host
    // buffers for two images each way and the events that say when the
    // device is done with each.
    struct Batch {
        float *hin[2] = {}, *hout[2] = {};
        hipEvent_t h2d[2] = {}, d2h[2] = {};  // input on the device; output in hout
        uint64_t n_in = 0, n_out = 0;
    } bt;

    // One pass over the image already in the arena, as mxh_run makes it
    // (graph replay when switched on, else the program's launches).
    void pass() {
        if (use_graph) run_graph();
        else if (fusion) run_range(0, n_ops);
        else for (uint64_t i = 0; i < n_ops; ++i) run_op(i);
    }

    void batch_setup(uint64_t n_in, uint64_t n_out) {
        if (bt.hin[0]) {
            if (bt.n_in != n_in || bt.n_out != n_out) throw Error("internal: batch staging sized for another plan");
            return;
        }
        bt.n_in = n_in;
        bt.n_out = n_out;
        for (int s = 0; s < 2; ++s) {
            check(H.hipHostMalloc((void **)&bt.hin[s], n_in * 4, 0), "hipHostMalloc(batch input)");
            check(H.hipHostMalloc((void **)&bt.hout[s], n_out * 4, 0), "hipHostMalloc(batch output)");
            for (hipEvent_t *e : {&bt.h2d[s], &bt.d2h[s]}) {
                check(H.hipEventCreate(e), "hipEventCreate");
                check(H.hipEventRecord(*e, stream), "hipEventRecord");  // complete before first use
            }
        }
        sync();
    }

    // n images through the pass, host arrays in and out, the host's copies
    // off the device's path: image k's input is staged into pinned memory
    // while pass k - 1 runs, copied in (DMA from pinned memory) right
    // before pass k and its output copied back right after it, and handed
    // to the caller while pass k + 1 runs. All on the executor's stream: the
    // device copies on a second stream overlapped the passes but slowed each
    // pass by more than they saved (measured at C4: 23.62 against 23.30 ms
    // per pass, for copies of 0.16 ms).
    void run_batch(uint64_t oi, uint64_t oo, const float *const *in, uint64_t n_in, float *const *out,
                   uint64_t n_out, uint64_t n) {
        if (n == 0) return;
        batch_setup(n_in, n_out);
        for (uint64_t k = 0; k <= n; ++k) {
            if (k < n) {
                const int s = k & 1;
                // the pinned buffer's last image (k - 2) is on the device
                check(H.hipEventSynchronize(bt.h2d[s]), "hipEventSynchronize(batch input)");
                memcpy(bt.hin[s], in[k], n_in * 4);
                check(H.hipMemcpyAsync(arena + oi, bt.hin[s], n_in * 4, kMemcpyH2D, stream), "hipMemcpyAsync(H2D)");
                check(H.hipEventRecord(bt.h2d[s], stream), "hipEventRecord");
                pass();
                // hout[s]'s last image (k - 2) went to the caller at k - 1
                check(H.hipMemcpyAsync(bt.hout[s], arena + oo, n_out * 4, kMemcpyD2H, stream), "hipMemcpyAsync(D2H)");
                check(H.hipEventRecord(bt.d2h[s], stream), "hipEventRecord");
            }
            if (k >= 1) {  // image k - 1 back to the caller, pass k (if any) queued behind it
                const int s = (k - 1) & 1;
                check(H.hipEventSynchronize(bt.d2h[s]), "hipEventSynchronize(batch output)");
                memcpy(out[k - 1], bt.hout[s], n_out * 4);
            }
        }
    }

    // The whole op list as one captured graph, instantiated on first use and
    // replayed after: one submission per pass instead of one per kernel.
    void run_graph() {
        if (!gexec) {
            check(H.hipStreamBeginCapture(stream, kCaptureModeThreadLocal), "hipStreamBeginCapture");
            const uint64_t l0 = launched, k0 = kernels;
            try {
                if (fusion) run_range(0, n_ops);
                else for (uint64_t i = 0; i < n_ops; ++i) run_op(i);
            } catch (...) {
                hipGraph_t g = nullptr;
                H.hipStreamEndCapture(stream, &g);
                if (g) H.hipGraphDestroy(g);
                throw;
            }
            launched = l0;
            graph_kernels = kernels - k0;
            kernels = k0;
            check(H.hipStreamEndCapture(stream, &graph), "hipStreamEndCapture");
            check(H.hipGraphInstantiate(&gexec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
        }
        check(H.hipGraphLaunch(gexec, stream), "hipGraphLaunch");
        launched += n_ops;
        kernels += graph_kernels;
    }
    uint64_t graph_kernels = 0;

    void check_plan(const mx_plan_desc *p) const {
        if (p->n_ops != n_ops || p->n_bufs != n_bufs || p->arena_len != plan_arena_len)
            throw Error("this executor was built for a different plan");
    }
    // on: the stream to launch on (the executor's own when null)
    void launch(Launch &l, hipStream_t on = nullptr) {
        void *params[2] = {l.a0, l.a1};
        check(H.hipModuleLaunchKernel(l.f, l.g[0], l.g[1], l.g[2], l.b[0], l.b[1], l.b[2], l.shm, on ? on : stream,
                                      params, nullptr),
              l.name);
        ++kernels;
    }
    void run_op(uint64_t i) {
        for (auto &l : ops[i]) launch(l);
        ++launched;
    }
    // Ops [first, last) through the fused program; a step that straddles the
    // range runs its ops one by one.
    void run_range(uint64_t first, uint64_t last) {
        for (const Step &st : prog) {
            if (st.last <= first || st.first >= last) continue;
            if (st.first >= first && st.last <= last) {
                if (st.so_from >= 0 && prog[st.so_from].first < first)
                    for (auto &l : st.pre) launch(const_cast<Launch &>(l));
                for (auto &l : st.launches) launch(const_cast<Launch &>(l));
                launched += st.last - st.first;
            } else {
                // A step the range cuts runs its ops one by one, each with its
                // own launch, reading what the earlier ops of the step left in
                // the arena (a contiguous run continues where the previous one
                // stopped). An elided forward permutation's output was never
                // written, as its readers take the source through a map when
                // they run fused: a reader run on its own gets it restored
                // first, from the source, which is intact until the step that
                // rewrites it has finished.
                std::set<int64_t> restored;
                for (uint64_t i = std::max(first, st.first); i < std::min(last, st.last); ++i) {
                    for (int64_t b : op_srcs[i]) {
                        auto it = elided_perm.find(b);
                        if (b < 0 || it == elided_perm.end() || it->second >= i || restored.count(b)) continue;
                        for (auto &l : ops[it->second]) launch(l);
                        restored.insert(b);
                    }
                    run_op(i);
                }
            }
        }
    }
    // The sources each op reads (a resize's intermediate plane excluded), and
    // each elided forward permutation's output -> its op.
    std::vector<std::array<int64_t, 2>> op_srcs;
    std::map<int64_t, uint64_t> elided_perm;
    std::vector<Step> prog;
    // The fused program with every scratch pointer in the code object's
    // static scratch (empty when this plan needs more than it holds).
    std::vector<Step> prog_na;
    bool fusion = true;
    Program pg;                   // the fusion decisions and the device layout
    std::vector<uint64_t> &doff;  // = pg.doff
    uint64_t plan_arena_len = 0;
    void build_program(const mx_plan_desc *p);
    void specialise(Launch &l);
    void pair_launches(const mx_plan_desc *p);
    void sync() { check(H.hipStreamSynchronize(stream), "hipStreamSynchronize"); }
    // All ops with an event before each and one after the last; one sync.
    // Every step (one op, or one fused launch standing for several) with an
    // event before each and one after the last; one synchronisation.
    // Every launch of the program (fused steps, or ops with fusion off) in
    // order, with the step or op it belongs to.
    std::vector<std::pair<uint64_t, const Launch *>> launch_list() const {
        std::vector<std::pair<uint64_t, const Launch *>> v;
        const uint64_t n = fusion ? prog.size() : n_ops;
        for (uint64_t i = 0; i < n; ++i)
            for (const Launch &l : fusion ? prog[i].launches : ops[i]) v.push_back({i, &l});
        return v;
    }
    // Every launch timed by the dispatch itself (hipExtModuleLaunchKernel's
    // start/stop events bracket the kernel's execution, not the gap before
    // it), one synchronisation: per-launch and per-step (the sum of its
    // launches) device milliseconds.
    void run_timed() {
        const uint64_t n = fusion ? prog.size() : n_ops;
        const auto seq = launch_list();
        std::vector<hipEvent_t> ev(2 * seq.size());
        for (auto &e : ev) check(H.hipEventCreate(&e), "hipEventCreate");
        for (size_t k = 0; k < seq.size(); ++k) {
            Launch &l = const_cast<Launch &>(*seq[k].second);
            void *params[2] = {l.a0, l.a1};
            const uint64_t gx = (uint64_t)l.g[0] * l.b[0], gy = (uint64_t)l.g[1] * l.b[1], gz = (uint64_t)l.g[2] * l.b[2];
            if (gx > 0xffffffffULL || gy > 0xffffffffULL || gz > 0xffffffffULL) throw Error("a timed launch exceeds 2^32 work-items");
            check(H.hipExtModuleLaunchKernel(l.f, (uint32_t)gx, (uint32_t)gy, (uint32_t)gz, l.b[0], l.b[1], l.b[2], l.shm,
                                             stream, params, nullptr, ev[2 * k], ev[2 * k + 1], 0),
                  l.name);
            ++kernels;
        }
        for (uint64_t i = 0; i < n; ++i) launched += fusion ? prog[i].last - prog[i].first : 1;
        sync();
        per_op_ms.assign(n, 0.0f);
        per_launch_ms.assign(seq.size(), 0.0f);
        total_ms = 0.0f;
        for (size_t k = 0; k < seq.size(); ++k) {
            check(H.hipEventElapsedTime(&per_launch_ms[k], ev[2 * k], ev[2 * k + 1]), "hipEventElapsedTime");
            per_op_ms[seq[k].first] += per_launch_ms[k];
            total_ms += per_launch_ms[k];
        }
        for (auto &e : ev) H.hipEventDestroy(e);
        have_timeline = true;
    }
    std::vector<float> per_launch_ms;
    void write(uint64_t off, const float *v, uint64_t n) {
        if (n == 0) return;
        if (off + n > arena_len) throw Error("a write of " + std::to_string(n) + " floats at " + std::to_string(off) + " runs past the arena");
        check(H.hipMemcpyAsync(arena + off, v, n * 4, kMemcpyH2D, stream), "hipMemcpyAsync(H2D)");
        sync();
    }
    void read(uint64_t off, float *v, uint64_t n) {
        if (n == 0) return;
        if (off + n > arena_len) throw Error("a read of " + std::to_string(n) + " floats at " + std::to_string(off) + " runs past the arena");
        check(H.hipMemcpyAsync(v, arena + off, n * 4, kMemcpyD2H, stream), "hipMemcpyAsync(D2H)");
        sync();
    }

private:
    std::vector<ConvCfg> ccfg;
    std::map<std::string, hipFunction_t> fns_;
    std::set<std::string> names_;
    const char *intern(const std::string &s) { return names_.insert(s).first->c_str(); }
    hipFunction_t fn(const char *name) {
        auto it = fns_.find(name);
        if (it != fns_.end()) return it->second;
        hipFunction_t f = nullptr;
        check(H.hipModuleGetFunction(&f, mod, name), (std::string("hipModuleGetFunction ") + name).c_str());
        fns_[name] = f;
        return f;
    }
    Launch mk(const std::string &kname) {
        Launch l;
        l.name = intern(kname);
        l.f = fn(l.name);
        return l;
    }
    // The streaming pointwise kernels (pointwise.h) for a Dense-shaped op,
    // when its shape and alignment allow them; `layout` 0 = channel-major
    // output, 1 = row-major. `alt` keeps the tiled-GEMM launch of each op that
    // got one, for fused steps whose extra operands are not 16-byte aligned.
    // fold (channel-major, batch > 1): tile the batches' columns as one axis
    // (GemmArgs fold), so a batch of N columns that is not a multiple of 64
    // leaves no ragged tile per batch.
    bool try_pw(int layout, const GemmArgs &a0, Launch &l, bool whole = false, bool fold = false) {
        if (no_pw) return false;
        GemmArgs a = a0;
        fold = fold && layout == 0 && a.batch > 1 && a.N % 4 == 0 && a.N % 64 != 0 &&
               (int64_t)a.batch * a.N < 0x7fffffffLL && a.sC == (int64_t)a.M * a.N;
        if (fold) {
            a.fold = a.N;
            div_magic((uint32_t)a.N, a.fmul, a.fsh);
        }
        const int64_t wout = layout == 0 ? a.M : a.N, slen = layout == 0 ? (fold ? (int64_t)a.batch * a.N : a.N) : a.M;
        if (a.K % 16 || a.N % 4 || a.K == 0 || wout <= 0 || slen <= 0) return false;
        if (!aligned(a.A, 16) || !aligned(a.B, 16) || !aligned(a.C, 16)) return false;
        if (layout == 1 && !aligned(a.bias, 16)) return false;
        if (a.sA % 4 || a.sB % 4 || a.sC % 4 || a.batch > 65535) return false;
        static const char *names[2][3] = {{"mx_pw_ch1", "mx_pw_ch2", "mx_pw_ch4"},
                                          {"mx_pw_rw1", "mx_pw_rw2", "mx_pw_rw4"}};
        // Tile width and reduction split, from measurements on MI355X: 32
        // weight outputs per wave in both layouts (64 for the row-major
        // form's long reductions reused each operand load twice as often
        // but held 186 VGPRs, two waves per SIMD: the GateMm mode-1 launches
        // run 2-7% faster at 32 at 224x320 and the same at 448x640; the
        // channel-major form is 3-12% faster at 32 for 1x1 convs of 256-512
        // inputs and GateMm over 256 tokens); the block's four waves split
        // reductions of 128 and more, and shorter ones when one wave per
        // tile would leave SIMDs idle.
        const int ti = wout <= 16 ? 0 : 1, tmw = 1 << ti;
        const int64_t nib = (wout + 16 * tmw - 1) / (16 * tmw);
        const int64_t tiles = nib * ((slen + 63) / 64);
        if (tiles > 0x7fffffffLL) return false;
        // whole: the reduction stays in one wave (a step whose epilogue
        // normalises bands across several waves of a block, which needs them
        // to hold whole tiles)
        const int64_t nbat = fold ? 1 : a.batch;
        const bool k4 = !whole && a.K % 64 == 0 && (a.K >= 128 || tiles * nbat < 2LL * 4 * cus);
        l = mk(std::string(names[layout][ti]).insert(8, fold ? "b" : "") + (k4 ? "_k4" : ""));
        const int64_t grid = k4 ? tiles : (tiles + 3) / 4;
        if (grid > 0x7fffffffLL) return false;
        l.g[0] = (unsigned)grid;
        l.g[1] = (unsigned)nbat;
        l.kind = 1;
        set_args(l, a);
        return true;
    }
    std::vector<std::vector<Launch>> alt;
    std::vector<char> whole_k;  // per op: keep a streaming GEMM's reduction in one wave
    bool no_pw = getenv("MAXIM_NO_PW") != nullptr;
    // keep the plan's order of arithmetic everywhere (fused = unfused to the bit)
    bool plan_order = getenv("MAXIM_PLAN_ORDER") != nullptr;
    void validate(const mx_plan_desc *p) const;
    void build_launches(const mx_plan_desc *p, const std::vector<int64_t> &woff,
                        const std::vector<std::array<int64_t, 4>> &extra,
                        const std::vector<std::array<int, 2>> &maxt);
};

// Every op is checked against the buffer table before anything touches the
// device: a wrong dimension would otherwise become an out-of-bounds kernel.
void Gpu::validate(const mx_plan_desc *p) const {
    auto len = [&](int64_t id) -> uint64_t {
        if (id < 0 || (uint64_t)id >= p->n_bufs) throw Error("an op names buffer " + std::to_string(id) + ", which does not exist");
        const mx_bufshape &s = p->bufs[id];
        uint64_t n = (uint64_t)(s.c * s.h * s.w);
        if (p->offs[id] + n > p->arena_len) throw Error("buffer " + std::to_string(id) + " runs past the arena");
        return n;
    };
    auto wlen = [&](int64_t id) -> uint64_t {
        if (id < 0 || (uint64_t)id >= p->n_weights) throw Error("an op names weight " + std::to_string(id) + ", which does not exist");
        return p->weight_lens[id];
    };
    auto shape = [&](int64_t id, int64_t c, int64_t h, int64_t w, const char *what) {
        const mx_bufshape &s = p->bufs[id];
        len(id);
        if (s.c != c || s.h != h || s.w != w)
            throw Error(std::string(what) + ": buffer " + std::to_string(id) + " is not [" + std::to_string(c) + "][" +
                        std::to_string(h) + "][" + std::to_string(w) + "]");
    };
    auto need = [](bool ok, const char *what) {
        if (!ok) throw Error(std::string("inconsistent op: ") + what);
    };
    for (uint64_t i = 0; i < p->n_ops; ++i) {
        const mx_op &o = p->ops[i];
        try {
            switch (o.kind) {
                case MX_OP_COPY:
                case MX_OP_GELU:
                case MX_OP_LRELU:
                case MX_OP_SIGMOID:
                    need(o.n >= 0 && (uint64_t)o.n <= len(o.dst) && (uint64_t)o.n <= len(o.src), "elementwise n");
                    break;
                case MX_OP_ADD:
                case MX_OP_MUL:
                case MX_OP_GATE_APPLY:
                    need((uint64_t)o.n == len(o.dst) && (uint64_t)o.n == len(o.src) && (uint64_t)o.n == len(o.src2), "binary n");
                    break;
                case MX_OP_CHAN_LN:
                    need(len(o.dst) == (uint64_t)(o.c * o.hw) && len(o.src) == (uint64_t)(o.c * o.hw), "chan_ln shape");
                    need(wlen(o.scale) == (uint64_t)o.c && wlen(o.bias) == (uint64_t)o.c, "chan_ln weights");
                    break;
                case MX_OP_CHAN_MEAN:
                    need(len(o.dst) == (uint64_t)o.c && len(o.src) == (uint64_t)(o.c * o.hw) && o.hw > 0, "chan_mean shape");
                    break;
                case MX_OP_CHAN_SCALE:
                    need(len(o.src2) == (uint64_t)o.c && len(o.dst) >= (uint64_t)(o.c * o.hw) && len(o.src) >= (uint64_t)(o.c * o.hw), "chan_scale shape");
                    break;
                case MX_OP_CONV1X1:
                    shape(o.dst, o.c_out, o.h, o.wd, "conv1x1 out");
                    shape(o.src, o.c_in, o.h, o.wd, "conv1x1 in");
                    need(wlen(o.w) == (uint64_t)(o.c_in * o.c_out), "conv1x1 weight");
                    if (o.bias >= 0) need(wlen(o.bias) == (uint64_t)o.c_out, "conv1x1 bias");
                    break;
                case MX_OP_CONV3X3:
                    shape(o.dst, o.c_out, o.h, o.wd, "conv3x3 out");
                    shape(o.src, o.c_in, o.h, o.wd, "conv3x3 in");
                    need(wlen(o.w) == (uint64_t)(9 * o.c_in * o.c_out), "conv3x3 weight");
                    if (o.bias >= 0) need(wlen(o.bias) == (uint64_t)o.c_out, "conv3x3 bias");
                    break;
                case MX_OP_CONV4X4S2:
                    shape(o.dst, o.c_out, o.oh, o.ow, "conv4x4 out");
                    shape(o.src, o.c_in, o.h, o.wd, "conv4x4 in");
                    need(wlen(o.w) == (uint64_t)(16 * o.c_in * o.c_out), "conv4x4 weight");
                    if (o.bias >= 0) need(wlen(o.bias) == (uint64_t)o.c_out, "conv4x4 bias");
                    need(o.p[0] >= 0 && o.p[0] < 4 && o.p[1] >= 0 && o.p[1] < 4, "conv4x4 padding");
                    break;
                case MX_OP_CONVT2X2:
                    shape(o.dst, o.c_out, 2 * o.h, 2 * o.wd, "convt out");
                    shape(o.src, o.c_in, o.h, o.wd, "convt in");
                    need(wlen(o.w) == (uint64_t)(4 * o.c_in * o.c_out), "convt weight");
                    if (o.bias >= 0) need(wlen(o.bias) == (uint64_t)o.c_out, "convt bias");
                    break;
                case MX_OP_GATE_MM: {
                    int64_t outer = o.p[0], inner = o.p[1], k = o.mode == 0 ? outer : inner;
                    shape(o.dst, o.c, outer, inner, "gate_mm out");
                    shape(o.src, o.c, outer, inner, "gate_mm in");
                    need(o.mode == 0 || o.mode == 1, "gate_mm mode");
                    need(wlen(o.w) == (uint64_t)(k * k), "gate_mm weight");
                    if (o.bias >= 0) need(wlen(o.bias) == (uint64_t)k, "gate_mm bias");
                    break;
                }
                case MX_OP_BLOCK_PERM: {
                    int64_t gh = o.p[0], gw = o.p[1], fh = o.p[2], fw = o.p[3];
                    need(gh > 0 && gw > 0 && fh > 0 && fw > 0 && gh * fh <= o.h && gw * fw <= o.wd, "block_perm cells");
                    need(len(o.src) >= (uint64_t)(o.c * o.h * o.wd) && len(o.dst) >= (uint64_t)(o.c * o.h * o.wd), "block_perm size");
                    need(len(o.src) == len(o.dst), "block_perm sizes differ");
                    break;
                }
                case MX_OP_RESIZE:
                    shape(o.dst, o.c, o.oh, o.ow, "resize out");
                    shape(o.src, o.c, o.h, o.wd, "resize in");
                    shape(o.src2, o.c, o.h, o.ow, "resize tmp");
                    break;
                case MX_OP_DOWN_S:
                    shape(o.dst, o.c, o.oh, o.ow, "down out");
                    shape(o.src, o.c, o.h, o.wd, "down in");
                    need((o.oh - 1) * o.p[0] + o.p[1] < o.h && (o.ow - 1) * o.p[0] + o.p[1] < o.wd, "down range");
                    break;
                default:
                    throw Error("unknown op kind " + std::to_string(o.kind));
            }
        } catch (const Error &e) {
            throw Error("op " + std::to_string(i) + ": " + e.what());
        }
    }
}

// A constructor that throws never runs the destructor, so every HIP object
// created before a refusal or a later failure (module, stream, arena,
// weights, scratch) is released here before the error propagates: a caller
// that retries at a smaller size finds the device as it was.
Gpu::Gpu(const mx_plan_desc *p) : H(hip()), doff(pg.doff) {
    try {
        init(p);
    } catch (...) {
        release();
        throw;
    }
}

void Gpu::init(const mx_plan_desc *p) {
    validate(p);
    op_srcs.assign(p->n_ops, {-1, -1});
    for (uint64_t i = 0; i < p->n_ops; ++i)
        op_srcs[i] = {p->ops[i].src, p->ops[i].kind == MX_OP_RESIZE ? -1 : p->ops[i].src2};
    check(H.hipInit(0), "hipInit");
    int ndev = 0;
    check(H.hipGetDeviceCount(&ndev), "hipGetDeviceCount");
    if (ndev < 1) throw Error("no HIP device");
    check(H.hipSetDevice(0), "hipSetDevice");
    char nm[256] = {0};
    if (H.hipDeviceGetName(nm, sizeof nm - 1, 0) == 0) name = nm;
    H.hipDeviceGetAttribute(&cus, kAttrMultiprocessorCount, 0);
    H.hipDeviceGetAttribute(&clock_khz, kAttrClockRate, 0);
    const DeviceCode &dc = device_code(H, 0);
    mod = dc.mod;
    // The runtime reports an empty marketing name for devices its name table
    // does not list; the code object only loads on gfx950, so that names it.
    if (name.empty()) name = "AMD gfx950 (" + std::to_string(cus) + " CUs)";
    check(H.hipStreamCreate(&stream), "hipStreamCreate");

    // Device weights, in the layout each kernel reads, packed into one blob.
    std::vector<float> blob;
    auto place = [&](const float *v, uint64_t n) -> int64_t {
        blob.resize((blob.size() + 63) & ~(size_t)63);
        int64_t off = (int64_t)blob.size();
        blob.insert(blob.end(), v, v + n);
        return off;
    };
    auto placev = [&](const std::vector<float> &v) { return place(v.data(), v.size()); };
    const size_t nw = p->n_weights;
    std::vector<int64_t> woff(nw, -1);
    auto as_is = [&](int64_t id) {
        if (id >= 0 && woff[id] < 0) woff[id] = place(p->weights[id], p->weight_lens[id]);
    };
    std::vector<std::array<int64_t, 4>> extra(p->n_ops, {-1, -1, -1, -1});  // per-op derived blobs
    std::vector<std::array<int, 2>> maxt(p->n_ops, {0, 0});
    ccfg.assign(p->n_ops, ConvCfg{});
    uint64_t mean_scratch = 0;
    for (uint64_t i = 0; i < p->n_ops; ++i) {
        const mx_op &o = p->ops[i];
        switch (o.kind) {
            case MX_OP_CHAN_LN:
                as_is(o.scale);
                as_is(o.bias);
                break;
            case MX_OP_CHAN_MEAN: {
                const int64_t chunk = mean_chunk(o.hw);
                const int64_t nchunk = (o.hw + chunk - 1) / chunk;
                mean_scratch = std::max<uint64_t>(mean_scratch, (uint64_t)(o.c * nchunk));
                break;
            }
            case MX_OP_CONV1X1:
                as_is(o.w);
                as_is(o.bias);
                break;
            case MX_OP_CONV3X3:
            case MX_OP_CONV4X4S2: {
                // [co][ci][k][k] -> the kernel's LDS tiles, [m-block][chunk][tap*CK + c][BM]
                const bool k3 = o.kind == MX_OP_CONV3X3;
                const int taps = k3 ? 9 : 16;
                const ConvCfg cc = pick_conv(o.c_out, o.c_in, k3 ? o.h : o.oh, k3 ? o.wd : o.ow, k3, cus);
                ccfg[i] = cc;
                const float *w = p->weights[o.w];
                const int64_t nmb = (o.c_out + cc.bm - 1) / cc.bm, nch = (o.c_in + cc.ck - 1) / cc.ck;
                const int64_t kc = (int64_t)taps * cc.ck;
                std::vector<float> t((size_t)(nmb * nch * kc * cc.bm), 0.0f);
                for (int64_t mb = 0; mb < nmb; ++mb)
                    for (int64_t ch = 0; ch < nch; ++ch)
                        for (int64_t k = 0; k < kc; ++k)
                            for (int64_t m = 0; m < cc.bm; ++m) {
                                const int64_t gm = mb * cc.bm + m, gc = ch * cc.ck + k % cc.ck, tp = k / cc.ck;
                                if (gm < o.c_out && gc < o.c_in)
                                    t[((mb * nch + ch) * kc + k) * cc.bm + m] = w[(gm * o.c_in + gc) * taps + tp];
                            }
                extra[i][0] = placev(t);
                if (k3 && o.c_in % 16 == 0 && o.c_in >= 128 && o.wd % 4 == 0) {
                    // the mx_c3 weight tiles: [m-block][chunk][BM][tap][16]
                    pick_c3(ccfg[i], o.c_out);
                    const int bm = ccfg[i].c3bm;
                    const int64_t nb = (o.c_out + bm - 1) / bm, nc = o.c_in / 16;
                    std::vector<float> u((size_t)(nb * nc * bm * 9 * 16), 0.0f);
                    for (int64_t mb = 0; mb < nb; ++mb)
                        for (int64_t ch = 0; ch < nc; ++ch)
                            for (int64_t m = 0; m < bm; ++m)
                                for (int tp = 0; tp < 9; ++tp)
                                    for (int c = 0; c < 16; ++c) {
                                        const int64_t gm = mb * bm + m, gc = ch * 16 + c;
                                        if (gm < o.c_out)
                                            u[(((mb * nc + ch) * bm + m) * 9 + tp) * 16 + c] = w[(gm * o.c_in + gc) * 9 + tp];
                                    }
                    extra[i][1] = placev(u);
                }
                if (k3 && o.c_out <= 4) {
                    // the vector-ALU kernel's [c_in][9 taps][4] (zero past c_out)
                    std::vector<float> q((size_t)(o.c_in * 36), 0.0f);
                    for (int64_t c = 0; c < o.c_in; ++c)
                        for (int tp = 0; tp < 9; ++tp)
                            for (int64_t m = 0; m < o.c_out; ++m) q[(c * 9 + tp) * 4 + m] = w[(m * o.c_in + c) * 9 + tp];
                    extra[i][3] = placev(q);
                }
                if (k3 && !std::getenv("MAXIM_NO_WINOGRAD")) {
                    ccfg[i].wtc = pick_wino(o.c_in, o.c_out, o.h, o.wd);
                    if (ccfg[i].wtc) extra[i][2] = placev(wino_weights(w, o.c_out, o.c_in));
                }
                as_is(o.bias);
                break;
            }
            case MX_OP_CONVT2X2: {
                // [ci][co][2][2] (flipped) -> [tap][co][ci]
                const float *w = p->weights[o.w];
                std::vector<float> t((size_t)(4 * o.c_out * o.c_in));
                for (int64_t c = 0; c < o.c_in; ++c)
                    for (int64_t m = 0; m < o.c_out; ++m)
                        for (int tp = 0; tp < 4; ++tp) t[(tp * o.c_out + m) * o.c_in + c] = w[(c * o.c_out + m) * 4 + tp];
                extra[i][0] = placev(t);
                // and rows ordered (ky, oc, kx) for the streaming kernels' _t form
                for (int64_t c = 0; c < o.c_in; ++c)
                    for (int64_t m = 0; m < o.c_out; ++m)
                        for (int tp = 0; tp < 4; ++tp)
                            t[(((tp >> 1) * o.c_out + m) * 2 + (tp & 1)) * o.c_in + c] = w[(c * o.c_out + m) * 4 + tp];
                extra[i][1] = placev(t);
                as_is(o.bias);
                break;
            }
            case MX_OP_GATE_MM: {
                as_is(o.w);  // [a][t]: the streaming kernels' layout, both modes
                if (o.mode == 1) {
                    // [a][t] -> [t][a], the B operand of the tiled X . W^T
                    const int64_t k = o.p[1];
                    const float *w = p->weights[o.w];
                    std::vector<float> t((size_t)(k * k));
                    for (int64_t a = 0; a < k; ++a)
                        for (int64_t tt = 0; tt < k; ++tt) t[tt * k + a] = w[a * k + tt];
                    extra[i][0] = placev(t);
                }
                as_is(o.bias);
                break;
            }
            case MX_OP_RESIZE: {
                extra[i][0] = placev(resize_table(o.wd, o.ow, maxt[i][0]));
                extra[i][1] = placev(resize_table(o.h, o.oh, maxt[i][1]));
                break;
            }
            default:
                break;
        }
    }
    blob.resize((blob.size() + 63) & ~(size_t)63);

    // The fused program and the device layout it implies.
    n_ops = p->n_ops;
    n_bufs = p->n_bufs;
    plan_arena_len = p->arena_len;
    const bool repack = p->alias_parent && p->alias_delta && !std::getenv("MAXIM_PLAN_LAYOUT");
    pg.plan_fusion(p, !repack);
    if (repack && !std::getenv("MAXIM_NO_PAIR")) pg.plan_regions(p);
    pg.layout(p, repack);
    arena_len = pg.arena_len;
    // A 1x1 conv whose step normalises (or takes the statistics of) output
    // bands of 128 channels needs whole tiles per wave, so four waves of a
    // block hold a band (64-channel bands fit one 64-wide wave with the
    // split reduction). Up to 128 inputs, with at least two 32-wide tiles per
    // SIMD, that costs the split reduction 1-2 us (measured at the MAXIM
    // 112x160 shapes) and saves a LayerNorm or statistics pass; with fewer
    // tiles (56x80) the whole reductions cost more than the pass. Its own
    // launch takes the same form, so the fused and unfused passes still
    // agree to the bit.
    whole_k.assign(p->n_ops, 0);
    for (const StepSpec &sp : pg.specs) {
        const uint64_t g = sp.ln >= 0 ? sp.first + 1 : sp.first;
        if (g >= p->n_ops || p->ops[g].kind != MX_OP_CONV1X1 || p->ops[g].c_in > 128) continue;
        const mx_op &c = p->ops[g];
        const int64_t band = sp.lno >= 0 ? p->ops[sp.lno].c : sp.so_nband > 0 ? sp.so_c : 0;
        const int64_t tiles = (c.c_out + 31) / 32 * ((c.h * c.wd + 63) / 64);
        if (band > 64 && tiles >= 8LL * cus) whole_k[g] = 1;
    }

    // Size the pass before allocating it, and refuse with the numbers.
    wbytes = blob.size() * 4;
    // Scratch: channel-mean partial sums, then the statistics of a folded
    // LayerNorm ([2][hw], one step at a time).
    ln_off = (mean_scratch + 63) & ~(uint64_t)63;
    uint64_t ln_need = 0;
    for (const StepSpec &sp : pg.specs)
        if (sp.ln >= 0) ln_need = std::max<uint64_t>(ln_need, 2 * (uint64_t)p->ops[sp.ln].hw);
    // then the statistics that steps' epilogues leave for later steps
    so_base = (ln_off + ln_need + 63) & ~(uint64_t)63;
    // then the low-resolution 1x1 conv outputs of commuted Resize -> Conv1x1
    // steps (one step at a time)
    uint64_t rs_need = 0;
    for (const StepSpec &sp : pg.specs)
        if (sp.rule == RULE_RS_CONV) {
            const mx_op &r = p->ops[sp.first], &c = p->ops[sp.first + 1];
            rs_need = std::max<uint64_t>(rs_need, (uint64_t)(c.c_out * r.h * r.wd));
        }
    rs_off = (so_base + pg.so_len + 63) & ~(uint64_t)63;
    // and, in the same region (a step uses one or the other, never both), the
    // partial outputs of split-reduction 4x4 convs (one op at a time)
    uint64_t cs_need = 0;
    for (uint64_t i = 0; i < p->n_ops; ++i)
        if (p->ops[i].kind == MX_OP_CONV4X4S2 && ccfg[i].nsplit > 1)
            cs_need = std::max<uint64_t>(cs_need, (uint64_t)(ccfg[i].nsplit * p->ops[i].c_out * p->ops[i].oh * p->ops[i].ow));
    cs_off = rs_off;
    scratch_len = std::max<uint64_t>(rs_off + std::max(rs_need, cs_need), 64);
    const uint64_t need = arena_len * 4 + wbytes + scratch_len * 4;
    size_t free_b = 0, total_b = 0;
    if (H.hipMemGetInfo(&free_b, &total_b) == 0 && need > free_b) {
        throw Error("not enough device memory for a " + std::to_string(p->bufs[p->input].w) + "x" +
                    std::to_string(p->bufs[p->input].h) + " pass\nmaxim: the arena needs " +
                    std::to_string((arena_len * 4) >> 20) + " MiB and the weights " + std::to_string(wbytes >> 20) +
                    " MiB; " + std::to_string(free_b >> 20) +
                    " MiB is free\nmaxim: the arena is exact - the packed size of this pass - so this is a hard limit");
    }
    void *ptr = nullptr;
    hipError_t rc = H.hipMalloc(&ptr, std::max<uint64_t>(arena_len, 1) * 4);
    if (rc != 0)
        throw Error("the arena (" + std::to_string((arena_len * 4) >> 20) + " MiB) did not fit after all, with " +
                    std::to_string(free_b >> 20) + " MiB free: " + H.hipGetErrorString(rc));
    arena = static_cast<float *>(ptr);
    check(H.hipMalloc(&ptr, std::max<uint64_t>(wbytes, 256)), "hipMalloc(weights)");
    wdev = static_cast<unsigned char *>(ptr);
    check(H.hipMalloc(&ptr, scratch_len * 4), "hipMalloc(scratch)");
    scratch = static_cast<float *>(ptr);
    if (wbytes) check(H.hipMemcpy(wdev, blob.data(), wbytes, kMemcpyH2D), "hipMemcpy(weights)");
    if (std::getenv("MAXIM_LOG_ALLOC"))
        fprintf(stderr, "maxim: arena [%p, %p) weights [%p, %p) scratch [%p, %p) static scratch [%p, %p)\n",
                (void *)arena, (void *)(arena + arena_len), (void *)wdev, (void *)(wdev + wbytes), (void *)scratch,
                (void *)(scratch + scratch_len), (void *)dc.scratch, (void *)((char *)dc.scratch + dc.scratch_bytes));

    build_launches(p, woff, extra, maxt);
    build_program(p);

    // The same program over the code object's static scratch, for
    // mxh_run_noalloc: the launches differ only in their scratch pointers.
    if (scratch_len * 4 <= dc.scratch_bytes) {
        float *own = scratch;
        auto ops0 = std::move(ops);
        auto alt0 = std::move(alt);
        auto prog0 = std::move(prog);
        scratch = dc.scratch;
        build_launches(p, woff, extra, maxt);
        build_program(p);
        prog_na = std::move(prog);
        ops = std::move(ops0);
        alt = std::move(alt0);
        prog = std::move(prog0);
        scratch = own;
    }
}

void Gpu::build_launches(const mx_plan_desc *p, const std::vector<int64_t> &woff,
                         const std::vector<std::array<int64_t, 4>> &extra,
                         const std::vector<std::array<int, 2>> &maxt) {
    auto B = [&](int64_t id) { return arena + doff[id]; };
    auto W = [&](int64_t id) -> const float * {
        if (id < 0) return nullptr;
        if (woff[id] < 0) throw Error("internal: weight " + std::to_string(id) + " was not uploaded");
        return reinterpret_cast<const float *>(wdev) + woff[id];
    };
    auto X = [&](uint64_t i, int k) { return reinterpret_cast<const float *>(wdev) + extra[i][k]; };
    ops.assign(p->n_ops, {});
    alt.assign(p->n_ops, {});
    for (uint64_t i = 0; i < p->n_ops; ++i) {
        const mx_op &o = p->ops[i];
        auto &L = ops[i];
        switch (o.kind) {
            case MX_OP_COPY:
            case MX_OP_ADD:
            case MX_OP_MUL:
            case MX_OP_GATE_APPLY:
            case MX_OP_GELU:
            case MX_OP_LRELU:
            case MX_OP_SIGMOID: {
                if (o.n == 0) break;
                static const char *v4[] = {"mx_copy_v4", "mx_add_v4", "mx_mul_v4", "mx_gate_apply_v4",
                                           "mx_gelu_v4", "mx_lrelu_v4", "mx_sigmoid_v4"};
                static const char *s1[] = {"mx_copy_s", "mx_add_s", "mx_mul_s", "mx_gate_apply_s",
                                           "mx_gelu_s", "mx_lrelu_s", "mx_sigmoid_s"};
                int k;
                switch (o.kind) {
                    case MX_OP_COPY: k = MXK_COPY; break;
                    case MX_OP_ADD: k = MXK_ADD; break;
                    case MX_OP_MUL: k = MXK_MUL; break;
                    case MX_OP_GATE_APPLY: k = MXK_GATE_APPLY; break;
                    case MX_OP_GELU: k = MXK_GELU; break;
                    case MX_OP_LRELU: k = MXK_LRELU; break;
                    default: k = MXK_SIGMOID; break;
                }
                EwArgs a{};
                a.a = B(o.src);
                a.b = o.src2 >= 0 ? B(o.src2) : nullptr;
                a.y = B(o.dst);
                a.n = o.n;
                a.op = k;
                a.slope = o.slope;
                bool vec = o.n % 4 == 0 && aligned(a.a, 16) && aligned(a.y, 16) && (!a.b || aligned(a.b, 16));
                Launch l = mk(vec ? v4[k] : s1[k]);
                l.g[0] = vec ? cdiv(o.n / 4, MXK_BLOCK * 4) : cdiv(o.n, MXK_BLOCK);
                set_args(l, a);
                L.push_back(l);
                break;
            }
            case MX_OP_CHAN_SCALE: {
                ChanScaleArgs a{B(o.src), B(o.src2), B(o.dst), o.hw, o.c, nullptr, nullptr};
                bool vec = o.hw % 4 == 0 && aligned(a.x, 16) && aligned(a.y, 16);
                Launch l = mk(vec ? "mx_chan_scale_v4" : "mx_chan_scale_s");
                l.g[0] = vec ? cdiv(o.hw / 4, MXK_BLOCK * 4) : cdiv(o.hw, MXK_BLOCK);
                l.g[1] = grid_yz(o.c);
                set_args(l, a);
                L.push_back(l);
                break;
            }
            case MX_OP_CHAN_LN: {
                ChanLnArgs a{B(o.src), W(o.scale), W(o.bias), B(o.dst), o.hw, (int32_t)o.c, mx::kEps};
                const char *k = "mx_chan_ln_any";
                int64_t per = MXK_BLOCK;  // pixels per block
                const bool vec = o.hw % 4 == 0 && aligned(a.x, 16) && aligned(a.y, 16);
                std::string kn = k;
                if (vec && (o.c == 32 || o.c == 64 || o.c == 128)) {
                    const auto t = ln_tile(o.c, o.hw, cus);
                    kn = "mx_chan_ln_c" + std::to_string(o.c) + t.second;
                    per = t.first;
                }
                Launch l = mk(kn);
                l.g[0] = cdiv(o.hw, per);
                set_args(l, a);
                L.push_back(l);
                break;
            }
            case MX_OP_CHAN_MEAN: {
                const int64_t chunk = mean_chunk(o.hw);
                const int32_t nchunk = (int32_t)((o.hw + chunk - 1) / chunk);
                ChanMeanArgs a{B(o.src), scratch, B(o.dst), o.hw, chunk, (int32_t)o.c, nchunk};
                const bool vec = o.hw % 4 == 0 && aligned(a.x, 16);
                Launch l1 = mk(vec ? "mx_chan_mean_part4" : "mx_chan_mean_part");
                l1.g[0] = (unsigned)nchunk;
                l1.g[1] = grid_yz(o.c);
                set_args(l1, a);
                L.push_back(l1);
                Launch l2 = mk("mx_chan_mean_final");
                l2.g[0] = cdiv(o.c, MXK_BLOCK);
                set_args(l2, a);
                L.push_back(l2);
                break;
            }
            case MX_OP_CONV1X1: {
                const int64_t plane = o.h * o.wd;
                if (plane == 1) {
                    GemvArgs a{W(o.w), B(o.src), W(o.bias), B(o.dst), (int32_t)o.c_in, (int32_t)o.c_out};
                    Launch l = mk("mx_gemv");
                    l.g[0] = cdiv(o.c_out, MXK_BLOCK);
                    set_args(l, a);
                    L.push_back(l);
                    break;
                }
                GemmArgs a{};
                a.A = W(o.w);
                a.B = B(o.src);
                a.bias = W(o.bias);
                a.C = B(o.dst);
                a.M = (int32_t)o.c_out;
                a.N = (int32_t)plane;
                a.K = (int32_t)o.c_in;
                a.batch = 1;
                a.bias_mode = o.bias >= 0 ? MXK_BIAS_ROW : MXK_BIAS_NONE;
                a.epi = MXK_EPI_PLAIN;
                if (plane > 0x7fffffff) throw Error("conv1x1 plane too large");
                a.cvec = aligned(a.C, 16) && plane % 4 == 0;
                Tile t = pick_tile(o.c_out, plane, 1, cus);
                Launch l = mk(gemm_name(t, o.c_in % 4 == 0 && aligned(a.A, 16)));
                l.g[0] = cdiv(plane, t.bn);
                l.g[1] = grid_yz((o.c_out + t.bm - 1) / t.bm);
                set_args(l, a);
                l.kind = 1;
                Launch q;
                if (try_pw(0, a, q, whole_k[i])) {
                    alt[i].push_back(l);
                    L.push_back(q);
                } else {
                    L.push_back(l);
                }
                break;
            }
            case MX_OP_CONV3X3:
            case MX_OP_CONV4X4S2: {
                const bool k3 = o.kind == MX_OP_CONV3X3;
                ConvArgs a{};
                a.x = B(o.src);
                a.w = X(i, 0);
                a.bias = W(o.bias);
                a.y = B(o.dst);
                a.ci = (int32_t)o.c_in;
                a.co = (int32_t)o.c_out;
                a.h = (int32_t)o.h;
                a.wd = (int32_t)o.wd;
                a.oh = (int32_t)(k3 ? o.h : o.oh);
                a.ow = (int32_t)(k3 ? o.wd : o.ow);
                a.pad_top = (int32_t)(k3 ? 1 : o.p[0]);
                a.pad_left = (int32_t)(k3 ? 1 : o.p[1]);
                a.cvec = aligned(a.y, 16) && a.ow % 4 == 0;
                const ConvCfg &cc = ccfg[i];
                // the vector halo fetch: 16-byte aligned input rows and whole
                // 16-wide tiles
                const bool xv = k3 && cc.ck == 8 && aligned(a.x, 16) && a.wd % 4 == 0 && a.ow % 16 == 0;
                std::string cn = conv_name(cc, k3);
                if (xv) cn = "mx_conv3x3v_" + cn.substr(strlen("mx_conv3x3_"));
                Launch l = mk(cn);
                const int64_t tiles = (int64_t)((a.oh + cc.th - 1) / cc.th) * ((a.ow + 15) / 16);
                l.g[0] = cdiv(tiles, 1);
                l.g[1] = grid_yz((o.c_out + cc.bm - 1) / cc.bm);
                set_args(l, a);
                l.kind = 2;
                if (!k3 && cc.nsplit > 1 && aligned(a.y, 16)) {
                    // the reduction in z-slices into scratch, then their sum
                    ConvArgs b = a;
                    b.y = scratch + cs_off;
                    b.bias = nullptr;
                    b.cvec = a.ow % 4 == 0;
                    b.ksplit = (int32_t)((o.c_in + 3) / 4 / cc.nsplit);
                    Launch q = mk(cn + "_s");
                    q.g[0] = l.g[0];
                    q.g[1] = l.g[1];
                    q.g[2] = (unsigned)cc.nsplit;
                    set_args(q, b);
                    q.kind = 2;
                    const int64_t n = o.c_out * o.oh * o.ow;
                    ConvSumArgs sa{scratch + cs_off, a.bias, a.y, n, o.oh * o.ow, cc.nsplit, 0};
                    Launch r = mk("mx_conv_split_sum");
                    r.g[0] = cdiv(n / 4, 256);
                    set_args(r, sa);
                    L.push_back(q);
                    L.push_back(r);
                    break;
                }
                if (k3 && o.c_out <= 4 && o.c_in >= 64) {
                    // at most four outputs from many inputs: the vector-ALU
                    // kernel (measured faster than 16-channel MFMA blocks
                    // from 64 inputs at the MAXIM shapes, slower at 32)
                    ConvArgs b = a;
                    b.w = X(i, 3);
                    Launch q = mk("mx_conv3x3_co4");
                    q.g[0] = cdiv((int64_t)((a.oh + 7) / 8) * ((a.ow + 7) / 8), 1);
                    set_args(q, b);
                    q.kind = 2;
                    alt[i].push_back(l);
                    L.push_back(q);
                } else if (k3 && cc.wtc && aligned(a.x, 16)) {
                    // Winograd F(2x2, 3x3): 32 output channels x TR x TC tiles
                    ConvArgs b = a;
                    b.w = X(i, 2);
                    b.cvec = aligned(a.y, 8) && a.ow % 2 == 0;
                    Launch q = mk("mx_wino3_t" + std::to_string(cc.wtc));
                    const int trows = cc.wtc == 16 ? 4 : 8;  // output rows per block
                    q.g[0] = cdiv((int64_t)((a.oh + trows - 1) / trows) * ((a.ow + 2 * cc.wtc - 1) / (2 * cc.wtc)), 1);
                    q.g[1] = grid_yz((o.c_out + 31) / 32);
                    set_args(q, b);
                    q.kind = 2;
                    alt[i].push_back(l);
                    L.push_back(q);
                } else if (k3 && extra[i][1] >= 0 && aligned(a.x, 16) && aligned(a.y, 16)) {
                    // mx_c3 (channel-last LDS tiles, 128-bit fragment reads)
                    ConvArgs b = a;
                    b.w = X(i, 1);
                    Launch q = mk("mx_c3_m" + std::to_string(cc.c3bm) + "_t" + std::to_string(cc.c3th));
                    q.g[0] = cdiv((int64_t)((a.oh + cc.c3th - 1) / cc.c3th) * ((a.ow + 15) / 16), 1);
                    q.g[1] = grid_yz((o.c_out + cc.c3bm - 1) / cc.c3bm);
                    set_args(q, b);
                    q.kind = 2;
                    alt[i].push_back(l);
                    L.push_back(q);
                } else {
                    L.push_back(l);
                }
                break;
            }
            case MX_OP_CONVT2X2: {
                const int64_t plane = o.h * o.wd;
                GemmArgs a{};
                a.A = X(i, 0);
                a.B = B(o.src);
                a.bias = W(o.bias);
                a.C = B(o.dst);
                a.M = (int32_t)(4 * o.c_out);
                a.N = (int32_t)plane;
                a.K = (int32_t)o.c_in;
                a.batch = 1;
                a.bias_mode = MXK_BIAS_NONE;
                a.epi = MXK_EPI_CONVT;
                a.co = (int32_t)o.c_out;
                a.wd = (int32_t)o.wd;
                if (o.wd % 4 == 0) {
                    // the streaming kernels: each lane pair stores eight
                    // contiguous outputs of one output row
                    GemmArgs pa = a;
                    pa.A = X(i, 1);
                    Launch pl;
                    if (try_pw(0, pa, pl)) {
                        pl.name = intern(std::string(pl.name) + "_t");
                        pl.f = fn(pl.name);
                        L.push_back(pl);
                        break;
                    }
                }
                Tile t = pick_tile(a.M, plane, 1, cus);
                Launch l = mk(gemm_name(t, o.c_in % 4 == 0 && aligned(a.A, 16)) + "_t");
                l.g[0] = cdiv(plane, t.bn);
                l.g[1] = grid_yz((a.M + t.bm - 1) / t.bm);
                set_args(l, a);
                L.push_back(l);
                break;
            }
            case MX_OP_GATE_MM: {
                const int64_t outer = o.p[0], inner = o.p[1];
                GemmArgs a{};
                a.bias = W(o.bias);
                a.C = B(o.dst);
                a.epi = MXK_EPI_PLAIN;
                if (o.mode == 0) {
                    // per channel: Y[c] = W . X[c], bias by row
                    a.A = W(o.w);
                    a.B = B(o.src);
                    a.sA = 0;
                    a.sB = a.sC = outer * inner;
                    a.M = (int32_t)outer;
                    a.K = (int32_t)outer;
                    a.N = (int32_t)inner;
                    a.batch = (int32_t)o.c;
                    a.bias_mode = o.bias >= 0 ? MXK_BIAS_ROW : MXK_BIAS_NONE;
                    a.cvec = aligned(a.C, 16) && inner % 4 == 0 && a.sC % 4 == 0;
                    Tile t = pick_tile(outer, inner, o.c, cus);
                    Launch l = mk(gemm_name(t, outer % 4 == 0 && aligned(a.A, 16)));
                    l.g[0] = cdiv(inner, t.bn);
                    l.g[1] = grid_yz((outer + t.bm - 1) / t.bm);
                    l.g[2] = grid_yz(o.c);
                    set_args(l, a);
                    l.kind = 1;
                    Launch q;
                    if (try_pw(0, a, q, false, true)) {
                        alt[i].push_back(l);
                        L.push_back(q);
                    } else {
                        L.push_back(l);
                    }
                } else {
                    // all channels at once: Y = X . W^T, bias by column
                    a.A = B(o.src);
                    a.B = X(i, 0);
                    a.M = (int32_t)(o.c * outer);
                    a.K = (int32_t)inner;
                    a.N = (int32_t)inner;
                    a.batch = 1;
                    a.bias_mode = o.bias >= 0 ? MXK_BIAS_COL : MXK_BIAS_NONE;
                    if (o.c * outer > 0x7fffffff) throw Error("gate_mm rows too many");
                    a.cvec = aligned(a.C, 16) && inner % 4 == 0;
                    Tile t = pick_tile(a.M, inner, 1, cus);
                    Launch l = mk(gemm_name(t, inner % 4 == 0 && aligned(a.A, 16)));
                    l.g[0] = cdiv(inner, t.bn);
                    l.g[1] = grid_yz((a.M + t.bm - 1) / t.bm);
                    set_args(l, a);
                    l.kind = 1;
                    // the streaming form reads the Dense kernel [a][t] as is
                    GemmArgs r = a;
                    r.A = W(o.w);
                    r.B = B(o.src);
                    Launch q;
                    if (try_pw(1, r, q)) {
                        alt[i].push_back(l);
                        L.push_back(q);
                    } else {
                        L.push_back(l);
                    }
                }
                break;
            }
            case MX_OP_BLOCK_PERM: {
                PermArgs a{};
                a.x = B(o.src);
                a.y = B(o.dst);
                a.c = o.c;
                a.h = (int32_t)o.h;
                a.wd = (int32_t)o.wd;
                a.gh = (int32_t)o.p[0];
                a.gw = (int32_t)o.p[1];
                a.fh = (int32_t)o.p[2];
                a.fw = (int32_t)o.p[3];
                a.swap = (o.mode & MX_PERM_SWAP) ? 1 : 0;
                a.forward = (o.mode & MX_PERM_FORWARD) ? 1 : 0;
                int v = 1;
                if (!a.swap && a.fw % 4 == 0 && a.wd % 4 == 0 && aligned(a.x, 16) && aligned(a.y, 16)) v = 4;
                else if (!a.swap && a.fw % 2 == 0 && a.wd % 2 == 0 && aligned(a.x, 8) && aligned(a.y, 8)) v = 2;
                Launch l = mk(v == 4 ? "mx_block_perm_v4" : v == 2 ? "mx_block_perm_v2" : "mx_block_perm_v1");
                const int64_t psz = o.p[2] * o.p[3];
                l.g[0] = cdiv(o.c * o.p[0] * o.p[1], 1);
                l.b[0] = psz / v <= 64 ? 64 : psz / v <= 128 ? 128 : MXK_BLOCK;
                set_args(l, a);
                L.push_back(l);
                break;
            }
            case MX_OP_RESIZE: {
                // One pass when the taps of both axes are at most 8 and a
                // block's input rows and columns fit its LDS: 256 output
                // columns per block (128-bit stores) unless the columns are
                // downsampled, then 64; the most output rows per block that
                // still leaves >= 2048 blocks, else the band with the most.
                if (maxt[i][0] <= kResizeTapsMax && maxt[i][1] <= kResizeTapsMax && !std::getenv("MAXIM_RESIZE_2PASS")) {
                    int mv = 0, mh = 0;
                    const std::vector<float> tv = resize_table(o.h, o.oh, mv);
                    const std::vector<float> th = resize_table(o.wd, o.ow, mh);
                    bool done = false;
                    for (int tw : {256, 64}) {
                        if (tw == 256 && (o.ow < o.wd || o.ow % 4 || !aligned(B(o.dst), 16))) continue;
                        int span = resize_band(th, mh, o.ow, tw);
                        if (span < 0) continue;
                        // rows staged with 128-bit loads from the 16-byte
                        // boundary at or before a block's first column: up to
                        // 6 more columns, rows a multiple of 4 apart in LDS
                        const bool vec = o.wd % 4 == 0 && aligned(B(o.src), 16);
                        if (vec) span = (span + 6 + 3) & ~3;
                        const int64_t tiles_x = cdiv(o.ow, tw);
                        int64_t pick = 0;
                        int pick_band = 0;
                        for (int64_t rows : {64, 32, 16, 8, 4, 2, 1}) {
                            const int band = resize_band(tv, mv, o.oh, rows);
                            if (band < 0 || 4 * (band * (span + tw) + rows * (3 + mv)) > kResizeLdsMax) continue;
                            pick = rows;
                            pick_band = band;
                            if (tiles_x * cdiv(o.oh, rows) * o.c >= 2048) break;
                        }
                        if (pick == 0) continue;
                        Resize2Args r{B(o.src), B(o.dst), X(i, 0), X(i, 1), (int32_t)o.h, (int32_t)o.wd,
                                      (int32_t)o.oh, (int32_t)o.ow, maxt[i][0], maxt[i][1], (int32_t)pick,
                                      (int32_t)tiles_x, pick_band, span, vec ? 1 : 0, 0};
                        const int mt = std::max(maxt[i][0], maxt[i][1]), ut = mt <= 2 ? 2 : mt <= 4 ? 4 : 8;
                        Launch l = mk(std::string(tw == 256 ? "mx_resize_hv4_t" : "mx_resize_hv_t") + std::to_string(ut));
                        l.g[0] = (uint32_t)(tiles_x * cdiv(o.oh, pick));
                        l.g[1] = (uint32_t)o.c;
                        l.shm = (unsigned)(4 * (pick_band * (span + tw) + pick * (3 + mv)));
                        set_args(l, r);
                        L.push_back(l);
                        done = true;
                        break;
                    }
                    if (done) break;
                }
                ResizeArgs h{};
                h.x = B(o.src);
                h.y = B(o.src2);
                h.rows = o.c * o.h;
                h.n_in = (int32_t)o.wd;
                h.n_out = (int32_t)o.ow;
                h.width = 1;
                h.axis = 2;
                ResizeTab th{X(i, 0), maxt[i][0], 0};
                Launch l1 = mk("mx_resize_h");
                l1.g[0] = cdiv(h.rows * o.ow, MXK_BLOCK);
                set_args(l1, h, th);
                L.push_back(l1);
                ResizeArgs v{};
                v.x = B(o.src2);
                v.y = B(o.dst);
                v.rows = o.c;
                v.n_in = (int32_t)o.h;
                v.n_out = (int32_t)o.oh;
                v.width = (int32_t)o.ow;
                v.axis = 1;
                ResizeTab tv{X(i, 1), maxt[i][1], 0};
                Launch l2 = mk("mx_resize_v");
                l2.g[0] = cdiv(o.c * o.oh * o.ow, MXK_BLOCK);
                set_args(l2, v, tv);
                L.push_back(l2);
                break;
            }
            case MX_OP_DOWN_S: {
                DownArgs a{B(o.src), B(o.dst), o.c, (int32_t)o.h, (int32_t)o.wd, (int32_t)o.p[0],
                           (int32_t)o.p[1], (int32_t)o.oh, (int32_t)o.ow};
                Launch l = mk("mx_down_s");
                l.g[0] = cdiv(o.c * o.oh * o.ow, MXK_BLOCK);
                set_args(l, a);
                L.push_back(l);
                break;
            }
            default:
                throw Error("op " + std::to_string(i) + ": no kernel for kind " + std::to_string(o.kind));
        }
    }
}

// The fused program. Each rule replaces an op whose output has exactly one
// reader with one launch that applies the reader in the producer's epilogue
// (see Epilogue in kargs.h: the same operations in the same order, so fused
// and unfused passes agree to the bit):
//   GEMM -> Gelu                       (every in-projection / MLP Dense)
//   GEMM -> Add [-> Add]               (out-projections + residuals)
//   GateMm -> GateApply                (the gMLP gate, u * (Dense(v) + 1))
//   GEMM -> Copy                       (a Dense written straight into its
//                                       slot of a channel concatenation)
//   Conv3x3 -> Lrelu                   (RCAB)
// "Exactly one reader" is decided on the plan's own arena: the bytes of the
// intermediate stay live until later writes have covered them all, and no op
// but the consumer may read a live byte in that window. With the plan's view
// table the executor then lays out its own device arena by steps (below), so
// a fused step's operands can never overlap; without it the plan layout is
// kept and a pair only fuses where its output overlaps nothing it reads.
void Program::plan_fusion(const mx_plan_desc *p, bool require_clear) {
    struct R {
        uint64_t a, b;
    };
    auto range = [&](int64_t id) -> R {
        const mx_bufshape &s = p->bufs[id];
        return R{p->offs[id], p->offs[id] + (uint64_t)(s.c * s.h * s.w)};
    };
    auto overlap = [](R x, R y) { return x.a < y.b && y.a < x.b; };
    const bool commute = !std::getenv("MAXIM_PLAN_ORDER");
    // Whether buffer `id` must stay intact to the end of a pass (a named
    // dump): the plan marks the storage owner, so a view is kept when its
    // root (following alias_parent) is.
    auto kept = [&](int64_t id) {
        if (!p->keep || id < 0) return false;
        for (int guard = 0; id >= 0 && guard < 64; ++guard) {
            if (p->keep[id]) return true;
            id = p->alias_parent ? p->alias_parent[id] : -1;
        }
        return false;
    };
    auto reads_of = [&](const mx_op &o) {
        std::vector<int64_t> v{o.src};
        if (o.src2 >= 0 && o.kind != MX_OP_RESIZE) v.push_back(o.src2);
        return v;
    };
    auto writes_of = [&](const mx_op &o) {
        std::vector<int64_t> v{o.dst};
        if (o.kind == MX_OP_RESIZE) v.push_back(o.src2);  // the tmp, written before it is read
        return v;
    };
    auto only_reader = [&](int64_t x, uint64_t i, uint64_t j) {
        std::vector<R> live{range(x)};
        for (uint64_t k = i + 1; k < p->n_ops && !live.empty(); ++k) {
            const mx_op &o = p->ops[k];
            if (k != j)
                for (int64_t s : reads_of(o))
                    for (const R &l : live)
                        if (overlap(range(s), l)) return false;
            for (int64_t d : writes_of(o)) {
                const R w = range(d);
                std::vector<R> rest;
                for (const R &l : live) {
                    if (!overlap(w, l)) { rest.push_back(l); continue; }
                    if (l.a < w.a) rest.push_back(R{l.a, w.a});
                    if (w.b < l.b) rest.push_back(R{w.b, l.b});
                }
                live.swap(rest);
            }
        }
        return true;
    };
    auto whole = [&](const mx_op &o, int64_t x) { return o.n == (int64_t)(range(x).b - range(x).a); };
    auto gemm_op = [&](const mx_op &o) {
        return (o.kind == MX_OP_CONV1X1 && o.h * o.wd > 1) || o.kind == MX_OP_GATE_MM;
    };
    auto clear_of = [&](int64_t dst, const std::vector<int64_t> &reads) {
        if (!require_clear) return true;
        for (int64_t r : reads)
            if (overlap(range(dst), range(r))) return false;
        return true;
    };

    // Extend `sp` with the reader of producer g's output, when a rule applies.
    auto epilogue = [&](uint64_t g, StepSpec &sp) {
        const mx_op &o = p->ops[g];
        if (!(g + 1 < p->n_ops && (gemm_op(o) || o.kind == MX_OP_CONV3X3) && only_reader(o.dst, g, g + 1))) return;
        const int64_t x = o.dst;
        const mx_op &n1 = p->ops[g + 1];
        std::vector<int64_t> reads = reads_of(o);
        if (sp.ln >= 0) reads.push_back(p->ops[sp.ln].src);
        if (sp.xmul >= 0) for (int64_t r : reads_of(p->ops[sp.xmul])) reads.push_back(r);
        StepSpec f = sp;
        if (o.kind == MX_OP_GATE_MM && n1.kind == MX_OP_GATE_APPLY && n1.src2 == x && n1.src != x &&
            whole(n1, x)) {
            f.u = n1.src;
            f.out = n1.dst;
            f.last = g + 2;
        } else if (o.kind == MX_OP_CONV1X1 && n1.kind == MX_OP_GELU && n1.src == x && whole(n1, x)) {
            f.act = MXK_ACT_GELU;
            f.out = n1.dst;
            f.last = g + 2;
        } else if (o.kind == MX_OP_CONV3X3 && n1.kind == MX_OP_LRELU && n1.src == x && whole(n1, x)) {
            f.act = MXK_ACT_LRELU;
            f.slope = n1.slope;
            f.out = n1.dst;
            f.last = g + 2;
        } else if (o.kind == MX_OP_CONV3X3 && n1.kind == MX_OP_SIGMOID && n1.src == x && whole(n1, x)) {
            // the supervised attention module's gate: sigmoid(conv) [* f] [+ r]
            f.act = MXK_ACT_SIGMOID;
            f.out = n1.dst;
            f.last = g + 2;
            if (g + 2 < p->n_ops) {
                const mx_op &n2 = p->ops[g + 2];
                const int64_t y = f.out;
                if (n2.kind == MX_OP_MUL && (n2.src == y) != (n2.src2 == y) && whole(n2, y) &&
                    only_reader(y, g + 1, g + 2)) {
                    const int64_t mf = n2.src == y ? n2.src2 : n2.src;
                    std::vector<int64_t> rr = reads;
                    rr.insert(rr.end(), {mf, y});
                    if (clear_of(n2.dst, rr)) {
                        f.m = mf;
                        f.out = n2.dst;
                        f.last = g + 3;
                        if (g + 3 < p->n_ops) {
                            const mx_op &n3 = p->ops[g + 3];
                            const int64_t z = f.out;
                            if (n3.kind == MX_OP_ADD && (n3.src == z) != (n3.src2 == z) && whole(n3, z) &&
                                only_reader(z, g + 2, g + 3)) {
                                const int64_t r1 = n3.src == z ? n3.src2 : n3.src;
                                rr.insert(rr.end(), {r1, z});
                                if (clear_of(n3.dst, rr)) {
                                    f.r1 = r1;
                                    f.out = n3.dst;
                                    f.last = g + 4;
                                }
                            }
                        }
                    }
                }
            }
        } else if (o.kind == MX_OP_CONV3X3 && n1.kind == MX_OP_ADD && (n1.src == x) != (n1.src2 == x) &&
                   whole(n1, x)) {
            f.r1 = n1.src == x ? n1.src2 : n1.src;
            f.out = n1.dst;
            f.last = g + 2;
        } else if (o.kind == MX_OP_CONV1X1 && n1.kind == MX_OP_COPY && n1.src == x && whole(n1, x)) {
            f.out = n1.dst;
            f.last = g + 2;
        } else if (o.kind == MX_OP_CONV1X1 && n1.kind == MX_OP_ADD && (n1.src == x) != (n1.src2 == x) &&
                   whole(n1, x)) {
            f.r1 = n1.src == x ? n1.src2 : n1.src;
            f.out = n1.dst;
            f.last = g + 2;
            if (g + 2 < p->n_ops) {
                const mx_op &n2 = p->ops[g + 2];
                const int64_t y = f.out;
                if (n2.kind == MX_OP_ADD && (n2.src == y) != (n2.src2 == y) && whole(n2, y) &&
                    only_reader(y, g + 1, g + 2)) {
                    const int64_t r2 = n2.src == y ? n2.src2 : n2.src;
                    std::vector<int64_t> rr = reads;
                    rr.insert(rr.end(), {f.r1, r2, y});
                    if (clear_of(n2.dst, rr)) {
                        f.r2 = r2;
                        f.out = n2.dst;
                        f.last = g + 3;
                    }
                }
            }
        }
        if (f.out >= 0) {
            for (int64_t r : {f.u, f.r1, f.r2, f.m})
                if (r >= 0) reads.push_back(r);
            f.epi = true;
            if (clear_of(f.out, reads)) sp = f;
        }
    };
    // A backward BlockPerm (no swap, full coverage) of a GEMM step's output:
    // the streaming kernels' stores go straight to the image positions.
    auto perm_out = [&](uint64_t g, StepSpec &sp) {
        const mx_op &o = p->ops[g];
        if (!gemm_op(o) || sp.last >= p->n_ops) return;
        const int64_t x = sp.out >= 0 ? sp.out : o.dst;
        const uint64_t j = sp.last;
        const mx_op &q = p->ops[j];
        if (q.kind != MX_OP_BLOCK_PERM || q.src != x || (q.mode & (MX_PERM_SWAP | MX_PERM_FORWARD))) return;
        const int64_t gh = q.p[0], gw = q.p[1], fh = q.p[2], fw = q.p[3];
        const uint64_t n = (uint64_t)(q.c * q.h * q.wd);
        if (gh * fh != q.h || gw * fw != q.wd || fw % 4 || range(x).b - range(x).a != n || n >= (1ULL << 31)) return;
        if (!only_reader(x, j - 1, j)) return;
        std::vector<int64_t> reads = reads_of(o);
        if (sp.ln >= 0) reads.push_back(p->ops[sp.ln].src);
        if (sp.xmul >= 0) for (int64_t r : reads_of(p->ops[sp.xmul])) reads.push_back(r);
        for (int64_t r : {sp.u, sp.r1, sp.r2, sp.m})
            if (r >= 0) reads.push_back(r);
        if (!clear_of(q.dst, reads)) return;
        sp.pout = x;
        sp.perm = (int64_t)j;
        sp.out = q.dst;
        sp.last = j + 1;
    };

    // Copy elision (own device layout only): a copy whose source x has one
    // writer (or is written only through the views inside it, slot by slot:
    // a concatenation copied whole into a larger one), and whose
    // destination's bytes nothing touches between x's first write and the
    // copy nor rewrites while x is still read after it, is served by laying
    // x (and its views) out on the destination's storage: the writers then
    // produce the destination directly (x's other readers, e.g. a skip
    // connection's, read it there) and the copy's step launches nothing (run
    // op by op it copies the destination onto itself). Checked per storage
    // owner (the view table's base), since the executor lays out every owner
    // itself.
    elide_to.assign(p->n_bufs, -1);
    std::vector<char> elided(p->n_ops, 0);
    if (!require_clear) {
        const uint64_t nb = p->n_bufs;
        std::vector<int64_t> base(nb);
        std::vector<uint64_t> delta(nb);
        std::vector<int> views(nb, 0), writers(nb, 0);
        std::vector<char> target(nb, 0);
        for (uint64_t b = 0; b < nb; ++b) {
            const int64_t par = p->alias_parent[b];
            base[b] = par < 0 ? (int64_t)b : base[par];
            delta[b] = par < 0 ? 0 : delta[par] + p->alias_delta[b];
            if (par >= 0) ++views[base[b]];
        }
        for (uint64_t k = 0; k < p->n_ops; ++k)
            for (int64_t d : writes_of(p->ops[k])) ++writers[d];
        auto blen = [&](int64_t b) { return (uint64_t)(p->bufs[b].c * p->bufs[b].h * p->bufs[b].w); };
        auto shares = [&](int64_t b, int64_t d) {
            return base[b] == base[d] && delta[b] < delta[d] + blen(d) && delta[d] < delta[b] + blen(b);
        };
        auto touches = [&](const mx_op &o, int64_t d) {
            for (int64_t b : reads_of(o))
                if (shares(b, d)) return true;
            for (int64_t b : writes_of(o))
                if (shares(b, d)) return true;
            return false;
        };
        // x's family: x and the views inside it (a concatenation written
        // slot by slot through its views)
        auto in_x = [&](int64_t b, int64_t x) { return b >= 0 && base[b] == x; };
        for (uint64_t j = 0; j < p->n_ops; ++j) {
            const mx_op &c = p->ops[j];
            if (c.kind != MX_OP_COPY) continue;
            const int64_t x = c.src, d = c.dst;
            if (x == d || base[x] != x || (!views[x] && writers[x] != 1) || (views[x] && writers[x]) || target[x] ||
                elide_to[d] >= 0 || elide_to[x] >= 0)  // x copied twice: it takes the first destination only
                continue;
            if ((uint64_t)x == p->input || (uint64_t)x == p->output || kept(x)) continue;
            if ((uint64_t)c.n != blen(x) || (uint64_t)c.n != blen(d)) continue;
            bool ok = true;
            // w: x's writer, or the first writer of one of its views; every
            // writer of the family before the copy reads no byte of d
            int64_t w = -1;
            for (uint64_t k = 0; k < j && ok; ++k)
                for (int64_t b : writes_of(p->ops[k]))
                    if (in_x(b, x)) {
                        if (views[x]) {
                            if (w < 0) w = (int64_t)k;
                        } else {
                            w = (int64_t)k;
                        }
                        for (int64_t r : reads_of(p->ops[k])) ok = ok && !shares(r, d);
                    }
            if (w < 0 || !ok) continue;
            uint64_t last_read = j;  // x's last reader (x may have others: a skip connection)
            for (uint64_t k = 0; k < p->n_ops; ++k)
                for (int64_t b : reads_of(p->ops[k]))
                    if (in_x(b, x)) {
                        if (k < (uint64_t)w) ok = false;  // nothing reads x before it is written
                        last_read = std::max(last_read, k);
                    }
            for (uint64_t k = (uint64_t)w + 1; k < j && ok; ++k) ok = !touches(p->ops[k], d);
            // d's bytes keep x's value for as long as x is read after the copy
            for (uint64_t k = j + 1; k <= last_read && ok; ++k)
                for (int64_t b : writes_of(p->ops[k])) ok = ok && !shares(b, d);
            if (!ok) continue;
            elide_to[x] = d;
            target[d] = 1;
            elided[j] = 1;
        }
    }

    specs.clear();
    fused_ops = 0;
    for (uint64_t i = 0; i < p->n_ops;) {
        const mx_op &o = p->ops[i];
        StepSpec sp;
        sp.first = i;
        sp.last = i + 1;
        if (elided[i]) {
            sp.rule = RULE_ELIDED;
            ++fused_ops;
            specs.push_back(sp);
            ++i;
            continue;
        }
        // The CALayer's MLP: plane-1 Conv1x1 -> Lrelu -> plane-1 Conv1x1 ->
        // Sigmoid, one block (mx_ca_mlp); with the ChanMean before it, that
        // block also finishes the means (mx_ca_mean_mlp).
        auto ca_mlp_at = [&](uint64_t k) {
            if (k + 3 >= p->n_ops) return false;
            const mx_op &c1 = p->ops[k], &n1 = p->ops[k + 1], &n2 = p->ops[k + 2], &n3 = p->ops[k + 3];
            return c1.kind == MX_OP_CONV1X1 && c1.h * c1.wd == 1 && c1.c_out <= 1024 && c1.c_in <= 1024 &&
                   n1.kind == MX_OP_LRELU && n1.src == c1.dst && n1.n == c1.c_out && n2.kind == MX_OP_CONV1X1 &&
                   n2.h * n2.wd == 1 && n2.src == n1.dst && n2.c_in == c1.c_out && n2.c_out == c1.c_in &&
                   n3.kind == MX_OP_SIGMOID && n3.src == n2.dst && n3.n == n2.c_out && only_reader(c1.dst, k, k + 1) &&
                   only_reader(n1.dst, k + 1, k + 2) && only_reader(n2.dst, k + 2, k + 3) && clear_of(n3.dst, {c1.src});
        };
        if (o.kind == MX_OP_CHAN_MEAN && o.c <= 1024 && i + 1 < p->n_ops && p->ops[i + 1].src == o.dst &&
            p->ops[i + 1].c_in == o.c && ca_mlp_at(i + 1) && only_reader(o.dst, i, i + 1) &&
            clear_of(p->ops[i + 4].dst, {o.src, o.dst})) {
            sp.rule = RULE_CA_MLP;
            sp.out = p->ops[i + 4].dst;
            sp.last = i + 5;
        } else if (o.kind == MX_OP_CONV1X1 && ca_mlp_at(i)) {
            sp.rule = RULE_CA_MLP;
            sp.out = p->ops[i + 3].dst;
            sp.last = i + 4;
        }
        // Upsampling Resize -> 1x1 conv to fewer channels (the reference's
        // UpSampleRatio): the conv runs first, at the input resolution, and the
        // resize then interpolates its c_out channels instead of the c_in
        // channels it was given. Both are linear, the resize acts on each
        // channel plane alone with taps that sum to 1, and the conv on each
        // pixel alone, so W R(x) + b = R(W x + b) up to rounding; the pair
        // moves and multiplies (c_out / c_in) x (input / output pixels) of the
        // data. Not bit-preserving: MAXIM_PLAN_ORDER=1 keeps the plan's order.
        if (sp.rule == RULE_NONE && commute && o.kind == MX_OP_RESIZE && i + 1 < p->n_ops) {
            const mx_op &n1 = p->ops[i + 1];
            if (n1.kind == MX_OP_CONV1X1 && n1.src == o.dst && n1.c_in == o.c && n1.c_out < o.c &&
                n1.h == o.oh && n1.wd == o.ow && o.oh >= o.h && o.ow >= o.wd && o.oh * o.ow > o.h * o.wd &&
                !kept(o.dst) && only_reader(o.dst, i, i + 1) && clear_of(n1.dst, {o.src})) {
                sp.rule = RULE_RS_CONV;
                sp.last = i + 2;
            }
        }
        // ChanScale -> Add: y = x * s + r in one pass.
        if (sp.rule == RULE_NONE && o.kind == MX_OP_CHAN_SCALE && i + 1 < p->n_ops) {
            const mx_op &n1 = p->ops[i + 1];
            if (n1.kind == MX_OP_ADD && (n1.src == o.dst) != (n1.src2 == o.dst) && whole(n1, o.dst) &&
                o.c * o.hw == n1.n && only_reader(o.dst, i, i + 1)) {
                const int64_t r = n1.src == o.dst ? n1.src2 : n1.src;
                if (clear_of(n1.dst, {o.src, o.src2, r})) {
                    sp.rule = RULE_SCALE_ADD;
                    sp.r1 = r;
                    sp.out = n1.dst;
                    sp.last = i + 2;
                    // and a second Add of that sum (a block's long skip), read by nothing else
                    if (i + 2 < p->n_ops) {
                        const mx_op &n2 = p->ops[i + 2];
                        const int64_t y = n1.dst;
                        if (n2.kind == MX_OP_ADD && (n2.src == y) != (n2.src2 == y) && whole(n2, y) &&
                            only_reader(y, i + 1, i + 2)) {
                            const int64_t r2 = n2.src == y ? n2.src2 : n2.src;
                            if (clear_of(n2.dst, {o.src, o.src2, r, r2, y})) {
                                sp.r2 = r2;
                                sp.out = n2.dst;
                                sp.last = i + 3;
                            }
                        }
                    }
                }
            }
        }
        // LayerNorm -> 1x1 conv: the conv's GEMM reads the LayerNorm's input
        // and normalises it on the way in (the streaming kernels' _ln form).
        if (sp.rule == RULE_NONE && o.kind == MX_OP_CHAN_LN && i + 1 < p->n_ops) {
            const mx_op &n1 = p->ops[i + 1];
            if (n1.kind == MX_OP_CONV1X1 && n1.src == o.dst && n1.h * n1.wd == o.hw && o.hw > 1 &&
                n1.c_in == o.c && o.hw % 4 == 0 && o.c % 16 == 0 && only_reader(o.dst, i, i + 1) &&
                clear_of(n1.dst, {o.src})) {
                sp.ln = (int64_t)i;
                sp.last = i + 2;
                epilogue(i + 1, sp);
                perm_out(i + 1, sp);
            }
        }
        // Mul -> 1x1 conv: the conv's streaming GEMM reads both factors and
        // multiplies them on the way in (the _mul form).
        if (sp.rule == RULE_NONE && sp.ln < 0 && o.kind == MX_OP_MUL && i + 1 < p->n_ops) {
            const mx_op &n1 = p->ops[i + 1];
            if (n1.kind == MX_OP_CONV1X1 && n1.src == o.dst && n1.h * n1.wd > 1 && whole(o, o.dst) &&
                o.n == n1.c_in * n1.h * n1.wd && only_reader(o.dst, i, i + 1) &&
                clear_of(n1.dst, {o.src, o.src2})) {
                sp.xmul = (int64_t)i;
                sp.last = i + 2;
                epilogue(i + 1, sp);
                perm_out(i + 1, sp);
            }
        }
        if (sp.rule == RULE_NONE && sp.ln < 0 && sp.xmul < 0) {
            epilogue(i, sp);
            perm_out(i, sp);
        }
        fused_ops += sp.last - sp.first - 1;
        specs.push_back(sp);
        i = sp.last;
    }

    // Forward BlockPerm elision. The gMLP branches permute x into blocked
    // order P, LayerNorm P straight into a 1x1 conv (folded above), and later
    // add P back as the residual of an out-projection whose stores are folded
    // into the backward permutation of the same geometry into x itself. LN
    // is per pixel, so both readers can take x in image order through the
    // block map instead: the folded LayerNorm's GEMM reads its columns (and
    // the statistics) at the mapped positions, and the residual is read at
    // the position the output is stored to. The permutation then launches
    // nothing. Requires: P read by exactly those two ops, x unwritten until
    // the backward permutation writes it back (each element then read and
    // rewritten by one thread), whole buffers, fw % 4 == 0, < 2^31 elements.
    auto readers_after = [&](int64_t x, uint64_t i) {
        std::vector<uint64_t> who;
        std::vector<R> live{range(x)};
        for (uint64_t k = i + 1; k < p->n_ops && !live.empty(); ++k) {
            const mx_op &o = p->ops[k];
            bool reads = false;
            for (int64_t s : reads_of(o))
                for (const R &l : live) reads = reads || overlap(range(s), l);
            if (reads) who.push_back(k);
            for (int64_t d : writes_of(o)) {
                const R w = range(d);
                std::vector<R> rest;
                for (const R &l : live) {
                    if (!overlap(w, l)) { rest.push_back(l); continue; }
                    if (l.a < w.a) rest.push_back(R{l.a, w.a});
                    if (w.b < l.b) rest.push_back(R{w.b, l.b});
                }
                live.swap(rest);
            }
        }
        return who;
    };
    std::vector<int64_t> spec_of(p->n_ops, -1);
    for (uint64_t s = 0; s < specs.size(); ++s)
        for (uint64_t k = specs[s].first; k < specs[s].last; ++k) spec_of[k] = (int64_t)s;
    for (uint64_t j = 0; j + 2 < p->n_ops; ++j) {
        const mx_op &q = p->ops[j];
        if (q.kind != MX_OP_BLOCK_PERM || !(q.mode & MX_PERM_FORWARD) || (q.mode & MX_PERM_SWAP)) continue;
        const int64_t P = q.dst, S = q.src;
        const uint64_t n = (uint64_t)(q.c * q.h * q.wd);
        if (q.p[0] * q.p[2] != q.h || q.p[1] * q.p[3] != q.wd || q.p[3] % 4 || q.wd % 4 || n >= (1ULL << 31)) continue;
        if (range(P).b - range(P).a != n || range(S).b - range(S).a != n || overlap(range(P), range(S))) continue;
        if ((uint64_t)P == p->output || kept(P)) continue;
        StepSpec &J = specs[spec_of[j]];
        if (J.first != j || J.last != j + 1 || J.rule != RULE_NONE) continue;
        // A GateMm straight on P (the cross-gating blocks): its X is P's
        // [cells][pixels] per channel, read from S through the token map.
        const mx_op &gm = p->ops[j + 1];
        if (gm.kind == MX_OP_GATE_MM && gm.src == P) {
            StepSpec &G = specs[spec_of[j + 1]];
            const bool adv = gm.mode == 0 ? 16 % q.p[1] == 0 : 16 % q.p[3] == 0;  // 16 k's = whole rows
            if (G.first != j + 1 || G.rule != RULE_NONE || G.ln >= 0 || !adv || gm.c != q.c ||
                gm.p[0] != q.p[0] * q.p[1] || gm.p[1] != q.p[2] * q.p[3])
                continue;
            const std::vector<uint64_t> who = readers_after(P, j);
            if (who.size() != 1 || who[0] != j + 1 || !clear_of(G.out >= 0 ? G.out : gm.dst, {S})) continue;
            J.rule = RULE_PERM_IN;
            G.xperm = (int64_t)j;
            G.xsrc = S;
            ++fused_ops;
            continue;
        }
        StepSpec &L = specs[spec_of[j + 1]];
        if (L.ln != (int64_t)(j + 1) || p->ops[j + 1].src != P) continue;
        int64_t sk = -1;
        for (uint64_t s = spec_of[j + 1] + 1; s < specs.size() && sk < 0; ++s)
            if (specs[s].r1 == P) sk = (int64_t)s;
        if (sk < 0) continue;
        StepSpec &K = specs[sk];
        if (!K.epi || K.perm < 0 || K.u == P || K.r2 == P) continue;
        const mx_op &bq = p->ops[K.perm];
        if (bq.dst != S || bq.c != q.c || bq.h != q.h || bq.wd != q.wd || bq.p[0] != q.p[0] || bq.p[1] != q.p[1] ||
            bq.p[2] != q.p[2] || bq.p[3] != q.p[3])
            continue;
        uint64_t add = 0;
        for (uint64_t k = K.first; k < K.last; ++k)
            if (p->ops[k].kind == MX_OP_ADD && (p->ops[k].src == P || p->ops[k].src2 == P)) add = k;
        const std::vector<uint64_t> who = readers_after(P, j);
        if (add == 0 || who.size() != 2 || who[0] != j + 1 || who[1] != add) continue;
        bool ok = clear_of(L.out >= 0 ? L.out : p->ops[j + 2].dst, {S});
        for (uint64_t k = j + 1; k < (uint64_t)K.perm && ok; ++k)
            for (int64_t d : writes_of(p->ops[k])) ok = ok && !overlap(range(d), range(S));
        if (!ok) continue;
        J.rule = RULE_PERM_IN;
        L.xperm = (int64_t)j;
        L.xsrc = S;
        K.rperm = (int64_t)j;
        K.r1p = P;
        K.r1 = S;
        ++fused_ops;
    }

    // LayerNorm of a 1x1 conv's output band in the conv's epilogue: a
    // stand-alone ChanLn of 32, 64 or 128 channels whose input is a whole
    // band of channels of the GEMM step just before it (the gMLP gate's v
    // half after its in-projection, the RCAB's input after an out-projection
    // + residual). One wave, or a few waves of one block, of the streaming
    // kernel hold every channel of the band for their pixels, so they
    // normalise them there; the LayerNorm's step joins the GEMM's.
    std::vector<StepSpec> merged;
    const bool lno_on = !std::getenv("MAXIM_NO_LN_EPILOGUE");
    for (uint64_t s = 0; s < specs.size(); ++s) {
        StepSpec sp = specs[s];
        if (lno_on && s + 1 < specs.size() && sp.rule == RULE_NONE && sp.perm < 0 && sp.xmul < 0 && sp.lno < 0) {
            const StepSpec &L = specs[s + 1];
            const uint64_t g = sp.ln >= 0 ? sp.first + 1 : sp.first;
            const mx_op &c = p->ops[g], &ln = p->ops[L.first];
            const int64_t y = sp.out >= 0 ? sp.out : c.dst, hw = c.h * c.wd;
            const R yr = range(y), lr = range(ln.src);
            if (L.first == sp.last && L.last == L.first + 1 && L.rule == RULE_NONE && ln.kind == MX_OP_CHAN_LN &&
                c.kind == MX_OP_CONV1X1 && hw > 1 && ln.hw == hw && (ln.c == 32 || ln.c == 64 || ln.c == 128) &&
                lr.a >= yr.a && lr.b <= yr.b && (lr.a - yr.a) % (uint64_t)hw == 0 &&
                ((lr.a - yr.a) / (uint64_t)hw) % (uint64_t)ln.c == 0) {
                std::vector<int64_t> reads = reads_of(c);
                if (sp.ln >= 0) reads.push_back(p->ops[sp.ln].src);
                for (int64_t r : {sp.u, sp.r1, sp.r2, sp.xsrc, y})
                    if (r >= 0) reads.push_back(r);
                if (clear_of(ln.dst, reads) && !overlap(range(ln.dst), lr)) {
                    sp.lno = (int64_t)L.first;
                    sp.lno_keep = !only_reader(ln.src, L.first - 1, L.first) || (uint64_t)ln.src == p->output ||
                                  (uint64_t)y == p->output || kept(ln.src) || kept(y);
                    sp.last = L.last;
                    ++fused_ops;
                    ++s;
                }
            }
        }
        merged.push_back(sp);
    }
    specs.swap(merged);

    // LayerNorm statistics from the producer. A folded LayerNorm's input x
    // (or, past an elided forward permutation, its source in image order)
    // is a whole band of output channels of an earlier streaming GEMM step,
    // and nothing writes it in between: that step's epilogue writes each
    // pixel's statistics of the band (the statistics pass's values, at the
    // pixel's image position) and the folded GEMM reads them instead of
    // running the statistics pass. Each producer's bands share one slot of
    // the statistics region, live from the producer to its last reader;
    // slots are packed first-fit over those spans.
    so_len = 0;
    if (!std::getenv("MAXIM_NO_LN_EPILOGUE")) {
        struct Req {
            uint64_t p = 0, last = 0, hw = 0;
            int64_t c = 0, lo = -1, hi = -1;
            std::vector<std::pair<uint64_t, int64_t>> qs;  // (consumer spec, band row)
        };
        std::map<uint64_t, Req> reqs;
        for (uint64_t q = 0; q < specs.size(); ++q) {
            const StepSpec &Q = specs[q];
            if (Q.ln < 0) continue;
            const mx_op &ln = p->ops[Q.ln];
            if (ln.c != 32 && ln.c != 64 && ln.c != 128) continue;
            const int64_t X = Q.xperm >= 0 ? Q.xsrc : ln.src;
            const R xr = range(X);
            int64_t P = -1;
            for (int64_t s2 = (int64_t)q - 1; s2 >= 0 && P < 0; --s2)
                for (uint64_t k = specs[s2].first; k < specs[s2].last && P < 0; ++k)
                    for (int64_t d : writes_of(p->ops[k]))
                        if (overlap(range(d), xr)) P = s2;
            if (P < 0) continue;
            const StepSpec &S = specs[P];
            int64_t y = -1;
            uint64_t hw = 0;
            if (S.rule == RULE_SCALE_ADD) {
                // the CALayer's scaled residual sum, the whole buffer one band
                const mx_op &c = p->ops[S.first];
                y = S.out;
                hw = (uint64_t)c.hw;
                if (y < 0 || ln.c != c.c) continue;
            } else {
                if (S.rule != RULE_NONE || S.lno >= 0 || S.xmul >= 0 || S.xperm >= 0) continue;
                const uint64_t g = S.ln >= 0 ? S.first + 1 : S.first;
                const mx_op &c = p->ops[g];
                if (c.kind != MX_OP_CONV1X1 || c.h * c.wd <= 1) continue;
                y = S.out >= 0 ? S.out : c.dst;
                hw = (uint64_t)(c.h * c.wd);
            }
            const R yr = range(y);
            if (ln.hw != (int64_t)hw || xr.a < yr.a || xr.b > yr.b || (xr.a - yr.a) % hw ||
                xr.b - xr.a != (uint64_t)ln.c * hw)
                continue;
            const int64_t row = (int64_t)((xr.a - yr.a) / hw);
            if (row % ln.c) continue;
            Req &r = reqs[(uint64_t)P];
            if (r.c && r.c != ln.c) continue;
            r.p = (uint64_t)P;
            r.c = ln.c;
            r.hw = hw;
            r.lo = r.lo < 0 ? row : std::min(r.lo, row);
            r.hi = std::max(r.hi, row + ln.c);
            r.last = std::max<uint64_t>(r.last, q);
            r.qs.push_back({q, row});
        }
        struct Slot {
            uint64_t a, b, off, len;
        };
        std::vector<Slot> slots;
        for (auto &kv : reqs) {
            Req &r = kv.second;
            const int nband = (int)((r.hi - r.lo) / r.c);
            const uint64_t len = ((uint64_t)nband * 2 * r.hw + 63) & ~(uint64_t)63;
            std::vector<uint64_t> cands{0};
            for (const Slot &t : slots) cands.push_back(t.off + t.len);
            std::sort(cands.begin(), cands.end());
            uint64_t off = 0;
            for (uint64_t cand : cands) {
                bool clash = false;
                for (const Slot &t : slots)
                    if (t.a <= r.last && r.p <= t.b && cand < t.off + t.len && t.off < cand + len) clash = true;
                if (!clash) {
                    off = cand;
                    break;
                }
            }
            slots.push_back({r.p, r.last, off, len});
            so_len = std::max(so_len, off + len);
            StepSpec &S = specs[r.p];
            S.so_row0 = r.lo;
            S.so_c = r.c;
            S.so_nband = nband;
            S.so_hw = r.hw;
            S.so_out = off;
            for (const auto &qr : r.qs) {
                specs[qr.first].so_from = (int64_t)r.p;
                specs[qr.first].so_in = off + (uint64_t)((qr.second - r.lo) / r.c) * 2 * r.hw;
            }
        }
    }
}

// The device arena: the plan's own packing rule (largest first, first use as
// the tie-break, first fit over {0} u {off + size}, src/model.rs:1091-1234)
// with live ranges counted in STEPS of the fused program, so every operand of
// a fused step - the eliminated intermediate included, which the unfused path
// still writes - is live at once and no two of them share storage. Views keep
// their delta inside their parent; kept (named) buffers live to the end.
// The buffer that owns every buffer's storage and its offset there: views
// sit in their parents, an elided copy's source (with the views inside it)
// takes its destination's storage, which may itself sit on another's.
void Program::storage(const mx_plan_desc *p, std::vector<int64_t> &base, std::vector<uint64_t> &delta) const {
    const uint64_t n = p->n_bufs;
    base.assign(n, 0);
    delta.assign(n, 0);
    for (uint64_t i = 0; i < n; ++i) {
        const int64_t par = p->alias_parent[i];
        if (par < 0) { base[i] = (int64_t)i; delta[i] = 0; }
        else {
            if ((uint64_t)par >= i) throw Error("the view table names a later buffer as a parent");
            base[i] = base[par];
            delta[i] = delta[par] + p->alias_delta[i];
        }
    }
    std::vector<char> done(n, 0);
    std::function<void(uint64_t)> resolve = [&](uint64_t i) {
        if (done[i]) return;
        done[i] = 1;
        const int64_t x = base[i];
        if (x < (int64_t)elide_to.size() && elide_to[x] >= 0) {
            const int64_t d = elide_to[x];
            resolve((uint64_t)d);
            const uint64_t dx = delta[i];  // offset inside x
            base[i] = base[d];
            delta[i] = delta[d] + dx;
        }
    };
    for (uint64_t i = 0; i < n; ++i) resolve(i);
}

// Regions (see `regions`): within a window of at most 12 consecutive steps
// made only of 1x1-conv/GateMm steps and the pointwise, LayerNorm,
// permutation and copy ops fused around them, every pair of steps with the
// same op sequence and shapes (the two branches' steps differ only in how
// their pixels are blocked, not in their sizes), or with the same GEMM,
// whose buffers do not meet with a write; the region runs from the first
// such step to the last.
void Program::plan_regions(const mx_plan_desc *p) {
    regions.clear();
    if (!p->alias_parent || !p->alias_delta) return;
    constexpr uint64_t W = 12;
    std::vector<int64_t> base;
    std::vector<uint64_t> delta;
    storage(p, base, delta);
    auto len = [&](int64_t b) { return (uint64_t)(p->bufs[b].c * p->bufs[b].h * p->bufs[b].w); };
    // (GEMMs over at most 80000 pixels: a full-resolution branch already
    // fills the chip on its own, and two of its memory-bound launches side
    // by side measured slower, not faster)
    auto member = [&](uint64_t s) {
        bool gemm = false;
        for (uint64_t k = specs[s].first; k < specs[s].last; ++k) {
            switch (p->ops[k].kind) {
                case MX_OP_CONV1X1:
                    if (p->ops[k].h * p->ops[k].wd > 80000) return 0;
                    gemm = true;
                    break;
                case MX_OP_GATE_MM: gemm = true; break;
                case MX_OP_GATE_APPLY: case MX_OP_GELU: case MX_OP_ADD: case MX_OP_MUL: case MX_OP_CHAN_LN:
                case MX_OP_BLOCK_PERM: case MX_OP_COPY: case MX_OP_LRELU: break;
                default: return 0;
            }
        }
        return gemm ? 2 : 1;  // 2: a step with a GEMM, 1: one that may sit between
    };
    auto sig = [&](uint64_t s) {
        std::vector<int64_t> v;
        for (uint64_t k = specs[s].first; k < specs[s].last; ++k) {
            const mx_op &o = p->ops[k];
            v.insert(v.end(), {(int64_t)o.kind, (int64_t)o.mode, o.c_in, o.c_out, o.h * o.wd, o.n, o.c, o.hw});
        }
        return v;
    };
    // the step's GEMM alone: two steps whose GEMMs match but whose fused
    // ops around them differ (one branch's output permutation folded into
    // the stores, the other's launched apart) pair as two kernels
    auto gsig = [&](uint64_t s) {
        std::vector<int64_t> v;
        for (uint64_t k = specs[s].first; k < specs[s].last; ++k) {
            const mx_op &o = p->ops[k];
            if (o.kind != MX_OP_CONV1X1 && o.kind != MX_OP_GATE_MM) continue;
            v.insert(v.end(), {(int64_t)o.kind, (int64_t)o.mode, o.c_in, o.c_out, o.h * o.wd, o.n, o.c, o.hw});
            break;
        }
        return v;
    };
    struct Iv { int64_t owner; uint64_t lo, hi; };
    auto touch = [&](uint64_t s, std::vector<Iv> &rd, std::vector<Iv> &wr) {
        auto iv = [&](int64_t b) { return Iv{base[b], delta[b], delta[b] + len(b)}; };
        for (uint64_t k = specs[s].first; k < specs[s].last; ++k) {
            const mx_op &o = p->ops[k];
            if (o.dst >= 0) { wr.push_back(iv(o.dst)); rd.push_back(iv(o.dst)); }
            if (o.src >= 0) rd.push_back(iv(o.src));
            if (o.src2 >= 0) rd.push_back(iv(o.src2));
        }
        for (int64_t b : {specs[s].xsrc, specs[s].r1, specs[s].u, specs[s].r2})
            if (b >= 0) rd.push_back(iv(b));
    };
    auto meets = [](const std::vector<Iv> &x, const std::vector<Iv> &y) {
        for (const Iv &u : x)
            for (const Iv &v : y)
                if (u.owner == v.owner && u.lo < v.hi && v.lo < u.hi) return true;
        return false;
    };
    uint64_t i = 0;
    const uint64_t S = specs.size();
    while (i < S) {
        if (member(i) != 2) { ++i; continue; }
        uint64_t j = i + 1;
        while (j < S && j - i < W && member(j)) ++j;
        std::vector<std::vector<Iv>> rd(j - i), wr(j - i);
        for (uint64_t s = i; s < j; ++s) touch(s, rd[s - i], wr[s - i]);
        uint64_t lo = UINT64_MAX, hi = 0;
        for (uint64_t u = i; u < j; ++u) {
            if (member(u) != 2) continue;
            const auto su = sig(u);
            for (uint64_t v = u + 1; v < j; ++v) {
                if (member(v) != 2 || (sig(v) != su && gsig(v) != gsig(u))) continue;
                const size_t a = u - i, b = v - i;
                if (meets(wr[a], rd[b]) || meets(wr[b], rd[a])) continue;
                lo = std::min(lo, u);
                hi = std::max(hi, v);
            }
        }
        if (lo != UINT64_MAX) {
            regions.push_back({lo, hi});
            i = hi + 1;
        } else {
            i = j;
        }
    }
}

void Program::layout(const mx_plan_desc *p, bool repack) {
    const uint64_t n = p->n_bufs;
    doff.assign(n, 0);
    dbase.assign(n, 0);
    if (!repack) {
        for (uint64_t i = 0; i < n; ++i) {
            doff[i] = p->offs[i];
            dbase[i] = (int64_t)i;
        }
        if (p->alias_parent)
            for (uint64_t i = 0; i < n; ++i)
                if (p->alias_parent[i] >= 0) dbase[i] = dbase[p->alias_parent[i]];
        arena_len = p->arena_len;
        return;
    }
    std::vector<int64_t> base;
    std::vector<uint64_t> delta;
    storage(p, base, delta);
    for (uint64_t i = 0; i < n; ++i) dbase[i] = base[i];
    const uint64_t DEAD = UINT64_MAX;
    std::vector<uint64_t> first(n, DEAD), last(n, 0);
    for (uint64_t s = 0; s < specs.size(); ++s) {
        auto use = [&](int64_t b) {
            if (b < 0) return;
            const int64_t r = base[b];
            if (first[r] == DEAD) first[r] = s;
            last[r] = std::max(last[r], s);
        };
        for (uint64_t k = specs[s].first; k < specs[s].last; ++k) {
            const mx_op &o = p->ops[k];
            for (int64_t b : {o.dst, o.src, o.src2}) use(b);
        }
        // buffers a step reads in place of an elided permutation's output
        use(specs[s].xsrc);
        use(specs[s].r1);
    }
    // every buffer a region touches is live across the whole region, so
    // that its steps may run in another order or side by side - except the
    // intermediates only one step touches, which its fused launch never
    // stores (op by op, the steps run in their own order)
    const std::vector<uint64_t> first0 = first, last0 = last;
    for (const auto &rg : regions)
        for (uint64_t s = rg.first; s <= rg.second; ++s) {
            auto span = [&](int64_t b) {
                if (b < 0) return;
                const int64_t r = base[b];
                if (first0[r] == last0[r]) return;
                first[r] = std::min(first[r], rg.first);
                last[r] = std::max(last[r], rg.second);
            };
            for (uint64_t k = specs[s].first; k < specs[s].last; ++k) {
                const mx_op &o = p->ops[k];
                for (int64_t b : {o.dst, o.src, o.src2}) span(b);
            }
            span(specs[s].xsrc);
            span(specs[s].r1);
        }
    if (p->keep)
        for (uint64_t i = 0; i < n; ++i)
            if (p->keep[i] && first[base[i]] != DEAD) last[base[i]] = specs.size() - 1;
    std::vector<int64_t> order;
    auto len = [&](int64_t b) { return (uint64_t)(p->bufs[b].c * p->bufs[b].h * p->bufs[b].w); };
    for (uint64_t i = 0; i < n; ++i)
        if (base[i] == (int64_t)i && first[i] != DEAD) order.push_back((int64_t)i);
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
        if (len(a) != len(b)) return len(a) > len(b);
        return first[a] < first[b];
    });
    struct Block { uint64_t start, end, off, size; };
    std::vector<Block> placed;
    std::vector<uint64_t> off(n, 0), cands;
    std::vector<const Block *> live;
    uint64_t total = 0;
    for (int64_t b : order) {
        const uint64_t size = len(b), st = first[b], en = last[b];
        cands.assign(1, 0);
        live.clear();
        for (auto &q : placed) {
            cands.push_back(q.off + q.size);
            if (st <= q.end && q.start <= en) live.push_back(&q);
        }
        std::sort(cands.begin(), cands.end());
        cands.erase(std::unique(cands.begin(), cands.end()), cands.end());
        uint64_t chosen = total;
        for (uint64_t c : cands) {
            bool clash = false;
            for (const Block *q : live)
                if (c < q->off + q->size && q->off < c + size) { clash = true; break; }
            if (!clash) { chosen = c; break; }
        }
        off[b] = chosen;
        total = std::max(total, chosen + size);
        placed.push_back({st, en, chosen, size});
    }
    for (uint64_t i = 0; i < n; ++i) doff[i] = off[base[i]] + delta[i];
    arena_len = std::max<uint64_t>(total, 1);
    repacked = true;
    // An elided copy launches nothing: its source must sit on its destination.
    for (const StepSpec &sp : specs)
        if (sp.rule == RULE_ELIDED && doff[p->ops[sp.first].src] != doff[p->ops[sp.first].dst])
            throw Error("internal: an elided copy whose source is not laid out on its destination");
}

// Materialise the program: single-op steps reuse the op's launches; a fused
// step is the producer's launch with its destination and epilogue patched.
void Gpu::build_program(const mx_plan_desc *p) {
    auto dev = [&](int64_t id) -> float * { return id >= 0 ? arena + doff[id] : nullptr; };
    // The producer g's launch with the step's epilogue applied (kernel + _f),
    // writing buffer `out`.
    auto with_epilogue = [&](const StepSpec &sp, uint64_t g, const Launch &base, int64_t out) {
        Epilogue e{};
        e.u = dev(sp.u);
        e.r1 = dev(sp.r1);
        e.r2 = dev(sp.r2);
        e.m = dev(sp.m);
        e.act = sp.act;
        e.slope = sp.slope;
        // 128-bit stores need every array the epilogue indexes like the
        // output on a 16-byte boundary.
        const bool ealign = aligned(e.u, 16) && aligned(e.r1, 16) && aligned(e.r2, 16) && aligned(e.m, 16);
        Launch l = base;
        if (!strncmp(l.name, "mx_pw_", 6) && !(ealign && aligned(dev(out), 16)))
            l = alt[g][0];  // the streaming kernels store 128 bits at a time
        if (!strncmp(l.name, "mx_c3_", 6) && !aligned(dev(out), 16)) l = alt[g][0];  // so does mx_c3
        // Up to 32 outputs with a residual read: 16-wide tiles (twice the
        // waves, each with half the epilogue) measured 9% faster at the
        // 448x640 shapes; the tile width changes no output's bits. A step whose
        // epilogue also normalises a 32-channel LayerNorm band then holds the
        // band in two waves of a block (44.8 -> 43.4 us for the 64 -> 32
        // out-projections at 448x640); not for steps that leave statistics.
        if (e.r1 && sp.so_nband <= 0 && l.kind == 1 &&
            (!strcmp(l.name, "mx_pw_ch2") || !strcmp(l.name, "mx_pw_ch2_mul"))) {
            GemmArgs a;
            memcpy(&a, l.a0, sizeof a);
            if (a.M <= 32 && a.batch == 1) {
                const int64_t tiles = (int64_t)((a.M + 15) / 16) * ((a.N + 63) / 64);
                l.name = intern(std::string("mx_pw_ch1") + (l.name + 9));
                l.f = fn(l.name);
                l.g[0] = (unsigned)((tiles + 3) / 4);
            }
        }
        l.name = intern(std::string(l.name) + "_f");
        l.f = fn(l.name);
        if (l.kind == 1) {
            GemmArgs a;
            memcpy(&a, l.a0, sizeof a);
            a.C = dev(out);
            a.e = e;
            a.cvec = a.N % 4 == 0 && a.sC % 4 == 0 && aligned(a.C, 16) && ealign;
            set_args(l, a);
        } else if (l.kind == 2) {
            ConvArgs a;
            memcpy(&a, l.a0, sizeof a);
            a.y = dev(out);
            a.e = e;
            a.cvec = a.ow % 4 == 0 && aligned(a.y, 16) && ealign;
            set_args(l, a);
        } else {
            throw Error("internal: a fused step whose producer has no epilogue");
        }
        return l;
    };
    // The launches of producer g: its epilogue, and a folded BlockPerm through
    // the streaming kernels' block map - or, where they cannot take it
    // (shape, alignment), the producer writing the permutation's source and
    // the permutation's own launch after it.
    // An elided forward permutation's step, by op, and what restores it
    // when a reader cannot take the block map after all.
    std::vector<int64_t> perm_step(p->n_ops, -1);
    auto restore_perm = [&](int64_t j) {
        if (j >= 0 && perm_step[j] >= 0) prog[perm_step[j]].launches = ops[j];
    };
    auto gemm_part = [&](const StepSpec &sp, uint64_t g) -> std::vector<Launch> {
        const Launch &base = ops[g][0];
        if (sp.perm < 0) {
            if (sp.epi) return {with_epilogue(sp, g, base, sp.out)};
            return ops[g];
        }
        const mx_op &q = p->ops[sp.perm];
        Launch l = base;
        if (sp.epi) {
            l = with_epilogue(sp, g, base, sp.out);
        } else if (l.kind == 1) {
            GemmArgs a;
            memcpy(&a, l.a0, sizeof a);
            a.C = dev(sp.out);
            set_args(l, a);
        }
        if (!strncmp(l.name, "mx_pw_", 6) && aligned(dev(sp.out), 16)) {
            GemmArgs a;
            memcpy(&a, l.a0, sizeof a);
            a.ymap = mx_block_map(q, sp.rperm >= 0 ? 1 : 0);
            set_args(l, a);
            return {l};
        }
        // no map: the residual is the permutation's output after all
        StepSpec s2 = sp;
        if (sp.rperm >= 0) {
            s2.r1 = sp.r1p;
            restore_perm(sp.rperm);
        }
        std::vector<Launch> v{s2.epi ? with_epilogue(s2, g, base, s2.pout) : base};
        for (const Launch &x : ops[sp.perm]) v.push_back(x);
        return v;
    };
    // A GateMm reading an elided forward permutation's source through the
    // token map (the streaming kernels' _xm form, layout by mode), or, where
    // the producer is not one of them, the permutation after all.
    auto token_map = [&](const StepSpec &sp, Launch &l) {
        const mx_op &o = p->ops[sp.first], &q = p->ops[sp.xperm];
        const char *want = o.mode == 0 ? "mx_pw_ch" : "mx_pw_rw";
        if (strncmp(l.name, want, 8) || !aligned(dev(sp.xsrc), 16)) {
            restore_perm(sp.xperm);
            return;
        }
        const std::string nm = l.name;
        const bool f = nm.size() > 2 && nm.compare(nm.size() - 2, 2, "_f") == 0;
        l.name = intern((f ? nm.substr(0, nm.size() - 2) : nm) + "_xm" + (f ? "_f" : ""));
        l.f = fn(l.name);
        GemmArgs a;
        memcpy(&a, l.a0, sizeof a);
        a.B = dev(sp.xsrc);
        a.xmap = mx_block_map(q, 0);
        set_args(l, a);
    };
    // A GEMM step that also computes the LayerNorm of an output band (lno):
    // its streaming kernel's _lo form with a wave-wide band, or, where the
    // step's kernel cannot take it (not streaming, another operand form, a
    // misaligned or overlapping LayerNorm output), the LayerNorm's own
    // launch after the step's.
    // The streaming kernel's _lo form on a step's main launch: LayerNorm
    // bands of c channels from output row r0 (mode 0: one band, normalised
    // into y; mode 1: nband bands' statistics into y). False where the launch
    // cannot take it (not streaming, another operand form, a misaligned or
    // overlapping y, a tile that cannot hold the band).
    auto lo_apply = [&](Step &st, int mode, int64_t r0, int64_t c, int nband, int keep, float *y, int64_t ylen,
                        const float *scale, const float *bias, float eps, bool need_ymap) -> bool {
        Launch &l = st.launches[st.main];
        if (strncmp(l.name, "mx_pw_ch", 8) || l.kind != 1 || !aligned(y, 16)) return false;
        const std::string nm = l.name;
        GemmArgs a;
        memcpy(&a, l.a0, sizeof a);
        if (a.batch != 1 || (mode == 0 && a.ymap.on) || (need_ymap && !a.ymap.on)) return false;
        // the name is mx_pw_ch<T>[_k4][_ln][_f]: nothing else may be folded in
        std::string rest = nm.substr(9);
        for (const char *t : {"_k4", "_ln", "_f"})
            if (!rest.compare(0, strlen(t), t)) rest = rest.substr(strlen(t));
        if (!rest.empty() || r0 < 0 || r0 % c || r0 + nband * c > a.M) return false;
        // y may overlap nothing the kernel reads or writes
        const float *lo = y, *hi = y + ylen;
        auto clash = [&](const float *b, int64_t n) { return b && b < hi && lo < b + n; };
        const int64_t xn = (int64_t)a.K * a.N, yn = (int64_t)a.M * a.N;
        if (clash(a.C, a.ymap.on ? std::max<int64_t>(yn, a.ymap.plane * a.M) : yn) || clash(a.B, xn) ||
            clash(a.B2, xn) || clash(a.e.u, yn) || clash(a.e.r1, yn) || clash(a.e.r2, yn) ||
            clash(a.A, (int64_t)a.M * a.K) || (a.xmap.on && clash(a.B, a.xmap.plane * a.K)) ||
            (a.ln.mean && clash(a.ln.mean, 2 * (int64_t)a.N)))
            return false;
        // The tile: the step's own width when G = c / width consecutive
        // waves of a block hold a band (G = 1 also with the split reduction;
        // G > 1 needs whole blocks of tiles, groups aligned to the block),
        // else a width of c itself. The reduction split stays as the step
        // has it: the tile width does not change any output's order of
        // accumulation, the split does, and the fused pass stays the unfused
        // one to the bit.
        auto fits = [&](int tmw, bool k4) {
            const int tw = 16 * tmw, G = (int)(c / tw);
            if (c % tw || (G != 1 && G != 2 && G != 4) || (k4 && G != 1)) return 0;
            const int64_t nib = (a.M + tw - 1) / tw, tiles = nib * ((a.N + 63) / 64);
            if (G > 1 && (nib % G || (r0 / tw) % G || tiles % 4)) return 0;
            return G;
        };
        const bool k4 = nm.find("_k4") != std::string::npos, lnn = nm.find("_ln") != std::string::npos;
        int tmw = nm[8] - '0', G = fits(tmw, k4);
        if (!G && (c == 32 || c == 64)) {
            tmw = (int)(c / 16);
            G = 1;
        }
        if (!G) return false;
        const int64_t tiles = ((a.M + 16 * tmw - 1) / (16 * tmw)) * ((a.N + 63) / 64);
        l.name = intern("mx_pw_ch" + std::to_string(tmw) + (k4 ? "_k4" : "") + (lnn ? "_ln" : "") + "_f_lo");
        l.f = fn(l.name);
        l.g[0] = (unsigned)(k4 ? tiles : (tiles + 3) / 4);
        l.g[1] = 1;
        // a group of waves of 32+ channels each sums its band per wave, then
        // adds the partials in wave order (not the LayerNorm kernels' order:
        // MAXIM_PLAN_ORDER=1 keeps theirs)
        a.lo = LnOut{scale, bias, y, eps, (int32_t)r0, keep, G, mode, nband, G > 1 && tmw >= 2 && !plan_order ? 1 : 0};
        set_args(l, a);
        return true;
    };
    // A GEMM step that also computes the LayerNorm of an output band (lno),
    // or, where its kernel cannot, the LayerNorm's own launch after it.
    auto lno_apply = [&](const StepSpec &sp, Step &st) {
        if (sp.lno < 0) return;
        const mx_op &ln = p->ops[sp.lno];
        ChanLnArgs la;
        memcpy(&la, ops[sp.lno][0].a0, sizeof la);
        const Launch &l = st.launches[st.main];
        GemmArgs a;
        memcpy(&a, l.a0, sizeof a);
        const int64_t d = l.kind == 1 ? la.x - a.C : -1;
        const int64_t r0 = d >= 0 && d % ln.hw == 0 && a.N == ln.hw ? d / ln.hw : -1;
        if (!lo_apply(st, 0, r0, ln.c, 1, sp.lno_keep ? 1 : 0, la.y, ln.c * ln.hw, la.scale, la.bias, la.eps, false))
            for (const Launch &x : ops[sp.lno]) st.launches.push_back(x);
    };
    // A GEMM step whose output bands later LayerNorms fold (so_*): their
    // statistics from its epilogue, into the statistics region.
    std::vector<char> so_ok(pg.specs.size(), 0);
    auto so_apply = [&](const StepSpec &sp, Step &st) {
        if (sp.so_nband <= 0) return;
        const int64_t hw = (int64_t)sp.so_hw;
        const Launch &l = st.launches[st.main];
        GemmArgs a;
        memcpy(&a, l.a0, sizeof a);
        if (l.kind != 1 || a.N != hw) return;
        so_ok[&sp - pg.specs.data()] =
            lo_apply(st, 1, sp.so_row0, sp.so_c, sp.so_nband, 1, scratch + so_base + sp.so_out,
                     2 * hw * sp.so_nband, nullptr, nullptr, mx::kEps, sp.perm >= 0);
    };
    prog.clear();
    for (const StepSpec &sp : pg.specs) {
        if (sp.rule == RULE_ELIDED) {
            prog.push_back(Step{sp.first, sp.last, {}});
            continue;
        }
        if (sp.rule == RULE_RS_CONV) {
            // the conv's own GEMM over the resize's input plane into scratch,
            // then the resize's own launch over the conv's c_out channels
            // into the conv's output
            const mx_op &r = p->ops[sp.first], &c = p->ops[sp.first + 1];
            const std::vector<Launch> &rl = ops[sp.first], &cl = ops[sp.first + 1];
            Step st{sp.first, sp.last, {}};
            if (rl.size() == 1 && !strncmp(rl[0].name, "mx_resize_hv", 12) && cl.size() == 1 && cl[0].kind == 1 &&
                (r.h * r.wd) % 4 == 0) {
                GemmArgs a;
                memcpy(&a, cl[0].a0, sizeof a);
                float *out = a.C;
                a.B = dev(r.src);
                a.N = (int32_t)(r.h * r.wd);
                a.C = scratch + rs_off;
                Launch g;
                // (the 256-column forms store 128 bits: the conv's output must be 16-byte aligned)
                const bool st_ok = strncmp(rl[0].name, "mx_resize_hv4", 13) != 0 || aligned(out, 16);
                if (a.batch == 1 && a.M == c.c_out && st_ok && try_pw(0, a, g)) {
                    Resize2Args z;
                    memcpy(&z, rl[0].a0, sizeof z);
                    z.x = scratch + rs_off;
                    z.y = out;
                    Launch zl = rl[0];
                    zl.g[1] = (unsigned)c.c_out;
                    set_args(zl, z);
                    st.launches = {g, zl};
                }
            }
            if (st.launches.empty())  // the plan's order, op by op
                for (uint64_t k = sp.first; k < sp.last; ++k)
                    for (const Launch &x : ops[k]) st.launches.push_back(x);
            prog.push_back(st);
            continue;
        }
        if (sp.rule == RULE_PERM_IN) {
            perm_step[sp.first] = (int64_t)prog.size();
            prog.push_back(Step{sp.first, sp.last, {}});
            continue;
        }
        if (sp.rule == RULE_CA_MLP) {
            const bool mean = p->ops[sp.first].kind == MX_OP_CHAN_MEAN;
            const uint64_t c1 = sp.first + (mean ? 1 : 0);
            GemvArgs g1, g2;
            memcpy(&g1, ops[c1][0].a0, sizeof g1);
            memcpy(&g2, ops[c1 + 2][0].a0, sizeof g2);
            CaArgs a{g1.x, g1.w, g1.bias, g2.w, g2.bias, dev(sp.out), g1.ci, g1.co, p->ops[c1 + 1].slope, 0};
            if (!mean) {
                Launch l = mk("mx_ca_mlp");
                set_args(l, a);
                prog.push_back(Step{sp.first, sp.last, {l}});
                continue;
            }
            // the ChanMean's partial sums, then the means and the MLP in one block
            ChanMeanArgs m;
            memcpy(&m, ops[sp.first][0].a0, sizeof m);
            CaMeanArgs cm{a, m.part, m.y, m.hw, m.nchunk, 0};
            Launch l = mk("mx_ca_mean_mlp");
            set_args(l, cm);
            prog.push_back(Step{sp.first, sp.last, {ops[sp.first][0], l}});
            continue;
        }
        if (sp.rule == RULE_SCALE_ADD) {
            ChanScaleArgs a;
            memcpy(&a, ops[sp.first][0].a0, sizeof a);
            a.y = dev(sp.out);
            a.r = dev(sp.r1);
            a.r2 = dev(sp.r2);
            const bool vec = a.hw % 4 == 0 && aligned(a.x, 16) && aligned(a.y, 16) && aligned(a.r, 16) &&
                             aligned(a.r2, 16);
            if (sp.so_nband == 1 && vec && (a.c == 32 || a.c == 64 || a.c == 128)) {
                // with the statistics of the sum for a later folded LayerNorm
                ScaleAddLnArgs b{a.x, a.s, a.r, a.r2, a.y, scratch + so_base + sp.so_out, a.hw, (int32_t)a.c,
                                 mx::kEps};
                const auto t = ln_tile(a.c, a.hw, cus);
                Launch l = mk("mx_chan_scale_add_stats_c" + std::to_string(a.c) + t.second);
                l.g[0] = cdiv(a.hw, t.first);
                set_args(l, b);
                so_ok[&sp - pg.specs.data()] = 1;
                prog.push_back(Step{sp.first, sp.last, {l}});
                continue;
            }
            Launch l = mk(vec ? "mx_chan_scale_add_v4" : "mx_chan_scale_add_s");
            l.g[0] = vec ? cdiv(a.hw / 4, MXK_BLOCK * 4) : cdiv(a.hw, MXK_BLOCK);
            l.g[1] = grid_yz(a.c);
            set_args(l, a);
            prog.push_back(Step{sp.first, sp.last, {l}});
            continue;
        }
        if (sp.xmul >= 0) {
            // the conv's GEMM reading both factors of the Mul, or, where it is
            // not a streaming kernel (or the factors are misaligned), the Mul
            // on its own before it
            const uint64_t g = sp.first + 1;
            const mx_op &m = p->ops[sp.first];
            std::vector<Launch> v = sp.out < 0 ? ops[g] : gemm_part(sp, g);
            Launch &l = v[0];
            if (!strncmp(l.name, "mx_pw_ch", 8) && aligned(dev(m.src), 16) && aligned(dev(m.src2), 16)) {
                const std::string nm = l.name;
                const bool f = nm.size() > 2 && nm.compare(nm.size() - 2, 2, "_f") == 0;
                l.name = intern((f ? nm.substr(0, nm.size() - 2) : nm) + "_mul" + (f ? "_f" : ""));
                l.f = fn(l.name);
                GemmArgs a;
                memcpy(&a, l.a0, sizeof a);
                a.B = dev(m.src);
                a.B2 = dev(m.src2);
                set_args(l, a);
                prog.push_back(Step{sp.first, sp.last, v});
            } else {
                Step st{sp.first, sp.last, ops[sp.first]};
                st.main = st.launches.size();
                for (const Launch &x : v) st.launches.push_back(x);
                prog.push_back(st);
            }
            continue;
        }
        if (sp.ln < 0) {
            std::vector<Launch> v = sp.out < 0 ? ops[sp.first] : gemm_part(sp, sp.first);
            if (sp.xperm >= 0) token_map(sp, v[0]);
            Step st{sp.first, sp.last, v};
            lno_apply(sp, st);
            so_apply(sp, st);
            prog.push_back(st);
            continue;
        }
        // A LayerNorm folded into the next op's streaming GEMM: the
        // statistics pass, then the GEMM reading the LayerNorm's input.
        const uint64_t g = sp.first + 1;
        const mx_op &ln = p->ops[sp.first];
        const Launch &conv = ops[g][0];
        ChanLnArgs la;
        memcpy(&la, ops[sp.first][0].a0, sizeof la);
        float *stats = scratch + ln_off;
        // an elided forward permutation: statistics and columns from its
        // source in image order, the GEMM reading through the block map
        const bool xmap = sp.xperm >= 0 && aligned(dev(sp.xsrc), 16);
        if (xmap) la.x = dev(sp.xsrc);
        const bool ok = !strncmp(conv.name, "mx_pw_ch", 8) && aligned(la.x, 16) && la.hw % 4 == 0;
        std::vector<Launch> gp = gemm_part(sp, g);
        Launch &gl = gp[0];
        if (!ok || strncmp(gl.name, "mx_pw_ch", 8) || (sp.xperm >= 0 && !xmap)) {
            // not streaming (shape or alignment): the LayerNorm runs on its own
            restore_perm(sp.xperm);
            Step st{sp.first, sp.last, ops[sp.first]};
            st.main = st.launches.size();
            for (const Launch &x : gp) st.launches.push_back(x);
            lno_apply(sp, st);
            so_apply(sp, st);
            prog.push_back(st);
            continue;
        }
        // statistics from the step that produced x (its _lo epilogue), or
        // a statistics pass here
        const bool so = sp.so_from >= 0 && so_ok[sp.so_from];
        if (so) stats = scratch + so_base + sp.so_in;
        ChanLnArgs sa = la;
        sa.y = stats;
        Launch sl;
        if (ln.c == 64 || ln.c == 128) {
            // the LayerNorm kernels' LDS tile (measured faster than the
            // register loop from 64 channels up)
            const auto t = ln_tile(ln.c, ln.hw, cus);
            sl = mk("mx_chan_ln_stats_c" + std::to_string(ln.c) + t.second);
            sl.g[0] = cdiv(ln.hw, t.first);
        } else {
            sl = mk("mx_chan_ln_stats");
            sl.g[0] = cdiv((ln.hw + 3) / 4, MXK_BLOCK);
        }
        set_args(sl, sa);
        const std::string gname = gl.name;
        const bool f = gname.size() > 2 && gname.compare(gname.size() - 2, 2, "_f") == 0;
        // With no statistics from a producer, a split-reduction GEMM over a
        // 128-channel LayerNorm (each of the block's waves holds 32 channels
        // of every pixel it reads) forms them itself (_ln2): no statistics
        // pass. Its sums run in another order than the LayerNorm kernels',
        // so MAXIM_PLAN_ORDER=1 keeps the pass.
        GemmArgs a;
        memcpy(&a, gl.a0, sizeof a);
        const bool ln2 = !so && !plan_order && gname.rfind("mx_pw_ch2_k4", 0) == 0 && a.K == 128 && ln.c == 128;
        gl.name = intern((f ? gname.substr(0, gname.size() - 2) : gname) + (ln2 ? "_ln2" : "_ln") + (f ? "_f" : ""));
        gl.f = fn(gl.name);
        a.B = la.x;
        a.ln = LnIn{ln2 ? nullptr : stats, ln2 ? nullptr : stats + ln.hw, la.scale, la.bias, la.eps, 0};
        if (xmap) {
            const mx_op &q = p->ops[sp.xperm];
            a.xmap = mx_block_map(q, 0);
        }
        set_args(gl, a);
        Step st{sp.first, sp.last, {}};
        if (so) {
            st.so_from = sp.so_from;
            st.pre.push_back(sl);
        } else if (!ln2) {
            st.launches.push_back(sl);
        }
        st.main = st.launches.size();
        for (const Launch &x : gp) st.launches.push_back(x);
        lno_apply(sp, st);
        so_apply(sp, st);
        prog.push_back(st);
    }
    for (Step &st : prog) {
        for (Launch &l : st.launches) specialise(l);
        for (Launch &l : st.pre) specialise(l);
    }
    elided_perm.clear();
    for (const Step &st : prog)
        if (st.launches.empty() && st.last == st.first + 1 && p->ops[st.first].kind == MX_OP_BLOCK_PERM &&
            !ops[st.first].empty())
            elided_perm[p->ops[st.first].dst] = st.first;
    if (!std::getenv("MAXIM_NO_PAIR")) pair_launches(p);
}

// Pairs of independent streaming-GEMM launches of one kernel within a few
// steps of each other (the grid and block branches of a multi-axis gMLP
// block: their in-projections, their out-projections) become one launch of
// the kernel's _x2 form, so that two grids too small to fill the chip share
// it and one tail. Within a window of consecutive steps with one launch each
// (or none), launches are list-scheduled over the steps' dependencies - any
// two steps whose device bytes (arena, and the scratch statistics their
// arguments name) overlap with a write keep their order - taking two ready
// launches of one kernel together where it can, and otherwise holding back a
// launch whose partner is still waiting on others. Streaming GEMMs and
// LayerNorms pair; the other kernels of a window (permutations, the general
// GEMM at shapes the streaming one does not take) keep their place among
// them.
// A window in which anything was paired becomes one step over all its ops:
// every op still computes exactly what it did, in a dependency-respecting
// order, so results are unchanged to the bit; a run of ops that cuts the
// window runs its ops one by one.
void Gpu::pair_launches(const mx_plan_desc *p) {
    constexpr size_t W = 12;
    struct Iv {
        int space;  // 0 arena, 1 scratch
        uint64_t lo, hi;
    };
    auto x2fn = [&](const char *name) -> hipFunction_t {
        const std::string n = std::string(name) + "_x2";
        auto it = fns_.find(n);
        if (it != fns_.end()) return it->second;
        hipFunction_t f = nullptr;
        if (H.hipModuleGetFunction(&f, mod, n.c_str()) != 0) f = nullptr;
        fns_[n] = f;
        return f;
    };
    // a kernel pairing two different launches: A__B_x2, A's blocks first
    auto hx2fn = [&](const char *a, const char *b) -> hipFunction_t {
        if (strncmp(b, "mx_pw_", 6)) return nullptr;
        return x2fn((std::string(a) + "__" + (b + 6)).c_str());
    };
    auto single = [&](const Step &st) {
        if (st.launches.size() != 1 || st.launches[0].kind != 1) return false;
        const char *n = st.launches[0].name;
        const size_t k = strlen(n);
        return strncmp(n, "mx_pw_", 6) == 0 && !(k > 2 && strcmp(n + k - 2, "_t") == 0);
    };
    // Any other kernel of a window never pairs; its bytes are taken from its
    // ops (sources read, destinations read and written, the step's fused
    // operands read and written, and all of the scratch both ways when its
    // argument block holds any address inside the scratch), a superset of
    // what it touches. A step of a streaming GEMM followed by the
    // LayerNorm of its output band (a LayerNorm kernel of its own, where the
    // band is wider than the GEMM's epilogue takes) gives two nodes, the
    // GEMM's ops and then the LayerNorm op.
    const bool specs_ok = pg.specs.size() == prog.size();
    auto is_pw = [&](const Launch &l) {
        const size_t k = strlen(l.name);
        return l.kind == 1 && strncmp(l.name, "mx_pw_", 6) == 0 && !(k > 2 && strcmp(l.name + k - 2, "_t") == 0);
    };
    // a LayerNorm launch (its own kernel, not a statistics pass): pairs with
    // another of the same kernel
    auto is_ln = [&](const Launch &l) { return l.kind == 0 && strncmp(l.name, "mx_chan_ln_c", 12) == 0; };
    auto other = [&](const Step &st) {
        return specs_ok && st.launches.size() == 1 && st.pre.empty() && st.launches[0].kind < 3 && !single(st);
    };
    auto banded = [&](const Step &st) {
        return specs_ok && st.launches.size() == 2 && st.pre.empty() && st.last - st.first >= 2 &&
               is_pw(st.launches[0]) && strncmp(st.launches[1].name, "mx_chan_ln_c", 12) == 0 &&
               p->ops[st.last - 1].kind == MX_OP_CHAN_LN;
    };
    auto member = [&](const Step &st) {
        return (st.launches.empty() && st.pre.empty()) || single(st) || other(st) || banded(st);
    };
    // the device memory a step's streaming-GEMM launch reads and writes,
    // from its arguments: X (and a folded Mul's second factor), the epilogue
    // operands and the folded LayerNorm's statistics are read; the output and
    // the output LayerNorm's band (or statistics) are written. Extents are
    // per batch (a block map permutes within them: X over its plane, Y
    // within M x N); weights and biases are never written and are left out.
    auto footprint = [&](const Launch &l, std::vector<Iv> &rd, std::vector<Iv> &wr) {
        GemmArgs a;
        memcpy(&a, l.a0, sizeof a);
        auto add = [&](std::vector<Iv> &v, const float *q, int64_t stride, uint64_t len) {
            if (!q || len == 0) return;
            const uint64_t span = (uint64_t)((a.batch > 1 ? (int64_t)(a.batch - 1) * stride : 0)) + len;
            if (q >= arena && q < arena + arena_len)
                v.push_back(Iv{0, (uint64_t)(q - arena), (uint64_t)(q - arena) + span});
            else if (q >= scratch && q < scratch + scratch_len)
                v.push_back(Iv{1, (uint64_t)(q - scratch), (uint64_t)(q - scratch) + span});
        };
        const bool rw = strncmp(l.name, "mx_pw_rw", 8) == 0;
        const uint64_t MN = (uint64_t)a.M * (uint64_t)a.N;
        uint64_t xlen = rw ? (uint64_t)a.M * (uint64_t)a.K : (uint64_t)a.K * (uint64_t)a.N;
        if (a.xmap.on) xlen = std::max<uint64_t>(xlen, (uint64_t)a.K * (uint64_t)a.xmap.plane);
        add(rd, a.B, a.sB, xlen);
        add(rd, a.B2, a.sB, xlen);
        add(rd, a.e.u, a.sC, MN);
        add(rd, a.e.r1, a.sC, MN);
        add(rd, a.e.r2, a.sC, MN);
        add(rd, a.ln.mean, 0, (uint64_t)a.N);
        add(rd, a.ln.rstd, 0, (uint64_t)a.N);
        add(wr, a.C, a.sC, MN);
        if (a.lo.y) {
            if (a.lo.mode)
                add(wr, a.lo.y, 0, (uint64_t)a.lo.nband * 2 * (uint64_t)a.N);
            else
                add(wr, a.lo.y, 0, (uint64_t)(a.M - a.lo.row0) * (uint64_t)a.N);
        }
    };
    auto uses_scratch = [&](const Launch &l) {
        const uintptr_t lo = (uintptr_t)scratch, hi = (uintptr_t)(scratch + scratch_len);
        auto scan = [&](const unsigned char *b, size_t n) {
            for (size_t o = 0; o + 8 <= n; o += 8) {
                uintptr_t v;
                memcpy(&v, b + o, 8);
                if (v >= lo && v < hi) return true;
            }
            return false;
        };
        return scan(l.a0, sizeof l.a0) || scan(l.a1, sizeof l.a1);
    };
    auto footprint_ops = [&](size_t k, const Launch &l, uint64_t first, uint64_t last, std::vector<Iv> &rd,
                             std::vector<Iv> &wr) {
        auto buf = [&](int64_t b, bool w) {
            if (b < 0) return;
            const uint64_t n = (uint64_t)(p->bufs[b].c * p->bufs[b].h * p->bufs[b].w);
            rd.push_back(Iv{0, doff[b], doff[b] + n});
            if (w) wr.push_back(Iv{0, doff[b], doff[b] + n});
        };
        for (uint64_t o = first; o < last; ++o) {
            buf(p->ops[o].src, false);
            buf(p->ops[o].src2, false);
            buf(p->ops[o].dst, true);
        }
        const StepSpec &sp = pg.specs[k];
        for (int64_t b : {sp.out, sp.u, sp.r1, sp.r2, sp.m, sp.xsrc, sp.r1p, sp.pout}) buf(b, true);
        if (uses_scratch(l)) {
            rd.push_back(Iv{1, 0, scratch_len});
            wr.push_back(Iv{1, 0, scratch_len});
        }
    };
    auto meets = [](const std::vector<Iv> &x, const std::vector<Iv> &y) {
        for (const Iv &u : x)
            for (const Iv &v : y)
                if (u.space == v.space && u.lo < v.hi && v.lo < u.hi) return true;
        return false;
    };
    std::vector<Step> out;
    out.reserve(prog.size());
    std::map<size_t, size_t> region_end;  // the layout's regions (steps are its specs here)
    for (const auto &rg : pg.regions)
        if (rg.second < prog.size()) region_end[rg.first] = rg.second + 1;
    size_t i = 0;
    while (i < prog.size()) {
        auto rg = region_end.find(i);
        if (rg == region_end.end()) {
            out.push_back(std::move(prog[i]));
            ++i;
            continue;
        }
        // the window: a region whose steps are all single streaming GEMMs (or
        // launch nothing), with at most one producer of folded-LayerNorm
        // statistics among their `pre` sources
        const size_t j = rg->second;
        int64_t so = -1;
        bool ok = true;
        for (size_t k = i; k < j && ok; ++k) {
            ok = member(prog[k]) && (prog[k].so_from < 0 || so < 0 || prog[k].so_from == so);
            if (prog[k].so_from >= 0) so = prog[k].so_from;
        }
        if (!ok || j - i > W) {
            for (size_t k = i; k < j; ++k) out.push_back(std::move(prog[k]));
            i = j;
            continue;
        }
        // window nodes: each launch of its steps, with the ops it computes
        std::vector<size_t> node;  // its step
        std::vector<const Launch *> ln;
        std::vector<std::array<uint64_t, 2>> spn;
        for (size_t k = i; k < j; ++k) {
            const Step &s = prog[k];
            for (size_t q = 0; q < s.launches.size(); ++q) {
                node.push_back(k);
                ln.push_back(&s.launches[q]);
                if (s.launches.size() == 1)
                    spn.push_back({s.first, s.last});
                else
                    spn.push_back(q == 0 ? std::array<uint64_t, 2>{s.first, s.last - 1}
                                         : std::array<uint64_t, 2>{s.last - 1, s.last});
            }
        }
        const size_t m = node.size();
        if (m > 32) {
            for (size_t k = i; k < j; ++k) out.push_back(std::move(prog[k]));
            i = j;
            continue;
        }
        std::vector<std::vector<Iv>> rd(m), wr(m);
        for (size_t u = 0; u < m; ++u) {
            if (is_pw(*ln[u]))
                footprint(*ln[u], rd[u], wr[u]);
            else
                footprint_ops(node[u], *ln[u], spn[u][0], spn[u][1], rd[u], wr[u]);
        }
        std::vector<uint32_t> pred(m, 0), reach(m, 0);
        for (size_t v = 0; v < m; ++v)
            for (size_t u = 0; u < v; ++u)
                if (node[u] == node[v] || meets(wr[u], rd[v]) || meets(wr[u], wr[v]) || meets(rd[u], wr[v]))
                    pred[v] |= 1u << u;
        for (size_t v = 0; v < m; ++v) {
            reach[v] = pred[v];
            for (size_t u = 0; u < v; ++u)
                if (pred[v] >> u & 1) reach[v] |= reach[u];
        }
        auto kname = [&](size_t u) { return ln[u]->name; };
        if (std::getenv("MAXIM_PAIR_LOG") && m > 1) {
            fprintf(stderr, "maxim: window steps [%zu, %zu):", i, j);
            for (size_t u = 0; u < m; ++u) fprintf(stderr, " %zu:%s(g%u/%u, pred %x)", node[u], kname(u), ln[u]->g[0], ln[u]->g[1], pred[u]);
            fprintf(stderr, "\n");
        }
        // one batch, and a grid of at most ten blocks per CU: a few rounds of
        // blocks, whose ragged last round a partner's blocks fill (with the
        // 224x320 GateMms paired too, C4 measured 23.06 -> 23.00 ms/image)
        auto one = [&](size_t u) {
            const Launch &l = *ln[u];
            return (is_pw(l) || is_ln(l)) && l.g[1] == 1 && l.g[2] == 1 && l.g[0] <= (unsigned)(10 * cus);
        };
        // the kernel running u and v in one grid (same kernel: its _x2 form;
        // two kernels: A__B_x2, with `swap` when v's blocks come first)
        auto pairfn = [&](size_t u, size_t v, bool &swap) -> hipFunction_t {
            swap = false;
            if (kname(u) == kname(v)) return x2fn(kname(u));
            if (std::getenv("MAXIM_NO_HPAIR") || !is_pw(*ln[u]) || !is_pw(*ln[v])) return nullptr;
            if (hipFunction_t f = hx2fn(kname(u), kname(v))) return f;
            swap = true;
            return hx2fn(kname(v), kname(u));
        };
        auto can_pair = [&](size_t u, size_t v) {
            const bool ok = one(u) && one(v) && !(reach[v] >> u & 1) && !(reach[u] >> v & 1);
            bool swap;
            if (ok && kname(u) == kname(v) && !x2fn(kname(u)) && std::getenv("MAXIM_PAIR_LOG"))
                fprintf(stderr, "maxim: no paired form of %s\n", kname(u));
            return ok && pairfn(u, v, swap) != nullptr;
        };
        // list scheduling: entries are (u) or (u, v)
        std::vector<std::pair<int, int>> seq;
        uint32_t done = 0;
        size_t pairs = 0;
        while (done != (m == 32 ? 0xffffffffu : (1u << m) - 1)) {
            std::vector<size_t> ready;
            for (size_t u = 0; u < m; ++u)
                if (!(done >> u & 1) && (pred[u] & ~done) == 0) ready.push_back(u);
            bool paired = false;
            for (size_t a = 0; a < ready.size() && !paired; ++a)
                for (size_t b = a + 1; b < ready.size() && !paired; ++b)
                    if (can_pair(ready[a], ready[b])) {
                        seq.push_back({(int)ready[a], (int)ready[b]});
                        done |= (1u << ready[a]) | (1u << ready[b]);
                        ++pairs;
                        paired = true;
                    }
            if (paired) continue;
            size_t pick = ready[0];
            for (size_t u : ready) {
                bool waits = false;
                for (size_t w = 0; w < m; ++w)
                    if (!(done >> w & 1) && w != u && (pred[w] & ~done) != 0 && can_pair(u, w)) waits = true;
                if (!waits) {
                    pick = u;
                    break;
                }
            }
            seq.push_back({(int)pick, -1});
            done |= 1u << pick;
        }
        if (pairs == 0) {
            for (size_t k = i; k < j; ++k) out.push_back(std::move(prog[k]));
            i = j;
            continue;
        }
        Step st(prog[i].first, prog[j - 1].last);
        st.so_from = so;
        for (size_t k = i; k < j; ++k)
            for (Launch &l : prog[k].pre) st.pre.push_back(l);
        for (auto &e : seq) {
            if (e.second < 0) {
                st.launches.push_back(*ln[e.first]);
                st.launches.back().span[0] = spn[e.first][0];
                st.launches.back().span[1] = spn[e.first][1];
                continue;
            }
            bool swap = false;
            const hipFunction_t pf = pairfn((size_t)e.first, (size_t)e.second, swap);
            const size_t u0 = swap ? e.second : e.first, u1 = swap ? e.first : e.second;
            const Launch &l0 = *ln[u0], &l1 = *ln[u1];
            Launch d = l0;
            d.span[0] = spn[u0][0];
            d.span[1] = spn[u0][1];
            d.span[2] = spn[u1][0];
            d.span[3] = spn[u1][1];
            d.name = intern(l0.name == l1.name ? std::string(l0.name) + "_x2"
                                               : std::string(l0.name) + "__" + (l1.name + 6) + "_x2");
            d.f = pf;
            d.g[0] = l0.g[0] + l1.g[0];
            if (is_ln(l0)) {
                DualLnArgs dl{};
                memcpy(&dl.a, l0.a0, sizeof(ChanLnArgs));
                memcpy(&dl.b, l1.a0, sizeof(ChanLnArgs));
                dl.na = l0.g[0];
                d.kind = 4;
                set_args(d, dl);
            } else {
                DualGemmArgs da{};
                memcpy(&da.a, l0.a0, sizeof(GemmArgs));
                memcpy(&da.b, l1.a0, sizeof(GemmArgs));
                da.na = l0.g[0];
                d.kind = 3;
                set_args(d, da);
            }
            st.main = st.launches.size();
            st.launches.push_back(d);
        }
        out.push_back(std::move(st));
        i = j;
    }
    // step indices of the statistics producers moved with the merging
    if (out.size() != prog.size()) {
        std::vector<int64_t> remap(prog.size(), -1);
        size_t o = 0;
        for (size_t k = 0; k < prog.size(); ++k) {
            while (o + 1 < out.size() && out[o].last <= prog[k].first) ++o;
            remap[k] = (int64_t)o;
        }
        for (Step &st : out)
            if (st.so_from >= 0) st.so_from = remap[st.so_from];
    }
    prog = std::move(out);
}

// A fused streaming kernel (mx_pw_..._f or _f_lo) specialised for the
// epilogue operand set its launch uses (..._e<mask>, the pw::EP_* bits),
// where the code object has one: the same arithmetic in the same order,
// without the per-slot tests of the argument block.
void Gpu::specialise(Launch &l) {
    if (l.kind == 2 && !strncmp(l.name, "mx_wino3_", 9)) {
        // the Winograd conv's fused epilogue when it is a LeakyReLU alone
        const size_t n = strlen(l.name);
        if (n < 2 || strcmp(l.name + n - 2, "_f")) return;
        ConvArgs a;
        memcpy(&a, l.a0, sizeof a);
        if (a.e.u || a.e.m || a.e.r1 || a.e.r2 || a.e.act != MXK_ACT_LRELU) return;
        const std::string sn = std::string(l.name) + "_e16";
        l.name = intern(sn);
        l.f = fn(l.name);
        return;
    }
    if (l.kind != 1 || strncmp(l.name, "mx_pw_", 6)) return;
    const std::string nm = l.name;
    auto ends = [&](const char *t) {
        const size_t n = strlen(t);
        return nm.size() > n && nm.compare(nm.size() - n, n, t) == 0;
    };
    if (!ends("_f") && !ends("_f_lo")) return;
    GemmArgs a;
    memcpy(&a, l.a0, sizeof a);
    const int ep = (a.e.u ? 1 : 0) | (a.e.r1 ? 2 : 0) | (a.e.r2 ? 4 : 0) | (a.e.act == MXK_ACT_GELU ? 8 : 0) |
                   (a.e.act == MXK_ACT_LRELU ? 16 : 0) | (a.ymap.on ? 32 : 0) | (a.bias ? 64 : 0) |
                   (a.ymap.on && a.ymap.r1map ? 128 : 0);
    const std::string sn = nm + "_e" + std::to_string(ep);
    auto it = fns_.find(sn);
    hipFunction_t f = nullptr;
    if (it != fns_.end()) {
        f = it->second;
    } else {
        if (H.hipModuleGetFunction(&f, mod, sn.c_str()) != 0) f = nullptr;
        fns_[sn] = f;
        if (!f && std::getenv("MAXIM_EP_LOG")) fprintf(stderr, "maxim: no specialised %s\n", sn.c_str());
    }
    if (!f) return;
    l.name = intern(sn);
    l.f = f;
}

Gpu::~Gpu() { release(); }

void Gpu::release() {
    if (stream) H.hipStreamSynchronize(stream);
    for (int s = 0; s < 2; ++s) {
        for (hipEvent_t e : {bt.h2d[s], bt.d2h[s]})
            if (e) H.hipEventDestroy(e);
        if (bt.hin[s]) H.hipHostFree(bt.hin[s]);
        if (bt.hout[s]) H.hipHostFree(bt.hout[s]);
    }
    bt = Batch{};
    if (gexec) H.hipGraphExecDestroy(gexec);
    if (graph) H.hipGraphDestroy(graph);
    if (arena) H.hipFree(arena);
    if (wdev) H.hipFree(wdev);
    if (scratch) H.hipFree(scratch);
    if (stream) H.hipStreamDestroy(stream);
    gexec = nullptr;
    graph = nullptr;
    arena = nullptr;
    wdev = nullptr;
    scratch = nullptr;
    stream = nullptr;
    mod = nullptr;
}

}  // namespace mxh

using mxh::Gpu;

namespace {

template <typename F>
int guard(F &&f) {
    try {
        f();
        return 0;
    } catch (const std::exception &e) {
        mx::set_error(e.what());
        return -1;
    }
}

Gpu *G(mxh_gpu *g) { return reinterpret_cast<Gpu *>(g); }

}  // namespace

extern "C" {

int mxh_driver_ready(void) {
    return guard([] {
        auto &H = mxh::hip();
        mxh::check(H.hipInit(0), "hipInit");
        int n = 0;
        mxh::check(H.hipGetDeviceCount(&n), "hipGetDeviceCount");
        if (n < 1) throw mx::Error("no HIP device");
    });
}

mxh_gpu *mxh_new(const mx_plan_desc *plan) {
    Gpu *g = nullptr;
    guard([&] {
        if (!plan) throw mx::Error("mxh_new: no plan");
        g = new Gpu(plan);
    });
    return reinterpret_cast<mxh_gpu *>(g);
}

void mxh_free(mxh_gpu *g) {
    try {
        delete G(g);
    } catch (...) {
    }
}

int mxh_begin(mxh_gpu *g, const mx_plan_desc *plan, const float *input, uint64_t n_in) {
    return guard([&] {
        G(g)->check_plan(plan);
        const mx_bufshape &s = plan->bufs[plan->input];
        if (n_in != (uint64_t)(s.c * s.h * s.w)) throw mx::Error("the input image and the plan's input buffer disagree");
        if (std::getenv("MAXIM_POISON")) mxh::check(G(g)->H.hipMemsetD8Async(G(g)->arena, 0xCD, G(g)->arena_len * 4, G(g)->stream), "poison");
        G(g)->write(G(g)->doff[plan->input], input, n_in);
    });
}

int mxh_step_op(mxh_gpu *g, const mx_plan_desc *plan, uint64_t i) {
    return guard([&] {
        G(g)->check_plan(plan);
        if (i >= plan->n_ops) throw mx::Error("op index out of range");
        G(g)->run_op(i);
        G(g)->sync();
    });
}

int mxh_run_ops(mxh_gpu *g, const mx_plan_desc *plan, uint64_t first, uint64_t last) {
    return guard([&] {
        G(g)->check_plan(plan);
        if (last > plan->n_ops || first > last) throw mx::Error("op range out of bounds");
        if (G(g)->fusion) G(g)->run_range(first, last);
        else for (uint64_t i = first; i < last; ++i) G(g)->run_op(i);
    });
}

int mxh_run(mxh_gpu *g, const mx_plan_desc *plan, const float *input, uint64_t n_in, float *output, uint64_t n_out) {
    return guard([&] {
        Gpu &x = *G(g);
        x.check_plan(plan);
        const mx_bufshape &so = plan->bufs[plan->output];
        if (n_out != (uint64_t)(so.c * so.h * so.w)) throw mx::Error("the output buffer and the plan's output disagree");
        if (mxh_begin(g, plan, input, n_in) != 0) throw mx::Error(mx_last_error());
        if (x.want_timeline) {
            x.run_timed();
        } else if (x.use_graph) {
            x.run_graph();
        } else {
            if (x.fusion) x.run_range(0, plan->n_ops);
            else for (uint64_t i = 0; i < plan->n_ops; ++i) x.run_op(i);
        }
        x.read(x.doff[plan->output], output, n_out);
    });
}

int mxh_run_batch(mxh_gpu *g, const mx_plan_desc *plan, const float *const *inputs, uint64_t n_in,
                  float *const *outputs, uint64_t n_out, uint64_t n_images) {
    return guard([&] {
        Gpu &x = *G(g);
        x.check_plan(plan);
        const mx_bufshape &si = plan->bufs[plan->input], &so = plan->bufs[plan->output];
        if (n_in != (uint64_t)(si.c * si.h * si.w)) throw mx::Error("the input image and the plan's input buffer disagree");
        if (n_out != (uint64_t)(so.c * so.h * so.w)) throw mx::Error("the output buffer and the plan's output disagree");
        if (n_images && (!inputs || !outputs)) throw mx::Error("mxh_run_batch: no input or output list");
        for (uint64_t k = 0; k < n_images; ++k)
            if (!inputs[k] || !outputs[k]) throw mx::Error("mxh_run_batch: image " + std::to_string(k) + " has no buffer");
        if (x.want_timeline) throw mx::Error("mxh_run_batch does not record the timeline (mxh_run does)");
        x.run_batch(x.doff[plan->input], x.doff[plan->output], inputs, n_in, outputs, n_out, n_images);
    });
}

int mxh_run_noalloc(mxh_gpu *g, const mx_plan_desc *plan, const float *d_input, uint64_t n_in, float *d_output,
                    uint64_t n_out, void *stream) {
    return guard([&] {
        Gpu &x = *G(g);
        x.check_plan(plan);
        const mx_bufshape &si = plan->bufs[plan->input], &so = plan->bufs[plan->output];
        if (n_in != (uint64_t)(si.c * si.h * si.w)) throw mx::Error("the input image and the plan's input buffer disagree");
        if (n_out != (uint64_t)(so.c * so.h * so.w)) throw mx::Error("the output buffer and the plan's output disagree");
        if (!d_input || !d_output) throw mx::Error("mxh_run_noalloc: no input or output");
        if (x.prog_na.empty())
            throw mx::Error("this pass needs " + std::to_string(x.scratch_len * 4) +
                            " bytes of scratch; the static scratch of mxh_run_noalloc holds " +
                            std::to_string((uint64_t)MXK_NOALLOC_SCRATCH_FLOATS * 4) + " (mxh_run has no such limit)");
        auto &H = x.H;
        // the caller's stream when given (stream order with its own work;
        // a capture of that stream records the pass), else the executor's
        const mxh::hipStream_t on = stream ? (mxh::hipStream_t)stream : x.stream;
        mxh::check(H.hipMemcpyAsync(x.arena + x.doff[plan->input], d_input, n_in * 4, mxh::kMemcpyD2D, on),
                   "hipMemcpyAsync(input)");
        for (mxh::Step &st : x.prog_na) {
            for (auto &l : st.launches) x.launch(l, on);
            x.launched += st.last - st.first;
        }
        mxh::check(H.hipMemcpyAsync(d_output, x.arena + x.doff[plan->output], n_out * 4, mxh::kMemcpyD2D, on),
                   "hipMemcpyAsync(output)");
    });
}

int mxh_run_graph(mxh_gpu *g, const mx_plan_desc *plan) {
    return guard([&] {
        G(g)->check_plan(plan);
        G(g)->run_graph();
    });
}

void mxh_set_graph(mxh_gpu *g, int on) { G(g)->use_graph = on != 0; }

void mxh_set_fusion(mxh_gpu *g, int on) {
    Gpu &x = *G(g);
    if (x.fusion != (on != 0) && x.gexec) {
        // the captured graph holds the other program: capture again on next use
        x.H.hipGraphExecDestroy(x.gexec);
        x.H.hipGraphDestroy(x.graph);
        x.gexec = nullptr;
        x.graph = nullptr;
    }
    x.fusion = on != 0;
}

int mxh_plan_program(const mx_plan_desc *plan, int repack, uint64_t *fused_ops, uint64_t *arena_len,
                     uint64_t *offs, uint64_t *step_first, uint64_t *step_last, uint64_t *n_steps) {
    return guard([&] {
        mxh::Program pg;
        const bool rp = repack && plan->alias_parent && plan->alias_delta;
        pg.plan_fusion(plan, !rp);
        if (rp && !std::getenv("MAXIM_NO_PAIR")) pg.plan_regions(plan);
        pg.layout(plan, rp);
        if (fused_ops) *fused_ops = pg.fused_ops;
        if (arena_len) *arena_len = pg.arena_len;
        if (offs) memcpy(offs, pg.doff.data(), sizeof(uint64_t) * pg.doff.size());
        if (n_steps) *n_steps = pg.specs.size();
        for (size_t i = 0; i < pg.specs.size(); ++i) {
            if (step_first) step_first[i] = pg.specs[i].first;
            if (step_last) step_last[i] = pg.specs[i].last;
        }
    });
}

int mxh_plan_storage(const mx_plan_desc *plan, int repack, int64_t *owner) {
    return guard([&] {
        mxh::Program pg;
        const bool rp = repack && plan->alias_parent && plan->alias_delta;
        pg.plan_fusion(plan, !rp);
        if (rp && !std::getenv("MAXIM_NO_PAIR")) pg.plan_regions(plan);
        pg.layout(plan, rp);
        if (owner) memcpy(owner, pg.dbase.data(), sizeof(int64_t) * pg.dbase.size());
    });
}

uint64_t mxh_fused_ops(mxh_gpu *g) { return G(g)->pg.fused_ops; }

uint64_t mxh_steps(mxh_gpu *g) { return G(g)->fusion ? G(g)->prog.size() : G(g)->n_ops; }

int mxh_step_info(mxh_gpu *g, uint64_t i, uint64_t *first, uint64_t *last, const char **kernel) {
    return guard([&] {
        Gpu &x = *G(g);
        if (i >= mxh_steps(g)) throw mx::Error("step index out of range");
        uint64_t a = i, b = i + 1;
        const char *k = "";
        if (x.fusion) {
            a = x.prog[i].first;
            b = x.prog[i].last;
            if (!x.prog[i].launches.empty()) k = x.prog[i].launches[x.prog[i].main].name;
        } else if (!x.ops[i].empty()) {
            k = x.ops[i][0].name;
        }
        if (first) *first = a;
        if (last) *last = b;
        if (kernel) *kernel = k;
    });
}

int mxh_run_timed(mxh_gpu *g, const mx_plan_desc *plan) {
    return guard([&] {
        G(g)->check_plan(plan);
        G(g)->run_timed();
    });
}

int mxh_read_buf(mxh_gpu *g, const mx_plan_desc *plan, uint64_t buf, float *out, uint64_t n) {
    return guard([&] {
        G(g)->check_plan(plan);
        if (buf >= plan->n_bufs) throw mx::Error("buffer index out of range");
        const mx_bufshape &s = plan->bufs[buf];
        if (n != (uint64_t)(s.c * s.h * s.w)) throw mx::Error("read_buf: wrong length");
        G(g)->read(G(g)->doff[buf], out, n);
    });
}

int mxh_write_buf(mxh_gpu *g, const mx_plan_desc *plan, uint64_t buf, const float *in, uint64_t n) {
    return guard([&] {
        G(g)->check_plan(plan);
        if (buf >= plan->n_bufs) throw mx::Error("buffer index out of range");
        const mx_bufshape &s = plan->bufs[buf];
        if (n != (uint64_t)(s.c * s.h * s.w)) throw mx::Error("write_buf: wrong length");
        G(g)->write(G(g)->doff[buf], in, n);
    });
}

uint64_t mxh_buf_offset(mxh_gpu *g, uint64_t buf) {
    return buf < G(g)->doff.size() ? G(g)->doff[buf] : UINT64_MAX;
}

int mxh_read_into(mxh_gpu *g, uint64_t off, float *out, uint64_t n) {
    return guard([&] { G(g)->read(off, out, n); });
}

int mxh_read_arena(mxh_gpu *g, float *out, uint64_t n) {
    return guard([&] {
        if (n != G(g)->arena_len) throw mx::Error("read_arena: wrong length");
        G(g)->read(0, out, n);
    });
}

int mxh_write_into(mxh_gpu *g, uint64_t off, const float *in, uint64_t n) {
    return guard([&] { G(g)->write(off, in, n); });
}

int mxh_poison(mxh_gpu *g) {
    return guard([&] {
        mxh::check(G(g)->H.hipMemsetD8Async(G(g)->arena, 0xCD, G(g)->arena_len * 4, G(g)->stream), "poison");
        mxh::check(G(g)->H.hipMemsetD8Async(G(g)->scratch, 0xCD, G(g)->scratch_len * 4, G(g)->stream), "poison");
        G(g)->sync();
    });
}

int mxh_sync(mxh_gpu *g) {
    return guard([&] { G(g)->sync(); });
}

void mxh_set_timeline(mxh_gpu *g, int on) { G(g)->want_timeline = on != 0; }

uint64_t mxh_launches(mxh_gpu *g) { return G(g)->launch_list().size(); }

int mxh_launch_info(mxh_gpu *g, uint64_t i, uint64_t *step, const char **kernel) {
    return guard([&] {
        const auto seq = G(g)->launch_list();
        if (i >= seq.size()) throw mx::Error("launch index out of range");
        if (step) *step = seq[i].first;
        if (kernel) *kernel = seq[i].second->name;
    });
}

int mxh_launch_span(mxh_gpu *g, uint64_t i, uint64_t *ops) {
    return guard([&] {
        Gpu &x = *G(g);
        const auto seq = x.launch_list();
        if (i >= seq.size()) throw mx::Error("launch index out of range");
        const mxh::Launch &l = *seq[i].second;
        uint64_t first = seq[i].first, last = seq[i].first + 1;
        if (x.fusion) {
            first = x.prog[seq[i].first].first;
            last = x.prog[seq[i].first].last;
        }
        const bool own = l.span[1] > l.span[0];
        ops[0] = own ? l.span[0] : first;
        ops[1] = own ? l.span[1] : last;
        ops[2] = l.span[2];
        ops[3] = l.span[3];
    });
}

int mxh_launch_timeline(mxh_gpu *g, float *ms, uint64_t n) {
    return guard([&] {
        Gpu &x = *G(g);
        if (!x.have_timeline) throw mx::Error("no timeline recorded (mxh_run_timed)");
        if (n != x.per_launch_ms.size()) throw mx::Error("launch_timeline: wrong length");
        if (ms) memcpy(ms, x.per_launch_ms.data(), sizeof(float) * n);
    });
}

int mxh_timeline(mxh_gpu *g, float *per_op_ms, uint64_t n, float *total_ms) {
    return guard([&] {
        Gpu &x = *G(g);
        if (!x.have_timeline) throw mx::Error("no timeline recorded (mxh_set_timeline, then mxh_run)");
        if (per_op_ms) memcpy(per_op_ms, x.per_op_ms.data(), sizeof(float) * std::min<uint64_t>(n, x.per_op_ms.size()));
        if (total_ms) *total_ms = x.total_ms;
    });
}

int mxh_time_graph(mxh_gpu *g, const mx_plan_desc *plan, int n, float *ms) {
    return guard([&] {
        Gpu &x = *G(g);
        x.check_plan(plan);
        if (n <= 0 || !ms) throw mx::Error("mxh_time_graph: no passes or no output");
        auto &H = x.H;
        std::vector<mxh::hipEvent_t> ev(2 * (size_t)n, nullptr);
        try {
            for (auto &e : ev) mxh::check(H.hipEventCreate(&e), "hipEventCreate");
            for (int k = 0; k < n; ++k) {
                mxh::check(H.hipEventRecord(ev[2 * k], x.stream), "hipEventRecord");
                x.run_graph();
                mxh::check(H.hipEventRecord(ev[2 * k + 1], x.stream), "hipEventRecord");
            }
            x.sync();
            for (int k = 0; k < n; ++k)
                mxh::check(H.hipEventElapsedTime(&ms[k], ev[2 * k], ev[2 * k + 1]), "hipEventElapsedTime");
        } catch (...) {
            for (auto &e : ev)
                if (e) H.hipEventDestroy(e);
            throw;
        }
        for (auto &e : ev) H.hipEventDestroy(e);
    });
}

int mxh_time_ops(mxh_gpu *g, const mx_plan_desc *plan, uint64_t first, uint64_t last, int iters, float *ms) {
    return guard([&] {
        Gpu &x = *G(g);
        x.check_plan(plan);
        if (last > plan->n_ops || first > last) throw mx::Error("op range out of bounds");
        auto &H = x.H;
        mxh::hipEvent_t a, b;
        mxh::check(H.hipEventCreate(&a), "hipEventCreate");
        mxh::check(H.hipEventCreate(&b), "hipEventCreate");
        mxh::check(H.hipEventRecord(a, x.stream), "hipEventRecord");
        for (int it = 0; it < iters; ++it)
            for (uint64_t i = first; i < last; ++i) x.run_op(i);
        mxh::check(H.hipEventRecord(b, x.stream), "hipEventRecord");
        mxh::check(H.hipEventSynchronize(b), "hipEventSynchronize");
        float t = 0.0f;
        mxh::check(H.hipEventElapsedTime(&t, a, b), "hipEventElapsedTime");
        H.hipEventDestroy(a);
        H.hipEventDestroy(b);
        if (ms) *ms = t;
    });
}

const char *mxh_device_name(mxh_gpu *g) { return G(g)->name.c_str(); }
uint64_t mxh_arena_bytes(mxh_gpu *g) { return G(g)->arena_len * 4; }
uint64_t mxh_weight_bytes(mxh_gpu *g) { return G(g)->wbytes; }
uint64_t mxh_pool_bytes(mxh_gpu *g) { return G(g)->scratch_len * 4; }
uint64_t mxh_ops_launched(mxh_gpu *g) { return G(g)->launched; }
uint64_t mxh_kernels_launched(mxh_gpu *g) { return G(g)->kernels; }

const char *mxh_op_kernel(mxh_gpu *g, uint64_t i) {
    Gpu &x = *G(g);
    if (i >= x.ops.size() || x.ops[i].empty()) return "";
    return x.ops[i][0].name;
}

int mxh_device_info(mxh_gpu *g, int *cus, int *clock_khz) {
    if (cus) *cus = G(g)->cus;
    if (clock_khz) *clock_khz = G(g)->clock_khz;
    return 0;
}

int mxh_enhance(const char *checkpoint, const float *image, int64_t h, int64_t w, float *out) {
    struct Owned {
        mx_weights *w = nullptr;
        mx_plan *p = nullptr;
        mxh_gpu *g = nullptr;
        ~Owned() {
            if (g) mxh_free(g);
            if (p) mx_plan_free(p);
            if (w) mx_weights_free(w);
        }
    } o;
    return guard([&] {
        if (!image || !out) throw mx::Error("mxh_enhance: no image or output");
        // The checkpoint says what it is (Weights::open derives the variant).
        o.w = mx_weights_open(checkpoint);
        if (!o.w) throw mx::Error(mx_last_error());
        // The reference pipeline's padding: even-ize, then a centred reflect
        // to a multiple of 64 (image::preprocess, src/image.rs:171-207).
        int64_t ph = 0, pw = 0, eh = 0, ew = 0;
        if (mx_preprocess(image, 3, h, w, 64, nullptr, &ph, &pw, &eh, &ew) != 0) throw mx::Error(mx_last_error());
        std::vector<float> padded((size_t)(3 * ph * pw));
        if (mx_preprocess(image, 3, h, w, 64, padded.data(), &ph, &pw, &eh, &ew) != 0)
            throw mx::Error(mx_last_error());
        // The release plan (no dump buffers), run on the device, cropped back
        // centred on the even shape (image::crop_out, src/image.rs:232-246).
        o.p = mx_plan_build(o.w, ph, pw, 0, 1, 0);
        if (!o.p) throw mx::Error(mx_last_error());
        mx_plan_desc d;
        mx_plan_describe(o.p, &d);
        o.g = mxh_new(&d);
        if (!o.g) throw mx::Error(mx_last_error());
        std::vector<float> pred((size_t)(3 * ph * pw));
        if (mxh_run(o.g, &d, padded.data(), padded.size(), pred.data(), pred.size()) != 0)
            throw mx::Error(mx_last_error());
        if (mx_crop_out(pred.data(), 3, ph, pw, eh, ew, h, w, out) != 0) throw mx::Error(mx_last_error());
    });
}

int mxh_device_memory(uint64_t *free_bytes, uint64_t *total_bytes) {
    return guard([&] {
        auto &H = mxh::hip();
        mxh::check(H.hipInit(0), "hipInit");
        mxh::check(H.hipSetDevice(0), "hipSetDevice");
        size_t f = 0, t = 0;
        mxh::check(H.hipMemGetInfo(&f, &t), "hipMemGetInfo");
        if (free_bytes) *free_bytes = f;
        if (total_bytes) *total_bytes = t;
    });
}

}  // extern "C"
