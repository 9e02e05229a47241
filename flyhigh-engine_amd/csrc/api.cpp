// The C ABI of the conv hot path (include/fhc_conv.h): plans, the MI355X planner and its choice table, weight
// packing into MFMA fragment order, and the launch of the kernels in conv_kernels.hip.
#include <algorithm>
#include <cmath>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "common.h"
#include "gm_corun.h"
#include "conv_kernels.h"
#include "direct_table.h"
#include "fhc_conv.h"

namespace fhc {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* msg) { g_last_error = msg ? msg : ""; }
void clear_error() { g_last_error.clear(); }

namespace {

constexpr size_t kLdsBudget = 64 * 1024;  // dynamic LDS per workgroup the planner stays within

uint32_t div_ceil(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// ---- the choice table (TuneTable, ops/conv/tune_cache.rs:6-9) ----------------------------------------------
// Key: the reference's (cin, cout, h, w, stride) plus the batch n and the kernel size k (the reference runs batch 1
// and 3x3 only). Batch 1 of a 3x3 conv is written in the reference's 5-field text; other keys carry n and k as
// fields 6 and 7, so the batch-1 and batched choices for one layer shape, or a 1x1 and a 3x3 conv over the same
// channels, do not overwrite each other.
using TuneKey = std::tuple<uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t>;
TuneKey tune_key(const fhc_conv_desc& d) { return TuneKey(d.cin, d.cout, d.h, d.w, d.stride, d.n, d.kh); }
std::mutex g_tune_mu;
std::map<TuneKey, uint32_t> g_tune;

// ---- variant codes -------------------------------------------------------------------------------------------
// The code space of the choice table (the reference table's value is a u8, tune_cache.rs:82; MI355X codes run to
// kCodeEnd - 1, and a committed table names its variants instead):
//   1..127   a K-chunked kernel: configuration (bits 0-4) | global split-K code (bits 5-6: 0 -> 1, 1 -> 2,
//            2 -> 4, 3 -> 8 splits); configuration 1..kNumCfg is the chunked implicit-GEMM kernel's tile
//            configuration, 16 + i the deep-layer kernel's configuration i of kGemmCfgs;
//   128+i    the direct kernel's configuration i of direct_table.h (weights resident in VGPRs).
constexpr uint32_t kSplitCodes[4] = {1, 2, 4, 8};
constexpr uint32_t kDirectBase = 128;
constexpr uint32_t kCodeEnd = kDirectBase + (uint32_t)kNumDirect;
constexpr int kGemmBase = 16;
static_assert(kNumCfg < kGemmBase && kGemmBase + kNumGemm <= 32, "configuration ids fit bits 0-4");

struct Variant {
    int family;   // 0 chunked implicit GEMM, 1 direct, 3 deep-layer (gemm_impl.h)
    int cfg;      // chunked: tile configuration id; direct: index into kDirectCfgs; deep-layer: into kGemmCfgs
    uint32_t ks;  // chunked, deep-layer: global split-K count
};

uint32_t make_code(int cfg, uint32_t ksplit, int family = 0) {
    uint32_t sc = 0;
    for (uint32_t i = 0; i < 4; i++)
        if (kSplitCodes[i] == ksplit) sc = i;
    return (uint32_t)(family == 3 ? kGemmBase + cfg : cfg) | (sc << 5);
}
uint32_t variant_code(const Variant& v) {
    return v.family == 1 ? kDirectBase + (uint32_t)v.cfg : make_code(v.cfg, v.ks, v.family);
}
bool decode_code(uint32_t code, Variant* v) {
    if (code >= kDirectBase) {
        if (code - kDirectBase >= (uint32_t)kNumDirect) return false;
        *v = Variant{1, (int)(code - kDirectBase), 1};
        return true;
    }
    const int c = (int)(code & 31u);
    const uint32_t ks = kSplitCodes[(code >> 5) & 3u];
    if (c >= kGemmBase && c < kGemmBase + kNumGemm) {
        *v = Variant{3, c - kGemmBase, ks};
        return true;
    }
    if (c < 1 || c > kNumCfg) return false;
    *v = Variant{0, c, ks};
    return true;
}
std::string code_name(uint32_t code) {
    Variant v;
    if (!decode_code(code, &v)) return "";
    std::ostringstream o;
    if (v.family == 1) {
        const DirectCfg& c = kDirectCfgs[v.cfg];
        o << "direct" << (c.ks == 1 ? ".k1" : c.stride == 2 ? ".s2" : "") << ".c" << c.cin32 << ".t" << c.fm << "x"
          << c.wm << ".n" << 16 * c.na * c.wn;
        if (c.na > 1) o << ".a" << c.na;
        if (c.wk > 1) o << "/rows";
        if (c.persist == 1) o << "/p";
        if (c.persist == 2) o << "/w";
        return o.str();
    }
    if (v.family == 3) {
        const GemmCfg& c = kGemmCfgs[v.cfg];
        o << "gemm" << (c.s == 2 ? ".s2" : "") << ".t" << c.fm * c.wm << "x16.n" << 16 * c.na * c.wn << ".f" << c.fm
          << "x" << c.na << ".w" << c.wm << "x" << c.wn << ".c" << c.ck << ".p" << c.st;
        if (v.ks > 1) o << "/k" << v.ks;
        return o.str();
    }
    const TileCfg& t = kTileCfgs[v.cfg];
    o << "igemm.t" << t.fm * t.wm << "x16.n" << t.fn * 16 * t.wn << ".w" << t.wm << "x" << t.wn << "x" << t.wk;
    if (v.ks > 1) o << "/k" << v.ks;
    return o.str();
}

struct Geometry {
    uint32_t hout, wout, taps, cin8;
};

bool valid_desc(const fhc_conv_desc& d, std::string* why) {
    char b[256];
    auto bad = [&](const char* m) {
        snprintf(b, sizeof b, "%s (n=%u h=%u w=%u cin=%u cout=%u k=%ux%u stride=%u pad=%u)", m, d.n, d.h, d.w, d.cin,
                 d.cout, d.kh, d.kw, d.stride, d.pad);
        *why = b;
        return false;
    };
    if (d.n == 0 || d.h == 0 || d.w == 0 || d.cin == 0 || d.cout == 0) return bad("empty tensor");
    if (!((d.kh == 3 && d.kw == 3 && d.pad == 1 && (d.stride == 1 || d.stride == 2)) ||
          (d.kh == 1 && d.kw == 1 && d.pad == 0 && d.stride == 1)))
        return bad("unsupported conv: 3x3 pad 1 stride 1/2 or 1x1 pad 0 stride 1");
    if (d.cin > 4096 || d.cout > 4096) return bad("channel count above 4096");
    if (d.h > 16384 || d.w > 16384 || d.n > 4096) return bad("tensor dimension too large");
    if (d.x_cstride < d.x_c0 + d.cin) return bad("input view: x_cstride < x_c0 + cin");
    if (d.y_cstride < d.y_c0 + d.cout) return bad("output view: y_cstride < y_c0 + cout");
    if (d.residual > 1) return bad("residual must be 0 or 1");
    if (d.residual && d.r_cstride < d.r_c0 + d.cout) return bad("residual view: r_cstride < r_c0 + cout");
    if (d.act > 2) return bad("unknown activation");
    if (d.act == FHC_ACT_LEAKY && !std::isfinite(d.alpha)) return bad("LeakyReLU alpha is not finite");
    const uint64_t pix_in = (uint64_t)d.n * d.h * d.w, pix_out = (uint64_t)d.n * d.h * d.w;  // hout <= h
    if (pix_in > (1ull << 31) || pix_out * d.y_cstride > (1ull << 40)) return bad("tensor too large");
    if (d.ksplit != 0 && d.ksplit != 1 && d.ksplit != 2 && d.ksplit != 4 && d.ksplit != 8)
        return bad("ksplit must be 0, 1, 2, 4 or 8");
    return true;
}

}  // namespace

}  // namespace fhc

using namespace fhc;

struct fhc_conv_plan {
    fhc_conv_desc d;
    Geometry g;
    uint32_t code;
    int family;       // 0 chunked implicit GEMM, 1 direct, 2 fused pair (this plan is the pair's first conv), 3
                      // deep-layer
    int cfg;          // chunked: tile configuration id; direct: index into kDirectCfgs; pair: into kPairCfgs;
                      // deep-layer: into kGemmCfgs
    uint32_t tiles;   // spatial output tiles (all images)
    uint32_t ksplit;  // effective global split count (1 = none)
    ConvKArgs args;   // kernel arguments with the tensor pointers left null
    dim3 grid;
    uint32_t threads;
    size_t lds;
    size_t ws_bytes;
    size_t packed_bytes;
    int device;
    void* dmem;  // packed weights | bias | negative-value multipliers (upload)
    LaunchFn launch;
    fhc_conv_plan* pair_b;  // fused pair: the second conv (its weights and output geometry), owned
    int res_mid;            // fused pair: the second conv's residual is the first's output
    int film_in;            // fused pair: FiLM on the first conv's input (runs with fhc_conv_pair_run_film)
    PairLaunchFn pair_launch;
};

namespace fhc {
namespace {

void fill_args(fhc_conv_plan& p) {
    const fhc_conv_desc& d = p.d;
    ConvKArgs& a = p.args;
    a = ConvKArgs{};
    a.n = (int)d.n;
    a.h = (int)d.h;
    a.w = (int)d.w;
    a.cin = (int)d.cin;
    a.cout = (int)d.cout;
    a.hout = (int)p.g.hout;
    a.wout = (int)p.g.wout;
    a.pad = (int)d.pad;
    a.xcs = (int)d.x_cstride;
    a.xc0 = (int)d.x_c0;
    a.ycs = (int)d.y_cstride;
    a.yc0 = (int)d.y_c0;
    a.rcs = (int)d.r_cstride;
    a.rc0 = (int)d.r_c0;
    a.act = (int)d.act;
    a.alpha = d.alpha;
    a.residual = (int)d.residual;
}

// Whether the direct kernel's configuration `idx` serves this conv: same kernel size and stride, and the input
// channels padded to 32 are exactly its channel count.
bool direct_fits(const fhc_conv_desc& d, int idx) {
    const DirectCfg& c = kDirectCfgs[idx];
    return c.ks == (int)d.kh && c.stride == (int)d.stride && (uint32_t)c.cin32 == div_ceil(d.cin, 32) * 32;
}

// The direct kernel's launch geometry for configuration `idx`: input channels padded to 32 in one pass, weights
// resident; one workgroup per spatial tile (grid x) and channel tile (grid y). False if it does not serve the conv.
bool configure_direct(fhc_conv_plan& p, int idx, std::string* why) {
    const fhc_conv_desc& d = p.d;
    if (idx < 0 || idx >= kNumDirect || !direct_fits(d, idx)) {
        *why = "the direct configuration does not serve " + std::to_string(d.kh) + "x" + std::to_string(d.kw) +
               " stride " + std::to_string(d.stride) + " with " + std::to_string(d.cin) + " input channels";
        return false;
    }
    const DirectCfg& c = kDirectCfgs[idx];
    LaunchFn fn = direct_launcher(idx, nullptr);
    if (!fn) {
        *why = "direct configuration not instantiated";
        return false;
    }
    // the wave-stream kernel moves whole 16-byte input groups by LDS DMA and has no residual path
    if (c.persist == 2 && (d.cin % 8 || d.x_cstride % 8 || d.x_c0 % 8 || d.cout % 4 || d.y_cstride % 4 ||
                           d.y_c0 % 4 || d.residual)) {
        *why = "the wave-stream configuration needs cin, the input channel stride and offset multiples of 8, cout "
               "and the output channel stride and offset multiples of 4, and no residual";
        return false;
    }
    const int TH = c.fm * c.wm;
    const uint32_t tiles_x = div_ceil(p.g.wout, 16), tiles_y = div_ceil(p.g.hout, TH);
    const uint64_t tiles = (uint64_t)d.n * tiles_y * tiles_x;
    const uint32_t ntn = div_ceil(d.cout, 16 * c.na * c.wn);
    if (tiles > 0x7fffffffull || ntn > 65535) {
        *why = "grid too large";
        return false;
    }
    fill_args(p);
    ConvKArgs& a = p.args;
    a.cc = c.cin32;
    a.nchunks = 1;
    a.ksteps = (int)(p.g.taps * c.cin32 / 32);
    a.tapgroups = (int)(p.g.taps * c.cin32 / 8);
    a.tiles_x = (int)tiles_x;
    a.tiles_y = (int)tiles_y;
    a.ntn = (int)ntn;
    a.chunks_per_split = 1;
    a.np = (int)(ntn * 16 * c.na * c.wn);
    p.family = 1;
    p.cfg = idx;
    p.tiles = (uint32_t)tiles;
    p.ksplit = 1;
    p.code = kDirectBase + (uint32_t)idx;
    // a persistent configuration gets no more workgroups than fit at once (set from the device at plan creation;
    // a dry plan assumes one per CU of an MI355X)
    const uint64_t units = c.persist == 2 ? (tiles + 3) / 4 : tiles;  // the wave-stream kernel: a tile per wave
    p.grid = dim3(c.persist ? (unsigned)std::min<uint64_t>(units, std::max(1u, 256u / ntn)) : (unsigned)tiles, ntn, 1);
    p.threads = c.persist == 2 ? 256u : 64u * c.wm * c.wn * c.wk;
    p.lds = 0;
    p.ws_bytes = 0;
    p.launch = fn;
    return true;
}

// Fill the launch geometry of `p` for the chunked kernel's configuration `cfg` and global split `ks`; false if it
// does not fit.
bool configure_igemm(fhc_conv_plan& p, int cfg, uint32_t ks, std::string* why) {
    const fhc_conv_desc& d = p.d;
    const TileCfg& t = kTileCfgs[cfg];
    const int KS = (int)d.kh, S = (int)d.stride;
    const int TH = t.fm * t.wm, BN = t.fn * 16 * t.wn;
    const int IH = (TH - 1) * S + KS, IW = 15 * S + KS;
    LaunchFn fn = conv_launcher(KS, S, cfg);
    if (!fn) {
        *why = "no kernel instantiated for this kernel size / stride / configuration";
        return false;
    }
    // channel chunk: everything at once when it fits the LDS budget, else equal chunks of a multiple of 8;
    // a global split needs at least `ks` chunks
    const uint32_t cin8 = p.g.cin8;
    const size_t per_ch = (size_t)IH * IW * 2;               // LDS bytes per staged channel
    const size_t table_max = (size_t)KS * KS * 512 / 8 * 4;  // offset table for cc <= 512
    long ccmax = (long)((kLdsBudget - table_max - 16) / per_ch) - 8;
    ccmax = ccmax / 8 * 8;
    if (ccmax > 512) ccmax = 512;
    if (ccmax < 8) {
        *why = "halo tile does not fit in LDS";
        return false;
    }
    uint32_t nchunks = div_ceil(cin8, (uint32_t)ccmax);
    if (ks > 1 && nchunks < ks) nchunks = std::min<uint32_t>(ks, cin8 / 8);
    uint32_t cc = div_ceil(div_ceil(cin8, nchunks), 8) * 8;
    nchunks = div_ceil(cin8, cc);
    const uint32_t cps = ks > 1 ? div_ceil(nchunks, ks) : nchunks;
    const uint32_t zcount = div_ceil(nchunks, cps);
    const uint32_t taps = p.g.taps;
    const uint32_t tapgroups = taps * cc / 8;
    const uint32_t ksteps = div_ceil(tapgroups, 4);
    size_t lds = (((size_t)tapgroups * 4 + 15) & ~(size_t)15) + (size_t)IH * IW * (cc + 8) * 2;
    if (t.wk > 1) {
        const size_t red = (size_t)(t.wk - 1) * t.wm * t.wn * t.fm * t.fn * 64 * 16;
        lds = std::max(lds, red);
    }
    if (lds > kLdsBudget) {
        *why = "LDS budget exceeded";
        return false;
    }
    const uint32_t tiles_x = div_ceil(p.g.wout, 16), tiles_y = div_ceil(p.g.hout, TH);
    const uint32_t ntn = div_ceil(d.cout, BN);
    const uint64_t blocks = (uint64_t)d.n * tiles_y * tiles_x * ntn;
    if (blocks > 0x7fffffffull) {
        *why = "grid too large";
        return false;
    }
    fill_args(p);
    ConvKArgs& a = p.args;
    a.cc = (int)cc;
    a.nchunks = (int)nchunks;
    a.ksteps = (int)ksteps;
    a.tapgroups = (int)tapgroups;
    a.tiles_x = (int)tiles_x;
    a.tiles_y = (int)tiles_y;
    a.ntn = (int)ntn;
    a.chunks_per_split = (int)cps;
    a.np = (int)(ntn * BN);
    p.family = 0;
    p.cfg = cfg;
    p.tiles = (uint32_t)(d.n * tiles_y * tiles_x);
    p.ksplit = zcount;
    p.code = make_code(cfg, zcount);
    p.grid = dim3((unsigned)blocks, zcount, 1);
    p.threads = 64u * t.wm * t.wn * t.wk;
    p.lds = lds;
    p.ws_bytes = zcount > 1 ? (size_t)zcount * d.n * p.g.hout * p.g.wout * a.np * sizeof(float) : 0;
    p.launch = fn;
    return true;
}

// The deep-layer kernel's launch geometry for configuration `idx` and global split `ks`: chunks of CK input
// channels (the packed weights of the chunked layout with cc = CK), one workgroup per spatial tile (grid x), channel
// tile (grid y) and split (grid z). False if it does not serve the conv: 3x3 of its stride, an input view of
// 16-byte groups below 2^31 bytes, at least `ks` chunks.
bool configure_gemm(fhc_conv_plan& p, int idx, uint32_t ks, std::string* why) {
    const fhc_conv_desc& d = p.d;
    if (idx < 0 || idx >= kNumGemm) {
        *why = "unknown deep-layer configuration";
        return false;
    }
    const GemmCfg& c = kGemmCfgs[idx];
    if (d.kh != 3 || (int)d.stride != c.s) {
        *why = "the deep-layer configuration serves 3x3 convs of stride " + std::to_string(c.s) + " only";
        return false;
    }
    if (d.x_cstride % 8 || d.x_c0 % 8 || (uint64_t)d.n * d.h * d.w * d.x_cstride * 2 >= (1ull << 31)) {
        *why = "the deep-layer kernel needs an input view of 16-byte channel groups below 2^31 bytes";
        return false;
    }
    LaunchFn fn = gemm_launcher(idx, nullptr);
    if (!fn) {
        *why = "deep-layer configuration not instantiated";
        return false;
    }
    const uint32_t nchunks = div_ceil(d.cin, (uint32_t)c.ck);
    if (ks > nchunks) {
        *why = "fewer input-channel chunks than splits";
        return false;
    }
    const uint32_t cps = div_ceil(nchunks, ks), zcount = div_ceil(nchunks, cps);
    const int TH = c.fm * c.wm, BN = 16 * c.na * c.wn;
    const uint32_t tiles_x = div_ceil(p.g.wout, 16), tiles_y = div_ceil(p.g.hout, (uint32_t)TH);
    const uint64_t tiles = (uint64_t)d.n * tiles_y * tiles_x;
    const uint32_t ntn = div_ceil(d.cout, (uint32_t)BN);
    if (tiles > 0x7fffffffull || ntn > 65535) {
        *why = "grid too large";
        return false;
    }
    fill_args(p);
    ConvKArgs& a = p.args;
    a.cc = c.ck;
    a.nchunks = (int)nchunks;
    a.ksteps = 9 * c.ck / 32;
    a.tapgroups = 9 * c.ck / 8;
    a.tiles_x = (int)tiles_x;
    a.tiles_y = (int)tiles_y;
    a.ntn = (int)ntn;
    a.chunks_per_split = (int)cps;
    a.np = (int)(ntn * BN);
    p.family = 3;
    p.cfg = idx;
    p.tiles = (uint32_t)tiles;
    p.ksplit = zcount;
    p.code = make_code(idx, zcount, 3);
    p.grid = dim3((unsigned)tiles, ntn, zcount);
    p.threads = 64u * c.wm * c.wn;
    p.lds = 0;
    p.ws_bytes = zcount > 1 ? (size_t)zcount * d.n * p.g.hout * p.g.wout * a.np * sizeof(float) : 0;
    p.launch = fn;
    return true;
}

int heuristic_cfg(const fhc_conv_desc& d, const Geometry& g);
void* static_scratch(int dev);

bool configure(fhc_conv_plan& p, const Variant& v, std::string* why) {
    if (v.family == 1) {
        if (v.ks > 1) {
            *why = "the direct kernel has no split-K";
            return false;
        }
        return configure_direct(p, v.cfg, why);
    }
    if (v.family == 3) return configure_gemm(p, v.cfg, v.ks, why);
    return configure_igemm(p, v.cfg, v.ks, why);
}

// The direct configuration the planner takes without a table entry, or -1: among the one-block-per-wave
// configurations that launch one workgroup per tile, the narrowest channel tile that covers cout in one tile (else
// the widest there is), and among the tile heights the tallest that still gives about two workgroups per CU (the
// small layers of a frame take short tiles: more, shorter-running workgroups). Up to 128 input channels the
// kernel-row K split is left to the autotuner.
int direct_default(const fhc_conv_desc& d, const Geometry& g) {
    const int need = (int)div_ceil(d.cout, 16);
    auto eligible = [&](int i) {
        return direct_fits(d, i) && kDirectCfgs[i].na == 1 && (kDirectCfgs[i].wk == 1 || kDirectCfgs[i].cin32 > 128);
    };
    int best_wn = 0;
    for (int i = 0; i < kNumDirect; i++) {
        if (!eligible(i)) continue;
        const int wn = kDirectCfgs[i].wn;
        if (best_wn == 0 || (best_wn < need && wn > best_wn) || (wn >= need && wn < best_wn)) best_wn = wn;
    }
    if (best_wn == 0) return -1;
    int pick = -1;
    uint64_t pick_wgs = 0;
    int pick_th = 0;
    for (int i = 0; i < kNumDirect; i++) {
        if (!eligible(i) || kDirectCfgs[i].wn != best_wn || kDirectCfgs[i].persist) continue;
        const int th = kDirectCfgs[i].fm * kDirectCfgs[i].wm;
        const uint64_t wgs = (uint64_t)d.n * div_ceil(g.hout, th) * div_ceil(g.wout, 16) * div_ceil(d.cout, 16 * best_wn);
        const bool enough = wgs >= 512;
        if (pick < 0 || (enough && (pick_wgs < 512 || th > pick_th)) || (!enough && pick_wgs < 512 && th < pick_th)) {
            pick = i;
            pick_wgs = wgs;
            pick_th = th;
        }
    }
    return pick;
}

// The deep-layer configuration the planner takes without a table entry: 8 rows x 48 channels, 4 waves of 2 rows x
// 3 channel blocks, two chunk buffers (the fastest or within a few percent of it on every deep layer of the frame
// and its batched form, and on the 128 -> 128 layer at 1080p/16).
constexpr int kGemmDefault = 11;

// The MI355X planner's default when neither the caller nor the table chose. The deep-layer kernel serves stride-1
// 3x3 convs over at least 64 input channels whose input view has 16-byte channel groups; it takes those over 64
// input channels with at least 4096 output pixels (on smaller ones its fixed cost per launch, the first chunk's
// load and the epilogue, outweighs the direct kernel's longer chains). Then the direct kernel whenever a
// configuration serves the input channels, then the deep-layer kernel where it serves, else the chunked kernel.
uint32_t heuristic_code(const fhc_conv_desc& d, const Geometry& g) {
    const bool gemm_ok = d.kh == 3 && d.stride == 1 && d.cin >= 64 && d.x_cstride % 8 == 0 && d.x_c0 % 8 == 0 &&
                         (uint64_t)d.n * d.h * d.w * d.x_cstride * 2 < (1ull << 31);
    if (gemm_ok && d.cin > 64 && (uint64_t)d.n * g.hout * g.wout >= 4096) return make_code(kGemmDefault, 1, 3);
    const int idx = direct_default(d, g);
    if (idx >= 0) return kDirectBase + (uint32_t)idx;
    if (gemm_ok) return make_code(kGemmDefault, 1, 3);
    return (uint32_t)heuristic_cfg(d, g);
}

int heuristic_cfg(const fhc_conv_desc& d, const Geometry& g) {
    struct Opt {
        int bn, cfg8, cfg4;
    };
    const Opt opts[] = {{128, 6, 0}, {64, 1, 4}, {48, 9, 0}, {32, 2, 5}, {16, 3, 10}};
    int cfg8 = 3, cfg4 = 10;
    for (const Opt& o : opts) {
        const uint32_t padded = div_ceil(d.cout, o.bn) * o.bn;
        if ((padded - d.cout) * 4 <= d.cout) {
            cfg8 = o.cfg8;
            cfg4 = o.cfg4 ? o.cfg4 : o.cfg8;
            break;
        }
    }
    const uint32_t tiles8 = d.n * div_ceil(g.hout, 8) * div_ceil(g.wout, 16) * div_ceil(d.cout, 64);
    if (g.taps * g.cin8 >= 1024 && tiles8 < 128 && d.cout > 32) return 7;
    return d.stride == 2 ? cfg4 : cfg8;
}

// Weights in MFMA A-fragment order, [nb16][chunk][kstep][lane][8]: lane l holds output channel nb*16 + l%16 and
// the 8 K positions of its lane group l/16 in that K-step. K order per chunk: the chunked kernel walks 8-channel
// groups j = 4*s + l/16 of k = tap * cc + ci; the direct kernel pads channels to 32 per tap, K-step s being tap
// s / (cc/32), channels 32 * (s % (cc/32)) + 8 * (l/16) .. +7.
void pack_weights(const fhc_conv_plan& p, const uint16_t* w, std::vector<uint16_t>& out) {
    const fhc_conv_desc& d = p.d;
    const ConvKArgs& a = p.args;
    const int nb16 = a.np / 16, gpt = a.cc / 8;
    out.assign((size_t)nb16 * a.nchunks * a.ksteps * 64 * 8, 0);
    size_t o = 0;
    if (p.family == 1) {
        const int m = a.cc / 32;
        for (int nb = 0; nb < nb16; nb++)
            for (int s = 0; s < a.ksteps; s++)
                for (int l = 0; l < 64; l++)
                    for (int i = 0; i < 8; i++, o++) {
                        const int tap = s / m;
                        const uint32_t ci = (uint32_t)((s % m) * 32 + (l >> 4) * 8 + i);
                        const uint32_t co = (uint32_t)(nb * 16 + (l & 15));
                        if (ci >= d.cin || co >= d.cout) continue;
                        const uint32_t ky = (uint32_t)tap / d.kw, kx = (uint32_t)tap % d.kw;
                        out[o] = w[(((size_t)co * d.cin + ci) * d.kh + ky) * d.kw + kx];
                    }
        return;
    }
    for (int nb = 0; nb < nb16; nb++)
        for (int c = 0; c < a.nchunks; c++)
            for (int s = 0; s < a.ksteps; s++)
                for (int l = 0; l < 64; l++)
                    for (int i = 0; i < 8; i++, o++) {
                        const int j = 4 * s + (l >> 4);  // 8-channel group of this K position
                        if (j >= a.tapgroups) continue;
                        const int tap = j / gpt, g = j % gpt;
                        const uint32_t ci = (uint32_t)(c * a.cc + g * 8 + i), co = (uint32_t)(nb * 16 + (l & 15));
                        if (ci >= d.cin || co >= d.cout) continue;
                        const uint32_t ky = (uint32_t)tap / d.kw, kx = (uint32_t)tap % d.kw;
                        out[o] = w[(((size_t)co * d.cin + ci) * d.kh + ky) * d.kw + kx];
                    }
}

// A pair's first conv with taps packed into its K-steps (cp = 8 or 16 input channels per tap, cin <= cp): the
// A-fragment order of pack_weights, [nb16][kstep][lane][8], K-step s holding taps s * (32 / cp) .. in cp-channel
// slots, lane l's 8 positions channels (g % (cp / 8)) * 8 .. +7 of tap s * (32 / cp) + g / (cp / 8), g = l / 16;
// positions past the 9th tap or the input channels are zero.
void pack_weights_taps(const fhc_conv_desc& d, int nb16, int ksteps, int cp, const uint16_t* w,
                       std::vector<uint16_t>& out) {
    const int tps = 32 / cp, gpt = cp / 8;
    out.assign((size_t)nb16 * ksteps * 64 * 8, 0);
    size_t o = 0;
    for (int nb = 0; nb < nb16; nb++)
        for (int s = 0; s < ksteps; s++)
            for (int l = 0; l < 64; l++)
                for (int i = 0; i < 8; i++, o++) {
                    const int g = l >> 4, tap = s * tps + g / gpt;
                    const uint32_t ci = (uint32_t)((g % gpt) * 8 + i), co = (uint32_t)(nb * 16 + (l & 15));
                    if (tap >= 9 || ci >= d.cin || co >= d.cout) continue;
                    const uint32_t ky = (uint32_t)tap / 3, kx = (uint32_t)tap % 3;
                    out[o] = w[(((size_t)co * d.cin + ci) * d.kh + ky) * d.kw + kx];
                }
}

// f16 bits -> f32 (exact)
static float half_bits_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t b;
    if (e == 0x1f) {
        b = s | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        b = s | ((e + 112) << 23) | (m << 13);
    } else if (m == 0) {
        b = s;
    } else {  // subnormal: normalize
        int k = 0;
        uint32_t mm = m;
        while (!(mm & 0x400)) {
            mm <<= 1;
            k++;
        }
        b = s | ((uint32_t)(113 - k) << 23) | ((mm & 0x3ff) << 13);
    }
    float f;
    memcpy(&f, &b, 4);
    return f;
}

// Device layout of a plan: packed weights | bias (f16, np) | negative-value multipliers (f32, np, 16-byte
// aligned). The multiplier folds the activation into one array, so that every epilogue computes
// t > 0 ? t : m * t without looking at the activation: the PReLU slope (f16 -> f32 is exact), the LeakyReLU alpha
// (f32, as the reference's uniform holds it), or 1 for no activation (m * t == t, signed zero included).
hipError_t upload(fhc_conv_plan& p, const std::vector<uint16_t>& packed, const uint16_t* bias, const uint16_t* slope) {
    const size_t np = (size_t)p.args.np;
    const size_t wbytes = (packed.size() * 2 + 255) & ~(size_t)255;
    const size_t bbytes = (np * 2 + 15) & ~(size_t)15;
    const size_t total = wbytes + bbytes + np * 4 + 256;
    std::vector<uint16_t> host(total / 2, 0);
    memcpy(host.data(), packed.data(), packed.size() * 2);
    uint16_t* hb = host.data() + wbytes / 2;
    std::vector<float> neg(np, 1.0f);
    for (uint32_t i = 0; i < p.d.cout; i++) {
        hb[i] = bias[i];
        if (p.d.act == FHC_ACT_PRELU) neg[i] = half_bits_to_float(slope[i]);
        if (p.d.act == FHC_ACT_LEAKY) neg[i] = p.d.alpha;
    }
    memcpy(reinterpret_cast<char*>(host.data()) + wbytes + bbytes, neg.data(), np * 4);
    hipError_t e = hipMalloc(&p.dmem, total);
    if (e != hipSuccess) {
        p.dmem = nullptr;
        return e;
    }
    e = hipMemcpy(p.dmem, host.data(), total, hipMemcpyHostToDevice);
    if (e != hipSuccess) return e;
    p.args.wpk = p.dmem;
    p.args.bias = reinterpret_cast<const uint16_t*>(static_cast<char*>(p.dmem) + wbytes);
    p.args.neg = reinterpret_cast<const float*>(static_cast<char*>(p.dmem) + wbytes + bbytes);
    p.packed_bytes = packed.size() * 2;
    return hipSuccess;
}

// The planner's choice for `d` (conv_pick, autotune.rs:186-233): a forced variant, else the table, else the
// heuristic; the caller's forced split-K (or the reference code's split nibble) applies on top.
bool plan_choose(const fhc_conv_desc& d, fhc_conv_plan& p, std::string* why) {
    p.d = d;
    p.dmem = nullptr;
    p.g.hout = (d.h + 2 * d.pad - d.kh) / d.stride + 1;
    p.g.wout = (d.w + 2 * d.pad - d.kw) / d.stride + 1;
    p.g.taps = d.kh * d.kw;
    p.g.cin8 = div_ceil(d.cin, 8) * 8;
    // the choice: forced variant, then the table, then the heuristic (conv_pick, autotune.rs:186-233)
    Variant v{};
    if (d.variant != 0) {
        if (!decode_code(d.variant, &v)) {
            *why = "unknown variant " + std::to_string(d.variant);
            return false;
        }
    } else {
        const int hit = fhc_tune_get_ex(d.cin, d.cout, d.h, d.w, d.stride, d.n, d.kh);
        if (hit < 0 || !decode_code((uint32_t)hit, &v)) decode_code(heuristic_code(d, p.g), &v);
    }
    // a forced split (or the reference code's split nibble, candidates.rs:4) moves to the chunked kernel
    uint32_t ks = 0;
    if (d.ksplit != 0)
        ks = d.ksplit;
    else if (d.ref_cand != 0xFFu && (d.ref_cand >> 4) != 0 && d.variant == 0) {
        const uint32_t rk = d.ref_cand >> 4;
        if (rk == 1 || rk == 2 || rk == 4) ks = rk;
    }
    if (ks != 0 && !(v.family == 1 && ks == 1)) {
        if (v.family == 1) {
            if (d.variant != 0) {
                *why = "the direct kernel has no split-K";
                return false;
            }
            v = Variant{0, heuristic_cfg(d, p.g), ks};
        } else {
            v.ks = ks;
        }
    }
    if (!configure(p, v, why)) {
        // a table entry or heuristic that does not fit this shape falls back to the chunked 4-row tile
        const uint32_t code = variant_code(v);
        if (d.variant != 0 || !configure(p, Variant{0, d.cout <= 32 ? 5 : 4, v.family == 1 ? 1u : v.ks}, why)) {
            *why += " (variant " + code_name(code) + ")";
            return false;
        }
    }
    return true;
}

std::string describe_json(const fhc_conv_plan* p) {
    const fhc_conv_desc& d = p->d;
    int rows, chans, wm, wnv, wk;
    if (p->family == 2) {
        const PairCfg& c = kPairCfgs[p->cfg];
        const fhc_conv_desc& b = p->pair_b->d;
        const double fa = 2.0 * d.n * p->g.hout * p->g.wout * d.cout * d.cin * 9;
        const double fb = 2.0 * b.n * p->g.hout * p->g.wout * b.cout * b.cin * 9;
        const double out_el = (double)b.n * p->g.hout * p->g.wout * b.cout;
        const double bytes = 2.0 * ((double)d.n * d.h * d.w * d.cin + out_el + 9.0 * (d.cout * d.cin + b.cout * b.cin) +
                                    d.cout + b.cout + (d.act == FHC_ACT_PRELU ? d.cout : 0) +
                                    (b.act == FHC_ACT_PRELU ? b.cout : 0) + (b.residual && !p->res_mid ? out_el : 0));
        char buf[700];
        snprintf(buf, sizeof buf,
                 "{\"variant\":0,\"name\":\"pair.s%d.c%dx%d.n%dx%d.t%dx%d.w%d%s%s\",\"family\":\"pair\",\"cfg\":%d,"
                 "\"tile_rows\":%d,\"tile_cols\":%d,\"wave_rows\":%d,\"persistent\":%d,\"res_mid\":%d,\"tiles\":%u,"
                 "\"grid\":[%u,%u,%u],\"threads\":%u,\"hout\":%u,\"wout\":%u,\"flops\":%.0f,\"bytes\":%.0f,"
                 "\"a_channels_per_tap\":%d,\"a_ksteps\":%d}",
                 c.sa, c.ca32, c.cb32, 16 * c.nba, 16 * c.nbb, c.th, kPairTileW, c.wm,
                 c.cpa == 8 ? ".k8" : c.cpa == 16 ? ".k16" : "", c.persist == 2 ? "/ws" : c.persist ? "/p" : "", p->cfg,
                 c.th, kPairTileW, c.wm, c.persist, p->res_mid, p->tiles, p->grid.x, p->grid.y, p->grid.z, p->threads,
                 p->g.hout, p->g.wout, fa + fb, bytes, c.cpa ? c.cpa : 32, p->args.ksteps);
        return buf;
    }
    if (p->family == 1) {
        const DirectCfg& c = kDirectCfgs[p->cfg];
        rows = c.fm * c.wm;
        chans = 16 * c.na * c.wn;
        wm = c.wm;
        wnv = c.wn;
        wk = c.wk;
    } else if (p->family == 3) {
        const GemmCfg& c = kGemmCfgs[p->cfg];
        rows = c.fm * c.wm;
        chans = 16 * c.na * c.wn;
        wm = c.wm;
        wnv = c.wn;
        wk = 1;
    } else {
        const TileCfg& t = kTileCfgs[p->cfg];
        rows = t.fm * t.wm;
        chans = t.fn * 16 * t.wn;
        wm = t.wm;
        wnv = t.wn;
        wk = t.wk;
    }
    const double flops = 2.0 * d.n * p->g.hout * p->g.wout * d.cout * d.cin * d.kh * d.kw;
    const double out_el = (double)d.n * p->g.hout * p->g.wout * d.cout;
    const double bytes = 2.0 * ((double)d.n * d.h * d.w * d.cin + out_el + (double)d.cout * d.cin * d.kh * d.kw +
                                d.cout + (d.act == FHC_ACT_PRELU ? d.cout : 0) + (d.residual ? out_el : 0));
    const size_t packed = (size_t)(p->args.np / 16) * p->args.nchunks * p->args.ksteps * 64 * 16;
    char b[1200];
    snprintf(b, sizeof b,
             "{\"variant\":%u,\"name\":\"%s\",\"family\":\"%s\",\"cfg\":%d,\"tile_rows\":%d,\"tile_cols\":16,"
             "\"tile_channels\":%d,\"waves\":[%d,%d,%d],\"ksplit\":%u,\"cc\":%d,\"nchunks\":%d,\"ksteps\":%d,"
             "\"tiles\":%u,\"ntn\":%d,\"grid\":[%u,%u,%u],\"threads\":%u,\"lds\":%zu,\"packed_weight_bytes\":%zu,"
             "\"workspace_bytes\":%zu,\"hout\":%u,\"wout\":%u,\"flops\":%.0f,\"bytes\":%.0f}",
             p->code, code_name(p->code).c_str(), p->family == 1 ? "direct" : p->family == 3 ? "gemm" : "igemm",
             p->cfg, rows, chans, wm, wnv, wk, p->ksplit, p->args.cc, p->args.nchunks, p->args.ksteps, p->tiles, p->args.ntn, p->grid.x, p->grid.y, p->grid.z,
             p->threads, p->lds, packed, p->ws_bytes, p->g.hout, p->g.wout, flops, bytes);
    return b;
}

}  // namespace
}  // namespace fhc

extern "C" const char* fhc_last_error(void) { return g_last_error.c_str(); }

extern "C" int fhc_conv_plan_create(const fhc_conv_desc* desc, const uint16_t* w_oihw, const uint16_t* bias,
                                    const uint16_t* slope, fhc_conv_plan** out) {
    return guard(-1, [&]() -> int {
        if (!out) return fail(-1, "fhc_conv_plan_create: NULL output handle");
        *out = nullptr;
        if (!desc) return fail(-1, "fhc_conv_plan_create: NULL descriptor");
        if (!w_oihw || !bias) return fail(-1, "fhc_conv_plan_create: NULL weights or bias");
        fhc_conv_desc d = *desc;
        if (d.x_cstride == 0) d.x_cstride = d.cin;
        if (d.y_cstride == 0) d.y_cstride = d.cout;
        if (d.r_cstride == 0) d.r_cstride = d.cout;
        std::string why;
        if (!valid_desc(d, &why)) return fail(-1, "fhc_conv_plan_create: %s", why.c_str());
        if (d.act == FHC_ACT_PRELU && !slope) return fail(-1, "fhc_conv_plan_create: PReLU needs a slope");
        auto p = std::make_unique<fhc_conv_plan>();
        if (!plan_choose(d, *p, &why)) return fail(-1, "fhc_conv_plan_create: %s", why.c_str());
        hipError_t e = hipGetDevice(&p->device);
        if (e != hipSuccess) return fail(-1, "fhc_conv_plan_create: hipGetDevice: %s", hipGetErrorString(e));
        if (p->family == 1 && kDirectCfgs[p->cfg].persist) {
            const void* k = nullptr;
            direct_launcher(p->cfg, &k, d.residual != 0);
            int per_cu = 0, cus = 0;
            if (!k || hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, (int)p->threads, 0) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device) != hipSuccess)
                return fail(-1, "fhc_conv_plan_create: occupancy query failed");
            const uint64_t resident = (uint64_t)std::max(1, per_cu) * (uint64_t)std::max(1, cus);
            // the wave-stream kernel runs a tile per wave (4 per workgroup) at a time
            const uint64_t units = kDirectCfgs[p->cfg].persist == 2 ? (p->tiles + 3) / 4 : p->tiles;
            p->grid.x = (unsigned)std::min<uint64_t>(units, std::max<uint64_t>(1, resident / p->grid.y));
        }
        std::vector<uint16_t> packed;
        pack_weights(*p, w_oihw, packed);
        e = upload(*p, packed, bias, slope);
        if (e != hipSuccess) {
            if (p->dmem) (void)hipFree(p->dmem);
            return fail(-1, "fhc_conv_plan_create: device upload: %s", hipGetErrorString(e));
        }
        // set-up of fhc_conv_run_noalloc: the static scratch's address on this device, looked up here, outside any
        // stream capture (a failure is reported again by fhc_conv_run_noalloc)
        if (p->ws_bytes > 0 && p->ws_bytes <= FHC_STATIC_SCRATCH_BYTES) (void)static_scratch(p->device);
        *out = p.release();
        clear_error();
        return 0;
    });
}

extern "C" size_t fhc_conv_workspace_bytes(const fhc_conv_plan* p) { return p ? p->ws_bytes : 0; }

extern "C" int fhc_conv_out_shape(const fhc_conv_plan* p, uint32_t* hout, uint32_t* wout) {
    if (!p) return fail(-1, "fhc_conv_out_shape: NULL plan");
    if (hout) *hout = p->g.hout;
    if (wout) *wout = p->g.wout;
    return 0;
}

namespace {
// the arguments of a fused pair plan's launch: x is the first conv's input, y and res the second's output and
// residual, film the FiLM vectors of a FHC_PAIR_FILM_IN plan
PairKArgs pair_args(const fhc_conv_plan* p, const void* x, void* y, const void* res, const void* film) {
    const fhc_conv_plan* q = p->pair_b;
    PairKArgs pk{p->args, q->args, p->res_mid};
    pk.a.x = static_cast<const uint16_t*>(x);
    pk.a.xvec = ((uintptr_t)x % 16 == 0) && pk.a.xcs % 8 == 0 && pk.a.xc0 % 8 == 0;
    pk.a.film = static_cast<const uint16_t*>(film);
    pk.b.y = static_cast<uint16_t*>(y);
    pk.b.res = static_cast<const uint16_t*>(res);
    pk.b.yvec = ((uintptr_t)y % 8 == 0) && pk.b.ycs % 4 == 0 && pk.b.yc0 % 4 == 0;
    pk.b.rvec = pk.b.residual && !p->res_mid && ((uintptr_t)res % 8 == 0) && pk.b.rcs % 4 == 0 &&
                pk.b.rc0 % 4 == 0 && pk.b.cout % 4 == 0;
    return pk;
}

// the launch of a fused pair plan (validated by the caller)
int run_pair(const fhc_conv_plan* p, const void* x, void* y, const void* res, const void* film, void* stream,
             const char* who) {
    if (p->pair_b->d.residual && !p->res_mid && !res)
        return fail(-1, "%s: the pair's second conv has a residual but res is NULL", who);
    const PairKArgs pk = pair_args(p, x, y, res, film);
    hipError_t e = p->pair_launch(pk, p->grid, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(-1, "%s: launch: %s", who, hipGetErrorString(e));
    return 0;
}
}  // namespace

extern "C" int fhc_conv_pair_run_film(const fhc_conv_plan* p, const void* x, const void* film, void* y, void* stream) {
    return guard(-1, [&]() -> int {
        if (!p) return fail(-1, "fhc_conv_pair_run_film: NULL plan");
        if (p->family != 2 || !p->film_in)
            return fail(-1, "fhc_conv_pair_run_film: not a pair plan created with FHC_PAIR_FILM_IN");
        if (!x || !y || !film) return fail(-1, "fhc_conv_pair_run_film: NULL input, output or FiLM vectors");
        if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)film) & 1u)
            return fail(-1, "fhc_conv_pair_run_film: f16 tensors must be 2-byte aligned");
        int dev = -1;
        if (hipGetDevice(&dev) != hipSuccess || dev != p->device)
            return fail(-1, "fhc_conv_pair_run_film: the plan belongs to device %d, the current device is %d",
                        p->device, dev);
        return run_pair(p, x, y, nullptr, film, stream, "fhc_conv_pair_run_film");
    });
}

extern "C" int fhc_conv_run(const fhc_conv_plan* p, const void* x, void* y, const void* res, void* workspace,
                            void* stream) {
    return guard(-1, [&]() -> int {
        if (!p) return fail(-1, "fhc_conv_run: NULL plan");
        if (!x || !y) return fail(-1, "fhc_conv_run: NULL input or output");
        if (p->d.residual && !res) return fail(-1, "fhc_conv_run: the plan has a residual but res is NULL");
        if (p->ws_bytes && !workspace)
            return fail(-1, "fhc_conv_run: the plan needs %zu bytes of workspace", p->ws_bytes);
        if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)res) & 1u)
            return fail(-1, "fhc_conv_run: f16 tensors must be 2-byte aligned");
        if ((uintptr_t)workspace & 15u) return fail(-1, "fhc_conv_run: workspace must be 16-byte aligned");
        int dev = -1;
        if (hipGetDevice(&dev) != hipSuccess || dev != p->device)
            return fail(-1, "fhc_conv_run: the plan belongs to device %d, the current device is %d", p->device, dev);
        if (p->args.split) return fail(-1, "fhc_conv_run: a sibling plan runs with fhc_conv_sibling_run");
        if (p->family == 2) {  // fused pair: x is the first conv's input, y and res the second's output and residual
            if (p->film_in) return fail(-1, "fhc_conv_run: the pair takes FiLM vectors: run it with fhc_conv_pair_run_film");
            return run_pair(p, x, y, res, nullptr, stream, "fhc_conv_run");
        }
        ConvKArgs a = p->args;
        a.x = static_cast<const uint16_t*>(x);
        a.y = static_cast<uint16_t*>(y);
        a.res = static_cast<const uint16_t*>(res);
        a.part = static_cast<float*>(workspace);
        a.xvec = ((uintptr_t)x % 16 == 0) && a.xcs % 8 == 0 && a.xc0 % 8 == 0;
        a.yvec = ((uintptr_t)y % 8 == 0) && a.ycs % 4 == 0 && a.yc0 % 4 == 0;
        a.rvec = a.residual && ((uintptr_t)res % 8 == 0) && a.rcs % 4 == 0 && a.rc0 % 4 == 0 && a.cout % 4 == 0;
        hipStream_t s = static_cast<hipStream_t>(stream);
        hipError_t e = p->launch(a, p->grid, p->lds, s);
        if (e != hipSuccess) return fail(-1, "fhc_conv_run: launch: %s", hipGetErrorString(e));
        if (p->ksplit > 1) {
            e = splitk_reduce_launch(a, (int)p->ksplit, s);
            if (e != hipSuccess) return fail(-1, "fhc_conv_run: split-K reduce launch: %s", hipGetErrorString(e));
        }
        return 0;
    });
}

extern "C" int fhc_conv_describe(const fhc_conv_plan* p, char* json, size_t cap) {
    return guard(-1, [&]() -> int {
        if (!p) return fail(-1, "fhc_conv_describe: NULL plan");
        return write_string(describe_json(p), json, cap);
    });
}

extern "C" int fhc_conv_plan_dry(const fhc_conv_desc* desc, char* json, size_t cap) {
    return guard(-1, [&]() -> int {
        if (!desc) return fail(-1, "fhc_conv_plan_dry: NULL descriptor");
        fhc_conv_desc d = *desc;
        if (d.x_cstride == 0) d.x_cstride = d.cin;
        if (d.y_cstride == 0) d.y_cstride = d.cout;
        if (d.r_cstride == 0) d.r_cstride = d.cout;
        std::string why;
        if (!valid_desc(d, &why)) return fail(-1, "fhc_conv_plan_dry: %s", why.c_str());
        fhc_conv_plan p{};
        if (!plan_choose(d, p, &why)) return fail(-1, "fhc_conv_plan_dry: %s", why.c_str());
        p.device = -1;
        return write_string(describe_json(&p), json, cap);
    });
}

extern "C" void fhc_conv_plan_destroy(fhc_conv_plan* p) {
    if (!p) return;
    if (p->pair_b) fhc_conv_plan_destroy(p->pair_b);
    if (p->dmem) (void)hipFree(p->dmem);
    delete p;
}

namespace fhc {
namespace {

// One conv of a fused pair as a direct-kernel weight layout (CIN32 input channels per tap, nb 16-channel blocks):
// the plan's geometry, arguments, packed weights and device arrays.
hipError_t pair_part(fhc_conv_plan& p, const fhc_conv_desc& d, int cin32, int nb, const uint16_t* w,
                     const uint16_t* bias, const uint16_t* slope, int cp = 32) {
    p.d = d;
    p.dmem = nullptr;
    p.pair_b = nullptr;
    p.g.hout = (d.h + 2 * d.pad - d.kh) / d.stride + 1;
    p.g.wout = (d.w + 2 * d.pad - d.kw) / d.stride + 1;
    p.g.taps = d.kh * d.kw;
    p.g.cin8 = div_ceil(d.cin, 8) * 8;
    fill_args(p);
    p.args.cc = cin32;
    p.args.nchunks = 1;
    p.args.ksteps = 9 * cin32 / 32;
    p.args.tapgroups = 9 * cin32 / 8;
    p.args.chunks_per_split = 1;
    p.args.ntn = 1;
    p.args.np = 16 * nb;
    p.family = 1;
    p.ksplit = 1;
    std::vector<uint16_t> packed;
    if (cp < 32) {  // taps packed into the K-steps (pair_impl.h, tap_chain)
        p.args.ksteps = (9 + 32 / cp - 1) / (32 / cp);
        p.args.tapgroups = p.args.ksteps * 4;
        pack_weights_taps(d, nb, p.args.ksteps, cp, w, packed);
    } else {
        pack_weights(p, w, packed);
    }
    return upload(p, packed, bias, slope);
}

}  // namespace
}  // namespace fhc

extern "C" int fhc_conv_pair_plan_create(const fhc_conv_desc* desc_a, const uint16_t* w_a, const uint16_t* bias_a,
                                         const uint16_t* slope_a, const fhc_conv_desc* desc_b, const uint16_t* w_b,
                                         const uint16_t* bias_b, const uint16_t* slope_b, uint32_t flags,
                                         fhc_conv_plan** out) {
    return guard(-1, [&]() -> int {
        if (!desc_a || !desc_b || !w_a || !bias_a || !w_b || !bias_b || !out)
            return fail(-1, "fhc_conv_pair_plan_create: NULL argument");
        *out = nullptr;
        fhc_conv_desc A = *desc_a, B = *desc_b;
        for (fhc_conv_desc* d : {&A, &B}) {
            if (d->x_cstride == 0) d->x_cstride = d->cin;
            if (d->y_cstride == 0) d->y_cstride = d->cout;
            if (d->r_cstride == 0) d->r_cstride = d->cout;
        }
        std::string why;
        if (!valid_desc(A, &why)) return fail(-1, "fhc_conv_pair_plan_create: first conv: %s", why.c_str());
        if (!valid_desc(B, &why)) return fail(-1, "fhc_conv_pair_plan_create: second conv: %s", why.c_str());
        const bool res_mid = (flags & FHC_PAIR_RES_MID) != 0, post = (flags & FHC_PAIR_AFFINE_OUT) != 0;
        const bool film = (flags & FHC_PAIR_FILM_IN) != 0, tap32 = (flags & FHC_PAIR_TAP32) != 0;
        const uint32_t th_req = (flags >> 8) & 0xffu, wm_req = (flags >> 16) & 0xfu;
        // affine_out after the second conv, FiLM before the first: the one-workgroup-per-tile loop applies them
        const uint32_t loop_req = post || film ? 1u : (flags >> 20) & 3u;
        if ((flags & ~(FHC_PAIR_RES_MID | FHC_PAIR_AFFINE_OUT | FHC_PAIR_FILM_IN | FHC_PAIR_TAP32 | 0x3fff00u)) != 0)
            return fail(-1, "fhc_conv_pair_plan_create: unknown flags");
        if (post && ((flags >> 20) & 3u) > 1)
            return fail(-1, "fhc_conv_pair_plan_create: affine_out runs in the one-workgroup-per-tile loop only");
        if (film && ((flags >> 20) & 3u) > 1)
            return fail(-1, "fhc_conv_pair_plan_create: FiLM on the input runs in the one-workgroup-per-tile loop "
                            "only");
        if (film && B.residual && !res_mid)
            return fail(-1, "fhc_conv_pair_plan_create: FiLM on the input leaves no argument for an external residual");
        if (post && (B.cout > 4 || B.residual))
            return fail(-1, "fhc_conv_pair_plan_create: affine_out needs a second conv of at most 4 output channels "
                            "without residual");
        const uint32_t ha = (A.h + 2 * A.pad - A.kh) / A.stride + 1, wa = (A.w + 2 * A.pad - A.kw) / A.stride + 1;
        if (A.kh != 3 || B.kh != 3 || B.stride != 1 || A.residual)
            return fail(-1, "fhc_conv_pair_plan_create: the pair is a 3x3 conv (stride 1 or 2, no residual) then a 3x3 "
                            "stride-1 conv");
        if (B.n != A.n || B.h != ha || B.w != wa || B.cin != A.cout)
            return fail(-1, "fhc_conv_pair_plan_create: the second conv must read the first's output (n %u/%u, h %u/%u, "
                            "w %u/%u, channels %u/%u)", B.n, A.n, B.h, ha, B.w, wa, B.cin, A.cout);
        if (res_mid && (!B.residual || B.cout != B.cin))
            return fail(-1, "fhc_conv_pair_plan_create: a residual from the first conv's output needs the second conv's "
                            "residual flag and cout == cin");
        if ((A.act == FHC_ACT_PRELU && !slope_a) || (B.act == FHC_ACT_PRELU && !slope_b))
            return fail(-1, "fhc_conv_pair_plan_create: PReLU needs a slope");
        const int ca32 = (int)div_ceil(A.cin, 32) * 32, cb32 = (int)div_ceil(B.cin, 32) * 32;
        const int nba = (int)div_ceil(A.cout, 16), nbb = (int)div_ceil(B.cout, 16);
        // the configuration at the requested tile height, wave rows and loop; by default the resident-grid loop
        // when it is instantiated and there are at least 8 tiles per CU of an MI355X (256), one wave row where that
        // is instantiated (else two), and the tallest instantiated tile that still gives 256 workgroups, else the
        // shortest
        auto tiles_at = [&](int th) { return (uint64_t)A.n * div_ceil(ha, (uint32_t)th) * div_ceil(wa, kPairTileW); };
        // A's channels per tap: 8 or 16 where its input has at most that many and a configuration at the requested
        // tile, wave split and loop packs them (the taps then share K-steps), else 32 (or 32 on request,
        // FHC_PAIR_TAP32)
        auto serves_cp = [&](const PairCfg& c, int cp) {
            return c.sa == (int)A.stride && c.ca32 == ca32 && c.cb32 == cb32 && c.nba == nba && c.nbb == nbb &&
                   (c.cpa ? c.cpa : 32) == cp && (!th_req || c.th == (int)th_req) && (!wm_req || c.wm == (int)wm_req);
        };
        // the configuration for channels per tap cp: by default the resident-grid loop when it is instantiated and
        // there are at least 8 tiles per CU of an MI355X (256), one wave row where that is instantiated (else two),
        // and the tallest instantiated tile that still gives 256 workgroups, else the shortest; -1 if none
        auto select = [&](int cp) {
            auto serves = [&](const PairCfg& c) { return serves_cp(c, cp); };
            int persist = loop_req >= 2 ? (int)loop_req - 1 : 0;
            if (loop_req == 0)  // the resident grid where instantiated and big enough, stages on separate waves first
                for (int i = 0; i < kNumPair; i++)
                    if (kPairCfgs[i].persist && serves(kPairCfgs[i]) && tiles_at(kPairCfgs[i].th) >= 8 * 256)
                        persist = std::max(persist, kPairCfgs[i].persist);
            int wm = wm_req ? (int)wm_req : 2;
            if (!wm_req)
                for (int i = 0; i < kNumPair; i++)
                    if (kPairCfgs[i].persist == persist && serves(kPairCfgs[i]) && kPairCfgs[i].wm == 1) wm = 1;
            int best = -1;
            for (int i = 0; i < kNumPair; i++) {
                const PairCfg& c = kPairCfgs[i];
                if (!serves(c) || c.wm != wm || c.persist != persist) continue;
                if (th_req) {
                    best = i;
                    continue;
                }
                const int cur = best < 0 ? 0 : kPairCfgs[best].th;
                const bool fills = tiles_at(c.th) >= 256, cur_fills = best >= 0 && tiles_at(cur) >= 256;
                if (best < 0 || (fills && (!cur_fills || c.th > cur)) || (!fills && !cur_fills && c.th < cur)) best = i;
            }
            return best;
        };
        int idx = -1, cpa = 32;
        if (!tap32 && !film)
            for (int cp : {8, 16})
                if (idx < 0 && (int)A.cin <= cp && (idx = select(cp)) >= 0) cpa = cp;
        if (idx < 0) idx = select(32);
        if (idx < 0)
            return fail(-1, "fhc_conv_pair_plan_create: no fused pair instantiated for stride %u, %u -> %u -> %u "
                            "channels%s", A.stride, A.cin, A.cout, B.cout,
                        th_req || wm_req || loop_req ? " at that tile height, wave split and loop" : "");
        const PairCfg& c = kPairCfgs[idx];
        auto pa = std::make_unique<fhc_conv_plan>();
        auto pb = std::make_unique<fhc_conv_plan>();
        hipError_t e = hipGetDevice(&pa->device);
        if (e != hipSuccess) return fail(-1, "fhc_conv_pair_plan_create: hipGetDevice: %s", hipGetErrorString(e));
        pb->device = pa->device;
        e = pair_part(*pb, B, cb32, nbb, w_b, bias_b, slope_b);
        if (e == hipSuccess) e = pair_part(*pa, A, ca32, nba, w_a, bias_a, slope_a, cpa);
        if (e != hipSuccess) {
            if (pa->dmem) (void)hipFree(pa->dmem);
            if (pb->dmem) (void)hipFree(pb->dmem);
            return fail(-1, "fhc_conv_pair_plan_create: device upload: %s", hipGetErrorString(e));
        }
        const uint32_t tiles_x = div_ceil(wa, kPairTileW), tiles_y = div_ceil(ha, (uint32_t)c.th);
        pb->args.tiles_x = (int)tiles_x;
        pb->args.tiles_y = (int)tiles_y;
        pb->args.post = post ? 1 : 0;
        pa->family = 2;
        pa->cfg = idx;
        pa->code = 0;
        pa->tiles = (uint32_t)((uint64_t)A.n * tiles_y * tiles_x);
        pa->grid = dim3(pa->tiles, 1, 1);
        pa->threads = c.persist == 2 ? 64u * (uint32_t)(c.nba + c.nbb)
                                     : 64u * (uint32_t)std::max(c.nba, c.nbb) * (uint32_t)c.wm;
        if (c.persist) {
            // the resident grid: as many workgroups as fit at once. The kernel is compiled for 2 waves per SIMD
            // (kPairResidentWaves per CU); the LDS per CU bounds it too. (The runtime's occupancy query counts
            // only the LDS limit for these kernels and over-reports.)
            const void* k = nullptr;
            pair_launcher(idx, &k);
            hipFuncAttributes fa{};
            int cus = 0, lds_cu = 0;
            if (!k || hipFuncGetAttributes(&fa, k) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, pa->device) != hipSuccess ||
                hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, pa->device) !=
                    hipSuccess) {
                (void)hipFree(pa->dmem);
                (void)hipFree(pb->dmem);
                return fail(-1, "fhc_conv_pair_plan_create: kernel attribute query failed");
            }
            const int waves = (int)pa->threads / 64;
            int per_cu = std::max(1, kPairResidentWaves / waves);
            if (fa.sharedSizeBytes > 0) per_cu = std::min(per_cu, std::max(1, lds_cu / (int)fa.sharedSizeBytes));
            pa->grid.x = (unsigned)std::min<uint64_t>(pa->tiles, (uint64_t)per_cu * std::max(1, cus));
        }
        pa->lds = 0;
        pa->ws_bytes = 0;
        pa->launch = nullptr;
        pa->res_mid = res_mid ? 1 : 0;
        pa->film_in = film ? 1 : 0;
        pa->pair_launch = pair_launcher(idx);
        pa->pair_b = pb.release();
        *out = pa.release();
        clear_error();
        return 0;
    });
}

// ---- choice table -------------------------------------------------------------------------------------------

extern "C" int fhc_tune_parse(const char* text) {
    return guard(-1, [&]() -> int {
        if (!text) return fail(-1, "fhc_tune_parse: NULL text");
        // parse_tune (tune_cache.rs:71-87): "cin,cout,h,w,stride=code" per line (batch 1, 3x3), or
        // "cin,cout,h,w,stride,n,k=code"; malformed lines skipped; the value may also be a variant name
        std::istringstream in(text);
        std::string line;
        int n = 0;
        std::lock_guard<std::mutex> lk(g_tune_mu);
        while (std::getline(in, line)) {
            const size_t eq = line.find('=');
            if (eq == std::string::npos) continue;
            std::vector<uint32_t> f;
            std::istringstream ks(line.substr(0, eq));
            std::string part;
            bool ok = true;
            while (std::getline(ks, part, ',')) {
                const size_t a = part.find_first_not_of(" \t\r"), b = part.find_last_not_of(" \t\r");
                if (a == std::string::npos) {
                    ok = false;
                    break;
                }
                const std::string v = part.substr(a, b - a + 1);
                if (v.find_first_not_of("0123456789") != std::string::npos || v.size() > 9) {
                    ok = false;
                    break;
                }
                f.push_back((uint32_t)std::stoul(v));
            }
            if (!ok || (f.size() != 5 && f.size() != 7)) continue;
            if (f.size() == 5) {
                f.push_back(1);
                f.push_back(3);
            }
            if (f[5] == 0 || (f[6] != 1 && f[6] != 3)) continue;
            std::string v = line.substr(eq + 1);
            const size_t a = v.find_first_not_of(" \t\r"), b = v.find_last_not_of(" \t\r");
            if (a == std::string::npos) continue;
            v = v.substr(a, b - a + 1);
            uint32_t code = 0;
            if (!v.empty() && v.size() <= 3 && v.find_first_not_of("0123456789") == std::string::npos) {
                const unsigned long c = std::stoul(v);
                if (c >= kCodeEnd) continue;
                code = (uint32_t)c;
            } else {
                // an MI355X variant name ("direct.c64.t1x2.n48"): stable across builds, unlike the code it maps to
                for (uint32_t c = 1; c < kCodeEnd && !code; c++)
                    if (code_name(c) == v) code = c;
                if (!code) continue;
            }
            g_tune[TuneKey(f[0], f[1], f[2], f[3], f[4], f[5], f[6])] = code;
            n++;
        }
        return n;
    });
}

extern "C" int fhc_tune_format(char* text, size_t cap) {
    return guard(-1, [&]() -> int {
        // format_tune (tune_cache.rs:88-94): lines sorted as strings, joined by newlines; batch 1 of a 3x3 conv in
        // the reference's 5 fields, other keys with n and k appended
        std::vector<std::string> lines;
        {
            std::lock_guard<std::mutex> lk(g_tune_mu);
            for (const auto& kv : g_tune) {
                const TuneKey& k = kv.first;
                std::string line = std::to_string(std::get<0>(k)) + "," + std::to_string(std::get<1>(k)) + "," +
                                   std::to_string(std::get<2>(k)) + "," + std::to_string(std::get<3>(k)) + "," +
                                   std::to_string(std::get<4>(k));
                if (std::get<5>(k) != 1 || std::get<6>(k) != 3)
                    line += "," + std::to_string(std::get<5>(k)) + "," + std::to_string(std::get<6>(k));
                lines.push_back(line + "=" + std::to_string(kv.second));
            }
        }
        std::sort(lines.begin(), lines.end());
        std::string s;
        for (size_t i = 0; i < lines.size(); i++) s += (i ? "\n" : "") + lines[i];
        return write_string(s, text, cap);
    });
}

extern "C" int fhc_tune_clear(void) {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    g_tune.clear();
    return 0;
}

extern "C" int fhc_tune_get(uint32_t cin, uint32_t cout, uint32_t h, uint32_t w, uint32_t stride) {
    return fhc_tune_get_ex(cin, cout, h, w, stride, 1, 3);
}

extern "C" int fhc_tune_get_ex(uint32_t cin, uint32_t cout, uint32_t h, uint32_t w, uint32_t stride, uint32_t n,
                               uint32_t k) {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    auto it = g_tune.find(TuneKey(cin, cout, h, w, stride, n, k));
    return it == g_tune.end() ? -1 : (int)it->second;
}

extern "C" int fhc_variant_name(uint32_t code, char* buf, size_t cap) {
    return guard(-1, [&]() -> int {
        const std::string s = code_name(code);
        if (s.empty()) return fail(-1, "fhc_variant_name: unknown variant %u", code);
        return write_string(s, buf, cap);
    });
}

extern "C" int fhc_variant_list(const fhc_conv_desc* desc, uint32_t* codes, size_t cap) {
    return guard(-1, [&]() -> int {
        if (!desc) return fail(-1, "fhc_variant_list: NULL descriptor");
        fhc_conv_desc d = *desc;
        if (d.x_cstride == 0) d.x_cstride = d.cin;
        if (d.y_cstride == 0) d.y_cstride = d.cout;
        if (d.r_cstride == 0) d.r_cstride = d.cout;
        std::string why;
        if (!valid_desc(d, &why)) return fail(-1, "fhc_variant_list: %s", why.c_str());
        fhc_conv_plan p{};
        p.d = d;
        p.g.hout = (d.h + 2 * d.pad - d.kh) / d.stride + 1;
        p.g.wout = (d.w + 2 * d.pad - d.kw) / d.stride + 1;
        p.g.taps = d.kh * d.kw;
        p.g.cin8 = div_ceil(d.cin, 8) * 8;
        // the direct kernel at every channel-tile width that is instantiated for this input and not mostly padding;
        // every chunked configuration that fits, without split, and with global splits where the tile grid is
        // small (the counterpart of cand_list's split-K variants, candidates.rs:52-57)
        std::vector<uint32_t> out;
        for (int i = 0; i < kNumDirect; i++) {
            if (!direct_fits(d, i)) continue;
            const int width = kDirectCfgs[i].na * kDirectCfgs[i].wn;  // 16-channel blocks per channel tile
            if (16u * width >= 2 * div_ceil(d.cout, 16) * 16 && width > 1) continue;
            if (configure_direct(p, i, &why)) out.push_back(p.code);
        }
        // the deep-layer kernel where the channels fill its tile and the input is too deep for the direct kernel's
        // registers or the work is large (at least 64 input channels)
        for (int i = 0; i < kNumGemm && d.kh == 3 && d.cin >= 64; i++) {
            const GemmCfg& c = kGemmCfgs[i];
            const uint32_t bn = (uint32_t)(16 * c.na * c.wn);
            if (bn >= 2 * div_ceil(d.cout, 16) * 16 && bn > 32) continue;  // mostly padding
            for (uint32_t ks : {1u, 2u, 4u, 8u}) {
                if (!configure_gemm(p, i, ks, &why)) continue;
                if (p.ksplit != ks) continue;
                if (ks > 1 && (uint64_t)p.grid.x * p.grid.y >= 512) continue;
                out.push_back(p.code);
            }
        }
        for (int cfg = 1; cfg <= kNumCfg; cfg++) {
            const TileCfg& t = kTileCfgs[cfg];
            const uint32_t bn = (uint32_t)(t.fn * 16 * t.wn);
            if (bn >= 2 * div_ceil(d.cout, 16) * 16 && bn > 16) continue;  // mostly padding
            for (uint32_t ks : {1u, 2u, 4u, 8u}) {
                if (!configure_igemm(p, cfg, ks, &why)) continue;
                if (p.ksplit != ks) continue;
                if (ks > 1 && p.grid.x >= 512) continue;
                out.push_back(p.code);
            }
        }
        if (!codes && cap) return fail(-1, "fhc_variant_list: NULL output");
        if (out.size() > cap) return fail(-1, "fhc_variant_list: %zu variants do not fit in %zu", out.size(), cap);
        for (size_t i = 0; i < out.size(); i++) codes[i] = out[i];
        return (int)out.size();
    });
}

extern "C" int fhc_conv_autotune(const fhc_conv_desc* desc, const uint16_t* w_oihw, const uint16_t* bias,
                                 const uint16_t* slope, const void* x, void* y, const void* res, int reps,
                                 float* best_us) {
    return guard(-1, [&]() -> int {
        if (!desc || !w_oihw || !bias || !x || !y) return fail(-1, "fhc_conv_autotune: NULL argument");
        if (desc->residual && !res) return fail(-1, "fhc_conv_autotune: the conv has a residual but res is NULL");
        if (reps < 1 || reps > 10000) return fail(-1, "fhc_conv_autotune: reps must be in 1..10000");
        std::vector<uint32_t> codes(256);
        const int n = fhc_variant_list(desc, codes.data(), codes.size());
        if (n < 0) return -1;
        hipStream_t s = nullptr;
        if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess)
            return fail(-1, "fhc_conv_autotune: stream creation failed");
        hipEvent_t e0 = nullptr, e1 = nullptr;
        (void)hipEventCreate(&e0);
        (void)hipEventCreate(&e1);
        float best = 0.0f;
        int best_code = -1;
        std::string err;
        for (int i = 0; i < n && err.empty(); i++) {
            fhc_conv_desc d = *desc;
            d.variant = codes[i];
            d.ksplit = 0;
            d.ref_cand = 0xFF;
            fhc_conv_plan* p = nullptr;
            if (fhc_conv_plan_create(&d, w_oihw, bias, slope, &p) != 0) continue;  // not servable: skip
            void* ws = nullptr;
            if (p->ws_bytes && hipMalloc(&ws, p->ws_bytes) != hipSuccess) {
                fhc_conv_plan_destroy(p);
                continue;
            }
            hipGraph_t g = nullptr;
            hipGraphExec_t ge = nullptr;
            bool ok = fhc_conv_run(p, x, y, res, ws, s) == 0 && hipStreamSynchronize(s) == hipSuccess;
            ok = ok && hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) == hipSuccess;
            if (ok) {
                for (int r = 0; r < reps && ok; r++) ok = fhc_conv_run(p, x, y, res, ws, s) == 0;
                ok = hipStreamEndCapture(s, &g) == hipSuccess && ok;
            }
            ok = ok && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) == hipSuccess;
            ok = ok && hipGraphLaunch(ge, s) == hipSuccess;  // warm
            float ms = 0.0f;
            ok = ok && hipEventRecord(e0, s) == hipSuccess && hipGraphLaunch(ge, s) == hipSuccess &&
                 hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
                 hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
            if (ge) (void)hipGraphExecDestroy(ge);
            if (g) (void)hipGraphDestroy(g);
            if (ws) (void)hipFree(ws);
            fhc_conv_plan_destroy(p);
            if (!ok) {
                err = std::string("timing variant ") + code_name(codes[i]) + " failed: " + fhc_last_error();
                break;
            }
            const float us = ms * 1000.0f / (float)reps;
            if (best_code < 0 || us < best) {
                best = us;
                best_code = (int)codes[i];
            }
        }
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        (void)hipStreamDestroy(s);
        if (!err.empty()) return fail(-1, "fhc_conv_autotune: %s", err.c_str());
        if (best_code < 0) return fail(-1, "fhc_conv_autotune: no variant could be planned");
        {
            std::lock_guard<std::mutex> lk(g_tune_mu);
            g_tune[tune_key(*desc)] = (uint32_t)best_code;
        }
        if (best_us) *best_us = best;
        clear_error();
        return best_code;
    });
}

extern "C" int fhc_probe_mfma_rate(uint32_t blocks, uint32_t iters, void* out, void* stream) {
    return guard(-1, [&]() -> int {
        if (!out) return fail(-1, "fhc_probe_mfma_rate: NULL output");
        if (blocks == 0 || blocks > 65535 || iters == 0 || iters > (1u << 24))
            return fail(-1, "fhc_probe_mfma_rate: blocks must be 1..65535 and iters 1..2^24");
        hipError_t e = mfma_rate_probe_launch(blocks, (int)iters, static_cast<float*>(out),
                                              static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return fail(-1, "fhc_probe_mfma_rate: %s", hipGetErrorString(e));
        return 0;
    });
}

extern "C" int fhc_probe_mfma_layout(const void* a, const void* b, void* d, void* stream) {
    return guard(-1, [&]() -> int {
        if (!a || !b || !d) return fail(-1, "fhc_probe_mfma_layout: NULL pointer");
        hipError_t e = mfma_probe_launch(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                                         static_cast<float*>(d), static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return fail(-1, "fhc_probe_mfma_layout: %s", hipGetErrorString(e));
        return 0;
    });
}

// ---- the run entry point that allocates nothing ------------------------------------------------------------
// fhc_conv_run_noalloc takes the plan's scratch (the split-K partials) from a file-scope device array instead of a
// caller workspace. Each device holds its own copy of the array, at its own address; host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol), but the address
// hipGetSymbolAddress gives with that device current, looked up once per device and kept here.
namespace fhc {
namespace {
constexpr size_t kStaticScratchBytes = FHC_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
__device__ __align__(256) float scratch[kStaticScratchBytes / sizeof(float)];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// the scratch array's device address on `dev` (the current device), or nullptr with the last error set
void* static_scratch(int dev) {
    if (dev < 0 || dev >= kMaxDevices) {
        fail(-1, "fhc_conv_run_noalloc: device %d is beyond the %d the library keeps scratch for", dev, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            fail(-1, "fhc_conv_run_noalloc: hipGetSymbolAddress of the scratch array: %s", hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}
}  // namespace
}  // namespace fhc

extern "C" int fhc_conv_run_noalloc(const fhc_conv_plan* p, const void* x, void* y, const void* res, void* stream) {
    return guard(-1, [&]() -> int {
        if (!p) return fail(-1, "fhc_conv_run_noalloc: NULL plan");
        if (p->ws_bytes > kStaticScratchBytes)
            return fail(-1, "fhc_conv_run_noalloc: the plan needs %zu bytes of scratch, the static scratch holds %zu "
                            "(use fhc_conv_run with a workspace, or a smaller split-K)",
                        p->ws_bytes, kStaticScratchBytes);
        void* ws = nullptr;
        if (p->ws_bytes) {
            int dev = -1;
            if (hipGetDevice(&dev) != hipSuccess || dev != p->device)
                return fail(-1, "fhc_conv_run_noalloc: the plan belongs to device %d, the current device is %d",
                            p->device, dev);
            ws = static_scratch(dev);
            if (!ws) return -1;
        }
        return fhc_conv_run(p, x, y, res, ws, stream);
    });
}

extern "C" int fhc_conv_sibling_plan_create(const fhc_conv_desc* desc_a, const uint16_t* w_a, const uint16_t* bias_a,
                                            const uint16_t* slope_a, const fhc_conv_desc* desc_b,
                                            const uint16_t* w_b, const uint16_t* bias_b, const uint16_t* slope_b,
                                            fhc_conv_plan** out) {
    return guard(-1, [&]() -> int {
        const char* who = "fhc_conv_sibling_plan_create";
        if (!out) return fail(-1, "%s: NULL output handle", who);
        *out = nullptr;
        if (!desc_a || !desc_b) return fail(-1, "%s: NULL descriptor", who);
        if (!w_a || !bias_a || !w_b || !bias_b) return fail(-1, "%s: NULL weights or bias", who);
        fhc_conv_desc A = *desc_a, B = *desc_b;
        for (fhc_conv_desc* d : {&A, &B}) {
            if (d->x_cstride == 0) d->x_cstride = d->cin;
            if (d->y_cstride == 0) d->y_cstride = d->cout;
            if (d->r_cstride == 0) d->r_cstride = d->cout;
        }
        std::string why;
        if (!valid_desc(A, &why)) return fail(-1, "%s: first conv: %s", who, why.c_str());
        if (!valid_desc(B, &why)) return fail(-1, "%s: second conv: %s", who, why.c_str());
        if (A.n != B.n || A.h != B.h || A.w != B.w || A.cin != B.cin || A.kh != B.kh || A.kw != B.kw ||
            A.stride != B.stride || A.pad != B.pad || A.x_cstride != B.x_cstride || A.x_c0 != B.x_c0)
            return fail(-1, "%s: the two convs must read the same input view with the same geometry", who);
        if (B.residual) return fail(-1, "%s: the second conv cannot take a residual", who);
        if (A.act == FHC_ACT_LEAKY || B.act == FHC_ACT_LEAKY)
            return fail(-1, "%s: identity or PReLU activations only", who);
        if ((A.act == FHC_ACT_PRELU && !slope_a) || (B.act == FHC_ACT_PRELU && !slope_b))
            return fail(-1, "%s: PReLU needs a slope", who);
        // the combined conv: A's channels, zero channels up to a multiple of 4, B's. Its K order per output channel
        // is the kernel-row split's or the plain chain's: the one the planner gives both convs alone when it gives
        // both a direct configuration with the same split (the outputs are then bit-identical), else the split's
        const uint32_t split = (A.cout + 3) & ~3u, total = split + B.cout, cin32 = div_ceil(A.cin, 32) * 32;
        int wk = 3;
        {
            fhc_conv_plan pa{}, pb{};
            std::string w1, w2;
            if (plan_choose(A, pa, &w1) && plan_choose(B, pb, &w2) && pa.family == 1 && pb.family == 1 &&
                kDirectCfgs[pa.cfg].na == 1 && kDirectCfgs[pb.cfg].na == 1 &&
                kDirectCfgs[pa.cfg].wk == kDirectCfgs[pb.cfg].wk && kDirectCfgs[pa.cfg].cin32 == (int)cin32 &&
                kDirectCfgs[pb.cfg].cin32 == (int)cin32)
                wk = kDirectCfgs[pa.cfg].wk;
        }
        int idx = -1;
        for (int i = 0; i < kNumDirect; i++) {
            const DirectCfg& c = kDirectCfgs[i];
            if (c.ks == (int)A.kh && c.stride == (int)A.stride && c.cin32 == (int)cin32 && c.na == 1 && c.wk == wk &&
                !c.persist && 16u * c.wn >= total && sibling_launcher(i) && (idx < 0 || c.wn < kDirectCfgs[idx].wn))
                idx = i;
        }
        if (idx < 0)
            return fail(-1, "%s: no sibling kernel for %u -> %u + %u channels (3x3 stride 1, 33-64 input channels, at "
                            "most 48 output channels with the first conv's padded to 4)", who, A.cin, A.cout, B.cout);
        fhc_conv_desc C = A;
        C.cout = total;
        C.act = A.act == FHC_ACT_PRELU || B.act == FHC_ACT_PRELU ? FHC_ACT_PRELU : FHC_ACT_NONE;
        C.variant = 0;
        C.ksplit = 0;
        auto p = std::make_unique<fhc_conv_plan>();
        p->d = C;  // A's output and residual views: the kernel stores A's channels through them, B's through y2
        p->dmem = nullptr;
        p->g.hout = (C.h + 2 * C.pad - C.kh) / C.stride + 1;
        p->g.wout = (C.w + 2 * C.pad - C.kw) / C.stride + 1;
        p->g.taps = C.kh * C.kw;
        p->g.cin8 = div_ceil(C.cin, 8) * 8;
        if (!configure_direct(*p, idx, &why)) return fail(-1, "%s: %s", who, why.c_str());
        p->launch = sibling_launcher(idx);
        p->args.split = (int)split;
        p->args.cout1 = (int)A.cout;
        p->args.y2cs = (int)B.y_cstride;
        p->args.y2c0 = (int)B.y_c0;
        hipError_t e = hipGetDevice(&p->device);
        if (e != hipSuccess) return fail(-1, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
        const size_t kk = (size_t)A.cin * A.kh * A.kw;
        std::vector<uint16_t> w(total * kk, 0), b(total, 0), sl(total, 0x3c00);  // slope 1: no activation
        memcpy(w.data(), w_a, A.cout * kk * 2);
        memcpy(w.data() + split * kk, w_b, B.cout * kk * 2);
        memcpy(b.data(), bias_a, A.cout * 2);
        memcpy(b.data() + split, bias_b, B.cout * 2);
        if (A.act == FHC_ACT_PRELU) memcpy(sl.data(), slope_a, A.cout * 2);
        if (B.act == FHC_ACT_PRELU) memcpy(sl.data() + split, slope_b, B.cout * 2);
        std::vector<uint16_t> packed;
        pack_weights(*p, w.data(), packed);
        e = upload(*p, packed, b.data(), sl.data());
        if (e != hipSuccess) {
            if (p->dmem) (void)hipFree(p->dmem);
            return fail(-1, "%s: device upload: %s", who, hipGetErrorString(e));
        }
        *out = p.release();
        clear_error();
        return 0;
    });
}

extern "C" int fhc_conv_sibling_run(const fhc_conv_plan* p, const void* x, void* y_a, const void* res_a, void* y_b,
                                    void* stream) {
    return guard(-1, [&]() -> int {
        const char* who = "fhc_conv_sibling_run";
        if (!p) return fail(-1, "%s: NULL plan", who);
        if (!p->args.split) return fail(-1, "%s: not a sibling plan", who);
        if (!x || !y_a || !y_b) return fail(-1, "%s: NULL input or output", who);
        if (p->d.residual && !res_a) return fail(-1, "%s: the first conv has a residual but res_a is NULL", who);
        if (((uintptr_t)x | (uintptr_t)y_a | (uintptr_t)res_a | (uintptr_t)y_b) & 1u)
            return fail(-1, "%s: f16 tensors must be 2-byte aligned", who);
        int dev = -1;
        if (hipGetDevice(&dev) != hipSuccess || dev != p->device)
            return fail(-1, "%s: the plan belongs to device %d, the current device is %d", who, p->device, dev);
        ConvKArgs a = p->args;
        a.x = static_cast<const uint16_t*>(x);
        a.y = static_cast<uint16_t*>(y_a);
        a.res = static_cast<const uint16_t*>(res_a);
        a.y2 = static_cast<uint16_t*>(y_b);
        a.xvec = ((uintptr_t)x % 16 == 0) && a.xcs % 8 == 0 && a.xc0 % 8 == 0;
        a.yvec = ((uintptr_t)y_a % 8 == 0) && a.ycs % 4 == 0 && a.yc0 % 4 == 0;
        a.y2vec = ((uintptr_t)y_b % 8 == 0) && a.y2cs % 4 == 0 && a.y2c0 % 4 == 0;
        a.rvec = a.residual && ((uintptr_t)res_a % 8 == 0) && a.rcs % 4 == 0 && a.rc0 % 4 == 0 && a.cout1 % 4 == 0;
        const hipError_t e = p->launch(a, p->grid, p->lds, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return fail(-1, "%s: launch: %s", who, hipGetErrorString(e));
        return 0;
    });
}

extern "C" int fhc_gmhs_film(const fhc_tensor* a, const fhc_tensor* b, uint32_t h, uint32_t w,
                             const fhc_tensor* flow, uint32_t h8, uint32_t w8, uint32_t full_w, uint32_t level,
                             void* ws, size_t ws_bytes, const fhc_conv_plan* pair, const void* pair_x,
                             const void* pair_film, void* pair_y, const fhc_conv_plan* conv, const void* conv_x,
                             void* conv_y, void* stream) {
    return guard(-1, [&]() -> int {
        const char* who = "fhc_gmhs_film";
        if (!pair) return fail(-1, "%s: NULL pair plan", who);
        if (pair->family != 2 || !pair->film_in)
            return fail(-1, "%s: not a pair plan created with FHC_PAIR_FILM_IN", who);
        const FitPairLaunchFn fn = fit_pair_launcher(pair->cfg);
        if (!fn)
            return fail(-1, "%s: no launch of the fit beside this pair's configuration (one tile per workgroup, 3 + 3 "
                            "channel blocks, one wave row)", who);
        if (!pair_x || !pair_y || !pair_film) return fail(-1, "%s: NULL pair input, output or FiLM vectors", who);
        if (((uintptr_t)pair_x | (uintptr_t)pair_y | (uintptr_t)pair_film) & 1u)
            return fail(-1, "%s: f16 tensors must be 2-byte aligned", who);
        int dev = -1;
        if (hipGetDevice(&dev) != hipSuccess || dev != pair->device)
            return fail(-1, "%s: the plan belongs to device %d, the current device is %d", who, pair->device, dev);
        GmCoRun co{fn, pair_args(pair, pair_x, pair_y, nullptr, pair_film), pair->tiles, nullptr, {}, dim3()};
        if (conv) {
            if (!conv_x || !conv_y) return fail(-1, "%s: NULL conv input or output", who);
            if (conv->family != 1 || conv->args.split || conv->d.residual || conv->ws_bytes || conv->device != dev)
                return fail(-1, "%s: the conv must be a one-launch direct plan without residual on this device", who);
            if (((uintptr_t)conv_x | (uintptr_t)conv_y) & 1u)
                return fail(-1, "%s: f16 tensors must be 2-byte aligned", who);
            co.cfn = fit_conv_launcher(conv->cfg);  // null: the conv runs in its own launch after the repair
            ConvKArgs& ca = co.ca;
            ca = conv->args;
            ca.x = static_cast<const uint16_t*>(conv_x);
            ca.y = static_cast<uint16_t*>(conv_y);
            ca.res = nullptr;
            ca.xvec = ((uintptr_t)conv_x % 16 == 0) && ca.xcs % 8 == 0 && ca.xc0 % 8 == 0;
            ca.yvec = ((uintptr_t)conv_y % 8 == 0) && ca.ycs % 4 == 0 && ca.yc0 % 4 == 0;
            ca.rvec = 0;
            co.cgrid = conv->grid;
        }
        if (level == 0) {  // no repair: the pair, then the conv
            const int rc = run_pair(pair, pair_x, pair_y, nullptr, pair_film, stream, who);
            return rc || !conv ? rc : fhc_conv_run(conv, conv_x, conv_y, nullptr, nullptr, stream);
        }
        const int rc = gmhs_run(a, b, h, w, flow, h8, w8, full_w, level, ws, ws_bytes, &co, stream);
        if (rc || !conv || co.cfn) return rc;
        return fhc_conv_run(conv, conv_x, conv_y, nullptr, nullptr, stream);  // no fused launch for its configuration
    });
}
