// Device-side contract of the conv kernels: the argument block every launch takes, the tile configurations the
// planner can choose from, and the launcher table. Shared by conv_kernels.hip (kernels) and api.cpp (host).
#pragma once
#include <cstddef>
#include <cstdint>

#include <hip/hip_runtime.h>

namespace fhc {

// One conv launch. Activations NHWC f16: element (img, y, x, c) of a view at ((img*H + y)*W + x)*cs + c0 + c.
struct ConvKArgs {
    const uint16_t* x;
    uint16_t* y;
    const uint16_t* res;
    const void* wpk;        // packed weights, MFMA A-fragment order: [nb16][chunk][kstep][lane 64][8 halves]
    const uint16_t* bias;   // f16, padded to np
    const float* neg;       // f32 multiplier of negative values, padded to np: the PReLU slope (exact in f32), the
                            // LeakyReLU alpha, or 1 without activation; 16-byte aligned
    float* part;            // split-K partials [z][n*hout*wout][np] f32 (global split only)
    int n, h, w, cin, cout, hout, wout, pad;
    int xcs, xc0, ycs, yc0, rcs, rc0;
    int act;
    float alpha;
    int residual;
    int cc;         // input channels staged per chunk (multiple of 8)
    int nchunks;    // ceil(cin8 / cc)
    int ksteps;     // MFMA K-steps (of 32) per chunk = ceil(taps * cc / 32)
    int tapgroups;  // 8-channel groups per chunk = taps * cc / 8
    int tiles_x, tiles_y, ntn;  // output tiles: columns of 16, rows of TH, channel tiles of BN
    int chunks_per_split;       // global split-K: chunks handled by one z
    int np;                     // output channels padded to ntn * BN
    int xvec, yvec, rvec;       // vector paths: 16-byte input loads, 8-byte output stores / residual loads
                                // (rvec also needs cout % 4 == 0)
    int post;                   // 1: the f16 output goes through affine_out, 2 / (1 + exp(-v)) - 1, rounded again
                                // (the one-tile pair kernel's second conv, cout <= 4, no residual)
    const uint16_t* film;       // the one-tile pair kernel's first conv: FiLM vectors [n][gamma cin | beta cin]
                                // (f16) applied to the input as it is staged, or null
    // sibling convs (two convs of one input in one launch, the one-tile direct kernel's SPLIT form): output channels
    // below `split` belong to the first conv (its cout1 of them stored through y with the residual), the rest to the
    // second, stored through y2 at channel co - split without residual
    int split, cout1;
    uint16_t* y2;
    int y2cs, y2c0, y2vec;
};

// A tile configuration: wave grid WM x WN x WK (WK > 1 splits K inside the workgroup), each wave FM output rows
// of 16 pixels by FN blocks of 16 channels. TH = FM * WM output rows per tile, BN = FN * 16 * WN channels.
struct TileCfg {
    int fm, fn, wm, wn, wk;
};

// Configuration ids 1..kNumCfg (0 is "none"); the table is the same on host and device side.
constexpr int kNumCfg = 10;
inline constexpr TileCfg kTileCfgs[kNumCfg + 1] = {
    {0, 0, 0, 0, 0},
    {2, 4, 4, 1, 1},  // 1: TH 8, BN 64
    {2, 2, 4, 1, 1},  // 2: TH 8, BN 32
    {2, 1, 4, 1, 1},  // 3: TH 8, BN 16
    {1, 4, 4, 1, 1},  // 4: TH 4, BN 64
    {1, 2, 4, 1, 1},  // 5: TH 4, BN 32
    {4, 4, 2, 2, 1},  // 6: TH 8, BN 128
    {4, 4, 1, 1, 4},  // 7: TH 4, BN 64, K split over 4 waves
    {2, 4, 2, 1, 2},  // 8: TH 4, BN 64, K split over 2 waves
    {2, 3, 4, 1, 1},  // 9: TH 8, BN 48
    {1, 1, 4, 1, 1},  // 10: TH 4, BN 16
};

using LaunchFn = hipError_t (*)(const ConvKArgs&, dim3 grid, size_t lds, hipStream_t);
// the SPLIT (sibling convs) launcher of direct configuration `index`, or null where it is not instantiated
LaunchFn sibling_launcher(int index);

// The launcher of configuration `cfg` for a (kernel size, stride) pair, or nullptr if not instantiated.
LaunchFn conv_launcher(int ks, int stride, int cfg);
// The launcher of the direct kernel's configuration `index` (direct_table.h), or nullptr; *kernel receives the
// kernel's address (for occupancy queries; persistent configurations have a variant per `residual`) when not null.
LaunchFn direct_launcher(int index, const void** kernel, bool residual = false);
hipError_t splitk_reduce_launch(const ConvKArgs& a, int ksplit, hipStream_t s);

// The deep-layer conv (gemm_impl.h, 3x3 only): stride S, chunks of CK input channels through LDS in a ring of ST
// buffers, waves WM x WN of FM rows x NA channel blocks each; TH = FM * WM rows x 16 columns x BN = 16 * NA * WN
// channels per workgroup. The 2-wave configurations fit two workgroups per CU.
struct GemmCfg {
    int s, ck, fm, na, wm, wn, st;
};
constexpr int kNumGemm = 14;
inline constexpr GemmCfg kGemmCfgs[kNumGemm] = {
    {1, 32, 4, 2, 2, 2, 3},  // 0: TH 8, BN 64, 4 waves
    {1, 32, 2, 2, 4, 2, 2},  // 1: TH 8, BN 64, 8 waves
    {1, 32, 4, 2, 2, 1, 2},  // 2: TH 8, BN 32, 2 waves
    {1, 32, 2, 2, 2, 2, 3},  // 3: TH 4, BN 64, 4 waves
    {1, 32, 4, 3, 2, 2, 2},  // 4: TH 8, BN 96, 4 waves
    {1, 32, 2, 3, 2, 2, 2},  // 5: TH 4, BN 96, 4 waves
    {1, 32, 4, 2, 4, 1, 3},  // 6: TH 16, BN 32, 4 waves
    {1, 32, 2, 3, 4, 1, 3},  // 7: TH 8, BN 48, 4 waves
    {1, 32, 2, 2, 2, 1, 2},  // 8: TH 4, BN 32, 2 waves
    {1, 32, 2, 3, 2, 1, 2},  // 9: TH 4, BN 48, 2 waves
    {1, 64, 2, 2, 4, 1, 2},  // 10: TH 8, BN 32, 4 waves, 64-channel chunks
    {1, 32, 2, 3, 4, 1, 2},  // 11: as 7 with two buffers
    {1, 32, 4, 2, 2, 2, 2},  // 12: as 0 with two buffers
    // 4 rows x 3 channel blocks a wave: 12 accumulators, each LDS operand read feeding 4 MFMAs (weights) or up to
    // 9 (halo rows); measured fastest where the image batch is large and cin is a few K-chunks (155 -> 48 at
    // 8 x 60 x 108)
    {1, 32, 4, 3, 4, 1, 2},  // 13: TH 16, BN 48, 4 waves
};
// The launcher of the deep-layer configuration `index`, or nullptr; *kernel receives the kernel's address.
LaunchFn gemm_launcher(int index, const void** kernel);

// A fused pair of 3x3 convs (pair_impl.h): B (stride 1) reads A's output, which stays in LDS.
struct PairKArgs {
    ConvKArgs a, b;  // a: x, A's weights, bias, multipliers, input geometry; b: y, res, B's weights, output geometry
    int res_mid;     // B's residual is A's output
};
constexpr int kPairTileW = 14;  // output columns per tile (B's 16-pixel MFMA block reads 16 + 2 columns of A)
// The instantiated pairs: A's stride, A's and B's input channels padded to 32, A's and B's output channel blocks
// of 16, the output rows per tile, the wave rows that split them, and the loop: 0 one workgroup per tile (weights
// loaded per tile: small frames), 1 a resident grid looping over tiles (weights loaded once: large tensors), 2 a
// resident grid whose A and B stages run on separate waves, pipelined across tiles (one wave row). cpa: A's input
// channels per tap in its K-steps, 0 (32: one tap per 32-wide step) or 8 / 16 (at most that many input channels:
// 4 or 2 taps packed into each step, 3 or 5 steps where one tap a step takes 9).
struct PairCfg {
    int sa, ca32, cb32, nba, nbb, th, wm, persist, cpa;
};
constexpr int kNumPair = 44;
inline constexpr PairCfg kPairCfgs[kNumPair] = {
    // the encoder's stride-2 conv and its successor (3 -> 36 -> 36)
    {2, 32, 64, 3, 3, 2, 1, 0}, {2, 32, 64, 3, 3, 4, 1, 0}, {2, 32, 64, 3, 3, 2, 2, 0}, {2, 32, 64, 3, 3, 4, 2, 0},
    // 48 -> 48 -> 48 (FiLM head, fine block)
    {1, 64, 64, 3, 3, 2, 1, 0}, {1, 64, 64, 3, 3, 4, 1, 0}, {1, 64, 64, 3, 3, 2, 2, 0}, {1, 64, 64, 3, 3, 4, 2, 0},
    // <= 32 -> 32 -> 32 (refine head)
    {1, 32, 32, 2, 2, 2, 1, 0}, {1, 32, 32, 2, 2, 4, 1, 0}, {1, 32, 32, 2, 2, 2, 2, 0}, {1, 32, 32, 2, 2, 4, 2, 0},
    // <= 32 -> 32 -> 16 (refine head output)
    {1, 32, 32, 2, 1, 2, 1, 0}, {1, 32, 32, 2, 1, 4, 1, 0}, {1, 32, 32, 2, 1, 2, 2, 0}, {1, 32, 32, 2, 1, 4, 2, 0},
    // the encoder's second stride-2 conv and its successor (36 -> 72 -> 72)
    {2, 64, 96, 5, 5, 1, 1, 0}, {2, 64, 96, 5, 5, 2, 1, 0},
    // resident-grid loops (2 waves per SIMD): 64 -> 64 -> 64 (the 1080p/4 ladder), then the frame's pairs at batch
    // scale (with 64-channel weights only two wave rows fit the 256 registers; the 36 -> 72 -> 72 pair spills)
    {1, 64, 64, 4, 4, 4, 2, 1},
    {1, 64, 64, 3, 3, 4, 2, 1},
    {2, 32, 64, 3, 3, 4, 2, 1},
    {1, 32, 32, 2, 2, 4, 1, 1}, {1, 32, 32, 2, 2, 4, 2, 1}, {1, 32, 32, 2, 2, 8, 2, 1},
    {1, 32, 32, 2, 1, 4, 1, 1}, {1, 32, 32, 2, 1, 4, 2, 1}, {1, 32, 32, 2, 1, 8, 2, 1},
    // resident grids with the A and B stages on separate waves (at most 8 waves: 2 per SIMD)
    {1, 64, 64, 4, 4, 4, 1, 2},
    {1, 64, 64, 3, 3, 4, 1, 2},
    {2, 32, 64, 3, 3, 4, 1, 2},
    {1, 32, 32, 2, 2, 4, 1, 2}, {1, 32, 32, 2, 2, 8, 1, 2},
    {1, 32, 32, 2, 1, 4, 1, 2}, {1, 32, 32, 2, 1, 8, 1, 2},
    // taps packed into A's K-steps: the encoder's first pair (3 input channels, 8 per tap: 3 steps) and the refine
    // head's first pair (14 input channels, 16 per tap: 5 steps), in each loop
    {2, 32, 64, 3, 3, 2, 1, 0, 8}, {2, 32, 64, 3, 3, 4, 1, 0, 8}, {2, 32, 64, 3, 3, 4, 2, 1, 8},
    {2, 32, 64, 3, 3, 4, 1, 2, 8},
    {1, 32, 32, 2, 2, 2, 1, 0, 16}, {1, 32, 32, 2, 2, 4, 1, 0, 16}, {1, 32, 32, 2, 2, 4, 2, 1, 16},
    {1, 32, 32, 2, 2, 8, 2, 1, 16}, {1, 32, 32, 2, 2, 4, 1, 2, 16}, {1, 32, 32, 2, 2, 8, 1, 2, 16},
};
constexpr int kPairResidentWaves = 8;  // waves per CU of the resident-grid pair (2 per SIMD)
using PairLaunchFn = hipError_t (*)(const PairKArgs&, dim3 grid, hipStream_t);
// The launcher of pair configuration `index`, or nullptr; *kernel receives the (persistent) kernel's address.
PairLaunchFn pair_launcher(int index, const void** kernel = nullptr);

// One round of the repair's affine fit (gm_fit.h) and the tiles of a FiLM pair (FHC_PAIR_FILM_IN) in one launch of
// 192-thread workgroups: workgroups 0-127 run the fit (workgroup g of channel c at c * 32 + g), the rest the pair's
// tiles. The two touch none of each other's data; the fit's workgroups are few and latency-bound, so the pair's
// work fills the machine beside them.
struct FitRoundArgs {
    const uint16_t* flow;  // the E8 flow, channel c at flow[i * cs + c0 + c]
    uint32_t cs, c0, h8, w8;
    float delta;
    uint32_t round;
    const float* part_in;
    float* part_out;
};
using FitPairLaunchFn = hipError_t (*)(const FitRoundArgs&, const PairKArgs&, uint32_t pair_tiles, hipStream_t);
// the launcher for pair configuration `index` (one tile per workgroup, 3 + 3 channel blocks on one wave row: 192
// threads), or nullptr
FitPairLaunchFn fit_pair_launcher(int index);
// The same with a conv plan's workgroups (conv_tile, 192 threads: tile t, channel tile ct at t + tiles * ct)
using FitConvLaunchFn = hipError_t (*)(const FitRoundArgs&, const ConvKArgs&, dim3 conv_grid, hipStream_t);
// the launcher for direct configuration `index` (one tile per workgroup, 192 threads), or nullptr
FitConvLaunchFn fit_conv_launcher(int index);

// Fragment-layout probe: D(16x16 f32) = A(16x32 f16) x B(32x16 f16) through one v_mfma_f32_16x16x32_f16 with the
// operand layouts the conv kernels assume. Device pointers.
hipError_t mfma_probe_launch(const uint16_t* a, const uint16_t* b, float* d, hipStream_t s);
// The sustained MFMA rate probe: `blocks` workgroups of 4 waves, each wave kRateAcc * iters 16x16x32 f16 MFMAs
// (16384 FLOPs each); out holds blocks * 256 * 4 floats.
constexpr int kRateAcc = 16;
hipError_t mfma_rate_probe_launch(unsigned blocks, int iters, float* out, hipStream_t s);

}  // namespace fhc
