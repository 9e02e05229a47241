// The direct conv kernel for layers whose input channels fit one pass (cin padded to 32 <= 128, or 160/288 with
// the kernel-row K split WK = 3): the weights of a wave's 16 * NA output channels stay in registers for the whole
// launch, input tiles stream through a halo tile in LDS.
//
// Workgroup: WN x WM (x WK) waves; wave (wn, wm) owns output channels [16 NA wn, 16 NA (wn + 1)) of the
// workgroup's channel tile and FM output rows of 16 pixels. Every B operand read from LDS feeds the wave's NA
// channel blocks (NA MFMAs), which is what bounds the LDS read traffic (1 KB per NA MFMAs). Per spatial tile (TH = FM * WM rows x 16 columns) the workgroup writes the
// input halo ((TH-1)*S + KS) x (15*S + KS) x CIN32 into LDS (zero outside the image and beyond cin), then each
// wave runs KSTEPS = KS*KS*CIN32/32 MFMA K-steps reading its shifted windows from LDS. K order: k = tap * CIN32 + ci
// (channels padded to 32 per tap), so K-step s is tap s / M, channels 32 (s % M) .. +31 with M = CIN32 / 32, and
// lane group l/16 reads channels +8 (l/16): every LDS read is a per-row base register plus a compile-time offset.
// The weights were packed in the same order (api.cpp, pack_weights).
// One workgroup per spatial tile (blockIdx.x) and channel tile (blockIdx.y), or, PERSIST, no more workgroups than
// can be resident, each looping over spatial tiles with the next tile's halo loading while the current one
// computes. Every global load a tile needs (halo, residual; weights and bias once) is issued before its first
// wait, so a tile costs at most one memory round trip; the MFMA chain reads LDS one K-step ahead of the MFMAs.
#pragma once
#include <type_traits>

#ifndef FULL_WAIT_BEFORE_CHAIN
#define FULL_WAIT_BEFORE_CHAIN
#endif

#include "conv_kernels.h"

namespace fhc {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// The activation with the plan's multiplier of negative values m (PReLU slope, LeakyReLU alpha, or 1: m * t == t
// for t <= 0, signed zero included): t > 0 ? t : m * t, both sides computed and selected, without a branch.
__device__ __forceinline__ float activate(float t, float m) {
    const float n = m * t;
    return t > 0.0f ? t : n;
}

// bias, activation, f16 round, residual add rounded again (shaders/conv_tiled.wgsl:57-67), store of 4
// consecutive channels co..co+3 of output pixel `pix`. ng: the negative-value multipliers; rv: the residual's 4
// halves (ignored without residual).
__device__ __forceinline__ void epilogue4r(const ConvKArgs& a, size_t pix, int co, f4 v, const float* b,
                                          const float* ng, uint2 rv) {
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = f2h(activate(v[i] + b[i], ng[i]));
    if (a.residual) {
        const uint16_t r[4] = {(uint16_t)(rv.x & 0xffffu), (uint16_t)(rv.x >> 16), (uint16_t)(rv.y & 0xffffu),
                               (uint16_t)(rv.y >> 16)};
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = f2h(h2f(o[i]) + h2f(r[i]));
    }
    uint16_t* yp = a.y + pix * (size_t)a.ycs + a.yc0 + co;
    if (a.yvec && co + 4 <= a.cout) {
        uint2 q;
        q.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
        q.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
        *reinterpret_cast<uint2*>(yp) = q;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (co + i < a.cout) yp[i] = o[i];
    }
}

// the residual's 4 halves at (pix, co..co+3), zeros past cout. Branch-free: a lane outside the output (!valid)
// reads pixel 0, channel 0 of the view instead, so no load sits in divergent control flow (a load there forces a
// wait for every outstanding memory operation, stores included, where the branches join). rvec (8-byte aligned
// view, cout a multiple of 4): one 8-byte load; else 4 clamped 2-byte loads, whose zeroing waits for them.
__device__ __forceinline__ uint2 load_res4(const ConvKArgs& a, size_t pix, int co, bool valid) {
    // without a residual the loads read the bias array (at least 16 halves), and the values go unused
    const uint16_t* rp = a.residual ? a.res + (valid ? pix * (size_t)a.rcs + co : 0) + a.rc0 : a.bias;
    if (a.rvec || !a.residual) return *reinterpret_cast<const uint2*>(rp);  // the bias array is 256-byte aligned
    const int rem = valid ? a.cout - co : a.cout;
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t v = rp[min(i, rem - 1)];
        r[i] = i < rem ? v : 0u;
    }
    return uint2{r[0] | (r[1] << 16), r[2] | (r[3] << 16)};
}

// 8 consecutive input channels ch..ch+7 of one pixel (p points at channel ch), zeros at and past cin. VEC: the
// view is 16-byte aligned (cstride, c0 multiples of 8), so a full group is one 16-byte load, and so is a partial
// group when the view's channel stride holds the whole group (`whole`: c0 + cin rounded up to 8 <= cstride); its
// channels past cin are then zeroed by the caller (mask_group) where the value is next used. Any other group is 8
// independent 2-byte loads at clamped in-bounds addresses, selected without branches.
template <bool VEC>
__device__ __forceinline__ uint4 load_group(const uint16_t* p, int ch, int cin, bool whole = false) {
    const int rem = cin - ch;
    if (VEC && (rem >= 8 || whole)) return *reinterpret_cast<const uint4*>(p);
    uint32_t q[4];
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        const uint32_t lo = p[min(k, rem - 1)], hi = p[min(k + 1, rem - 1)];
        q[k >> 1] = (k < rem ? lo : 0u) | ((k + 1 < rem ? hi : 0u) << 16);
    }
    return uint4{q[0], q[1], q[2], q[3]};
}

// zeroes the halves of an 8-channel group at and past `rem` valid channels (rem >= 8: unchanged)
__device__ __forceinline__ uint4 mask_group(uint4 v, int rem) {
    auto keep = [&](int h) { return (2 * h < rem ? 0xffffu : 0u) | (2 * h + 1 < rem ? 0xffff0000u : 0u); };
    return uint4{v.x & keep(0), v.y & keep(1), v.z & keep(2), v.w & keep(3)};
}

// The MFMA schedule of one tile (WK == 1). The distinct B operands of a wave are the halo rows r = 0 .. R-1 it
// touches (R = (FM-1)*S + KS) at each column step c = (kx, m); operand q = c*R + r feeds the MFMAs of every output
// row f with ky = r - f*S in [0, KS), for each of the NA channel blocks. uses() counts those (f, ky) pairs.
template <int FM, int S, int KS>
__host__ __device__ constexpr int row_uses(int r) {
    int u = 0;
    for (int f = 0; f < FM; f++) u += (r - f * S >= 0 && r - f * S < KS) ? 1 : 0;
    return u;
}

// Pins the order the scheduler keeps for the unrolled chain: the first D LDS reads, then per operand q the read of
// operand q + D, q's MFMAs and, for q < NSQ, one global store (the previous tile's outputs, persistent grid).
// Left alone, the scheduler issues each read about one MFMA before its use and bunches the stores.
template <int Q, int NQ, int D, int R, int FM, int S, int KS, int NA, int NSQ>
__device__ __forceinline__ void pin_mfma_pipeline() {
    if constexpr (Q == 0) __builtin_amdgcn_sched_group_barrier(0x100, D, 0);
    if constexpr (Q < NQ) {
        if constexpr (Q + D < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, row_uses<FM, S, KS>(Q % R) * NA, 0);
        if constexpr (Q < NSQ) __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);
        pin_mfma_pipeline<Q + 1, NQ, D, R, FM, S, KS, NA, NSQ>();
    }
}

// Buffer accesses at this byte offset are out of range: loads return zeros, stores are dropped.
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Bytes a view spans from its tensor's first element: pixels * cstride + c0 + channels, in halves.
__host__ __device__ inline uint64_t view_bytes(uint64_t pixels, int cstride, int c0, int channels) {
    return pixels == 0 ? 0 : ((pixels - 1) * (uint64_t)cstride + (uint64_t)c0 + (uint64_t)channels) * 2;
}

// Waves per SIMD a persistent configuration is compiled for: one workgroup per CU, or two of 4 waves. Left to aim
// for a higher occupancy that the resident grid cannot use, the scheduler trades away the LDS read pipeline for
// registers (every MFMA then waits for its own LDS read).
constexpr int persist_waves_per_simd(int waves) { return (waves + 3) / 4 < 2 ? 2 : (waves + 3) / 4; }

template <int KS, int S, int CIN32, int FM, int WM, int WN, int NA, int WK, bool PERSIST, int MODE>
__global__ __launch_bounds__(64 * WM * WN * WK)
__attribute__((amdgpu_waves_per_eu(1, PERSIST ? persist_waves_per_simd(WM * WN * WK) : 8))) void conv_direct(
    ConvKArgs a) {
    static_assert(WK == 1 || (WK == 3 && KS == 3), "the K split runs one kernel row per wave");
    static_assert(!PERSIST || MODE >= 2, "the persistent configurations run the buffer loop");
    constexpr bool VEC = MODE > 0;  // 16-byte aligned input
    constexpr int TH = FM * WM, TW = 16, BN = 16 * NA * WN, NT = 64 * WM * WN * WK;
    constexpr int IH = (TH - 1) * S + KS, IW = (TW - 1) * S + KS;
    constexpr int GPT = CIN32 / 8, PSTR = CIN32 + 8, M = CIN32 / 32;
    constexpr int KSTEPS = KS * KS * M, KW = KSTEPS / WK;  // K-steps of the whole conv / of one wave
    constexpr int HALO = IH * IW * GPT, NLD = (HALO + NT - 1) / NT;
    // LDS: the halo, padded so that the last staging round writes without a branch (its elements past the halo
    // hold zeros), or the K-split partial sums
    constexpr int HALO_BYTES = ((NLD * NT + GPT - 1) / GPT) * PSTR * 2, RED_BYTES = (WK - 1) * WM * WN * FM * NA * 64 * 16;
    constexpr int NS = FM * NA;  // 8-byte output stores per lane and tile
    __shared__ __align__(16) uint16_t halo[(HALO_BYTES > RED_BYTES ? HALO_BYTES : RED_BYTES) / 2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wk = wave / (WM * WN), wmn = wave - wk * (WM * WN);
    const int wn = wmn % WN, wm = wmn / WN;
    const int co_w = blockIdx.y * BN + wn * 16 * NA;  // the wave's first output channel; block j at co_w + 16 j
    const int co = co_w + 4 * (lane >> 4);            // the lane's 4 output channels of block 0 in the accumulator
    const int tiles = a.n * a.tiles_y * a.tiles_x;

    // this wave's weights (its K-steps, once per workgroup) in the order the MFMA chain first uses them, then
    // bias and negative-value multipliers
    h8 wr[NA][KW];
    float bias[NA][4], neg[NA][4];
    auto load_weights = [&]() {
#pragma unroll
        for (int j = 0; j < NA; j++) {
            const h8* wp =
                reinterpret_cast<const h8*>(a.wpk) + ((size_t)((co_w >> 4) + j) * KSTEPS + wk * KW) * 64 + lane;
            if constexpr (WK == 1) {
#pragma unroll
                for (int c = 0; c < KS * M; c++)
#pragma unroll
                    for (int ky = 0; ky < KS; ky++) {
                        const int st = (ky * KS + c / M) * M + c % M;
                        wr[j][st] = wp[st * 64];
                    }
            } else {
#pragma unroll
                for (int st = 0; st < KW; st++) wr[j][st] = wp[st * 64];
            }
        }
#pragma unroll
        for (int j = 0; j < NA; j++) {
            // unconditional loads (both arrays span np channels): a load under a branch would make the compiler
            // wait for every outstanding load where the branches join
#pragma unroll
            for (int i = 0; i < 4; i++) bias[j][i] = h2f(a.bias[co + 16 * j + i]);
            const float4 m = *reinterpret_cast<const float4*>(a.neg + co + 16 * j);
            neg[j][0] = m.x;
            neg[j][1] = m.y;
            neg[j][2] = m.z;
            neg[j][3] = m.w;
        }
    };


    auto tile_origin = [&](int t, int& img, int& oy0, int& ox0) {
        const int tx = t % a.tiles_x, r = t / a.tiles_x;
        const int ty = r % a.tiles_y;
        img = r / a.tiles_y;
        oy0 = ty * TH;
        ox0 = tx * TW;
    };

    // the halo of tile t, staged in registers: element e = tid + i*NT is 8 channels (group g) of halo pixel pix.
    // MODE 1: 16-byte loads; MODE 0: 2-byte loads at clamped addresses. (MODE 2 and 3, the persistent loop without
    // and with a residual, have their own buffer-instruction versions below.)
    uint4 pre[NLD];
    // the input resource of the persistent loop spans the full strided extent (n*h*w*xcs halves, which the input
    // buffer holds): a 16-byte group that crossed the resource's end would read zeros, valid channels included
    const auto rx = buffer_rsrc(a.x, MODE >= 2 ? (uint32_t)((uint64_t)a.n * a.h * a.w * a.xcs * 2) : 0u);
    auto load_halo = [&](int t) {
        int img, oy0, ox0;
        tile_origin(t, img, oy0, ox0);
        const int iy0 = oy0 * S - a.pad, ix0 = ox0 * S - a.pad;
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = tid + i * NT;
            const int pix = e / GPT, g = e - pix * GPT;
            const int iy = pix / IW, ix = pix - iy * IW;
            const int gy = iy0 + iy, gx = ix0 + ix, ch = g * 8;
            const bool ok = ((i + 1) * NT <= HALO || e < HALO) & (gy >= 0) & (gy < a.h) & (gx >= 0) & (gx < a.w) &
                            (ch < a.cin);
            pre[i] = uint4{0u, 0u, 0u, 0u};
            if (ok)
                pre[i] = load_group<VEC>(a.x + (((size_t)img * a.h + gy) * a.w + gx) * (size_t)a.xcs + a.xc0 + ch, ch,
                                         a.cin);
        }
    };
    auto write_halo = [&]() {  // the staged halo into LDS (elements past the halo land in the padding)
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = tid + i * NT;
            const int pix = e / GPT, g = e - pix * GPT;
            *reinterpret_cast<uint4*>(halo + pix * PSTR + g * 8) = pre[i];
        }
    };

    // LDS base of the lane's pixel and channel group per output row; with the K split, wave wk runs kernel row wk
    int pb[FM];
#pragma unroll
    for (int f = 0; f < FM; f++)
        pb[f] = (((wm * FM + f) * S + wk * (WK > 1)) * IW + (lane & 15) * S) * PSTR + (lane >> 4) * 8;
    auto koff = [](int s) {  // LDS offset of K-step s (of this wave) relative to pb
        const int tap = s / M, m = s % M;
        return WK > 1 ? tap * PSTR + m * 32 : ((tap / KS) * IW + tap % KS) * PSTR + m * 32;
    };

    // the MFMA chain over the LDS halo; every LDS read is a base register plus a compile-time offset, and each read
    // feeds the NA channel blocks of the wave. side(k), k < NSQ, issues one global store between MFMA groups.
    auto compute = [&](f4 (&acc)[FM][NA], auto side, auto nsq) {
        constexpr int NSQ = decltype(nsq)::value;
#pragma unroll
        for (int f = 0; f < FM; f++)
#pragma unroll
            for (int j = 0; j < NA; j++) acc[f][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (WK == 1) {
            // each distinct B operand is read once and feeds all its (f, ky) uses; reads run D operands ahead
            // through a ring of D + 1 registers, in the order pin_mfma_pipeline fixes
            constexpr int R = (FM - 1) * S + KS, NQ = KS * M * R, D = NQ < 4 ? NQ : 4;
            static_assert(NSQ <= NQ, "more stores than pipeline steps");
            const int pr = (wm * FM * S * IW + (lane & 15) * S) * PSTR + (lane >> 4) * 8;
            auto rd = [&](int q) {
                const int c = q / R, r = q % R, kx = c / M, m = c % M;
                return *reinterpret_cast<const h8*>(halo + pr + (r * IW + kx) * PSTR + m * 32);
            };
            h8 b[D + 1];
#pragma unroll
            for (int q = 0; q < D; q++) b[q] = rd(q);
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                if (q + D < NQ) b[(q + D) % (D + 1)] = rd(q + D);
                const int c = q / R, r = q % R, kx = c / M, m = c % M;
#pragma unroll
                for (int f = FM - 1; f >= 0; f--) {
                    const int ky = r - f * S;
                    if (ky < 0 || ky >= KS) continue;
                    const int st = (ky * KS + kx) * M + m;
#pragma unroll
                    for (int j = 0; j < NA; j++)
                        acc[f][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wr[j][st], b[q % (D + 1)], acc[f][j], 0, 0, 0);
                }
                if (q < NSQ) side(q);
            }
            pin_mfma_pipeline<0, NQ, D, R, FM, S, KS, NA, NSQ>();
        } else {
            // one kernel row per wave: LDS reads one K-step ahead of the MFMAs that consume them
            h8 bx[2][FM];
#pragma unroll
            for (int f = 0; f < FM; f++) bx[0][f] = *reinterpret_cast<const h8*>(halo + pb[f]);
#pragma unroll
            for (int s = 0; s < KW; s++) {
                if (s + 1 < KW) {
#pragma unroll
                    for (int f = 0; f < FM; f++)
                        bx[(s + 1) & 1][f] = *reinterpret_cast<const h8*>(halo + pb[f] + koff(s + 1));
                }
#pragma unroll
                for (int f = 0; f < FM; f++)
#pragma unroll
                    for (int j = 0; j < NA; j++)
                        acc[f][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wr[j][s], bx[s & 1][f], acc[f][j], 0, 0, 0);
            }
            // waves of kernel rows 1 and 2 hand their partial sums to the row-0 wave of the same (wm, wn), which
            // adds them in row order
            f4* red = reinterpret_cast<f4*>(halo);
            __syncthreads();
            if (wk > 0) {
#pragma unroll
                for (int f = 0; f < FM; f++)
#pragma unroll
                    for (int j = 0; j < NA; j++)
                        red[((((wk - 1) * WM * WN + wmn) * FM + f) * NA + j) * 64 + lane] = acc[f][j];
            }
            __syncthreads();
            if (wk == 0) {
#pragma unroll
                for (int k = 1; k < WK; k++)
#pragma unroll
                    for (int f = 0; f < FM; f++)
#pragma unroll
                        for (int j = 0; j < NA; j++)
                            acc[f][j] += red[((((k - 1) * WM * WN + wmn) * FM + f) * NA + j) * 64 + lane];
            }
        }
    };

    f4 acc[FM][NA];
    uint2 rres[FM][NA];
    if constexpr (MODE < 2) {
        // one tile per workgroup: every load issued up front, the weights first (at one tile per workgroup they are
        // the larger transfer), and the chain starts once all have landed
        const int t = blockIdx.x;
        load_weights();
        load_halo(t);
        int img, oy0, ox0;
        tile_origin(t, img, oy0, ox0);
#pragma unroll
        for (int f = 0; f < FM; f++)
#pragma unroll
            for (int j = 0; j < NA; j++) {
                const int oy = oy0 + wm * FM + f, ox = ox0 + (lane & 15);
                const bool valid = (oy < a.hout) & (ox < a.wout) & (co + 16 * j < a.cout);
                rres[f][j] = load_res4(a, ((size_t)img * a.hout + oy) * a.wout + ox, co + 16 * j, valid);
            }
        write_halo();
        __syncthreads();
        FULL_WAIT_BEFORE_CHAIN
        compute(acc, [](int) {}, std::integral_constant<int, 0>{});
        if (wk == 0) {
#pragma unroll
            for (int f = 0; f < FM; f++) {
                const int oy = oy0 + wm * FM + f, ox = ox0 + (lane & 15);
                if (oy < a.hout && ox < a.wout) {
#pragma unroll
                    for (int j = 0; j < NA; j++)
                        if (co + 16 * j < a.cout)
                            epilogue4r(a, ((size_t)img * a.hout + oy) * a.wout + ox, co + 16 * j, acc[f][j], bias[j],
                                       neg[j], rres[f][j]);
                }
            }
        }
    } else {
        // The persistent configurations: G = gridDim.x resident workgroups loop over tiles. Input, residual and
        // output go through buffer instructions (out-of-range lanes: zero loads, dropped stores), so no memory access
        // sits in a branch and the compiler's waits are exact. Per tile: the MFMA chain, which also issues the
        // previous tile's stores one per pipeline step; the next tile's halo (in registers since the previous tile)
        // into LDS; this tile's epilogue into registers; then the halo loads of the tile after next and the next
        // tile's residual loads. Every wait is for
        // operations issued a whole chain earlier (the hardware counter that tracks loads also tracks stores, so a
        // load issued before a store cannot be waited for alone), and the stores of all workgroups spread over the
        // chain instead of leaving every CU at once. The first halo is loaded before the weights, so that its wait
        // does not include them and the chain starts as the weights arrive. The launcher checks the alignment and the
        // 2^31-byte extents this needs.
        // Tile order: workgroup b takes tiles b, b + G, ... (G = gridDim.x), so the tiles in flight at any time are
        // consecutive in row-major order and their loads stream through contiguous rows of the input. (Ordering the
        // tiles in column strips per XCD, for L2 locality of the shared halo rows, measured slower: the halo re-reads
        // already hit in the caches, and the strips break up the row streams.)
        const int G = gridDim.x;
        int t = blockIdx.x;
        if (t >= tiles) return;  // uniform over the workgroup
        const uint64_t pix_out = (uint64_t)a.n * a.hout * a.wout;
        const auto ry = buffer_rsrc(a.y, (uint32_t)view_bytes(pix_out, a.ycs, a.yc0, a.cout));
        // MODE 3 adds the residual; MODE 2 issues no residual load at all (each one costs the CU's address unit
        // as much as a store of the tile)
        constexpr bool RES = MODE == 3;
        const auto rr = buffer_rsrc(a.res, RES ? (uint32_t)view_bytes(pix_out, a.rcs, a.rc0, a.cout) : 0u);

        // Every address splits into a per-tile scalar base and a lane part fixed for the whole launch, computed
        // here once: the loop then spends a few full-rate VALU instructions per memory access. Offsets are 32-bit
        // unsigned (the launcher keeps every view below 2^31 bytes); a base that wraps below zero at the image's
        // top-left corner comes back in range for every lane whose access is valid.
        uint32_t hoff[NLD];  // halo element i: byte offset from the tile's first halo pixel
        int hpos[NLD];       // its halo row << 16 | column
        bool hst[NLD];       // inside the halo and below cin (tile-invariant part of its validity)
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = tid + i * NT;
            const int pix = e / GPT, g = e - pix * GPT;
            const int iy = pix / IW, ix = pix - iy * IW;
            hoff[i] = ((uint32_t)(iy * a.w + ix) * (uint32_t)a.xcs + (uint32_t)(a.xc0 + g * 8)) * 2u;
            hpos[i] = (iy << 16) | ix;
            hst[i] = ((i + 1) * NT <= HALO || e < HALO) & (g * 8 < a.cin);
        }
        const int lx = lane & 15;
        const uint32_t rl = ((uint32_t)lx * (uint32_t)a.rcs + (uint32_t)(a.rc0 + co)) * 2u;
        const uint32_t yl = ((uint32_t)lx * (uint32_t)a.ycs + (uint32_t)(a.yc0 + co)) * 2u;
        const uint32_t rrow = (uint32_t)a.wout * (uint32_t)a.rcs * 2u, yrow = (uint32_t)a.wout * (uint32_t)a.ycs * 2u;

        // tile tt's halo into registers (a tile past the last reads zeros)
        auto load_halo_b = [&](int tt) {
            int img, oy0, ox0;
            tile_origin(tt, img, oy0, ox0);
            const int iy0 = oy0 * S - a.pad, ix0 = ox0 * S - a.pad;
            const uint32_t base =
                (((uint32_t)(img * a.h + iy0) * (uint32_t)a.w + (uint32_t)ix0) * (uint32_t)a.xcs) * 2u;
            const bool tv = tt < tiles;
#pragma unroll
            for (int i = 0; i < NLD; i++) {
                const int gy = iy0 + (hpos[i] >> 16), gx = ix0 + (hpos[i] & 0xffff);
                const bool ok = hst[i] & tv & ((uint32_t)gy < (uint32_t)a.h) & ((uint32_t)gx < (uint32_t)a.w);
                pre[i] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? base + hoff[i] : kOOB, 0, 0));
            }
        };
        // the staged halo into LDS; the channels of a partial last group past cin are zeroed only when cin is not
        // a multiple of 8 (a uniform branch around arithmetic)
        auto write_halo_b = [&]() {
            if ((a.cin & 7) == 0) {
#pragma unroll
                for (int i = 0; i < NLD; i++) {
                    const int e = tid + i * NT;
                    const int pix = e / GPT, g = e - pix * GPT;
                    *reinterpret_cast<uint4*>(halo + pix * PSTR + g * 8) = pre[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < NLD; i++) {
                    const int e = tid + i * NT;
                    const int pix = e / GPT, g = e - pix * GPT;
                    *reinterpret_cast<uint4*>(halo + pix * PSTR + g * 8) = mask_group(pre[i], a.cin - g * 8);
                }
            }
        };
        // validity of output row f, channel block j of tile (oy0, ox0) for this lane
        auto out_ok = [&](int oy0, int ox0, int f, int j) {
            return (wk == 0) & (oy0 + wm * FM + f < a.hout) & (ox0 + lx < a.wout) & (co + 16 * j < a.cout);
        };
        auto load_res_buf = [&](int tt) {  // waves of kernel rows 1, 2 (K split) load nothing
            if constexpr (!RES) return;
            int img, oy0, ox0;
            tile_origin(tt, img, oy0, ox0);
            const uint32_t base = ((uint32_t)(img * a.hout + oy0 + wm * FM) * (uint32_t)a.wout + (uint32_t)ox0) *
                                  (uint32_t)a.rcs * 2u;
            const bool tv = tt < tiles;
#pragma unroll
            for (int f = 0; f < FM; f++)
#pragma unroll
                for (int j = 0; j < NA; j++) {
                    const uint32_t off = (out_ok(oy0, ox0, f, j) & tv) ? base + f * rrow + rl + 32u * j : kOOB;
                    rres[f][j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rr, off, 0, 0));
                }
        };
        // tile t's outputs, packed, and their byte offsets (kOOB: nothing to store). The residual add is an f16
        // add: f16(f32(h) + f32(r)) of two f16 values is their sum rounded once to f16 (the f32 sum is exact, or,
        // when the exponents are more than 12 apart, off by less than a quarter of an f16 ulp of the larger).
        uint2 ov[FM][NA];
        uint32_t ooff[FM][NA];
        typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
        auto epilogue_pack = [&](int tt) {
            int img, oy0, ox0;
            tile_origin(tt, img, oy0, ox0);
            const uint32_t base = ((uint32_t)(img * a.hout + oy0 + wm * FM) * (uint32_t)a.wout + (uint32_t)ox0) *
                                  (uint32_t)a.ycs * 2u;
#pragma unroll
            for (int f = 0; f < FM; f++)
#pragma unroll
                for (int j = 0; j < NA; j++) {
                    ooff[f][j] = out_ok(oy0, ox0, f, j) ? base + f * yrow + yl + 32u * j : kOOB;
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) v[i] = activate(acc[f][j][i] + bias[j][i], neg[j][i]);
                    hh2 p0 = hh2{(_Float16)v[0], (_Float16)v[1]}, p1 = hh2{(_Float16)v[2], (_Float16)v[3]};
                    if constexpr (RES) {
                        p0 += __builtin_bit_cast(hh2, rres[f][j].x);
                        p1 += __builtin_bit_cast(hh2, rres[f][j].y);
                    }
                    ov[f][j] = uint2{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1)};
                }
        };
        auto store_one = [&](int k) {
            const int f = k / NA, j = k % NA;
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) uint32_t, ov[f][j]),
                                                  ry, ooff[f][j], 0, 0);
        };
        // stores interleaved with the next tile's chain (the K-split chain takes none: its tile's stores go out
        // right after the epilogue)
        constexpr int NSQ = WK == 1 ? NS : 0;

        load_halo_b(t);
        load_weights();
        write_halo_b();
        __syncthreads();
        load_halo_b(t + G);
        load_res_buf(t);
#pragma unroll
        for (int f = 0; f < FM; f++)
#pragma unroll
            for (int j = 0; j < NA; j++) {
                ov[f][j] = uint2{0u, 0u};
                ooff[f][j] = kOOB;
            }
        // The loads ahead are unconditional (a tile past the last reads zeros): a conditional load makes the
        // compiler copy its registers where the paths join, and the copy waits for every outstanding load.
        for (; t < tiles; t += G) {
            compute(acc, store_one, std::integral_constant<int, NSQ>{});
            __syncthreads();  // every wave is done reading tile t's halo
            write_halo_b();
            __syncthreads();
            epilogue_pack(t);
            if constexpr (NSQ == 0) {
#pragma unroll
                for (int k = 0; k < NS; k++) store_one(k);
            }
            load_halo_b(t + 2 * G);
            load_res_buf(t + G);
        }
        if constexpr (NSQ > 0) {
#pragma unroll
            for (int k = 0; k < NS; k++) store_one(k);
        }
    }
}

// The one-tile-per-workgroup kernel of the configurations with one channel block per wave: every global load of
// the tile issued before the first wait (weights, halo, residual, then bias and multipliers), the halo into LDS, the
// MFMA chain reading LDS one K-step ahead, the epilogue per wave. Measured faster at one tile per workgroup than
// the buffer loop above, whose deeper pipelining only pays over several tiles. SPLIT: sibling convs (the fields
// split, cout1, y2 of ConvKArgs): the same K loop for every output channel, two epilogues.
// The LDS of one conv_tile workgroup: the input halo, or the K split's partial sums
template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK>
struct TileLds {
    static constexpr int TH = FM * WM, IH = (TH - 1) * S + KS, IW = 15 * S + KS, PSTR = CIN32 + 8;
    static constexpr int HALO_BYTES = IH * IW * PSTR * 2, RED_BYTES = (WK - 1) * WM * WN * FM * 64 * 16;
    uint16_t halo[(HALO_BYTES > RED_BYTES ? HALO_BYTES : RED_BYTES) / 2];
};

// the body of one conv_tile workgroup: spatial tile t, channel tile ct (conv_tile's blockIdx.x, .y; a launch that
// runs other work beside the conv passes its own numbering), in the workgroup's LDS L
template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK, bool VEC, bool SPLIT = false>
__device__ __forceinline__ void conv_tile_body(const ConvKArgs& a, const int t, const int ct,
                                               TileLds<KS, S, CIN32, FM, WM, WN, WK>& L) {
    static_assert(WK == 1 || (WK == 3 && KS == 3), "the K split runs one kernel row per wave");
    constexpr int TH = FM * WM, TW = 16, BN = 16 * WN, NT = 64 * WM * WN * WK;
    constexpr int IH = (TH - 1) * S + KS, IW = (TW - 1) * S + KS;
    constexpr int GPT = CIN32 / 8, PSTR = CIN32 + 8, M = CIN32 / 32;
    constexpr int KSTEPS = KS * KS * M, KW = KSTEPS / WK;  // K-steps of the whole conv / of one wave
    constexpr int HALO = IH * IW * GPT, NLD = (HALO + NT - 1) / NT;
    uint16_t* const halo = L.halo;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wk = wave / (WM * WN), wmn = wave - wk * (WM * WN);
    const int wn = wmn % WN, wm = wmn / WN;
    const int co_w = ct * BN + wn * 16;
    const int co = co_w + 4 * (lane >> 4);  // the lane's 4 output channels in the accumulator
    const int tx = t % a.tiles_x, r = t / a.tiles_x;
    const int ty = r % a.tiles_y, img = r / a.tiles_y;
    const int oy0 = ty * TH, ox0 = tx * TW;

    h8 wr[KW];
    {
        const h8* wp = reinterpret_cast<const h8*>(a.wpk) + ((size_t)(co_w >> 4) * KSTEPS + wk * KW) * 64 + lane;
#pragma unroll
        for (int s = 0; s < KW; s++) wr[s] = wp[s * 64];
    }
    uint4 pre[NLD];
    const bool whole = VEC && a.xc0 + ((a.cin + 7) & ~7) <= a.xcs;  // partial groups load as one 16-byte group
    {
        const int iy0 = oy0 * S - a.pad, ix0 = ox0 * S - a.pad;
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = tid + i * NT;
            const int pix = e / GPT, g = e - pix * GPT;
            const int iy = pix / IW, ix = pix - iy * IW;
            const int gy = iy0 + iy, gx = ix0 + ix, ch = g * 8;
            pre[i] = uint4{0u, 0u, 0u, 0u};
            if ((i + 1) * NT <= HALO || e < HALO)
                if (gy >= 0 && gy < a.h && gx >= 0 && gx < a.w && ch < a.cin)
                    pre[i] = load_group<VEC>(
                        a.x + (((size_t)img * a.h + gy) * a.w + gx) * (size_t)a.xcs + a.xc0 + ch, ch, a.cin, whole);
        }
    }
    uint2 rres[FM];
#pragma unroll
    for (int f = 0; f < FM; f++) {
        rres[f] = uint2{0u, 0u};
        const int oy = oy0 + wm * FM + f, ox = ox0 + (lane & 15);
        if constexpr (SPLIT) {  // the first conv's channels only, cout1 of them
            ConvKArgs a1 = a;
            a1.cout = a.cout1;
            if (wk == 0 && a.residual && oy < a.hout && ox < a.wout && co < a.split)
                rres[f] = load_res4(a1, ((size_t)img * a.hout + oy) * a.wout + ox, co, true);
        } else {
            if (wk == 0 && a.residual && oy < a.hout && ox < a.wout && co < a.cout)
                rres[f] = load_res4(a, ((size_t)img * a.hout + oy) * a.wout + ox, co, true);
        }
    }
    float bias[4], neg[4];
#pragma unroll
    for (int i = 0; i < 4; i++) bias[i] = h2f(a.bias[co + i]);
    {
        const float4 m = *reinterpret_cast<const float4*>(a.neg + co);
        neg[0] = m.x;
        neg[1] = m.y;
        neg[2] = m.z;
        neg[3] = m.w;
    }

#pragma unroll
    for (int i = 0; i < NLD; i++) {
        const int e = tid + i * NT;
        if ((i + 1) * NT <= HALO || e < HALO) {
            const int pix = e / GPT, g = e - pix * GPT;
            *reinterpret_cast<uint4*>(halo + pix * PSTR + g * 8) = whole ? mask_group(pre[i], a.cin - g * 8) : pre[i];
        }
    }
    __syncthreads();

    f4 acc[FM];
#pragma unroll
    for (int f = 0; f < FM; f++) acc[f] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // LDS base of the lane's pixel and channel group per output row; with the K split, wave wk runs kernel row wk
    int pb[FM];
#pragma unroll
    for (int f = 0; f < FM; f++)
        pb[f] = (((wm * FM + f) * S + wk * (WK > 1)) * IW + (lane & 15) * S) * PSTR + (lane >> 4) * 8;
    // LDS reads run one K-step ahead of the MFMAs that consume them (two register sets, selected at compile time
    // once the loop is unrolled); every read is a base register plus a compile-time offset
    auto koff = [](int s) {  // LDS offset of K-step s (of this wave) relative to pb
        const int tap = s / M, m = s % M;
        return WK > 1 ? tap * PSTR + m * 32 : ((tap / KS) * IW + tap % KS) * PSTR + m * 32;
    };
    h8 bx[2][FM];
#pragma unroll
    for (int f = 0; f < FM; f++) bx[0][f] = *reinterpret_cast<const h8*>(halo + pb[f]);
#pragma unroll
    for (int s = 0; s < KW; s++) {
        if (s + 1 < KW) {
#pragma unroll
            for (int f = 0; f < FM; f++)
                bx[(s + 1) & 1][f] = *reinterpret_cast<const h8*>(halo + pb[f] + koff(s + 1));
        }
#pragma unroll
        for (int f = 0; f < FM; f++)
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wr[s], bx[s & 1][f], acc[f], 0, 0, 0);
    }

    if constexpr (WK > 1) {
        // waves of kernel rows 1 and 2 hand their partial sums to the row-0 wave of the same (wm, wn), which adds
        // them in row order and runs the epilogue
        f4* red = reinterpret_cast<f4*>(halo);
        __syncthreads();
        if (wk > 0) {
#pragma unroll
            for (int f = 0; f < FM; f++) red[(((wk - 1) * WM * WN + wmn) * FM + f) * 64 + lane] = acc[f];
        }
        __syncthreads();
        if (wk > 0) return;
#pragma unroll
        for (int k = 1; k < WK; k++)
#pragma unroll
            for (int f = 0; f < FM; f++) acc[f] += red[(((k - 1) * WM * WN + wmn) * FM + f) * 64 + lane];
    }

    if constexpr (SPLIT) {
        // channel groups below split: the first conv (cout1 stored, with its residual); the rest: the second conv
        ConvKArgs o = a;
        int c = co;
        if (co < a.split) {
            o.cout = a.cout1;
        } else {
            o.y = a.y2, o.ycs = a.y2cs, o.yc0 = a.y2c0, o.yvec = a.y2vec;
            o.residual = 0, o.cout = a.cout - a.split;
            c = co - a.split;
        }
        if (co < a.cout) {
#pragma unroll
            for (int f = 0; f < FM; f++) {
                const int oy = oy0 + wm * FM + f, ox = ox0 + (lane & 15);
                if (oy < a.hout && ox < a.wout)
                    epilogue4r(o, ((size_t)img * a.hout + oy) * a.wout + ox, c, acc[f], bias, neg, rres[f]);
            }
        }
    } else if (co < a.cout) {
#pragma unroll
        for (int f = 0; f < FM; f++) {
            const int oy = oy0 + wm * FM + f, ox = ox0 + (lane & 15);
            if (oy < a.hout && ox < a.wout)
                epilogue4r(a, ((size_t)img * a.hout + oy) * a.wout + ox, co, acc[f], bias, neg, rres[f]);
        }
    }
}

template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK, bool VEC, bool SPLIT = false>
__global__ __launch_bounds__(64 * WM * WN * WK) void conv_tile(ConvKArgs a) {
    __shared__ __align__(16) TileLds<KS, S, CIN32, FM, WM, WN, WK> lds;
    conv_tile_body<KS, S, CIN32, FM, WM, WN, WK, VEC, SPLIT>(a, blockIdx.x, blockIdx.y, lds);
}

// The sibling convs' launch of a one-tile configuration (one workgroup per tile, one channel tile)
template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK>
hipError_t launch_tile_split(const ConvKArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    (void)lds;
    const dim3 block(64 * WM * WN * WK);
    if (a.xvec)
        hipLaunchKernelGGL((conv_tile<KS, S, CIN32, FM, WM, WN, WK, true, true>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((conv_tile<KS, S, CIN32, FM, WM, WN, WK, false, true>), grid, block, 0, s, a);
    return hipGetLastError();
}

// Whether a launch can take the buffer-instruction loop of the persistent configurations: 16-byte aligned input
// whose last 8-channel group lies inside the pixel's stride (the group loads whole), 8-byte aligned output and
// residual with cout a multiple of 4, and extents within the 2^31 bytes a buffer offset reaches.
inline bool buffer_path_ok(const ConvKArgs& a) {
    const uint64_t pin = (uint64_t)a.n * a.h * a.w, pout = (uint64_t)a.n * a.hout * a.wout;
    const uint64_t lim = 1ull << 31;
    return a.xvec && a.yvec && a.cout % 4 == 0 && (!a.residual || a.rvec) && a.xc0 + ((a.cin + 7) & ~7) <= a.xcs &&
           pin * (uint64_t)a.xcs * 2 < lim && view_bytes(pout, a.ycs, a.yc0, a.cout) < lim &&
           (!a.residual || view_bytes(pout, a.rcs, a.rc0, a.cout) < lim);
}

// Launches a persistent configuration on its resident grid when the views allow the buffer loop, else one
// workgroup per tile, with 16-byte input loads when the input view is 16-byte aligned.
template <int KS, int S, int CIN32, int FM, int WM, int WN, int NA, int WK, bool PERSIST>
hipError_t launch_direct(const ConvKArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    (void)lds;
    const dim3 block(64 * WM * WN * WK);
    if constexpr (PERSIST) {
        if (buffer_path_ok(a)) {
            if (a.residual)
                hipLaunchKernelGGL((conv_direct<KS, S, CIN32, FM, WM, WN, NA, WK, true, 3>), grid, block, 0, s, a);
            else
                hipLaunchKernelGGL((conv_direct<KS, S, CIN32, FM, WM, WN, NA, WK, true, 2>), grid, block, 0, s, a);
            return hipGetLastError();
        }
        grid.x = (unsigned)(a.n * a.tiles_y * a.tiles_x);
    }
    if constexpr (NA == 1) {
        if (a.xvec)
            hipLaunchKernelGGL((conv_tile<KS, S, CIN32, FM, WM, WN, WK, true>), grid, block, 0, s, a);
        else
            hipLaunchKernelGGL((conv_tile<KS, S, CIN32, FM, WM, WN, WK, false>), grid, block, 0, s, a);
    } else {
        if (a.xvec)
            hipLaunchKernelGGL((conv_direct<KS, S, CIN32, FM, WM, WN, NA, WK, false, 1>), grid, block, 0, s, a);
        else
            hipLaunchKernelGGL((conv_direct<KS, S, CIN32, FM, WM, WN, NA, WK, false, 0>), grid, block, 0, s, a);
    }
    return hipGetLastError();
}

// the kernel of a configuration, for occupancy queries (the persistent loop's variant with or without a residual)
template <int KS, int S, int CIN32, int FM, int WM, int WN, int NA, int WK, bool PERSIST>
const void* direct_kernel(bool residual) {
    if constexpr (PERSIST)
        return residual ? reinterpret_cast<const void*>(&conv_direct<KS, S, CIN32, FM, WM, WN, NA, WK, true, 3>)
                        : reinterpret_cast<const void*>(&conv_direct<KS, S, CIN32, FM, WM, WN, NA, WK, true, 2>);
    else if constexpr (NA > 1)
        return reinterpret_cast<const void*>(&conv_direct<KS, S, CIN32, FM, WM, WN, NA, WK, false, 1>);
    else
        return reinterpret_cast<const void*>(&conv_tile<KS, S, CIN32, FM, WM, WN, WK, true>);
}

}  // namespace fhc
