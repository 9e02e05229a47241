// The wave-stream direct conv kernel, for large layers (the persistent configurations named "/w"): every wave of a
// 4-wave workgroup (one per SIMD) runs its own stream of output tiles with no workgroup barrier in its loop.
//
// - A wave computes FM output rows of 16 pixels for all 16 * NA output channels of the workgroup's channel tile,
//   so each B operand read from LDS feeds NA MFMAs and the wave keeps FM * NA independent accumulators in flight
//   (a dependent MFMA waits ~50 cycles for its predecessor against 16 cycles of issue).
// - The weights of the channel tile (K order and packing as in direct_impl.h) are staged once per workgroup in LDS
//   through LDS DMA and copied into every wave's registers.
// - Input halos go from global memory straight into the wave's own LDS buffers by LDS DMA (buffer_load ... lds:
//   lane i writes its 16 bytes at the buffer base + 16 i, an out-of-range offset writes zeros), so padding, the
//   channels past cin and a tile past the last all arrive as zeros, and no register holds a staged halo. The halo
//   layout is slot-major: pixel p's 8-channel group g at slot p * (CIN32 / 8 + 1) + g, the extra slot per pixel
//   (always zero) padding the pixel stride to CIN32 + 8 halves as in direct_impl.h.
// - Two halo buffers per wave in two distinct LDS arrays, the loop unrolled by two: while the chain reads one, the
//   DMA of the wave's next tile fills the other. The DMA instructions are issued inside the chain after its first
//   LDS reads: the compiler's wait for the DMA that filled the buffer being read (it waits for every LDS DMA in
//   flight that may write the array it reads) then lands before them, and the later reads, of the other array,
//   wait for nothing.
// - The previous tile's stores go out one per pipeline step of the chain, as in the persistent loop of
//   direct_impl.h.
// Registers: no waves-per-EU attribute is needed; the compiler already gives these kernels up to 512 registers
// per lane (one or two waves per SIMD).
// Requirements, checked by the planner and, at run time, by the launcher (which otherwise runs conv_tile with the
// same tiles): cin a multiple of 8 (whole 16-byte groups), a 16-byte aligned input view, cout a multiple of 4 and
// an 8-byte aligned output view, no residual, every view below 2^31 bytes.
#pragma once
#include "direct_impl.h"

namespace fhc {

template <int KS, int S, int CIN32, int FM, int NA>
struct WaveGeom {
    static constexpr int TW = 16, IH = (FM - 1) * S + KS, IW = (TW - 1) * S + KS;
    static constexpr int GPT = CIN32 / 8, SLOTS = GPT + 1, M = CIN32 / 32;
    static constexpr int KSTEPS = KS * KS * M;
    static constexpr int NDMA = (IH * IW * SLOTS + 63) / 64;  // DMA instructions per halo
    static constexpr int BUF = NDMA * 64;                     // 16-byte slots per halo buffer
    static constexpr int WU4 = NA * KSTEPS * 64;              // 16-byte slots of the channel tile's weights
    static constexpr int B1 = 4 * BUF > WU4 ? 4 * BUF : WU4;  // the second buffer array also stages the weights
    static constexpr int R = (FM - 1) * S + KS, NQ = KS * M * R;  // chain steps (distinct B operands)
    static constexpr int LDS_BYTES = (4 * BUF + B1) * 16 + 2 * 16 * NA * 4;
};

// Pins the chain's order: the first D LDS reads, then per step q the read of operand q + D, q's MFMAs, one store
// for q < NSQ, and the DMA instructions DMA0 .. whose slot is q (dma_step).
template <int NQ, int NDMA>
__host__ __device__ constexpr int dma_step(int k) {
    return 1 + (k * (NQ - 1)) / NDMA;
}
template <int Q, int NQ, int D, int R, int FM, int S, int KS, int NA, int NSQ, int NDMA>
__device__ __forceinline__ void pin_wave_pipeline() {
    if constexpr (Q == 0) __builtin_amdgcn_sched_group_barrier(0x100, D, 0);
    if constexpr (Q < NQ) {
        if constexpr (Q + D < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, row_uses<FM, S, KS>(Q % R) * NA, 0);
        if constexpr (Q < NSQ) __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);
        constexpr int nd = [] {
            int c = 0;
            for (int k = 0; k < NDMA; k++) c += dma_step<NQ, NDMA>(k) == Q ? 1 : 0;
            return c;
        }();
        if constexpr (nd > 0) __builtin_amdgcn_sched_group_barrier(0x020, nd, 0);
        pin_wave_pipeline<Q + 1, NQ, D, R, FM, S, KS, NA, NSQ, NDMA>();
    }
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One LDS DMA instruction: lane i's 16 bytes at byte offset `off` of resource r (zeros when out of range) into LDS
// at lds + 16 i; lds must be the same for the whole wave. The LDS address-space cast exists only in the device pass.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint4* lds, uint32_t off) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, off, 0, 0, 0);
#else
    (void)r, (void)lds, (void)off;
#endif
}


template <int KS, int S, int CIN32, int FM, int NA>
__global__ __launch_bounds__(256) void conv_wave(ConvKArgs a) {
    using Gm = WaveGeom<KS, S, CIN32, FM, NA>;
    constexpr int TW = Gm::TW, IW = Gm::IW, GPT = Gm::GPT, SLOTS = Gm::SLOTS, M = Gm::M;
    constexpr int KSTEPS = Gm::KSTEPS, NDMA = Gm::NDMA, BUF = Gm::BUF, R = Gm::R, NQ = Gm::NQ;
    constexpr int NS = FM * NA, D = NQ < 4 ? NQ : 4;
    static_assert(NS <= NQ, "more stores than chain steps");
    static_assert(NDMA < NQ, "more DMA instructions than chain steps");
    __shared__ __align__(16) uint4 hb0[4 * BUF];   // halo buffer 0 of each wave
    __shared__ __align__(16) uint4 hb1[Gm::B1];    // halo buffer 1 of each wave; first, the staged weights
    __shared__ __align__(16) float bn[2][16 * NA];  // bias and negative-value multipliers of the channel tile

    // the wave index as a scalar: the tile loop, the tile decode and the DMA's LDS base are per wave
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lx = lane & 15;
    const int co_w = blockIdx.y * 16 * NA;   // the channel tile's first output channel
    const int co = co_w + 4 * (lane >> 4);   // the lane's 4 channels of block 0 in the accumulator
    const int tiles = a.n * a.tiles_y * a.tiles_x;
    const int GW = (int)gridDim.x * 4;
    int t = (int)blockIdx.x * 4 + wave;  // the wave's first tile; then t + GW, ...

    const auto rx = buffer_rsrc(a.x, (uint32_t)((uint64_t)a.n * a.h * a.w * a.xcs * 2));
    const uint64_t pix_out = (uint64_t)a.n * a.hout * a.wout;
    const auto ry = buffer_rsrc(a.y, (uint32_t)view_bytes(pix_out, a.ycs, a.yc0, a.cout));

    auto tile_origin = [&](int k, int& img, int& oy0, int& ox0) {
        const int tx = k % a.tiles_x, r = k / a.tiles_x;
        img = r / a.tiles_y;
        oy0 = (r - img * a.tiles_y) * FM;
        ox0 = tx * TW;
    };

    // Halo DMA, lane parts fixed for the launch: instruction k covers slots 64 k .. 64 k + 63; the lane's slot is
    // pixel p = s / SLOTS (halo row p / IW, column p % IW), group g = s % SLOTS (g == GPT: the zero pad slot).
    // hoffm: the lane's byte offset from the tile's first halo pixel, or kOOB for a pad slot, a slot past the halo
    // or channels past cin (offsets stay below 2^31, so kOOB marks them)
    uint32_t hoffm[NDMA];
    int hpos[NDMA];
#pragma unroll
    for (int k = 0; k < NDMA; k++) {
        const int s = k * 64 + lane, p = s / SLOTS, g = s - p * SLOTS;
        const int iy = p / IW, ix = p - iy * IW;
        const bool st = (s < Gm::IH * IW * SLOTS) & (g < GPT) & (g * 8 < a.cin);
        hoffm[k] = st ? ((uint32_t)(iy * a.w + ix) * (uint32_t)a.xcs + (uint32_t)(a.xc0 + g * 8)) * 2u : kOOB;
        hpos[k] = (iy << 16) | ix;
    }
    // the DMA offsets of tile tt's halo, computed before the chain that issues them, so that the chain carries no
    // address arithmetic. A tile whose halo lies inside the image (most of them) needs one add per instruction: a
    // masked lane's kOOB plus the base stays at or above 2^31, out of range; the others check rows and columns.
    uint32_t doff[NDMA];
    auto dma_offsets = [&](int tt) {
        int img, oy0, ox0;
        tile_origin(tt, img, oy0, ox0);
        const int iy0 = oy0 * S - a.pad, ix0 = ox0 * S - a.pad;
        const uint32_t base = (((uint32_t)(img * a.h + iy0) * (uint32_t)a.w + (uint32_t)ix0) * (uint32_t)a.xcs) * 2u;
        const bool tv = tt < tiles;
        if (tv && iy0 >= 0 && iy0 + Gm::IH <= a.h && ix0 >= 0 && ix0 + IW <= a.w) {
#pragma unroll
            for (int k = 0; k < NDMA; k++) doff[k] = base + hoffm[k];
        } else {
#pragma unroll
            for (int k = 0; k < NDMA; k++) {
                const int gy = iy0 + (hpos[k] >> 16), gx = ix0 + (hpos[k] & 0xffff);
                const bool ok = (hoffm[k] < kOOB) & tv & ((uint32_t)gy < (uint32_t)a.h) & ((uint32_t)gx < (uint32_t)a.w);
                doff[k] = ok ? base + hoffm[k] : kOOB;
            }
        }
    };
    auto dma_halo = [&](uint4* buf, int k) {  // k: a constant after unrolling
        lds_dma16(rx, buf + wave * BUF + k * 64, doff[k]);
    };

    // ---- prologue: the first halo, the channel tile's weights (staged in hb1), bias and multipliers
    dma_offsets(t);
#pragma unroll
    for (int k = 0; k < NDMA; k++) dma_halo(hb0, k);
    {
        const auto rw = buffer_rsrc(reinterpret_cast<const char*>(a.wpk) + (size_t)(co_w >> 4) * KSTEPS * 1024,
                                    (uint32_t)Gm::WU4 * 16u);
#pragma unroll
        for (int k = wave; k < NA * KSTEPS; k += 4)
            lds_dma16(rw, hb1 + k * 64, (uint32_t)(k * 64 + lane) * 16u);
        if (tid < 16 * NA) {
            bn[0][tid] = h2f(a.bias[co_w + tid]);
            bn[1][tid] = a.neg[co_w + tid];
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // every counter at zero: this wave's DMAs have landed
    __syncthreads();
    h8 wr[NA][KSTEPS];
#pragma unroll
    for (int j = 0; j < NA; j++)
#pragma unroll
        for (int st = 0; st < KSTEPS; st++) wr[j][st] = __builtin_bit_cast(h8, hb1[(j * KSTEPS + st) * 64 + lane]);
    __syncthreads();  // the weights are in registers: hb1 becomes halo buffer 1
    if (t >= tiles) return;  // uniform over the wave; no workgroup barrier follows

    // ---- the chain of one tile over halo buffer `buf`; during it, the previous tile's stores and the DMA of the
    // wave's next tile into `nbuf`
    f4 acc[FM][NA];
    uint2 ov[FM][NA];
    uint32_t ooff[FM][NA];
#pragma unroll
    for (int f = 0; f < FM; f++)
#pragma unroll
        for (int j = 0; j < NA; j++) {
            ov[f][j] = uint2{0u, 0u};
            ooff[f][j] = kOOB;
        }
    const int pr = (lx * S * SLOTS + (lane >> 4)) * 8;  // halves: the lane's pixel and channel group, row 0
    auto chain = [&](const uint4* buf, uint4* nbuf, int tn) {
        // This wave's DMA into `buf` (issued during the previous chain) must have landed: wait for every memory
        // operation of the wave (the previous tile's stores, issued as long ago, included). The compiler does not
        // place this wait reliably across the loop's back edge, so it is explicit, fenced against the scheduler.
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), lgkmcnt and expcnt left alone
        __builtin_amdgcn_sched_barrier(0);
        const uint16_t* hv = reinterpret_cast<const uint16_t*>(buf + wave * BUF) + pr;
        auto rd = [&](int q) {
            const int c = q / R, r = q % R, kx = c / M, m = c % M;
            return *reinterpret_cast<const h8*>(hv + ((r * IW + kx) * SLOTS + 4 * m) * 8);
        };
#pragma unroll
        for (int f = 0; f < FM; f++)
#pragma unroll
            for (int j = 0; j < NA; j++) acc[f][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        dma_offsets(tn);
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
            if (q < NS)
                __builtin_amdgcn_raw_buffer_store_b64(
                    __builtin_bit_cast(__attribute__((ext_vector_type(2))) uint32_t, ov[q / NA][q % NA]), ry,
                    ooff[q / NA][q % NA], 0, 0);
#pragma unroll
            for (int k = 0; k < NDMA; k++)
                if (dma_step<NQ, NDMA>(k) == q) dma_halo(nbuf, k);
        }
        pin_wave_pipeline<0, NQ, D, R, FM, S, KS, NA, NS, NDMA>();
    };
    // tile tt's outputs, packed, and their byte offsets (kOOB: nothing to store)
    typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
    const uint32_t yl = ((uint32_t)lx * (uint32_t)a.ycs + (uint32_t)(a.yc0 + co)) * 2u;
    const uint32_t yrow = (uint32_t)a.wout * (uint32_t)a.ycs * 2u;
    auto epilogue_pack = [&](int tt) {
        int img, oy0, ox0;
        tile_origin(tt, img, oy0, ox0);
        const uint32_t base =
            ((uint32_t)(img * a.hout + oy0) * (uint32_t)a.wout + (uint32_t)ox0) * (uint32_t)a.ycs * 2u;
#pragma unroll
        for (int j = 0; j < NA; j++) {
            const float4 bj = *reinterpret_cast<const float4*>(&bn[0][16 * j + 4 * (lane >> 4)]);
            const float4 nj = *reinterpret_cast<const float4*>(&bn[1][16 * j + 4 * (lane >> 4)]);
            const float bb[4] = {bj.x, bj.y, bj.z, bj.w}, nn[4] = {nj.x, nj.y, nj.z, nj.w};
#pragma unroll
            for (int f = 0; f < FM; f++) {
                const bool ok = (oy0 + f < a.hout) & (ox0 + lx < a.wout) & (co + 16 * j < a.cout);
                ooff[f][j] = ok ? base + f * yrow + yl + 32u * j : kOOB;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = activate(acc[f][j][i] + bb[i], nn[i]);
                const hh2 p0 = hh2{(_Float16)v[0], (_Float16)v[1]}, p1 = hh2{(_Float16)v[2], (_Float16)v[3]};
                ov[f][j] = uint2{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1)};
            }
        }
    };

    // ---- the wave's loop, two tiles per round (halo buffers hb0, hb1 alternate)
    for (;;) {
        chain(hb0, hb1, t + GW);
        epilogue_pack(t);
        t += GW;
        if (t >= tiles) break;
        chain(hb1, hb0, t + GW);
        epilogue_pack(t);
        t += GW;
        if (t >= tiles) break;
    }
#pragma unroll
    for (int f = 0; f < FM; f++)
#pragma unroll
        for (int j = 0; j < NA; j++)
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) uint32_t, ov[f][j]),
                                                  ry, ooff[f][j], 0, 0);
}

// Whether a launch can take the wave kernel: whole 16-byte input groups at 16-byte aligned addresses, 8-byte output
// stores, no residual, and 32-bit buffer offsets.
inline bool wave_path_ok(const ConvKArgs& a) {
    return !a.residual && a.cin % 8 == 0 && buffer_path_ok(a);
}

template <int KS, int S, int CIN32, int FM, int NA>
hipError_t launch_wave(const ConvKArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    (void)lds;
    if (wave_path_ok(a)) {
        hipLaunchKernelGGL((conv_wave<KS, S, CIN32, FM, NA>), grid, dim3(256), 0, s, a);
        return hipGetLastError();
    }
    // the same tiles and channel tiles, one workgroup (NA waves of 16 channels) per tile
    grid.x = (unsigned)(a.n * a.tiles_y * a.tiles_x);
    if (a.xvec)
        hipLaunchKernelGGL((conv_tile<KS, S, CIN32, FM, 1, NA, 1, true>), grid, dim3(64 * NA), 0, s, a);
    else
        hipLaunchKernelGGL((conv_tile<KS, S, CIN32, FM, 1, NA, 1, false>), grid, dim3(64 * NA), 0, s, a);
    return hipGetLastError();
}

template <int KS, int S, int CIN32, int FM, int NA>
const void* wave_kernel() {
    return reinterpret_cast<const void*>(&conv_wave<KS, S, CIN32, FM, NA>);
}

}  // namespace fhc
