// The deep-layer conv (configurations named "gemm."): a 3x3 conv over any input channel count, the weights streamed
// through LDS chunk by chunk with the input, for layers whose weights do not fit a wave's registers (cin 155, 279)
// or whose work is large enough to tile as a GEMM (cin >= 64 on big or batched tensors).
//
// - Workgroup tile: TH = FM * WM output rows x 16 columns x BN = 16 * NA * WN output channels. Wave (wm, wn) owns
//   FM rows x NA 16-channel blocks: FM * NA independent accumulators, so consecutive MFMAs never wait on each
//   other, and every LDS operand read feeds several MFMAs: per kernel column kx and 32-channel step m a wave reads
//   the R = (FM - 1) * S + 3 halo rows it touches once and the 3 * NA weight fragments once, then runs the
//   3 * FM * NA MFMAs (ky-major, so the same accumulator comes back only after FM * NA - 1 others).
// - K runs over chunks of CK input channels (all 9 taps per chunk). A chunk's input halo ((TH-1)*S+3) x (15*S+3)
//   pixels x CK channels and its weights (BN channels x 9 * CK) go from global memory straight into LDS by LDS DMA
//   (lane i writes its 16 bytes at the base + 16 i; an out-of-range offset writes zeros: the padding and the
//   channels past cin) into a ring of ST chunk buffers: chunks c + 1 .. c + ST - 1 load while chunk c computes,
//   one barrier per chunk (with one workgroup per CU nothing else hides the DMA's latency, which is several times
//   a chunk's MFMA time). Every wave issues the same number of DMA instructions per chunk (the halo's and the
//   weights' instruction counts are padded to multiples of the wave count), so the wait for chunk c is an exact
//   count of the wave's outstanding operations: those of the chunks issued after c. The halo
//   is slot-major (pixel p's 8-channel group g at slot p * (CK/8 + 1) + g; the extra slot pads the pixel stride to
//   CK + 8 halves); the weights keep the packed fragment order [block][chunk][k-step][lane] of the chunked layout
//   (k = tap * CK + ci within a chunk; api.cpp, pack_weights).
// - A partial last 8-channel group (cin not a multiple of 8) arrives whole with the channels next to it in the
//   tensor; its channels past cin are zeroed in LDS before the chunk computes (they may hold anything, NaN
//   included, and zero weights do not cancel NaN).
// - Global split-K (grid.z = z splits of chunks_per_split chunks): f32 partials [z][pixel][np], summed in z order
//   by splitk_reduce, which then runs the epilogue; without a split the epilogue (bias, activation, f16, residual)
//   runs straight from the accumulators.
// - The input view must be 16-byte aligned (channel stride and offset multiples of 8, the base pointer aligned) and
//   below 2^31 bytes; the launcher runs the chunked kernel (the same packed weights) on any other view.
#pragma once
#include "wave_impl.h"

namespace fhc {

template <int S, int CK, int FM, int NA, int WM, int WN, int ST>
struct GemmGeom {
    static constexpr int TH = FM * WM, TW = 16, BN = 16 * NA * WN, NW = WM * WN;
    static constexpr int IH = (TH - 1) * S + 3, IW = (TW - 1) * S + 3, R = (FM - 1) * S + 3;
    static constexpr int GPC = CK / 8, SLOTS = GPC + 1, MC = CK / 32, KSC = 9 * MC;
    static constexpr int NDH0 = (IH * IW * SLOTS + 63) / 64;   // halo DMA instructions per chunk
    static constexpr int NDW0 = NA * WN * KSC;                  // weight DMA instructions (1 KB each) per chunk
    static constexpr int NDH = (NDH0 + NW - 1) / NW * NW, NDW = (NDW0 + NW - 1) / NW * NW;  // padded
    static constexpr int PER = (NDH + NDW) / NW;                // DMA instructions per wave and chunk
    static constexpr int LDS_BYTES = ST * (NDH + NDW) * 64 * 16;
    static_assert(CK % 32 == 0, "chunks of whole 32-channel K-steps");
    static_assert(ST >= 2 && PER * (ST - 2) < 64, "the wait count fits vmcnt");
    static_assert(LDS_BYTES <= 160 * 1024, "the chunk buffers exceed the CU's LDS");
};

// s_waitcnt with vmcnt(n) (bits 3:0 and 15:14), expcnt and lgkmcnt left at their maxima
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

template <int S, int CK, int FM, int NA, int WM, int WN, int ST>
__global__ __launch_bounds__(64 * WM * WN) void conv_gemm(ConvKArgs a) {
    using Gm = GemmGeom<S, CK, FM, NA, WM, WN, ST>;
    constexpr int TH = Gm::TH, TW = Gm::TW, BN = Gm::BN, NW = Gm::NW, IH = Gm::IH, IW = Gm::IW, R = Gm::R;
    constexpr int GPC = Gm::GPC, SLOTS = Gm::SLOTS, MC = Gm::MC, KSC = Gm::KSC, NDH = Gm::NDH, NDW = Gm::NDW;
    constexpr int DHW = NDH / NW, DWW = NDW / NW, PER = Gm::PER;
    // one LDS object per buffer: the compiler's wait for LDS DMA then covers only the DMA into the buffer a read
    // uses (with one array it waits for every DMA in flight before any LDS read, serializing load and compute)
    __shared__ __align__(16) uint4 hb0[NDH * 64], hb1[NDH * 64], hb2[ST > 2 ? NDH * 64 : 1];
    __shared__ __align__(16) uint4 wb0[NDW * 64], wb1[NDW * 64], wb2[ST > 2 ? NDW * 64 : 1];
    static_assert(ST <= 3, "three buffers at most");
    auto hbuf = [&](int b) -> uint4* { return b == 0 ? hb0 : b == 1 ? hb1 : hb2; };
    auto wbuf = [&](int b) -> uint4* { return b == 0 ? wb0 : b == 1 ? wb1 : wb2; };

    const int tid = threadIdx.x, lane = tid & 63, lx = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: the DMA's LDS base is per wave
    const int wn = wave % WN, wm = wave / WN;
    const int co = blockIdx.y * BN + wn * 16 * NA + 4 * (lane >> 4);  // the lane's 4 channels of block 0
    const int t = blockIdx.x;
    const int tx = t % a.tiles_x, r0 = t / a.tiles_x;
    const int ty = r0 % a.tiles_y, img = r0 / a.tiles_y;
    const int oy0 = ty * TH, ox0 = tx * TW;
    const int iy0 = oy0 * S - a.pad, ix0 = ox0 * S - a.pad;
    const int nch = a.nchunks;
    const int cbeg = blockIdx.z * a.chunks_per_split, cend = min(nch, cbeg + a.chunks_per_split);
    const bool split = gridDim.z > 1;

    const auto rx = buffer_rsrc(a.x, (uint32_t)((uint64_t)a.n * a.h * a.w * a.xcs * 2));
    const auto rw = buffer_rsrc(a.wpk, (uint32_t)((uint64_t)(a.np / 16) * nch * KSC * 1024));

    // the lane's slot of each of this wave's halo DMA instructions (instruction k = wave + NW * i), the same for
    // every chunk: its byte offset in chunk 0 (kOOB: padding, a pad slot or past the halo) and its first channel
    uint32_t hoff[DHW];
    int hch[DHW];
#pragma unroll
    for (int i = 0; i < DHW; i++) {
        const int k = wave + NW * i, s = k * 64 + lane, p = s / SLOTS, g = s - p * SLOTS;
        const int iy = p / IW, ix = p - iy * IW, gy = iy0 + iy, gx = ix0 + ix;
        const bool ok = (s < IH * IW * SLOTS) & (g < GPC) & (gy >= 0) & (gy < a.h) & (gx >= 0) & (gx < a.w);
        hoff[i] = ok ? ((((uint32_t)(img * a.h + gy) * (uint32_t)a.w + (uint32_t)gx) * (uint32_t)a.xcs) +
                        (uint32_t)(a.xc0 + g * 8)) * 2u
                     : kOOB;
        hch[i] = g * 8;
    }
    // chunk c into buffer b: every wave issues DHW halo and DWW weight instructions (the padding ones write zeros)
    auto dma_chunk = [&](int b, int c) {
        const int c0 = c * CK;
#pragma unroll
        for (int i = 0; i < DHW; i++)
            lds_dma16(rx, hbuf(b) + (wave + NW * i) * 64,
                      ((hoff[i] != kOOB) & (c0 + hch[i] < a.cin)) ? hoff[i] + (uint32_t)c0 * 2u : kOOB);
#pragma unroll
        for (int i = 0; i < DWW; i++) {
            const int k = wave + NW * i;  // weight instruction k: block k / KSC of the tile, k-step k % KSC
            const int j = k / KSC, st = k - j * KSC;
            const uint32_t blk = (uint32_t)(blockIdx.y * (BN / 16) + j);
            lds_dma16(rw, wbuf(b) + k * 64,
                      k < Gm::NDW0 ? (((blk * (uint32_t)nch + (uint32_t)c) * KSC + st) * 64 + lane) * 16u : kOOB);
        }
    };
    // the last chunk's partial 8-channel group: channels past cin zeroed in LDS (after every wave's DMA landed)
    const int rem_last = a.cin - (nch - 1) * CK;
    auto fix_partial = [&](int b) {
        if ((rem_last & 7) == 0) return;  // uniform
        const int g = rem_last >> 3, keep = rem_last & 7;
        uint4* hb = hbuf(b);
        for (int p = tid; p < IH * IW; p += 64 * NW) hb[p * SLOTS + g] = mask_group(hb[p * SLOTS + g], keep);
    };

    // the first chunks' DMA goes out first; the residual and parameter loads queue behind it
#pragma unroll
    for (int q = 0; q < ST - 1; q++)
        if (cbeg + q < cend) dma_chunk(q, cbeg + q);

    // residual, bias, multipliers: global loads ahead of the first wait
    uint2 rres[FM][NA];
#pragma unroll
    for (int f = 0; f < FM; f++)
#pragma unroll
        for (int j = 0; j < NA; j++) {
            const int oy = oy0 + wm * FM + f, ox = ox0 + lx;
            const bool valid = (oy < a.hout) & (ox < a.wout) & (co + 16 * j < a.cout);
            rres[f][j] = load_res4(a, ((size_t)img * a.hout + oy) * a.wout + ox, co + 16 * j, valid);
        }
    float bias[NA][4], neg[NA][4];
#pragma unroll
    for (int j = 0; j < NA; j++) {
#pragma unroll
        for (int i = 0; i < 4; i++) bias[j][i] = h2f(a.bias[co + 16 * j + i]);
        const float4 m = *reinterpret_cast<const float4*>(a.neg + co + 16 * j);
        neg[j][0] = m.x, neg[j][1] = m.y, neg[j][2] = m.z, neg[j][3] = m.w;
    }

    f4 acc[FM][NA];
#pragma unroll
    for (int f = 0; f < FM; f++)
#pragma unroll
        for (int j = 0; j < NA; j++) acc[f][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // B operands: the lane's pixel (the wave's first halo row, column lx * S) and channel group lane / 16
    const int pb = ((wm * FM * S) * IW + lx * S) * SLOTS + (lane >> 4);
    const int wa = (wn * NA) * KSC * 64 + lane;  // A operands: the wave's first block
    auto compute = [&](int b) {
        const uint4* hb = hbuf(b);
        const uint4* wb = wbuf(b);
#pragma unroll
        for (int m = 0; m < MC; m++)
#pragma unroll
            for (int kx = 0; kx < 3; kx++) {
                h8 bv[R], av[3][NA];
#pragma unroll
                for (int r = 0; r < R; r++) bv[r] = __builtin_bit_cast(h8, hb[pb + (r * IW + kx) * SLOTS + 4 * m]);
#pragma unroll
                for (int ky = 0; ky < 3; ky++)
#pragma unroll
                    for (int j = 0; j < NA; j++)
                        av[ky][j] = __builtin_bit_cast(h8, wb[wa + (j * KSC + (ky * 3 + kx) * MC + m) * 64]);
#pragma unroll
                for (int ky = 0; ky < 3; ky++)
#pragma unroll
                    for (int f = 0; f < FM; f++)
#pragma unroll
                        for (int j = 0; j < NA; j++)
                            acc[f][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[ky][j], bv[f * S + ky], acc[f][j],
                                                                               0, 0, 0);
            }
    };
    // chunk c has landed for this wave when at most the DMA of the `after` chunks issued after it is outstanding
    // (vmcnt counts in issue order; in the first round the residual and parameter loads queue behind chunk
    // cbeg + ST - 2, which then has to land too: conservative), then for every wave. The barrier
    // carries no release fence (one would wait for every DMA in flight): the wave's LDS reads are complete
    // (lgkmcnt(0)) and its LDS writes happen only before the last chunk, behind a full barrier of their own; the
    // acquire fence keeps later LDS reads below the barrier.
    auto landed = [&](int after) {
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (ST >= 3) {
            if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER) & ~0x0F00);  // and lgkmcnt(0)
        }
        if (after == 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~0x0F00);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };

    // the ring: chunk cbeg + q lives in buffer q % ST; chunk c + ST - 1 goes out into the buffer chunk c - 1 used,
    // once every wave is past the barrier of chunk c (done reading it)
    for (int c = cbeg;; c += ST) {
        bool done = false;
#pragma unroll
        for (int u = 0; u < ST; u++) {
            const int cc = c + u;
            landed(min(ST - 2, cend - 1 - cc));
            if (cc == nch - 1) {
                fix_partial(u);
                __syncthreads();
            }
            if (cc + ST - 1 < cend) dma_chunk((u + ST - 1) % ST, cc + ST - 1);
            compute(u);
            if (cc + 1 >= cend) {
                done = true;
                break;
            }
        }
        if (done) break;
    }

    const size_t mtot = (size_t)a.n * a.hout * a.wout;
#pragma unroll
    for (int f = 0; f < FM; f++) {
        const int oy = oy0 + wm * FM + f, ox = ox0 + lx;
        if (oy < a.hout && ox < a.wout) {
            const size_t pix = ((size_t)img * a.hout + oy) * a.wout + ox;
#pragma unroll
            for (int j = 0; j < NA; j++) {
                if (co + 16 * j >= a.cout) continue;
                if (split)
                    *reinterpret_cast<f4*>(a.part + ((size_t)blockIdx.z * mtot + pix) * a.np + co + 16 * j) = acc[f][j];
                else
                    epilogue4r(a, pix, co + 16 * j, acc[f][j], bias[j], neg[j], rres[f][j]);
            }
        }
    }
}

// Whether the kernel's input path serves these views: 16-byte aligned groups, offsets below 2^31.
inline bool gemm_path_ok(const ConvKArgs& a) {
    return a.xvec && (uint64_t)a.n * a.h * a.w * a.xcs * 2 < (1ull << 31);
}

// The chunked kernel's configuration that stands in on views the DMA path cannot read: 8 rows x 16 channels, which
// divides every np; same packed weights (chunks of cc = CK channels), same split.
constexpr int kGemmFallbackCfg = 3;

template <int S, int CK, int FM, int NA, int WM, int WN, int ST>
hipError_t launch_gemm(const ConvKArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    (void)lds;
    if (gemm_path_ok(a)) {
        hipLaunchKernelGGL((conv_gemm<S, CK, FM, NA, WM, WN, ST>), grid, dim3(64 * WM * WN), 0, s, a);
        return hipGetLastError();
    }
    constexpr TileCfg t = kTileCfgs[kGemmFallbackCfg];
    constexpr int TH = t.fm * t.wm, BN = t.fn * 16 * t.wn;
    ConvKArgs b = a;
    b.tiles_y = (a.hout + TH - 1) / TH;
    b.ntn = a.np / BN;
    const size_t ih = (size_t)(TH - 1) * S + 3, iw = (size_t)15 * S + 3;
    const size_t flds = (((size_t)b.tapgroups * 4 + 15) & ~(size_t)15) + ih * iw * (size_t)(b.cc + 8) * 2;
    const dim3 fgrid((unsigned)((size_t)b.n * b.tiles_y * b.tiles_x * b.ntn), grid.z, 1);
    return conv_launcher(3, S, kGemmFallbackCfg)(b, fgrid, flds, s);
}

template <int S, int CK, int FM, int NA, int WM, int WN, int ST>
const void* gemm_kernel() {
    return reinterpret_cast<const void*>(&conv_gemm<S, CK, FM, NA, WM, WN, ST>);
}

}  // namespace fhc
