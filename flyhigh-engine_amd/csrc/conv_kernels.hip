// The conv kernels for gfx950 (MI355X): an implicit-GEMM 3x3 / 1x1 convolution on v_mfma_f32_16x16x32_f16 with
// f32 accumulation, reading NHWC f16 activations through a halo tile in LDS and writing f16 through a fused
// bias + PReLU / LeakyReLU + residual epilogue.
//
// GEMM view (the reference's, shaders/conv_tiled.wgsl:4-5): Out[pixel][co] = sum_k X[pixel][k] * W[k][co]. Here the
// MFMA's A operand is the weights (rows = output channels) and its B operand the activations (columns = pixels), so
// the accumulator gives each lane 4 consecutive output channels of one pixel: NHWC stores of 8 bytes per lane.
//
// Per workgroup: an output tile of TH rows x 16 columns x BN channels. For each chunk of `cc` input channels the
// workgroup stages the input halo tile ((TH-1)*S+KS) x (15*S+KS) pixels x cc channels into LDS once (128-bit loads,
// zero padding and channel tails written as zeros: the caller's buffers are never assumed zeroed), and every tap
// (ky, kx) then reads its shifted window from LDS: im2col happens in the LDS addressing, nothing is materialised.
// K order inside a chunk: k = tap * cc + ci, walked in 8-channel groups; a per-chunk table maps group j to its LDS
// offset, so one K-step of 32 may span two taps and cin needs padding to 8 only.
//
// Weights arrive pre-packed (api.cpp) in A-fragment order: for 16-channel block nb, chunk c, K-step s, lane l the
// 8 halves W[co = nb*16 + l%16][k = 32*s + 8*(l/16) + i], i = 0..7: one coalesced 16-byte load per lane.
//
// Split-K: WK > 1 waves of one workgroup take interleaved K-steps of the same tile and are summed through LDS
// before the epilogue; a global split (grid.y = z) instead writes f32 partials that splitk_reduce sums in z order.
#include "conv_kernels.h"
#include "direct_impl.h"
#include "direct_table.h"
#include "gm_fit.h"

namespace fhc {

// bias, activation, f16 round, residual (rounded again), store: 4 consecutive channels co..co+3 of pixel `pix`.
// The order is the reference's epilogue (shaders/conv_tiled.wgsl:57-67; splitk_reduce.wgsl:21-23).
__device__ __forceinline__ void epilogue4(const ConvKArgs& a, size_t pix, int co, f4 v) {
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o[i] = f2h(activate(v[i] + h2f(a.bias[co + i]), a.neg[co + i]));
    }
    const bool full = co + 4 <= a.cout;
    if (a.residual) {
        const uint16_t* rp = a.res + pix * (size_t)a.rcs + a.rc0 + co;
        uint16_t rv[4];
        if (a.rvec && full) {
            const uint2 q = *reinterpret_cast<const uint2*>(rp);
            rv[0] = (uint16_t)(q.x & 0xffffu);
            rv[1] = (uint16_t)(q.x >> 16);
            rv[2] = (uint16_t)(q.y & 0xffffu);
            rv[3] = (uint16_t)(q.y >> 16);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) rv[i] = co + i < a.cout ? rp[i] : (uint16_t)0;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = f2h(h2f(o[i]) + h2f(rv[i]));
    }
    uint16_t* yp = a.y + pix * (size_t)a.ycs + a.yc0 + co;
    if (a.yvec && full) {
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

template <int KS, int S, int FM, int FN, int WM, int WN, int WK>
__global__ __launch_bounds__(64 * WM * WN * WK) void conv_igemm(ConvKArgs a) {
    constexpr int TH = FM * WM, TW = 16, BN = FN * 16 * WN, NT = 64 * WM * WN * WK;
    constexpr int IH = (TH - 1) * S + KS, IW = (TW - 1) * S + KS;
    extern __shared__ __align__(16) unsigned char smem[];
    int* toff = reinterpret_cast<int*>(smem);
    const int tabn = a.tapgroups;
    uint16_t* halo = reinterpret_cast<uint16_t*>(smem + ((tabn * 4 + 15) & ~15));
    const int pstr = a.cc + 8;  // LDS pixel stride in halves (8 halves of padding against bank conflicts)
    const int gpt = a.cc >> 3;  // 8-channel groups per pixel in a chunk

    int bid = blockIdx.x;
    const int nt = bid % a.ntn;
    bid /= a.ntn;
    const int tx = bid % a.tiles_x;
    bid /= a.tiles_x;
    const int ty = bid % a.tiles_y;
    const int img = bid / a.tiles_y;
    const int z = blockIdx.y;
    const int oy0 = ty * TH, ox0 = tx * TW;
    const int iy0 = oy0 * S - a.pad, ix0 = ox0 * S - a.pad;
    const int co0 = nt * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wk = wave % WK, wmn = wave / WK, wn = wmn % WN, wm = wmn / WN;

    for (int j = tid; j < tabn; j += NT) {
        const int tap = j / gpt, g = j - tap * gpt;
        const int ky = tap / KS, kx = tap - ky * KS;
        toff[j] = (ky * IW + kx) * pstr + g * 8;
    }
    int pb[FM];
#pragma unroll
    for (int f = 0; f < FM; f++) pb[f] = (((wm * FM + f) * S) * IW + (lane & 15) * S) * pstr;

    f4 acc[FM][FN];
#pragma unroll
    for (int f = 0; f < FM; f++)
#pragma unroll
        for (int q = 0; q < FN; q++) acc[f][q] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    const h8* wp = reinterpret_cast<const h8*>(a.wpk);
    const size_t nb_stride = (size_t)a.nchunks * a.ksteps * 64;
    const int nb0 = (co0 >> 4) + wn * FN;
    const int c_begin = z * a.chunks_per_split;
    const int c_end = min(c_begin + a.chunks_per_split, a.nchunks);
    const size_t img_base = (size_t)img * a.h;

    for (int c = c_begin; c < c_end; ++c) {
        __syncthreads();  // the table is written (first chunk) / the previous chunk's readers are done
        const int total = IH * IW * gpt;
        const int cbase = c * a.cc;
        for (int e = tid; e < total; e += NT) {
            const int pix = e / gpt, g = e - pix * gpt;
            const int iy = pix / IW, ix = pix - iy * IW;
            const int gy = iy0 + iy, gx = ix0 + ix, ch = cbase + g * 8;
            uint4 v = {0u, 0u, 0u, 0u};
            if (gy >= 0 && gy < a.h && gx >= 0 && gx < a.w && ch < a.cin) {
                const uint16_t* p = a.x + ((img_base + gy) * a.w + gx) * (size_t)a.xcs + a.xc0 + ch;
                if (a.xvec && ch + 8 <= a.cin) {
                    v = *reinterpret_cast<const uint4*>(p);
                } else {
                    uint32_t t[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        if (ch + i < a.cin) t[i >> 1] |= (uint32_t)p[i] << ((i & 1) * 16);
                    v = uint4{t[0], t[1], t[2], t[3]};
                }
            }
            *reinterpret_cast<uint4*>(halo + pix * pstr + g * 8) = v;
        }
        __syncthreads();
        const h8* wc = wp + (size_t)c * a.ksteps * 64 + lane;
        for (int s = wk; s < a.ksteps; s += WK) {
            const int j = 4 * s + (lane >> 4);
            const bool valid = j < tabn;
            const int off = valid ? toff[j] : 0;
            h8 bx[FM];
#pragma unroll
            for (int f = 0; f < FM; f++) {
                bx[f] = *reinterpret_cast<const h8*>(halo + pb[f] + off);
                if (!valid) bx[f] = h8{0, 0, 0, 0, 0, 0, 0, 0};
            }
            h8 aw[FN];
#pragma unroll
            for (int q = 0; q < FN; q++) aw[q] = wc[(size_t)(nb0 + q) * nb_stride + (size_t)s * 64];
#pragma unroll
            for (int f = 0; f < FM; f++)
#pragma unroll
                for (int q = 0; q < FN; q++)
                    acc[f][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[q], bx[f], acc[f][q], 0, 0, 0);
        }
    }

    if constexpr (WK > 1) {
        // intra-workgroup split-K: waves wk > 0 hand their partial tiles to wave wk == 0 through LDS
        f4* red = reinterpret_cast<f4*>(smem);
        __syncthreads();
        if (wk > 0) {
#pragma unroll
            for (int f = 0; f < FM; f++)
#pragma unroll
                for (int q = 0; q < FN; q++)
                    red[((((wk - 1) * WM * WN + wmn) * FM + f) * FN + q) * 64 + lane] = acc[f][q];
        }
        __syncthreads();
        if (wk > 0) return;
#pragma unroll
        for (int k = 1; k < WK; k++)
#pragma unroll
            for (int f = 0; f < FM; f++)
#pragma unroll
                for (int q = 0; q < FN; q++) acc[f][q] += red[((((k - 1) * WM * WN + wmn) * FM + f) * FN + q) * 64 + lane];
    }

    const bool split = gridDim.y > 1;
    const size_t mtot = (size_t)a.n * a.hout * a.wout;
#pragma unroll
    for (int f = 0; f < FM; f++) {
        const int oy = oy0 + wm * FM + f, ox = ox0 + (lane & 15);
        if (oy >= a.hout || ox >= a.wout) continue;
        const size_t pix = ((size_t)img * a.hout + oy) * a.wout + ox;
#pragma unroll
        for (int q = 0; q < FN; q++) {
            const int co = co0 + (wn * FN + q) * 16 + 4 * (lane >> 4);
            if (co >= a.cout) continue;
            if (split)
                *reinterpret_cast<f4*>(a.part + ((size_t)z * mtot + pix) * a.np + co) = acc[f][q];
            else
                epilogue4(a, pix, co, acc[f][q]);
        }
    }
}

// Finish a global split-K: sum the f32 partials in z order (the reference's splitk_reduce.wgsl:17-18), then the
// epilogue. One thread per 4 consecutive output channels of one pixel.
__global__ __launch_bounds__(256) void splitk_reduce(ConvKArgs a, int ksplit) {
    const int cq = (a.cout + 3) >> 2;
    const size_t mtot = (size_t)a.n * a.hout * a.wout;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= mtot * cq) return;
    const size_t pix = idx / cq;
    const int co = (int)(idx - pix * cq) * 4;
    f4 s = *reinterpret_cast<const f4*>(a.part + pix * a.np + co);
    for (int z = 1; z < ksplit; z++) s += *reinterpret_cast<const f4*>(a.part + ((size_t)z * mtot + pix) * a.np + co);
    epilogue4(a, pix, co, s);
}

template <int KS, int S, int CFG>
hipError_t launch_cfg(const ConvKArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    constexpr TileCfg c = kTileCfgs[CFG];
    auto k = conv_igemm<KS, S, c.fm, c.fn, c.wm, c.wn, c.wk>;
    hipLaunchKernelGGL(k, grid, dim3(64 * c.wm * c.wn * c.wk), lds, s, a);
    return hipGetLastError();
}

template <int KS, int S>
LaunchFn pick(int cfg) {
    switch (cfg) {
        case 1: return launch_cfg<KS, S, 1>;
        case 2: return launch_cfg<KS, S, 2>;
        case 3: return launch_cfg<KS, S, 3>;
        case 4: return launch_cfg<KS, S, 4>;
        case 5: return launch_cfg<KS, S, 5>;
        case 6: return launch_cfg<KS, S, 6>;
        case 7: return launch_cfg<KS, S, 7>;
        case 8: return launch_cfg<KS, S, 8>;
        case 9: return launch_cfg<KS, S, 9>;
        case 10: return launch_cfg<KS, S, 10>;
        default: return nullptr;
    }
}

LaunchFn conv_launcher(int ks, int stride, int cfg) {
    if (ks == 3 && stride == 1) return pick<3, 1>(cfg);
    if (ks == 3 && stride == 2) return pick<3, 2>(cfg);
    if (ks == 1 && stride == 1) return pick<1, 1>(cfg);
    return nullptr;
}

hipError_t splitk_reduce_launch(const ConvKArgs& a, int ksplit, hipStream_t s) {
    const size_t total = (size_t)a.n * a.hout * a.wout * ((a.cout + 3) / 4);
    hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a, ksplit);
    return hipGetLastError();
}

// The sibling convs' configurations, 33-64 input channels, 2 or 3 channel blocks (the frame's fine.out + up.w:
// 48 -> 7 + 36): one row of 16 pixels with the kernel-row K split (3 waves per channel block, the configuration the
// committed choice table gives both), or two rows without it (the K order of the planner's default for both)
constexpr int find_direct(int ks, int s, int cin32, int fm, int wm, int wn, int na, int wk) {
    for (int i = 0; i < kNumDirect; i++) {
        const DirectCfg& c = kDirectCfgs[i];
        if (c.ks == ks && c.stride == s && c.cin32 == cin32 && c.fm == fm && c.wm == wm && c.wn == wn && c.na == na &&
            c.wk == wk && !c.persist)
            return i;
    }
    return -1;
}

LaunchFn sibling_launcher(int index) {
    constexpr int k64_2 = find_direct(3, 1, 64, 1, 1, 2, 1, 3), k64_3 = find_direct(3, 1, 64, 1, 1, 3, 1, 3);
    constexpr int r64_2 = find_direct(3, 1, 64, 1, 2, 2, 1, 1), r64_3 = find_direct(3, 1, 64, 1, 2, 3, 1, 1);
    static_assert(k64_2 >= 0 && k64_3 >= 0 && r64_2 >= 0 && r64_3 >= 0, "sibling configurations in the table");
    if (index < 0) return nullptr;
    if (index == k64_2) return launch_tile_split<3, 1, 64, 1, 1, 2, 3>;
    if (index == k64_3) return launch_tile_split<3, 1, 64, 1, 1, 3, 3>;
    if (index == r64_2) return launch_tile_split<3, 1, 64, 1, 2, 2, 1>;
    if (index == r64_3) return launch_tile_split<3, 1, 64, 1, 2, 3, 1>;
    return nullptr;
}

namespace {

template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK>
union FitTileLds {
    gmfit::RoundLds fit;
    TileLds<KS, S, CIN32, FM, WM, WN, WK> tile;
};

// one fit round of the repair (workgroups 0-127, gm_fit.h at 192 threads) and a conv plan's workgroups (the rest:
// tile t, channel tile ct at 128 + t + tiles * ct) in one launch
template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK, bool VEC>
__global__ __launch_bounds__(192) void fit_conv_kernel(FitRoundArgs f, ConvKArgs a, uint32_t tiles) {
    static_assert(64 * WM * WN * WK == 192, "the conv's workgroup is 192 threads");
    constexpr uint32_t NFIT = gmfit::kNwg * 4;
    __shared__ __align__(16) FitTileLds<KS, S, CIN32, FM, WM, WN, WK> lds;
    if (blockIdx.x < NFIT) {  // uniform over the workgroup
        gmfit::round_body<192>(f.flow, f.cs, f.c0, f.h8, f.w8, f.delta, f.round, f.part_in, f.part_out,
                               blockIdx.x % gmfit::kNwg, blockIdx.x / gmfit::kNwg, lds.fit);
    } else {
        const uint32_t b = blockIdx.x - NFIT;
        conv_tile_body<KS, S, CIN32, FM, WM, WN, WK, VEC>(a, (int)(b % tiles), (int)(b / tiles), lds.tile);
    }
}

template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK>
hipError_t fit_conv_launch(const FitRoundArgs& f, const ConvKArgs& a, dim3 cg, hipStream_t s) {
    const dim3 grid(gmfit::kNwg * 4 + cg.x * cg.y);
    if (a.xvec)
        hipLaunchKernelGGL((fit_conv_kernel<KS, S, CIN32, FM, WM, WN, WK, true>), grid, dim3(192), 0, s, f, a, cg.x);
    else
        hipLaunchKernelGGL((fit_conv_kernel<KS, S, CIN32, FM, WM, WN, WK, false>), grid, dim3(192), 0, s, f, a, cg.x);
    return hipGetLastError();
}

}  // namespace

FitConvLaunchFn fit_conv_launcher(int index) {
    // the FiLM head's output conv (48 -> 5 at one row of 16 pixels per workgroup, the kernel-row split)
    constexpr int k64_1 = find_direct(3, 1, 64, 1, 1, 1, 1, 3);
    static_assert(k64_1 >= 0, "the FiLM output conv's configuration");
    if (index == k64_1) return fit_conv_launch<3, 1, 64, 1, 1, 1, 3>;
    return nullptr;
}

}  // namespace fhc
