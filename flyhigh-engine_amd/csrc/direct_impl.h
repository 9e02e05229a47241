// The direct conv kernel for layers whose input channels fit one pass (cin padded to 32 <= 128): the weights of a
// wave's 16 output channels stay in VGPRs for the whole launch, input tiles stream through a halo tile in LDS.
//
// Workgroup: WN x WM waves; wave (wn, wm) owns output channels [16 wn, 16 wn + 16) of the workgroup's channel
// tile and FM output rows of 16 pixels. Per spatial tile (TH = FM * WM rows x 16 columns) the workgroup writes the
// input halo ((TH-1)*S + KS) x (15*S + KS) x CIN32 into LDS (zero outside the image and beyond cin), then each
// wave runs KSTEPS = KS*KS*CIN32/32 MFMA K-steps reading its shifted windows from LDS. K order: k = tap * CIN32 + ci
// (channels padded to 32 per tap), so K-step s is tap s / M, channels 32 (s % M) .. +31 with M = CIN32 / 32, and
// lane group l/16 reads channels +8 (l/16): every LDS read is a per-row base register plus a compile-time offset.
// The weights were packed in the same order (api.cpp, pack_weights).
// One workgroup per spatial tile (blockIdx.x) and channel tile (blockIdx.y). Every global load the tile needs
// (weights, halo, residual, bias) is issued before the first wait, so a tile costs one memory round trip; the
// registers of the staging are dead before the MFMA chain, which reads LDS one K-step ahead of the MFMAs.
#pragma once
#include "conv_kernels.h"

namespace fhc {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// bias, activation, f16 round, residual add rounded again (shaders/conv_tiled.wgsl:57-67), store of 4
// consecutive channels co..co+3 of output pixel `pix`. rv: the residual's 4 halves (ignored without residual).
__device__ __forceinline__ void epilogue4r(const ConvKArgs& a, size_t pix, int co, f4 v, const float* b,
                                          const float* sl, uint2 rv) {
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float t = v[i] + b[i];
        if (a.act == 1)
            t = t > 0.0f ? t : sl[i] * t;
        else if (a.act == 2)
            t = t > 0.0f ? t : a.alpha * t;
        o[i] = f2h(t);
    }
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

// the residual's 4 halves at (pix, co..co+3), zeros past cout
__device__ __forceinline__ uint2 load_res4(const ConvKArgs& a, size_t pix, int co) {
    const uint16_t* rp = a.res + pix * (size_t)a.rcs + a.rc0 + co;
    if (a.rvec && co + 4 <= a.cout) return *reinterpret_cast<const uint2*>(rp);
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = co + i < a.cout ? rp[i] : 0u;
    return uint2{r[0] | (r[1] << 16), r[2] | (r[3] << 16)};
}

// 8 consecutive input channels ch..ch+7 of one pixel (p points at channel ch), zeros at and past cin. VEC: the
// view is 16-byte aligned (cstride, c0 multiples of 8), so a full group is one 16-byte load; a partial group (and
// every group without VEC) is 8 independent 2-byte loads at clamped in-bounds addresses, selected without branches.
template <bool VEC>
__device__ __forceinline__ uint4 load_group(const uint16_t* p, int ch, int cin) {
    const int rem = cin - ch;
    if (VEC && rem >= 8) return *reinterpret_cast<const uint4*>(p);
    uint32_t q[4];
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        const uint32_t lo = p[min(k, rem - 1)], hi = p[min(k + 1, rem - 1)];
        q[k >> 1] = (k < rem ? lo : 0u) | ((k + 1 < rem ? hi : 0u) << 16);
    }
    return uint4{q[0], q[1], q[2], q[3]};
}

template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK, bool VEC>
__global__ __launch_bounds__(64 * WM * WN * WK) void conv_direct(ConvKArgs a) {
    static_assert(WK == 1 || (WK == 3 && KS == 3), "the K split runs one kernel row per wave");
    constexpr int TH = FM * WM, TW = 16, BN = 16 * WN, NT = 64 * WM * WN * WK;
    constexpr int IH = (TH - 1) * S + KS, IW = (TW - 1) * S + KS;
    constexpr int GPT = CIN32 / 8, PSTR = CIN32 + 8, M = CIN32 / 32;
    constexpr int KSTEPS = KS * KS * M, KW = KSTEPS / WK;  // K-steps of the whole conv / of one wave
    constexpr int HALO = IH * IW * GPT, NLD = (HALO + NT - 1) / NT;
    constexpr int HALO_BYTES = IH * IW * PSTR * 2, RED_BYTES = (WK - 1) * WM * WN * FM * 64 * 16;
    __shared__ __align__(16) uint16_t halo[(HALO_BYTES > RED_BYTES ? HALO_BYTES : RED_BYTES) / 2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wk = wave / (WM * WN), wmn = wave - wk * (WM * WN);
    const int wn = wmn % WN, wm = wmn / WN;
    const int co_w = blockIdx.y * BN + wn * 16;
    const int co = co_w + 4 * (lane >> 4);  // the lane's 4 output channels in the accumulator
    const int t = blockIdx.x;
    const int tx = t % a.tiles_x, r = t / a.tiles_x;
    const int ty = r % a.tiles_y, img = r / a.tiles_y;
    const int oy0 = ty * TH, ox0 = tx * TW;

    // every global load of the tile is issued before the first wait: weights (this wave's K-steps), input halo,
    // residual, bias
    h8 wr[KW];
    {
        const h8* wp = reinterpret_cast<const h8*>(a.wpk) + ((size_t)(co_w >> 4) * KSTEPS + wk * KW) * 64 + lane;
#pragma unroll
        for (int s = 0; s < KW; s++) wr[s] = wp[s * 64];
    }
    uint4 pre[NLD];
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
                        a.x + (((size_t)img * a.h + gy) * a.w + gx) * (size_t)a.xcs + a.xc0 + ch, ch, a.cin);
        }
    }
    uint2 rres[FM];
#pragma unroll
    for (int f = 0; f < FM; f++) {
        rres[f] = uint2{0u, 0u};
        const int oy = oy0 + wm * FM + f, ox = ox0 + (lane & 15);
        if (wk == 0 && a.residual && oy < a.hout && ox < a.wout && co < a.cout)
            rres[f] = load_res4(a, ((size_t)img * a.hout + oy) * a.wout + ox, co);
    }
    float bias[4], slope[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        bias[i] = h2f(a.bias[co + i]);
        slope[i] = h2f(a.slope[co + i]);
    }

#pragma unroll
    for (int i = 0; i < NLD; i++) {
        const int e = tid + i * NT;
        if ((i + 1) * NT <= HALO || e < HALO) {
            const int pix = e / GPT, g = e - pix * GPT;
            *reinterpret_cast<uint4*>(halo + pix * PSTR + g * 8) = pre[i];
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

    if (co < a.cout) {
#pragma unroll
        for (int f = 0; f < FM; f++) {
            const int oy = oy0 + wm * FM + f, ox = ox0 + (lane & 15);
            if (oy < a.hout && ox < a.wout)
                epilogue4r(a, ((size_t)img * a.hout + oy) * a.wout + ox, co, acc[f], bias, slope, rres[f]);
        }
    }
}

// launches the 16-byte-load instantiation when the input view allows it (args.xvec), else the 2-byte one
template <int KS, int S, int CIN32, int FM, int WM, int WN, int WK>
hipError_t launch_direct(const ConvKArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    (void)lds;
    const dim3 block(64 * WM * WN * WK);
    if (a.xvec)
        hipLaunchKernelGGL((conv_direct<KS, S, CIN32, FM, WM, WN, WK, true>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((conv_direct<KS, S, CIN32, FM, WM, WN, WK, false>), grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace fhc
