// Two 3x3 convs fused into one launch, B after A (B: stride 1, pad 1, reading A's output), with A's output tile
// kept in LDS: the chains of small layers that a frame runs back to back (the encoder's conv pairs, the FiLM and
// refine heads, the fine block) pay one launch and one round of weight and halo loads instead of two.
//
// One workgroup per output tile of B: TH rows x 14 columns. B's 16-pixel MFMA column block then reads 16 + 2
// columns of A's output, so A is computed on (TH + 2) rows x 16 columns (one MFMA column block) around the tile,
// from an input halo of ((TH + 1) * SA + 3) x (15 * SA + 3) pixels. A's output is rounded to f16 as the unfused
// path stores it, and written to LDS as zero outside the image (B's zero padding), so both layers compute exactly
// what the two separate launches compute.
//
// WN x WM waves, WN = max(NBA, NBB): wave (wn, wm) runs A's 16-channel block wn (if wn < NBA) over its share
// (1 / WM) of A's rows, then B's block wn (if wn < NBB) over its share of B's rows, weights of both resident in
// registers (WM = 2 halves the chains and doubles the workgroup's weight loads). K order, packing and LDS pixel stride are
// those of direct_impl.h (k = tap * CIN32 + ci, channels padded to 32 per tap, pixel stride CIN32 + 8 halves).
// B's residual is either the external tensor of the descriptor or A's output at the same pixel (read from LDS).
#pragma once
#include "direct_impl.h"

namespace fhc {

// The value, made opaque to the optimizer (an empty asm that takes and returns it in VGPRs): a select between a
// value loaded from LDS and a register array element is otherwise rewritten into one load from a select of the
// two addresses, which puts the register array in scratch memory and reads it through a flat load.
__device__ __forceinline__ uint2 opaque_u2(uint2 v) {
    asm volatile("" : "+v"(v.x), "+v"(v.y));
    return v;
}

// The q-ring MFMA chain over an LDS tile (as direct_impl.h's WK == 1 chain, one channel block): output rows
// f = 0 .. FM-1 of stride S read tile rows f * S + ky; operand q = (kx * M + m) * R + r is read once and feeds every
// (f, ky) use; reads run D operands ahead. base: the lane's pixel (row 0, column (lane & 15) * S) and channel group.
template <int FM, int S, int M, int IW, int PSTR>
__device__ __forceinline__ void pair_chain(f4 (&acc)[FM], const h8* wr, const uint16_t* base) {
    constexpr int KS = 3, R = (FM - 1) * S + KS, NQ = KS * M * R, D = NQ < 4 ? NQ : 4;
    auto rd = [&](int q) {
        const int c = q / R, r = q % R, kx = c / M, m = c % M;
        return *reinterpret_cast<const h8*>(base + (r * IW + kx) * PSTR + m * 32);
    };
#pragma unroll
    for (int f = 0; f < FM; f++) acc[f] = f4{0.0f, 0.0f, 0.0f, 0.0f};
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
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wr[(ky * KS + kx) * M + m], b[q % (D + 1)], acc[f], 0, 0, 0);
        }
    }
    pin_mfma_pipeline<0, NQ, D, R, FM, S, KS, 1, 0>();
}

// A's K-steps for CP input channels per tap: CP = 32 one tap per 32-wide K-step (M = CA32 / 32 steps per tap); CP
// = 8 or 16 (at most that many input channels): 32 / CP taps packed into each K-step, 3 or 5 steps for the 9 taps
template <int CP, int MA>
constexpr int pair_ksteps() { return CP == 32 ? 9 * MA : (9 + 32 / CP - 1) / (32 / CP); }

// The chain of A over an LDS tile with CP < 32: K-step s holds taps s * T .. s * T + T - 1 (T = 32 / CP), tap t's
// input channels c in K positions (t - s * T) * CP + c. Lane group g (lane >> 4) feeds 8 of them: channels
// (g % (CP / 8)) * 8 .. +7 of tap s * T + g / (CP / 8), one 16-byte LDS read at the lane's pixel shifted by the
// tap; past the 9th tap (zero weights) it reads channels CP .. CP + 7 of the lane's own pixel, zero in the staged
// halo (at most CP input channels), so no value of the tensor meets a padding weight. base: the lane's pixel (row
// 0, column (lane & 15) * S), channel 0. Output rows f = 0 .. FM - 1 read tile rows f * S + ky.
template <int FM, int S, int CP, int IW, int PSTR>
__device__ __forceinline__ void tap_chain(f4 (&acc)[FM], const h8* wr, const uint16_t* base, int g) {
    constexpr int T = 32 / CP, KS = pair_ksteps<CP, 1>(), GPT = CP / 8;
    static_assert(CP == 8 || CP == 16, "8 or 16 channels per tap");
    const int tg = g / GPT, c8 = (g % GPT) * 8;
    int off[KS];
#pragma unroll
    for (int s = 0; s < KS; s++) {
        const int tap = s * T + tg;
        off[s] = tap < 9 ? ((tap / 3) * IW + tap % 3) * PSTR + c8 : CP;
    }
    h8 v[KS][FM];
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
        for (int f = 0; f < FM; f++) v[s][f] = *reinterpret_cast<const h8*>(base + f * S * IW * PSTR + off[s]);
#pragma unroll
    for (int f = 0; f < FM; f++) acc[f] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
        for (int f = 0; f < FM; f++) acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wr[s], v[s][f], acc[f], 0, 0, 0);
}

// A's chain: per tap (pair_chain) at CP = 32, taps packed (tap_chain) below
template <int FM, int S, int MA, int CP, int IW, int PSTR>
__device__ __forceinline__ void a_chain(f4 (&acc)[FM], const h8* wr, const uint16_t* px, int lane) {
    if constexpr (CP == 32) pair_chain<FM, S, MA, IW, PSTR>(acc, wr, px + (lane >> 4) * 8);
    else tap_chain<FM, S, CP, IW, PSTR>(acc, wr, px, lane >> 4);
}

// film_modulate (film.wgsl) on one staged 8-channel group: channel j < n becomes f16(v * gm[j] + bt[j]) with
// gm = 1 + gamma, bt = beta in f32, as the op computes it; channels past n stay as they are (zero)
__device__ __forceinline__ uint4 film_group(uint4 q, const float* gm, const float* bt, int n) {
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t lo = w[k] & 0xffffu, hi = w[k] >> 16;
        if (2 * k < n) lo = f2h(h2f((uint16_t)lo) * gm[2 * k] + bt[2 * k]);
        if (2 * k + 1 < n) hi = f2h(h2f((uint16_t)hi) * gm[2 * k + 1] + bt[2 * k + 1]);
        w[k] = lo | (hi << 16);
    }
    return uint4{w[0], w[1], w[2], w[3]};
}

// The LDS of one conv_pair tile: A's input halo, A's output tile
template <int SA, int CA32, int CB32, int TH>
struct PairLds {
    static constexpr int IHA = (TH + 1) * SA + 3, IWA = 15 * SA + 3, PSA = CA32 + 8, MW = 18, PSB = CB32 + 8;
    uint16_t hin[IHA * IWA * PSA];
    uint16_t mid[(TH + 2) * MW * PSB];
};

// FILM: A's input goes through film_modulate as it is staged (a.film, the one-tile loop only). The body of one
// tile t (conv_pair's workgroup t; a launch that runs other work beside the pair passes its own numbering) in the
// workgroup's LDS L; the block is 64 * WN * WM threads.
template <int SA, int CA32, int CB32, int NBA, int NBB, int TH, int WM, bool VEC, bool FILM = false, int CPA = 32>
__device__ __forceinline__ void conv_pair_tile(const PairKArgs& pk, const int t, PairLds<SA, CA32, CB32, TH>& L) {
    constexpr int WN = NBA > NBB ? NBA : NBB, NT = 64 * WN * WM, TWB = kPairTileW;
    constexpr int FA = TH + 2;                                  // A's rows per tile
    constexpr int FAW = FA / WM, THW = TH / WM;                 // rows per wave
    static_assert(FA % WM == 0 && TH % WM == 0, "rows split evenly over the wave rows");
    constexpr int IHA = (FA - 1) * SA + 3, IWA = 15 * SA + 3;   // A's input halo
    constexpr int GPA = CA32 / 8, PSA = CA32 + 8, MA = CA32 / 32, KA = pair_ksteps<CPA, MA>();
    constexpr int MW = 18, PSB = CB32 + 8, MB = CB32 / 32;     // A's output tile in LDS: FA rows x 18 pixels
    constexpr int HALO = IHA * IWA * GPA, NLD = (HALO + NT - 1) / NT;
    static_assert(NBA * 16 <= CB32, "A's channel blocks exceed B's input channels");
    static_assert(CPA == 32 || CA32 == 32, "packed taps read the zero channels CPA .. CPA + 7 of the staged halo");
    static_assert(sizeof(L.hin) == IHA * IWA * PSA * 2 && sizeof(L.mid) == FA * MW * PSB * 2, "the tile's LDS");
    uint16_t* const hin = L.hin;
    uint16_t* const mid = L.mid;
    const ConvKArgs& a = pk.a;
    const ConvKArgs& b = pk.b;

    const int tid = threadIdx.x, lane = tid & 63, wn = (tid >> 6) % WN, wm = (tid >> 6) / WN, lx = lane & 15;
    const int tx = t % b.tiles_x, rr = t / b.tiles_x;
    const int ty = rr % b.tiles_y, img = rr / b.tiles_y;
    const int oy0 = ty * TH, ox0 = tx * TWB;  // B's tile origin; A's tile starts one row and column earlier
    const int wa = wn < NBA ? wn : NBA - 1, wb = wn < NBB ? wn : NBB - 1;  // loads stay unconditional
    const int coa = wa * 16 + 4 * (lane >> 4), cob = wb * 16 + 4 * (lane >> 4);

    // every global load first: both layers' weights, A's input halo, B's external residual, biases, multipliers
    h8 wra[KA], wrb[9 * MB];
    {
        const h8* wp = reinterpret_cast<const h8*>(a.wpk) + (size_t)wa * KA * 64 + lane;
#pragma unroll
        for (int s = 0; s < KA; s++) wra[s] = wp[s * 64];
        const h8* wq = reinterpret_cast<const h8*>(b.wpk) + (size_t)wb * 9 * MB * 64 + lane;
#pragma unroll
        for (int s = 0; s < 9 * MB; s++) wrb[s] = wq[s * 64];
    }
    uint4 pre[NLD];
    uint32_t inside = 0;  // bit i: pre[i] holds input values (not the zero padding)
    static_assert(NLD <= 32 && NT % GPA == 0, "a lane stages the same channel group in every round");
    const bool whole = VEC && a.xc0 + ((a.cin + 7) & ~7) <= a.xcs;  // partial groups load as one 16-byte group
    {
        const int iy0 = (oy0 - 1) * SA - a.pad, ix0 = (ox0 - 1) * SA - a.pad;
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = tid + i * NT;
            const int pix = e / GPA, g = e - pix * GPA;
            const int iy = pix / IWA, ix = pix - iy * IWA;
            const int gy = iy0 + iy, gx = ix0 + ix, ch = g * 8;
            pre[i] = uint4{0u, 0u, 0u, 0u};
            if ((i + 1) * NT <= HALO || e < HALO)
                if (gy >= 0 && gy < a.h && gx >= 0 && gx < a.w && ch < a.cin) {
                    pre[i] = load_group<VEC>(
                        a.x + (((size_t)img * a.h + gy) * a.w + gx) * (size_t)a.xcs + a.xc0 + ch, ch, a.cin, whole);
                    if constexpr (FILM) inside |= 1u << i;
                }
        }
    }
    // FiLM on A's input (film_modulate, graph op 50, before film.h1): this lane's channel group tid % GPA, the
    // tile's image's vector; the zero padding stays zero, as the modulated tensor's padding is
    float fgm[8], fbt[8];
    if constexpr (FILM) {
        const uint16_t* gv = a.film + (size_t)img * 2 * a.cin;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int c = (tid % GPA) * 8 + j, cc = c < a.cin ? c : 0;
            fgm[j] = 1.0f + h2f(gv[cc]);
            fbt[j] = h2f(gv[a.cin + cc]);
        }
    }
    uint2 rres[THW];
#pragma unroll
    for (int f = 0; f < THW; f++) {
        rres[f] = uint2{0u, 0u};
        const int oy = oy0 + wm * THW + f, ox = ox0 + lx;
        if (b.residual && !pk.res_mid && lx < TWB && oy < b.hout && ox < b.wout && cob < b.cout)
            rres[f] = load_res4(b, ((size_t)img * b.hout + oy) * b.wout + ox, cob, true);
    }
    float biasa[4], nega[4], biasb[4], negb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        biasa[i] = h2f(a.bias[coa + i]);
        biasb[i] = h2f(b.bias[cob + i]);
    }
    {
        const float4 m = *reinterpret_cast<const float4*>(a.neg + coa);
        const float4 n = *reinterpret_cast<const float4*>(b.neg + cob);
        nega[0] = m.x, nega[1] = m.y, nega[2] = m.z, nega[3] = m.w;
        negb[0] = n.x, negb[1] = n.y, negb[2] = n.z, negb[3] = n.w;
    }

    // A's output channels past its blocks (up to B's padded input channels) are zero for every pixel
    if constexpr (NBA * 16 < CB32) {
        constexpr int G0 = NBA * 2, GN = CB32 / 8 - G0, NZ = FA * MW * GN;
        for (int e = tid; e < NZ; e += NT) {
            const int pix = e / GN, g = G0 + e % GN;
            *reinterpret_cast<uint4*>(mid + pix * PSB + g * 8) = uint4{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int i = 0; i < NLD; i++) {
        const int e = tid + i * NT;
        if ((i + 1) * NT <= HALO || e < HALO) {
            const int pix = e / GPA, g = e - pix * GPA;
            uint4 q = whole ? mask_group(pre[i], a.cin - g * 8) : pre[i];
            if constexpr (FILM)
                if ((inside >> i) & 1u) q = film_group(q, fgm, fbt, a.cin - g * 8);
            *reinterpret_cast<uint4*>(hin + pix * PSA + g * 8) = q;
        }
    }
    __syncthreads();

    // A over FA rows x 16 columns; its f16 output (zero outside the image) into the LDS tile
    if (wn < NBA) {
        f4 acc[FAW];
        a_chain<FAW, SA, MA, CPA, IWA, PSA>(acc, wra, hin + (wm * FAW * SA * IWA + lx * SA) * PSA, lane);
#pragma unroll
        for (int fw = 0; fw < FAW; fw++) {
            const int f = wm * FAW + fw;
            const int oy = oy0 - 1 + f, ox = ox0 - 1 + lx;  // A's output pixel
            const bool in = (oy >= 0) & (oy < a.hout) & (ox >= 0) & (ox < a.wout);
            uint16_t o[4];
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = in ? f2h(activate(acc[fw][i] + biasa[i], nega[i])) : (uint16_t)0;
            *reinterpret_cast<uint2*>(mid + (f * MW + lx) * PSB + coa) =
                uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
        }
    }
    __syncthreads();

    // B over TH rows x 16 columns (the first 14 stored); columns 16 and 17 of the LDS tile feed only the two
    // discarded lanes
    if (wn < NBB && b.post) {  // uniform
        // B then affine_out (B.cout <= 4, no residual: the host checks). B's outputs sit in lanes 0-15, the 4
        // channels of pixel lx each; lane group g = lane / 16 takes rows g, g + 4, ... of the wave from them, so
        // all 64 lanes share the exponentials and divisions (unary.wgsl's op 2 on the f16 output, rounded again)
        f4 acc[THW];
        pair_chain<THW, 1, MB, MW, PSB>(acc, wrb, mid + (wm * THW * MW + lx) * PSB + (lane >> 4) * 8);
        const int g = lane >> 4;
#pragma unroll
        for (int fw0 = 0; fw0 < THW; fw0 += 4) {
            float mine[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // row fw0 + g, pixel lx
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if (fw0 + k >= THW) break;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float v = h2f(f2h(activate(acc[fw0 + k][i] + biasb[i], negb[i])));
                    const float s = __shfl(v, lx);
                    mine[i] = g == k ? s : mine[i];
                }
            }
            const int fw = fw0 + g, oy = oy0 + wm * THW + fw, ox = ox0 + lx;
            if (fw < THW && lx < TWB && oy < b.hout && ox < b.wout) {
                uint16_t* yp = b.y + (((size_t)img * b.hout + oy) * b.wout + ox) * (size_t)b.ycs + b.yc0;
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (i < b.cout) yp[i] = f2h(2.0f / (1.0f + expf(-mine[i])) - 1.0f);
            }
        }
    } else if (wn < NBB) {
        f4 acc[THW];
        pair_chain<THW, 1, MB, MW, PSB>(acc, wrb, mid + (wm * THW * MW + lx) * PSB + (lane >> 4) * 8);
#pragma unroll
        for (int fw = 0; fw < THW; fw++) {
            const int f = wm * THW + fw;
            const int oy = oy0 + f, ox = ox0 + lx;
            if (lx < TWB && oy < b.hout && ox < b.wout && cob < b.cout) {
                // both values read, then selected as values (opaque_u2); the LDS read is in bounds for every lane
                const uint2 mv = opaque_u2(*reinterpret_cast<const uint2*>(mid + ((f + 1) * MW + lx + 1) * PSB + cob));
                const uint2 rv = pk.res_mid ? mv : rres[fw];
                epilogue4r(b, ((size_t)img * b.hout + oy) * b.wout + ox, cob, acc[fw], biasb, negb, rv);
            }
        }
    }
}

template <int SA, int CA32, int CB32, int NBA, int NBB, int TH, int WM, bool VEC, bool FILM = false, int CPA = 32>
__global__ __launch_bounds__(64 * (NBA > NBB ? NBA : NBB) * WM) void conv_pair(PairKArgs pk) {
    __shared__ __align__(16) PairLds<SA, CA32, CB32, TH> lds;
    conv_pair_tile<SA, CA32, CB32, NBA, NBB, TH, WM, VEC, FILM, CPA>(pk, blockIdx.x, lds);
}

// The persistent pair: G = gridDim.x resident workgroups loop over B's output tiles t, t + G, ... with both layers'
// weights, biases and multipliers loaded once. Input, external residual and output go through buffer instructions
// (out-of-range lanes: zero loads, dropped stores), so no memory access sits in a branch and the compiler's waits
// stay exact; waves without a channel block of A or B skip only the MFMAs and the LDS traffic. Per tile: A's chain
// and epilogue into the LDS tile; a barrier; the next tile's halo (in registers since the previous tile) into LDS
// and the loads of the tile after it, which then fly during B's chain and the next tile's A chain; B's chain and
// epilogue with its stores; the next tile's residual loads; a barrier. The intermediate never leaves the CU.
// Compiled for exactly 2 waves per SIMD (at most 256 registers per lane, AGPRs included), so that the resident
// grid the planner sizes (kPairResidentWaves waves per CU, or the LDS limit) is the one that fits.
template <int SA, int CA32, int CB32, int NBA, int NBB, int TH, int WM, int CPA = 32>
__global__ __launch_bounds__(64 * (NBA > NBB ? NBA : NBB) * WM)
__attribute__((amdgpu_waves_per_eu(2, 2))) void conv_pair_p(PairKArgs pk) {
    constexpr int WN = NBA > NBB ? NBA : NBB, NT = 64 * WN * WM, TWB = kPairTileW;
    constexpr int FA = TH + 2, FAW = FA / WM, THW = TH / WM;
    static_assert(FA % WM == 0 && TH % WM == 0, "rows split evenly over the wave rows");
    constexpr int IHA = (FA - 1) * SA + 3, IWA = 15 * SA + 3;
    constexpr int GPA = CA32 / 8, PSA = CA32 + 8, MA = CA32 / 32, KA = pair_ksteps<CPA, MA>();
    static_assert(CPA == 32 || CA32 == 32, "packed taps read the zero channels CPA .. CPA + 7 of the staged halo");
    constexpr int MW = 18, PSB = CB32 + 8, MB = CB32 / 32;
    constexpr int HALO = IHA * IWA * GPA, NLD = (HALO + NT - 1) / NT;
    static_assert(NBA * 16 <= CB32, "A's channel blocks exceed B's input channels");
    __shared__ __align__(16) uint16_t hin[IHA * IWA * PSA];
    __shared__ __align__(16) uint16_t mid[FA * MW * PSB];
    const ConvKArgs& a = pk.a;
    const ConvKArgs& b = pk.b;

    const int tid = threadIdx.x, lane = tid & 63, lx = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: the A / B branches are uniform
    const int wn = wave % WN, wm = wave / WN;
    const int wa = wn < NBA ? wn : NBA - 1, wb = wn < NBB ? wn : NBB - 1;
    const int coa = wa * 16 + 4 * (lane >> 4), cob = wb * 16 + 4 * (lane >> 4);
    const int tiles = b.n * b.tiles_y * b.tiles_x, G = gridDim.x;
    int t = blockIdx.x;
    if (t >= tiles) return;  // uniform over the workgroup
    const bool ext_res = b.residual && !pk.res_mid;
    const uint64_t pix_out = (uint64_t)b.n * b.hout * b.wout;
    const auto rx = buffer_rsrc(a.x, (uint32_t)((uint64_t)a.n * a.h * a.w * a.xcs * 2));
    const auto ry = buffer_rsrc(b.y, (uint32_t)view_bytes(pix_out, b.ycs, b.yc0, b.cout));
    const auto rr = buffer_rsrc(b.res, ext_res ? (uint32_t)view_bytes(pix_out, b.rcs, b.rc0, b.cout) : 0u);

    auto tile_origin = [&](int tt, int& img, int& oy0, int& ox0) {
        const int tx = tt % b.tiles_x, r0 = tt / b.tiles_x;
        oy0 = (r0 % b.tiles_y) * TH;
        img = r0 / b.tiles_y;
        ox0 = tx * TWB;
    };
    // lane parts of the halo addresses, fixed for the launch (as in the persistent direct loop)
    uint32_t hoff[NLD];
    int hpos[NLD];
    bool hst[NLD];
#pragma unroll
    for (int i = 0; i < NLD; i++) {
        const int e = tid + i * NT;
        const int pix = e / GPA, g = e - pix * GPA;
        const int iy = pix / IWA, ix = pix - iy * IWA;
        hoff[i] = ((uint32_t)(iy * a.w + ix) * (uint32_t)a.xcs + (uint32_t)(a.xc0 + g * 8)) * 2u;
        hpos[i] = (iy << 16) | ix;
        hst[i] = ((i + 1) * NT <= HALO || e < HALO) & (g * 8 < a.cin);
    }
    uint4 pre[NLD];
    auto load_halo = [&](int tt) {  // tile tt's A input halo into registers (a tile past the last reads zeros)
        int img, oy0, ox0;
        tile_origin(tt, img, oy0, ox0);
        const int iy0 = (oy0 - 1) * SA - a.pad, ix0 = (ox0 - 1) * SA - a.pad;
        const uint32_t base = (((uint32_t)(img * a.h + iy0) * (uint32_t)a.w + (uint32_t)ix0) * (uint32_t)a.xcs) * 2u;
        const bool tv = tt < tiles;
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int gy = iy0 + (hpos[i] >> 16), gx = ix0 + (hpos[i] & 0xffff);
            const bool ok = hst[i] & tv & ((uint32_t)gy < (uint32_t)a.h) & ((uint32_t)gx < (uint32_t)a.w);
            pre[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? base + hoff[i] : kOOB, 0, 0));
        }
    };
    auto write_halo = [&]() {
        const bool part = (a.cin & 7) != 0;  // uniform
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = tid + i * NT;
            if ((i + 1) * NT <= HALO || e < HALO) {
                const int pix = e / GPA, g = e - pix * GPA;
                *reinterpret_cast<uint4*>(hin + pix * PSA + g * 8) = part ? mask_group(pre[i], a.cin - g * 8) : pre[i];
            }
        }
    };
    // B's output and external residual: per-tile scalar base + lane part; validity of row f for this lane
    const uint32_t yl = ((uint32_t)lx * (uint32_t)b.ycs + (uint32_t)(b.yc0 + cob)) * 2u;
    const uint32_t rl = ((uint32_t)lx * (uint32_t)b.rcs + (uint32_t)(b.rc0 + cob)) * 2u;
    const uint32_t yrow = (uint32_t)b.wout * (uint32_t)b.ycs * 2u, rrow = (uint32_t)b.wout * (uint32_t)b.rcs * 2u;
    auto out_ok = [&](int oy0, int ox0, int f) {
        return (wn < NBB) & (lx < TWB) & (oy0 + wm * THW + f < b.hout) & (ox0 + lx < b.wout) & (cob < b.cout);
    };
    uint2 rres[THW];
    auto load_res = [&](int tt) {
        int img, oy0, ox0;
        tile_origin(tt, img, oy0, ox0);
        const uint32_t base =
            ((uint32_t)(img * b.hout + oy0 + wm * THW) * (uint32_t)b.wout + (uint32_t)ox0) * (uint32_t)b.rcs * 2u;
        const bool tv = (tt < tiles) & ext_res;
#pragma unroll
        for (int f = 0; f < THW; f++)
            rres[f] = __builtin_bit_cast(
                uint2, __builtin_amdgcn_raw_buffer_load_b64(rr, (out_ok(oy0, ox0, f) & tv) ? base + f * rrow + rl : kOOB,
                                                            0, 0));
    };

    // once: the first halo, both layers' weights, biases and multipliers, the zero channels of the LDS tile
    load_halo(t);
    h8 wra[KA], wrb[9 * MB];
    {
        const h8* wp = reinterpret_cast<const h8*>(a.wpk) + (size_t)wa * KA * 64 + lane;
#pragma unroll
        for (int s = 0; s < KA; s++) wra[s] = wp[s * 64];
        const h8* wq = reinterpret_cast<const h8*>(b.wpk) + (size_t)wb * 9 * MB * 64 + lane;
#pragma unroll
        for (int s = 0; s < 9 * MB; s++) wrb[s] = wq[s * 64];
    }
    float biasa[4], nega[4], biasb[4], negb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        biasa[i] = h2f(a.bias[coa + i]);
        biasb[i] = h2f(b.bias[cob + i]);
    }
    {
        const float4 m = *reinterpret_cast<const float4*>(a.neg + coa);
        const float4 n = *reinterpret_cast<const float4*>(b.neg + cob);
        nega[0] = m.x, nega[1] = m.y, nega[2] = m.z, nega[3] = m.w;
        negb[0] = n.x, negb[1] = n.y, negb[2] = n.z, negb[3] = n.w;
    }
    if constexpr (NBA * 16 < CB32) {
        constexpr int G0 = NBA * 2, GN = CB32 / 8 - G0, NZ = FA * MW * GN;
        for (int e = tid; e < NZ; e += NT) {
            const int pix = e / GN, g = G0 + e % GN;
            *reinterpret_cast<uint4*>(mid + pix * PSB + g * 8) = uint4{0u, 0u, 0u, 0u};
        }
    }
    write_halo();
    __syncthreads();
    load_halo(t + G);
    load_res(t);

    typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
    for (; t < tiles; t += G) {
        int img, oy0, ox0;
        tile_origin(t, img, oy0, ox0);
        // A over FA rows x 16 columns; its f16 output (zero outside the image) into the LDS tile
        if (wn < NBA) {
            f4 acc[FAW];
            a_chain<FAW, SA, MA, CPA, IWA, PSA>(acc, wra, hin + (wm * FAW * SA * IWA + lx * SA) * PSA, lane);
#pragma unroll
            for (int fw = 0; fw < FAW; fw++) {
                const int f = wm * FAW + fw;
                const int oy = oy0 - 1 + f, ox = ox0 - 1 + lx;
                const bool in = (oy >= 0) & (oy < a.hout) & (ox >= 0) & (ox < a.wout);
                uint16_t o[4];
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] = in ? f2h(activate(acc[fw][i] + biasa[i], nega[i])) : (uint16_t)0;
                *reinterpret_cast<uint2*>(mid + (f * MW + lx) * PSB + coa) =
                    uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
            }
        }
        __syncthreads();  // the LDS tile is complete and every wave is done reading the halo
        write_halo();     // the next tile's halo
        load_halo(t + 2 * G);
        // B over TH rows x 16 columns (the first 14 stored)
        f4 acc[THW];
#pragma unroll
        for (int fw = 0; fw < THW; fw++) acc[fw] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if (wn < NBB)
            pair_chain<THW, 1, MB, MW, PSB>(acc, wrb, mid + (wm * THW * MW + lx) * PSB + (lane >> 4) * 8);
        const uint32_t ybase =
            ((uint32_t)(img * b.hout + oy0 + wm * THW) * (uint32_t)b.wout + (uint32_t)ox0) * (uint32_t)b.ycs * 2u;
#pragma unroll
        for (int fw = 0; fw < THW; fw++) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = activate(acc[fw][i] + biasb[i], negb[i]);
            hh2 p0 = hh2{(_Float16)v[0], (_Float16)v[1]}, p1 = hh2{(_Float16)v[2], (_Float16)v[3]};
            if (b.residual) {  // uniform; A's output at the same pixel, or the external tensor
                // both values read, then selected as values (opaque_u2)
                const uint2 mv =
                    opaque_u2(*reinterpret_cast<const uint2*>(mid + ((wm * THW + fw + 1) * MW + lx + 1) * PSB + cob));
                const uint2 rv = pk.res_mid ? mv : rres[fw];
                p0 += __builtin_bit_cast(hh2, rv.x);
                p1 += __builtin_bit_cast(hh2, rv.y);
            }
            const uint32_t off = out_ok(oy0, ox0, fw) ? ybase + fw * yrow + yl : kOOB;
            __builtin_amdgcn_raw_buffer_store_b64(
                __builtin_bit_cast(__attribute__((ext_vector_type(2))) uint32_t,
                                   uint2{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1)}),
                ry, off, 0, 0);
        }
        load_res(t + G);
        __syncthreads();  // the next halo is in LDS and every wave is done reading the LDS tile
    }
}

// The warp-specialized resident pair: NBA waves run only A (one channel block each, all FA rows) and NBB waves
// run only B, so each wave holds one layer's weights, and the two stages pipeline across tiles: in step s the A
// waves compute tile s from halo buffer s % 2 into LDS tile s % 2 while the B waves compute tile s - 1 from LDS
// tile (s - 1) % 2, one barrier per step. Each SIMD then interleaves an A chain and a B chain instead of the whole
// workgroup alternating between them. The A waves also stage the halos (tile s + 1 into LDS from registers, tile
// s + 2 into registers); the B waves load the residual a step ahead and store. Every load and store is
// unconditional through buffer instructions (tiles past the last read zeros and store nothing).
template <int SA, int CA32, int CB32, int NBA, int NBB, int TH, int CPA = 32>
__global__ __launch_bounds__(64 * (NBA + NBB))
__attribute__((amdgpu_waves_per_eu(2, 2))) void conv_pair_ws(PairKArgs pk) {
    constexpr int NW = NBA + NBB, NTA = 64 * NBA, TWB = kPairTileW;
    constexpr int FA = TH + 2;
    constexpr int IHA = (FA - 1) * SA + 3, IWA = 15 * SA + 3;
    constexpr int GPA = CA32 / 8, PSA = CA32 + 8, MA = CA32 / 32, KA = pair_ksteps<CPA, MA>();
    static_assert(CPA == 32 || CA32 == 32, "packed taps read the zero channels CPA .. CPA + 7 of the staged halo");
    constexpr int MW = 18, PSB = CB32 + 8, MB = CB32 / 32;
    constexpr int HALO = IHA * IWA * GPA, NLD = (HALO + NTA - 1) / NTA;  // the A waves stage the halo
    constexpr int HB = IHA * IWA * PSA, MBUF = FA * MW * PSB;
    static_assert(NBA * 16 <= CB32, "A's channel blocks exceed B's input channels");
    __shared__ __align__(16) uint16_t hin[2 * HB];
    __shared__ __align__(16) uint16_t mid[2 * MBUF];
    const ConvKArgs& a = pk.a;
    const ConvKArgs& b = pk.b;

    const int tid = threadIdx.x, lane = tid & 63, lx = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool is_a = wave < NBA;  // uniform: this wave's stage
    const int wa = is_a ? wave : 0, wb = is_a ? 0 : wave - NBA;
    const int coa = wa * 16 + 4 * (lane >> 4), cob = wb * 16 + 4 * (lane >> 4);
    const int tiles = b.n * b.tiles_y * b.tiles_x, G = gridDim.x, first = blockIdx.x;
    if (first >= tiles) return;  // uniform over the workgroup
    const int K = (tiles - first + G - 1) / G;  // this workgroup's tiles: first, first + G, ...
    const bool ext_res = b.residual && !pk.res_mid;
    const uint64_t pix_out = (uint64_t)b.n * b.hout * b.wout;
    const auto rx = buffer_rsrc(a.x, (uint32_t)((uint64_t)a.n * a.h * a.w * a.xcs * 2));
    const auto ry = buffer_rsrc(b.y, (uint32_t)view_bytes(pix_out, b.ycs, b.yc0, b.cout));
    const auto rr = buffer_rsrc(b.res, ext_res ? (uint32_t)view_bytes(pix_out, b.rcs, b.rc0, b.cout) : 0u);

    auto tile_origin = [&](int tt, int& img, int& oy0, int& ox0) {
        const int tx = tt % b.tiles_x, r0 = tt / b.tiles_x;
        oy0 = (r0 % b.tiles_y) * TH;
        img = r0 / b.tiles_y;
        ox0 = tx * TWB;
    };
    // the A waves' lane parts of the halo addresses (thread tid < NTA stages halo elements tid + i * NTA)
    uint32_t hoff[NLD];
    int hpos[NLD];
    bool hst[NLD];
#pragma unroll
    for (int i = 0; i < NLD; i++) {
        const int e = tid + i * NTA;
        const int pix = e / GPA, g = e - pix * GPA;
        const int iy = pix / IWA, ix = pix - iy * IWA;
        hoff[i] = ((uint32_t)(iy * a.w + ix) * (uint32_t)a.xcs + (uint32_t)(a.xc0 + g * 8)) * 2u;
        hpos[i] = (iy << 16) | ix;
        hst[i] = ((i + 1) * NTA <= HALO || e < HALO) & (g * 8 < a.cin);
    }
    uint4 pre[NLD];
    auto load_halo = [&](int k) {  // tile number k of this workgroup into registers (past the last: zeros)
        const int tt = first + k * G;
        int img, oy0, ox0;
        tile_origin(tt, img, oy0, ox0);
        const int iy0 = (oy0 - 1) * SA - a.pad, ix0 = (ox0 - 1) * SA - a.pad;
        const uint32_t base = (((uint32_t)(img * a.h + iy0) * (uint32_t)a.w + (uint32_t)ix0) * (uint32_t)a.xcs) * 2u;
        const bool tv = k < K;
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int gy = iy0 + (hpos[i] >> 16), gx = ix0 + (hpos[i] & 0xffff);
            const bool ok = hst[i] & tv & ((uint32_t)gy < (uint32_t)a.h) & ((uint32_t)gx < (uint32_t)a.w);
            pre[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? base + hoff[i] : kOOB, 0, 0));
        }
    };
    auto write_halo = [&](int buf) {
        const bool part = (a.cin & 7) != 0;  // uniform
        uint16_t* h = hin + buf * HB;
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int e = tid + i * NTA;
            if ((i + 1) * NTA <= HALO || e < HALO) {
                const int pix = e / GPA, g = e - pix * GPA;
                *reinterpret_cast<uint4*>(h + pix * PSA + g * 8) = part ? mask_group(pre[i], a.cin - g * 8) : pre[i];
            }
        }
    };
    // the B waves' output and residual addresses; validity of row f of tile (oy0, ox0) for this lane
    const uint32_t yl = ((uint32_t)lx * (uint32_t)b.ycs + (uint32_t)(b.yc0 + cob)) * 2u;
    const uint32_t rl = ((uint32_t)lx * (uint32_t)b.rcs + (uint32_t)(b.rc0 + cob)) * 2u;
    const uint32_t yrow = (uint32_t)b.wout * (uint32_t)b.ycs * 2u, rrow = (uint32_t)b.wout * (uint32_t)b.rcs * 2u;
    auto out_ok = [&](int oy0, int ox0, int f) {
        return (lx < TWB) & (oy0 + f < b.hout) & (ox0 + lx < b.wout) & (cob < b.cout);
    };
    uint2 rres[TH];
    auto load_res = [&](int k) {
        const int tt = first + k * G;
        int img, oy0, ox0;
        tile_origin(tt, img, oy0, ox0);
        const uint32_t base = ((uint32_t)(img * b.hout + oy0) * (uint32_t)b.wout + (uint32_t)ox0) * (uint32_t)b.rcs * 2u;
        const bool tv = (k < K) & ext_res;
#pragma unroll
        for (int f = 0; f < TH; f++)
            rres[f] = __builtin_bit_cast(
                uint2, __builtin_amdgcn_raw_buffer_load_b64(rr, (out_ok(oy0, ox0, f) & tv) ? base + f * rrow + rl : kOOB,
                                                            0, 0));
    };

    // once: this wave's layer's weights, bias and multipliers; the first two halos (A) or the first residual (B);
    // the zero channels of both LDS tiles
    constexpr int NWR = KA > 9 * MB ? KA : 9 * MB;
    h8 wr[NWR];
    float bias[4], neg[4];
    {
        const ConvKArgs& l = is_a ? a : b;
        const int blk = is_a ? wa : wb, nk = is_a ? KA : 9 * MB, co = is_a ? coa : cob;
        const h8* wp = reinterpret_cast<const h8*>(l.wpk) + (size_t)blk * nk * 64 + lane;
#pragma unroll
        for (int s = 0; s < NWR; s++) wr[s] = wp[(s < nk ? s : 0) * 64];
#pragma unroll
        for (int i = 0; i < 4; i++) bias[i] = h2f(l.bias[co + i]);
        const float4 m = *reinterpret_cast<const float4*>(l.neg + co);
        neg[0] = m.x, neg[1] = m.y, neg[2] = m.z, neg[3] = m.w;
    }
    if (is_a) {
        load_halo(0);
        write_halo(0);
        load_halo(1);
    }
    if constexpr (NBA * 16 < CB32) {
        constexpr int G0 = NBA * 2, GN = CB32 / 8 - G0, NZ = 2 * FA * MW * GN;
        for (int e = tid; e < NZ; e += 64 * NW) {
            const int pix = e / GN, g = G0 + e % GN;  // pixels of both buffers (MBUF = FA * MW * PSB apart)
            *reinterpret_cast<uint4*>(mid + pix * PSB + g * 8) = uint4{0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();

    typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
    for (int s = 0; s <= K; s++) {
        if (is_a) {
            if (s < K) {  // A over FA rows x 16 columns of tile s; its f16 output (zero outside the image)
                int img, oy0, ox0;
                tile_origin(first + s * G, img, oy0, ox0);
                f4 acc[FA];
                a_chain<FA, SA, MA, CPA, IWA, PSA>(acc, wr, hin + (s & 1) * HB + (lx * SA) * PSA, lane);
                uint16_t* m = mid + (s & 1) * MBUF;
#pragma unroll
                for (int f = 0; f < FA; f++) {
                    const int oy = oy0 - 1 + f, ox = ox0 - 1 + lx;
                    const bool in = (oy >= 0) & (oy < a.hout) & (ox >= 0) & (ox < a.wout);
                    uint16_t o[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) o[i] = in ? f2h(activate(acc[f][i] + bias[i], neg[i])) : (uint16_t)0;
                    *reinterpret_cast<uint2*>(m + (f * MW + lx) * PSB + coa) =
                        uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
                }
                write_halo((s + 1) & 1);  // tile s + 1 (zeros past the last)
            }
            load_halo(s + 2);
        } else {
            if (s >= 1) {  // B over TH rows x 16 columns of tile s - 1 (the first 14 stored)
                int img, oy0, ox0;
                tile_origin(first + (s - 1) * G, img, oy0, ox0);
                const uint16_t* m = mid + ((s - 1) & 1) * MBUF;
                f4 acc[TH];
                pair_chain<TH, 1, MB, MW, PSB>(acc, wr, m + lx * PSB + (lane >> 4) * 8);
                const uint32_t ybase =
                    ((uint32_t)(img * b.hout + oy0) * (uint32_t)b.wout + (uint32_t)ox0) * (uint32_t)b.ycs * 2u;
#pragma unroll
                for (int f = 0; f < TH; f++) {
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) v[i] = activate(acc[f][i] + bias[i], neg[i]);
                    hh2 p0 = hh2{(_Float16)v[0], (_Float16)v[1]}, p1 = hh2{(_Float16)v[2], (_Float16)v[3]};
                    if (b.residual) {  // uniform: A's output at the same pixel, or the external tensor
                        const uint2 mv = opaque_u2(*reinterpret_cast<const uint2*>(m + ((f + 1) * MW + lx + 1) * PSB + cob));
                        const uint2 rv = pk.res_mid ? mv : rres[f];
                        p0 += __builtin_bit_cast(hh2, rv.x);
                        p1 += __builtin_bit_cast(hh2, rv.y);
                    }
                    const uint32_t off = out_ok(oy0, ox0, f) ? ybase + f * yrow + yl : kOOB;
                    __builtin_amdgcn_raw_buffer_store_b64(
                        __builtin_bit_cast(__attribute__((ext_vector_type(2))) uint32_t,
                                           uint2{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1)}),
                        ry, off, 0, 0);
                }
            }
            load_res(s);  // tile s's residual, for the next step
        }
        __syncthreads();  // LDS tile s and halo s + 1 are written; LDS tile s - 1 and halo s are read
    }
}

// Whether the persistent pair's buffer loop serves these views (16-byte input groups, 8-byte output and
// residual quads, every view below 2^31 bytes); else the one-tile kernel runs.
inline bool pair_buffer_ok(const PairKArgs& pk) {
    const ConvKArgs &a = pk.a, &b = pk.b;
    const uint64_t lim = 1ull << 31, pout = (uint64_t)b.n * b.hout * b.wout;
    const bool ext = b.residual && !pk.res_mid;
    return a.xvec && b.yvec && b.cout % 4 == 0 && (!ext || b.rvec) &&
           (uint64_t)a.n * a.h * a.w * (uint64_t)a.xcs * 2 < lim && view_bytes(pout, b.ycs, b.yc0, b.cout) < lim &&
           (!ext || view_bytes(pout, b.rcs, b.rc0, b.cout) < lim);
}

template <int SA, int CA32, int CB32, int NBA, int NBB, int TH, int CPA = 32>
hipError_t launch_pair_ws(const PairKArgs& pk, dim3 grid, hipStream_t s) {
    if (pair_buffer_ok(pk)) {
        hipLaunchKernelGGL((conv_pair_ws<SA, CA32, CB32, NBA, NBB, TH, CPA>), grid, dim3(64 * (NBA + NBB)), 0, s, pk);
        return hipGetLastError();
    }
    // views the buffer loop cannot serve: one workgroup per tile
    grid.x = (unsigned)(pk.b.n * pk.b.tiles_y * pk.b.tiles_x);
    const dim3 block(64 * (NBA > NBB ? NBA : NBB));
    if (pk.a.xvec)
        hipLaunchKernelGGL((conv_pair<SA, CA32, CB32, NBA, NBB, TH, 1, true, false, CPA>), grid, block, 0, s, pk);
    else
        hipLaunchKernelGGL((conv_pair<SA, CA32, CB32, NBA, NBB, TH, 1, false, false, CPA>), grid, block, 0, s, pk);
    return hipGetLastError();
}

template <int SA, int CA32, int CB32, int NBA, int NBB, int TH, int WM, int CPA = 32>
hipError_t launch_pair_p(const PairKArgs& pk, dim3 grid, hipStream_t s) {
    const dim3 block(64 * (NBA > NBB ? NBA : NBB) * WM);
    if (pair_buffer_ok(pk)) {
        hipLaunchKernelGGL((conv_pair_p<SA, CA32, CB32, NBA, NBB, TH, WM, CPA>), grid, block, 0, s, pk);
        return hipGetLastError();
    }
    grid.x = (unsigned)(pk.b.n * pk.b.tiles_y * pk.b.tiles_x);  // one workgroup per tile
    if (pk.a.xvec)
        hipLaunchKernelGGL((conv_pair<SA, CA32, CB32, NBA, NBB, TH, WM, true, false, CPA>), grid, block, 0, s, pk);
    else
        hipLaunchKernelGGL((conv_pair<SA, CA32, CB32, NBA, NBB, TH, WM, false, false, CPA>), grid, block, 0, s, pk);
    return hipGetLastError();
}

template <int SA, int CA32, int CB32, int NBA, int NBB, int TH, int WM, int CPA = 32>
hipError_t launch_pair(const PairKArgs& pk, dim3 grid, hipStream_t s) {
    const dim3 block(64 * (NBA > NBB ? NBA : NBB) * WM);
    if (pk.a.film) {  // FiLM on the input: its own instantiations, so the others stage as before
        if (pk.a.xvec)
            hipLaunchKernelGGL((conv_pair<SA, CA32, CB32, NBA, NBB, TH, WM, true, true, CPA>), grid, block, 0, s, pk);
        else
            hipLaunchKernelGGL((conv_pair<SA, CA32, CB32, NBA, NBB, TH, WM, false, true, CPA>), grid, block, 0, s, pk);
    } else if (pk.a.xvec) {
        hipLaunchKernelGGL((conv_pair<SA, CA32, CB32, NBA, NBB, TH, WM, true, false, CPA>), grid, block, 0, s, pk);
    } else {
        hipLaunchKernelGGL((conv_pair<SA, CA32, CB32, NBA, NBB, TH, WM, false, false, CPA>), grid, block, 0, s, pk);
    }
    return hipGetLastError();
}

}  // namespace fhc
