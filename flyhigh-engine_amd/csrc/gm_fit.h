// One round of the periodic-structure repair's affine fit (gmhs.rs:149-206; gm_fit_reduce.wgsl:15-44 with the solve
// of gm_fit_solve.wgsl:11-24 of the round before), as a workgroup body: the repair's own fit launches run it with
// 256 threads, and a launch that also runs other work's workgroups at 192 threads runs it there. Either way the sums
// are gm_fit_reduce's: 32 workgroups of 256 lanes, lane t of workgroup g summing cells g * 256 + t + k * 8192 in
// order, then the pairwise lane tree (t, t + off) for off = 128 .. 1, the first levels through LDS; with 192
// threads, threads 0-63 also take lanes 192-255. Self-contained (raw pointers, its own f16 conversion), so the conv
// kernels' translation unit can include it.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace fhc {
namespace gmfit {

constexpr uint32_t kNwg = 32, kWg = 256;  // gm_fit_reduce's workgroups and lanes per workgroup (gmhs.rs:160)
constexpr uint32_t kPart = kNwg * 4 * 9;  // one round's partial sums [workgroup][channel][9]

__device__ __forceinline__ float half_to_float(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// gm_fit_solve.wgsl:13-24: the normal equations of one flow channel, s = its summed partials; o = a0, a1, a2
__device__ inline void solve(const float* s, float* o) {
    const float m00 = s[0] + 1e-6f, m01 = s[1], m02 = s[2], m11 = s[3] + 1e-6f, m12 = s[4], m22 = s[5] + 1e-6f;
    const float det = m00 * (m11 * m22 - m12 * m12) - m01 * (m01 * m22 - m12 * m02) + m02 * (m01 * m12 - m11 * m02);
    if (fabsf(det) < 1e-12f) {
        o[0] = s[6] / fmaxf(s[0], 1e-6f), o[1] = 0.0f, o[2] = 0.0f;
        return;
    }
    const float i00 = (m11 * m22 - m12 * m12) / det, i01 = (m02 * m12 - m01 * m22) / det;
    const float i02 = (m01 * m12 - m02 * m11) / det, i11 = (m00 * m22 - m02 * m02) / det;
    const float i12 = (m01 * m02 - m00 * m12) / det, i22 = (m00 * m11 - m01 * m01) / det;
    o[0] = i00 * s[6] + i01 * s[7] + i02 * s[8];
    o[1] = i01 * s[6] + i11 * s[7] + i12 * s[8];
    o[2] = i02 * s[6] + i12 * s[7] + i22 * s[8];
}

// the coefficients of the channels `chans` (bit c: channel c) from a round's partials, into cf[c][0..2]: lane
// c * 9 + k sums partial k over the workgroups in order (gm_fit_solve.wgsl:11-12; the 32 loads issued together),
// lane c solves. Every thread of the block (at least 36) takes part in the barriers.
__device__ inline void solve_block(const float* part, uint32_t chans, float (*ss)[9], float (*cf)[3]) {
    const uint32_t t = threadIdx.x;
    if (t < 36 && (chans >> (t / 9) & 1u)) {
        const uint32_t c = t / 9, k = t % 9;
        float v[kNwg];
#pragma unroll
        for (uint32_t g = 0; g < kNwg; g++) v[g] = part[(g * 4 + c) * 9 + k];
        float a = 0.0f;
#pragma unroll
        for (uint32_t g = 0; g < kNwg; g++) a = a + v[g];
        ss[c][k] = a;
    }
    __syncthreads();
    if (t < 4 && (chans >> t & 1u)) solve(ss[t], cf[t]);
    __syncthreads();
}

// v of lane l + N for lanes l with l % 16 + N < 16 (a DPP row shift; the other lanes read 0): the tree's last
// levels, whose lanes that matter (l < N) read lanes below 16
template <int N>
__device__ __forceinline__ float row_down(float v) {
    static_assert(N >= 1 && N <= 8, "a row shift within 16 lanes");
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 | N, 0xf, 0xf, true));
}

// the LDS a round needs
struct RoundLds {
    float sh[9][kWg / 2];
    float ss[4][9], cf[4][3];
};

// one fit round for workgroup g of channel c, NTH threads (256, or 192 with threads 0-63 taking lanes 192-255 too):
// flow channel c of the E8 flow at p[i * cs + c0 + c]; rounds after the first weight each element by
// delta / max(delta, |residual|) against the coefficients of the previous round's partials
template <uint32_t NTH>
__device__ inline void round_body(const uint16_t* fp, uint32_t cs, uint32_t c0, uint32_t h8, uint32_t w8, float delta,
                                  uint32_t round, const float* part_in, float* part_out, uint32_t g, uint32_t c,
                                  RoundLds& L) {
    static_assert(NTH == 256 || NTH == 192, "the fit runs on 256 or 192 threads");
    constexpr uint32_t NV = NTH == 256 ? 1 : 2;  // lanes per thread (the second for threads below 256 - NTH)
    const uint32_t t = threadIdx.x;
    const uint32_t n = h8 * w8, stride = kWg * kNwg;
    uint32_t lanes[NV];
    lanes[0] = t;
    if constexpr (NV == 2) lanes[1] = t + NTH;
    float f0[NV];
#pragma unroll
    for (uint32_t v = 0; v < NV; v++) {  // in flight while the previous round is solved
        const uint32_t i0 = g * kWg + lanes[v];
        f0[v] = lanes[v] < kWg && i0 < n ? half_to_float(fp[(size_t)i0 * cs + c0 + c]) : 0.0f;
    }
    if (round > 0) solve_block(part_in, 1u << c, L.ss, L.cf);
    const float sx = 2.0f / (float)max(w8 - 1, 1u), sy = 2.0f / (float)max(h8 - 1, 1u);
    float s[NV][9];
#pragma unroll
    for (uint32_t v = 0; v < NV; v++) {
#pragma unroll
        for (uint32_t k = 0; k < 9; k++) s[v][k] = 0.0f;
        if (lanes[v] >= kWg) continue;
        const uint32_t i0 = g * kWg + lanes[v];
        for (uint32_t i = i0; i < n; i += stride) {
            const uint32_t yy = i / w8, xx = i - yy * w8;
            const float x = -1.0f + sx * (float)xx, y = -1.0f + sy * (float)yy;
            const float f = i == i0 ? f0[v] : half_to_float(fp[(size_t)i * cs + c0 + c]);
            float w2 = 1.0f;
            if (round > 0) w2 = delta / fmaxf(delta, fabsf(f - (L.cf[c][0] + L.cf[c][1] * x + L.cf[c][2] * y)));
            s[v][0] = s[v][0] + w2, s[v][1] = s[v][1] + w2 * x, s[v][2] = s[v][2] + w2 * y;
            s[v][3] = s[v][3] + w2 * x * x, s[v][4] = s[v][4] + w2 * x * y, s[v][5] = s[v][5] + w2 * y * y;
            s[v][6] = s[v][6] + w2 * f, s[v][7] = s[v][7] + w2 * x * f, s[v][8] = s[v][8] + w2 * y * f;
        }
    }
    // the lane tree, pairs (l, l + off) for off = 128 .. 1: the first level through LDS (lanes 128-255 write), the
    // rest in the first wave (offsets 32 and 16 across rows, 8 .. 1 as row shifts)
#pragma unroll
    for (uint32_t v = 0; v < NV; v++)
        if (lanes[v] >= kWg / 2 && lanes[v] < kWg)
#pragma unroll
            for (uint32_t k = 0; k < 9; k++) L.sh[k][lanes[v] - kWg / 2] = s[v][k];
    __syncthreads();
    if (t < kWg / 2)
#pragma unroll
        for (uint32_t k = 0; k < 9; k++) L.sh[k][t] = s[0][k] + L.sh[k][t];
    __syncthreads();
    if (t < 64) {
#pragma unroll
        for (uint32_t k = 0; k < 9; k++) {
            float v = L.sh[k][t] + L.sh[k][t + 64];
            v = v + __shfl_down(v, 32);
            v = v + __shfl_down(v, 16);
            v = v + row_down<8>(v);
            v = v + row_down<4>(v);
            v = v + row_down<2>(v);
            v = v + row_down<1>(v);
            if (t == 0) part_out[(g * 4 + c) * 9 + k] = v;
        }
    }
}

}  // namespace gmfit
}  // namespace fhc
