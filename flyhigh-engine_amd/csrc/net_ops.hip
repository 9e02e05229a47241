// The FlyHighFG network ops between the convs (include/fhc_ops.h): stencil and elementwise kernels on NHWC f16
// views. Each is bound by HBM (a few bytes per output, tens of FLOPs at most), so the design is about access
// shape, not arithmetic: one thread per pixel, or per pixel and group of 4 channels, so that consecutive lanes read
// and write consecutive channels of consecutive pixels (one 8-byte access per lane where the views are 4-channel
// aligned); neighbour reads of a stencil hit L2 behind the first. Arithmetic is f32 in the reference kernels' order
// (the library is built with -ffp-contract=off, so no product is fused into a sum), rounded once to f16 (RTNE) on
// store, so results equal the reference kernels' bit for bit up to the ulp of expf where a softmax is involved.
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.h"
#include "fhc_ops.h"

#include "gm_corun.h"
#include "gm_fit.h"

namespace fhc {

namespace {

constexpr uint32_t kThreads = 256;

struct View {  // an input view: element (pixel, ch) at p[pixel * cs + c0 + ch], read times scale where the op says
    const uint16_t* p;
    uint32_t cs, c0;
    float scale;
};
struct OView {
    uint16_t* p;
    uint32_t cs, c0;
};

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
// f32 -> f16, RTNE (the default rounding mode), of the f32 value as rounded: the conversion is written as its
// instruction, because the compiler otherwise contracts a product or sum feeding it into one mixed-precision FMA
// (v_fma_mixlo_f16) that rounds the exact result once, where the reference rounds it to f32 and then to f16 (the two
// differ next to f16 midpoints). A pure asm: the compiler may move or merge it, but cannot look inside it.
__device__ __forceinline__ uint16_t f2h(float f) {
    uint32_t r;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(f));
    return (uint16_t)r;
}
__device__ __forceinline__ float ld(const View& v, size_t pix, uint32_t ch) { return h2f(v.p[pix * v.cs + v.c0 + ch]); }
__device__ __forceinline__ void st(const OView& v, size_t pix, uint32_t ch, float x) {
    v.p[pix * v.cs + v.c0 + ch] = f2h(x);
}
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
// luma of f32 B, G, R at read scale 1: luma.wgsl:9-12
__device__ __forceinline__ float lum3(float b, float g, float r) { return 0.299f * r + 0.587f * g + 0.114f * b; }

// channels ch .. ch + 3 (those below c; 0 for the rest) of pixel pix. VEC: one 8-byte load, valid when the view's
// cs and c0, ch and the base address are 4-channel (8-byte) aligned and c is a multiple of 4.
template <bool VEC>
__device__ __forceinline__ void ld4(const View& v, size_t pix, uint32_t ch, uint32_t c, float (&o)[4]) {
    if constexpr (VEC) {
        const uint2 q = *reinterpret_cast<const uint2*>(v.p + pix * v.cs + v.c0 + ch);
        o[0] = h2f((uint16_t)q.x), o[1] = h2f((uint16_t)(q.x >> 16));
        o[2] = h2f((uint16_t)q.y), o[3] = h2f((uint16_t)(q.y >> 16));
    } else {
        // the channel index clamped to the view, the load unconditional and the value selected afterwards: a load
        // under a condition becomes a branch that waits for it, one memory latency per load
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const float val = ld(v, pix, min(ch + i, c - 1));
            o[i] = ch + i < c ? val : 0.0f;
        }
    }
}
template <bool VEC>
__device__ __forceinline__ void st4(const OView& v, size_t pix, uint32_t ch, uint32_t c, const float (&x)[4]) {
    if constexpr (VEC) {
        *reinterpret_cast<uint2*>(v.p + pix * v.cs + v.c0 + ch) =
            uint2{(uint32_t)f2h(x[0]) | ((uint32_t)f2h(x[1]) << 16), (uint32_t)f2h(x[2]) | ((uint32_t)f2h(x[3]) << 16)};
    } else {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++)
            if (ch + i < c) st(v, pix, ch + i, x[i]);
    }
}

// ---- warp: shaders/warp.wgsl:14-28 ----------------------------------------------------------------------------
// channels ch .. ch + 3 of image img0 / h of `img` (img0 = image * h) sampled at (x + fx, y + fy), bilinear with the
// coordinates clamped, times the view's scale
template <bool VEC>
__device__ __forceinline__ void warp4(const View& img, uint32_t img0, uint32_t x, uint32_t y, uint32_t h, uint32_t w,
                                      float fx, float fy, uint32_t ch, uint32_t c, float (&o)[4]) {
    const float gx = (float)x + fx, gy = (float)y + fy;
    const int x0 = (int)floorf(gx), y0 = (int)floorf(gy);
    const float ax = gx - (float)x0, ay = gy - (float)y0;
    const int x0c = clampi(x0, 0, (int)w - 1), x1c = clampi(x0 + 1, 0, (int)w - 1);
    const int y0c = clampi(y0, 0, (int)h - 1), y1c = clampi(y0 + 1, 0, (int)h - 1);
    const size_t r0 = (size_t)(img0 + y0c) * w, r1 = (size_t)(img0 + y1c) * w;
    float v00[4], v01[4], v10[4], v11[4];
    ld4<VEC>(img, r0 + x0c, ch, c, v00);
    ld4<VEC>(img, r0 + x1c, ch, c, v01);
    ld4<VEC>(img, r1 + x0c, ch, c, v10);
    ld4<VEC>(img, r1 + x1c, ch, c, v11);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float top = v00[i] * (1.0f - ax) + v01[i] * ax, bot = v10[i] * (1.0f - ax) + v11[i] * ax;
        o[i] = (top * (1.0f - ay) + bot * ay) * img.scale;
    }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void warp_kernel(View img, View flow, OView out, uint32_t h, uint32_t w,
                                                        uint32_t c, uint32_t groups, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t pix = t / groups, ch = (t - pix * groups) * 4;
    const uint32_t x = pix % w, row = pix / w, y = row % h, img0 = row - y;  // img0 = image * h
    float o[4];
    warp4<VEC>(img, img0, x, y, h, w, ld(flow, pix, 0) * flow.scale, ld(flow, pix, 1) * flow.scale, ch, c, o);
    st4<VEC>(out, pix, ch, c, o);
}

// ---- luma / luma_grad: shaders/luma.wgsl:9-28 (channel 2 R, 1 G, 0 B) --------------------------------------
__device__ __forceinline__ float lum(const View& v, size_t pix) {
    return (0.299f * ld(v, pix, 2) + 0.587f * ld(v, pix, 1) + 0.114f * ld(v, pix, 0)) * v.scale;
}
template <bool GRAD>
__global__ __launch_bounds__(kThreads) void luma_kernel(View x, OView out, uint32_t h, uint32_t w, uint32_t items) {
    const uint32_t pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= items) return;
    const float c = lum(x, pix);
    if constexpr (!GRAD) {
        st(out, pix, 0, c);
    } else {
        const uint32_t xx = pix % w, y = (pix / w) % h;
        const float gx = xx + 1 < w ? lum(x, pix + 1) - c : 0.0f;
        const float gy = y + 1 < h ? lum(x, (size_t)pix + w) - c : 0.0f;
        st(out, pix, 0, fabsf(gx) + fabsf(gy));
    }
}

// ---- sad_volume: shaders/sad.wgsl:12-28; one lane per (pixel, displacement), so a wave stores consecutive
// channels of the cost volume -----------------------------------------------------------------------------------
__device__ __forceinline__ void sad_at(const View& la, const View& lb, const OView& out, uint32_t h, uint32_t w,
                                       uint32_t r, uint32_t span2, uint32_t t) {
    const uint32_t pix = t / span2, d = t - pix * span2, span = 2 * r + 1;
    const uint32_t x = pix % w, row = pix / w, y = row % h, img0 = row - y;
    const int dy = (int)(d / span) - (int)r, dx = (int)(d % span) - (int)r;
    float acc = 0.0f;
#pragma unroll
    for (int wy = -1; wy <= 1; wy++)
#pragma unroll
        for (int wx = -1; wx <= 1; wx++) {
            // every load unconditional (clamped coordinates), so the 18 loads issue together; a tap outside the
            // image adds +0, which leaves the sum as the reference's skipped tap does
            const int yy = (int)y + wy, xx = (int)x + wx;
            const bool in = yy >= 0 && yy < (int)h && xx >= 0 && xx < (int)w;
            const int cy = clampi(yy, 0, (int)h - 1), cx = clampi(xx, 0, (int)w - 1);
            const float lav = ld(la, (size_t)(img0 + cy) * w + cx, 0);
            const int syy = clampi(yy + dy, 0, (int)h - 1), sxx = clampi(xx + dx, 0, (int)w - 1);
            const float d = fabsf(lav - ld(lb, (size_t)(img0 + syy) * w + sxx, 0));
            acc = acc + (in ? d : 0.0f);
        }
    st(out, pix, d, acc / 9.0f);
}
__global__ __launch_bounds__(kThreads) void sad_kernel(View la, View lb, OView out, uint32_t h, uint32_t w,
                                                       uint32_t r, uint32_t span2, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t < items) sad_at(la, lb, out, h, w, r, span2, t);
}

// ---- convex upsample: shaders/convex.wgsl:12-34 ------------------------------------------------------------------
// A workgroup (one wave) computes 8 x 8 output pixels (4 x 4 input pixels, 4 sub-pixels each): it stages the 36
// weight channels of its input pixels and the 6 x 6 neighbourhood of x (zeros outside the image: adding 0 * weight
// is what the reference's zero branch adds) in LDS with coalesced reads, then one lane per output pixel computes its
// softmax once and every channel from LDS, in the reference's order. Small tiles: the frame's quarter maps are
// 60 x 108 input pixels, and one wave per 16 outputs' worth of inputs spreads them over every CU.
constexpr uint32_t kCvIn = 4, kCvHalo = kCvIn + 2, kCvThreads = 4 * kCvIn * kCvIn;

// FVT: x is mid()'s flow_t | vis_t (7 channels), computed while staging from fv (flow 0-3, vis 4-6) and the FiLM
// head's output df (d_flow 0-3, d_mask 4) with flow_vis_t_kernel's arithmetic, so that x is never stored: the same
// f16 values the two launches produce
// (fpix: the pixel's index in fv, dpix: in df)
__device__ __forceinline__ void flow_vis_t_at(const View& fv, const View& df, size_t fpix, size_t dpix, float af,
                                              float ab, uint16_t (&o)[7]) {
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        const float lin = h2f(f2h(ld(fv, fpix, i) * fv.scale * (i < 2 ? af : ab)));
        o[i] = f2h(lin + ld(df, dpix, i) * df.scale);
    }
    const uint16_t dm = df.p[dpix * df.cs + df.c0 + 4];
    const float dv[3] = {h2f(dm), h2f(f2h(h2f(dm) * -1.0f)), 0.0f};
#pragma unroll
    for (uint32_t j = 0; j < 3; j++) o[4 + j] = f2h(ld(fv, fpix, 4 + j) * fv.scale + dv[j]);
}

// the softmax of an output pixel's 9 mask weights pw[4 k] (k: its 3 x 3 neighbourhood, row-major)
__device__ __forceinline__ void convex_weights(const uint16_t* pw, float (&ws)[9]) {
    float m = -3.0e38f;
#pragma unroll
    for (uint32_t k = 0; k < 9; k++) {
        ws[k] = h2f(pw[k * 4]);
        m = fmaxf(m, ws[k]);
    }
    float denom = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 9; k++) {
        ws[k] = expf(ws[k] - m);
        denom = denom + ws[k];
    }
#pragma unroll
    for (uint32_t k = 0; k < 9; k++) ws[k] = ws[k] / denom;
}

// FVT with several phases: image i of df and out is phase i / per of pair i % per, whose wt and fv are image i % per
// and whose mul_t factors are ph.af[i / per], ph.ab[i / per]
constexpr uint32_t kMaxPhases = 8;
struct PhaseT {
    float af[kMaxPhases], ab[kMaxPhases];
};
template <bool FVT>
__global__ __launch_bounds__(kCvThreads) void convex_tile_kernel(View wt, View x, OView out, uint32_t h, uint32_t w,
                                                               uint32_t c, uint32_t tiles_x, uint32_t tiles_y,
                                                               View fv, View df, PhaseT ph, uint32_t per) {
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t* lw = lds;                       // [kCvIn * kCvIn][36]
    uint16_t* lx = lds + kCvIn * kCvIn * 36;  // [kCvHalo * kCvHalo][c]
    const uint32_t tid = threadIdx.x, tx = tid % (2 * kCvIn), ty = tid / (2 * kCvIn);
    const uint32_t bt = blockIdx.x, txi = bt % tiles_x, r = bt / tiles_x, tyi = r % tiles_y, img = r / tiles_y;
    const uint32_t pimg = img % per;  // the image of wt and fv
    const float af = ph.af[img / per], ab = ph.ab[img / per];
    const int ix0 = (int)(txi * kCvIn), iy0 = (int)(tyi * kCvIn);
    // staging with every load unconditional (clamped to the image / the view) and unrolled, so they issue together
#pragma unroll
    for (uint32_t k = 0; k < (kCvIn * kCvIn * 9 + kCvThreads - 1) / kCvThreads; k++) {  // 9 quads of 4 channels a pixel
        const uint32_t e = min(tid + k * kCvThreads, kCvIn * kCvIn * 9 - 1);
        const uint32_t p = e / 9, q = e - p * 9, py = p / kCvIn, px = p % kCvIn;
        const int gy = min(iy0 + (int)py, (int)h - 1), gx = min(ix0 + (int)px, (int)w - 1);
        const uint16_t* src = wt.p + (((size_t)pimg * h + gy) * w + gx) * wt.cs + wt.c0 + q * 4;
        // lanes past the last quad rewrite that quad with its own value (a conditional store would pull the load
        // into the branch and serialise the loads again)
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) lw[p * 36 + q * 4 + i] = src[i];
    }
    if (FVT && tid < kCvHalo * kCvHalo) {  // one lane per halo pixel: flow_t | vis_t from fv and df
        const uint32_t py = tid / kCvHalo, px = tid % kCvHalo;
        const int gy = iy0 - 1 + (int)py, gx = ix0 - 1 + (int)px;
        const bool in = gy >= 0 && gy < (int)h && gx >= 0 && gx < (int)w;
        uint16_t v[7];
        const size_t pix = (size_t)clampi(gy, 0, (int)h - 1) * w + clampi(gx, 0, (int)w - 1);
        flow_vis_t_at(fv, df, (size_t)pimg * h * w + pix, (size_t)img * h * w + pix, af, ab, v);
#pragma unroll
        for (uint32_t cc = 0; cc < 7; cc++) lx[tid * 7 + cc] = in ? v[cc] : (uint16_t)0;
    } else if (!FVT && tid < kCvHalo * kCvHalo) {  // one lane per halo pixel, channels 8 at a time
        const uint32_t py = tid / kCvHalo, px = tid % kCvHalo;
        const int gy = iy0 - 1 + (int)py, gx = ix0 - 1 + (int)px;
        const bool in = gy >= 0 && gy < (int)h && gx >= 0 && gx < (int)w;
        const uint16_t* src =
            x.p + (((size_t)img * h + clampi(gy, 0, (int)h - 1)) * w + clampi(gx, 0, (int)w - 1)) * x.cs + x.c0;
        for (uint32_t c8 = 0; c8 < c; c8 += 8) {
            // channels past c rewrite channel c - 1 with its own value: unconditional loads and stores
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) {
                const uint32_t cc = min(c8 + i, c - 1);
                const uint16_t v = src[cc];
                lx[tid * c + cc] = in ? v : (uint16_t)0;
            }
        }
    }
    __syncthreads();
    const uint32_t ox = txi * 2 * kCvIn + tx, oy = tyi * 2 * kCvIn + ty;
    if (ox >= 2 * w || oy >= 2 * h) return;
    const uint32_t lix = tx / 2, liy = ty / 2, sub = (ty % 2) * 2 + tx % 2;
    float ws[9];
    convex_weights(lw + (liy * kCvIn + lix) * 36 + sub, ws);
    const size_t opix = ((size_t)img * 2 * h + oy) * 2 * w + ox;
    // each product as an FMA with +0, which takes the f16 value as it is (one mixed-precision FMA): the product's
    // value, or +0 for a product of -0, which the sum cannot tell apart (it starts at +0, and a sum of f32 values is
    // -0 only when both are)
    for (uint32_t co = 0; co < c; co++) {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < 9; k++)
            acc = acc + __builtin_fmaf(h2f(lx[((liy + k / 3) * kCvHalo + lix + k % 3) * c + co]), ws[k], 0.0f);
        st(out, opix, co, acc);
    }
}

// ---- film_modulate: shaders/film.wgsl:11-14 ---------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(kThreads) void film_kernel(View hv, const uint16_t* g, OView out, uint32_t hw,
                                                        uint32_t c, uint32_t groups, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t pix = t / groups, ch = (t - pix * groups) * 4;
    const uint16_t* gi = g + (size_t)(pix / hw) * 2 * c;
    float v[4], o[4];
    ld4<VEC>(hv, pix, ch, c, v);
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        const uint32_t cc = ch + i < c ? ch + i : 0;  // channels past c are not stored
        o[i] = v[i] * (1.0f + h2f(gi[cc])) + h2f(gi[c + cc]);
    }
    st4<VEC>(out, pix, ch, c, o);
}

// ---- blend_weights and blendmix: shaders/blend.wgsl:11-20, blendmix.wgsl:14-27 ------------------------------------
__device__ __forceinline__ void soft3v(float a, float b, float c, float& ea, float& eb, float& ec, float& s) {
    const float m = fmaxf(a, fmaxf(b, c));
    ea = expf(a - m), eb = expf(b - m), ec = expf(c - m);
    s = ea + eb + ec;
}
__device__ __forceinline__ void soft3(const View& vis, size_t pix, float& ea, float& eb, float& ec, float& s) {
    soft3v(ld(vis, pix, 0) * vis.scale, ld(vis, pix, 1) * vis.scale, ld(vis, pix, 2) * vis.scale, ea, eb, ec, s);
}
__global__ __launch_bounds__(kThreads) void blend_kernel(View vis, OView out, uint32_t items) {
    const uint32_t pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= items) return;
    float ea, eb, ec, s;
    soft3(vis, pix, ea, eb, ec, s);
    const float p0 = ea / s, p1 = eb / s, p2 = ec / s;
    st(out, pix, 0, p0 + 0.5f * p2);
    st(out, pix, 1, p1 + 0.5f * p2);
}
__global__ __launch_bounds__(kThreads) void blendmix_kernel(View wa, View wb, View vis, OView out, uint32_t items) {
    const uint32_t pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= items) return;
    float ea, eb, ec, s;
    soft3(vis, pix, ea, eb, ec, s);
    const float pa = h2f(f2h((ea + 0.5f * ec) / s)), pb = h2f(f2h((eb + 0.5f * ec) / s));
#pragma unroll
    for (uint32_t ch = 0; ch < 3; ch++) {
        const float t1 = h2f(f2h(ld(wa, pix, ch) * pa)), t2 = h2f(f2h(ld(wb, pix, ch) * pb));
        st(out, pix, ch, t1 + t2);
    }
}

// ---- avgpool: shaders/avgpool.wgsl:10-18 -------------------------------------------------------------------------
// K > 0: the pool size at compile time (the loads of the window then issue together); K == 0: k at run time
template <bool VEC, int K>
__global__ __launch_bounds__(kThreads) void avgpool_kernel(View x, OView out, uint32_t h, uint32_t w, uint32_t oh,
                                                           uint32_t ow, uint32_t c, uint32_t kr, uint32_t groups,
                                                           uint32_t items) {
    const uint32_t k = K > 0 ? (uint32_t)K : kr;
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t opix = t / groups, ch = (t - opix * groups) * 4;
    const uint32_t ox = opix % ow, row = opix / ow, oy = row % oh, img = row / oh;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, v[4];
#pragma unroll
    for (uint32_t ky = 0; ky < k; ky++)
#pragma unroll
        for (uint32_t kx = 0; kx < k; kx++) {
            ld4<VEC>(x, ((size_t)img * h + oy * k + ky) * w + ox * k + kx, ch, c, v);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = acc[i] + v[i];
        }
    const float kk = (float)(k * k);
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = acc[i] / kk;
    st4<VEC>(out, opix, ch, c, acc);
}

// ---- interpolate: shaders/interp.wgsl:13-44; the taps' weights are shared by a lane's 4 channels -----------------
template <bool VEC, bool AA>
__global__ __launch_bounds__(kThreads) void interp_kernel(View x, OView out, uint32_t ih, uint32_t iw, uint32_t oh,
                                                          uint32_t ow, uint32_t c, uint32_t groups, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t opix = t / groups, ch = (t - opix * groups) * 4;
    const uint32_t ox = opix % ow, row = opix / ow, oy = row % oh, img = row / oh;
    const float sh = (float)ih / (float)oh, sw = (float)iw / (float)ow;
    const size_t base = (size_t)img * ih;
    float val[4];
    if constexpr (!AA) {
        const float fiy = ((float)oy + 0.5f) * sh - 0.5f, fix = ((float)ox + 0.5f) * sw - 0.5f;
        const int y0 = (int)floorf(fiy), x0 = (int)floorf(fix);
        const float fy = fiy - (float)y0, fx = fix - (float)x0;
        const int y0c = clampi(y0, 0, (int)ih - 1), y1c = clampi(y0 + 1, 0, (int)ih - 1);
        const int x0c = clampi(x0, 0, (int)iw - 1), x1c = clampi(x0 + 1, 0, (int)iw - 1);
        float v00[4], v01[4], v10[4], v11[4];
        ld4<VEC>(x, (base + y0c) * iw + x0c, ch, c, v00);
        ld4<VEC>(x, (base + y0c) * iw + x1c, ch, c, v01);
        ld4<VEC>(x, (base + y1c) * iw + x0c, ch, c, v10);
        ld4<VEC>(x, (base + y1c) * iw + x1c, ch, c, v11);
#pragma unroll
        for (int i = 0; i < 4; i++)
            val[i] = (v00[i] * (1.0f - fx) + v01[i] * fx) * (1.0f - fy) + (v10[i] * (1.0f - fx) + v11[i] * fx) * fy;
    } else {
        const float fsh = fmaxf(sh, 1.0f), fsw = fmaxf(sw, 1.0f);
        const float cy = ((float)oy + 0.5f) * sh, cx = ((float)ox + 0.5f) * sw;
        const int ymin = max(0, (int)floorf(cy - fsh + 0.5f)), ymax = min((int)ih, (int)floorf(cy + fsh + 0.5f));
        const int xmin = max(0, (int)floorf(cx - fsw + 0.5f)), xmax = min((int)iw, (int)floorf(cx + fsw + 0.5f));
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, norm = 0.0f, v[4];
        for (int y = ymin; y < ymax; y++) {
            const float wy = fmaxf(0.0f, 1.0f - fabsf(((float)y + 0.5f - cy) / fsh));
            for (int xx = xmin; xx < xmax; xx++) {
                const float wx = fmaxf(0.0f, 1.0f - fabsf(((float)xx + 0.5f - cx) / fsw));
                const float wgt = wx * wy;
                ld4<VEC>(x, (base + y) * iw + xx, ch, c, v);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = acc[i] + v[i] * wgt;
                norm = norm + wgt;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) val[i] = acc[i] / norm;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) val[i] = val[i] * x.scale;
    st4<VEC>(out, opix, ch, c, val);
}

// The antialiased resize with its taps unrolled to a compile-time bound KM per dimension (the host picks the
// smallest KM that covers every output's window, from the same f32 formulas): every tap loads from a clamped,
// in-bounds address unconditionally, so a lane's loads issue together instead of one tap per memory latency; a tap
// outside the window gets weight 0 and value 0, and adding +0 leaves acc and norm as the reference's loop leaves
// them (neither is ever -0). The per-column weights are computed once per lane (the reference recomputes the same
// value per tap). The sum runs rows, then columns, as in the reference.
template <int KM>
__global__ __launch_bounds__(kThreads) void interp_aa_kernel(View x, OView out, uint32_t ih, uint32_t iw, uint32_t oh,
                                                             uint32_t ow, uint32_t c, uint32_t groups,
                                                             uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t opix = t / groups, ch = (t - opix * groups) * 4;
    const uint32_t ox = opix % ow, row = opix / ow, oy = row % oh, img = row / oh;
    const float sh = (float)ih / (float)oh, sw = (float)iw / (float)ow;
    const float fsh = fmaxf(sh, 1.0f), fsw = fmaxf(sw, 1.0f);
    const float cy = ((float)oy + 0.5f) * sh, cx = ((float)ox + 0.5f) * sw;
    const int ymin = max(0, (int)floorf(cy - fsh + 0.5f)), ymax = min((int)ih, (int)floorf(cy + fsh + 0.5f));
    const int xmin = max(0, (int)floorf(cx - fsw + 0.5f)), xmax = min((int)iw, (int)floorf(cx + fsw + 0.5f));
    float wx[KM];
    int xs[KM];
#pragma unroll
    for (int j = 0; j < KM; j++) {
        const int xx = xmin + j;
        wx[j] = xx < xmax ? fmaxf(0.0f, 1.0f - fabsf(((float)xx + 0.5f - cx) / fsw)) : 0.0f;
        xs[j] = min(xx, (int)iw - 1);
    }
    const size_t base = (size_t)img * ih;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, norm = 0.0f;
#pragma unroll
    for (int jy = 0; jy < KM; jy++) {
        const int y = ymin + jy;
        const float wy = y < ymax ? fmaxf(0.0f, 1.0f - fabsf(((float)y + 0.5f - cy) / fsh)) : 0.0f;
        const size_t rbase = (base + min(y, (int)ih - 1)) * iw;
#pragma unroll
        for (int jx = 0; jx < KM; jx++) {
            const bool in = (y < ymax) & (xmin + jx < xmax);
            const float wgt = wx[jx] * wy;
            float v[4];
            ld4<false>(x, rbase + xs[jx], ch, c, v);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = acc[i] + (in ? v[i] : 0.0f) * wgt;
            norm = norm + wgt;
        }
    }
    float val[4];
#pragma unroll
    for (int i = 0; i < 4; i++) val[i] = acc[i] / norm * x.scale;
    st4<false>(out, opix, ch, c, val);
}

// The same resize for views of at most 4 channels through LDS: a workgroup computes 16 x 16 output pixels from the
// union of their windows (at most kAaExt x kAaExt input pixels, the host checks the worst tile), staged once with
// coalesced loads, 4 channels a pixel (one 8-byte LDS read per tap); the L1 then serves no overlapping windows.
// Staging is a fixed kAaR x kAaR grid of clamped, unconditional loads per lane (lanes past the window rewrite its
// last row / column with the same values), so it takes one memory round trip. The per-output sum is the one above.
constexpr uint32_t kAaT = 16, kAaR = 5, kAaExt = kAaT * kAaR;

// PYR (3 channels, pairs of pictures: images 2k, 2k + 1 are pair k's): the tile's outputs also go through the pair()
// pyramid (avgpool k 2 twice and the luma, graph.json ops 14-18, 21-24) from LDS: a 16 x 16 tile holds whole 2 x 2
// and 4 x 4 blocks, so i8 (8 x 8 of them), i16 (4 x 4, into channels 3 * (image % 2) of its image k) and l16
// (channel image % 2 of image k) need no other launch; each pool reads the f16 values the previous stage stores, in
// avgpool's order.
struct PyrOut {
    OView i8, i16, l16;
};

// V4: the input view's pixels are 8-byte aligned 4-channel groups (cs and c0 multiples of 4): one load a pixel
template <int KM, bool PYR, bool V4>
__global__ __launch_bounds__(kThreads) void interp_aa_lds_kernel(View x, OView out, uint32_t ih, uint32_t iw,
                                                                 uint32_t oh, uint32_t ow, uint32_t c,
                                                                 uint32_t tiles_x, uint32_t tiles_y, PyrOut pyr) {
    // rows of kAaExt + 1 cells: the last cell of each row, and a whole extra row, hold zeros, the value every tap
    // outside its pixel's window reads (times its weight +0 it adds +0 to the sums, which never hold -0: what the
    // reference's skipped tap leaves, for any input values)
    constexpr uint32_t S = kAaExt + 1;
    __shared__ uint2 tile[S * kAaExt + S];
    __shared__ float qt[PYR ? kAaT * kAaT * 3 : 1], q8[PYR ? 64 * 3 : 1];
    const uint32_t tid = threadIdx.x, tx = tid % kAaT, ty = tid / kAaT;
    const uint32_t bt = blockIdx.x, txi = bt % tiles_x, r = bt / tiles_x, tyi = r % tiles_y, img = r / tiles_y;
    const uint32_t ox0 = txi * kAaT, oy0 = tyi * kAaT;
    const uint32_t ox_last = min(ox0 + kAaT, ow) - 1, oy_last = min(oy0 + kAaT, oh) - 1;
    const float sh = (float)ih / (float)oh, sw = (float)iw / (float)ow;
    const float fsh = fmaxf(sh, 1.0f), fsw = fmaxf(sw, 1.0f);
    const int ylo = max(0, (int)floorf(((float)oy0 + 0.5f) * sh - fsh + 0.5f));
    const int yhi = min((int)ih, (int)floorf(((float)oy_last + 0.5f) * sh + fsh + 0.5f));
    const int xlo = max(0, (int)floorf(((float)ox0 + 0.5f) * sw - fsw + 0.5f));
    const int xhi = min((int)iw, (int)floorf(((float)ox_last + 0.5f) * sw + fsw + 0.5f));
    const int ny = max(1, min(yhi - ylo, (int)kAaExt)), nx = max(1, min(xhi - xlo, (int)kAaExt));
    // the window's first pixel (uniform), then 32-bit byte offsets of the lane's rows and columns (the window is at
    // most kAaExt pixels square, so row * iw * cs stays far below 2^32 for any frame)
    const char* wbase = reinterpret_cast<const char*>(x.p + (((size_t)img * ih + ylo) * iw + xlo) * x.cs + x.c0);
    uint32_t roff[kAaR], coff[kAaR];
#pragma unroll
    for (uint32_t i = 0; i < kAaR; i++) {
        roff[i] = (uint32_t)min((int)(ty + kAaT * i), ny - 1) * iw * x.cs * 2u;
        coff[i] = (uint32_t)min((int)(tx + kAaT * i), nx - 1) * x.cs * 2u;
    }
#pragma unroll
    for (uint32_t i = 0; i < kAaR; i++)
#pragma unroll
        for (uint32_t j = 0; j < kAaR; j++) {
            const int row = min((int)(ty + kAaT * i), ny - 1), col = min((int)(tx + kAaT * j), nx - 1);
            const uint16_t* src = reinterpret_cast<const uint16_t*>(wbase + (roff[i] + coff[j]));
            if constexpr (V4) {  // channels past c are never read from the tile
                tile[row * S + col] = *reinterpret_cast<const uint2*>(src);
            } else {
                uint16_t v[4];
#pragma unroll
                for (uint32_t k = 0; k < 4; k++) v[k] = src[min(k, c - 1)];
                tile[row * S + col] =
                    uint2{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16)};
            }
        }
    if (tid < kAaExt) tile[tid * S + kAaExt] = uint2{0u, 0u};  // the zero column
    if (tid < S) tile[kAaExt * S + tid] = uint2{0u, 0u};       // the zero row
    // The tap weights and LDS offsets of the tile's columns (threads 0 .. 16 KM - 1: column t / KM, tap t % KM) and
    // rows (threads 128 ..), computed once for the tile: an invalid column or row (past the output) takes the
    // clamped pixel's, whose lanes store nothing. A tap outside its pixel's window gets weight 0 and the zero cell.
    __shared__ float wxs[kAaT * KM], wys[kAaT * KM];
    __shared__ int lcs[kAaT * KM], lrs[kAaT * KM];
    if (tid < kAaT * KM) {
        const uint32_t k = tid / KM, j = tid % KM;
        const float cx = ((float)min(ox0 + k, ow - 1) + 0.5f) * sw;
        const int xmin = max(0, (int)floorf(cx - fsw + 0.5f)), xmax = min((int)iw, (int)floorf(cx + fsw + 0.5f));
        const int xx = xmin + (int)j;
        wxs[tid] = xx < xmax ? fmaxf(0.0f, 1.0f - fabsf(((float)xx + 0.5f - cx) / fsw)) : 0.0f;
        lcs[tid] = xx < xmax ? xx - xlo : (int)kAaExt;
    } else if (tid >= 128 && tid < 128 + kAaT * KM) {
        const uint32_t k = (tid - 128) / KM, j = (tid - 128) % KM;
        const float cy = ((float)min(oy0 + k, oh - 1) + 0.5f) * sh;
        const int ymin = max(0, (int)floorf(cy - fsh + 0.5f)), ymax = min((int)ih, (int)floorf(cy + fsh + 0.5f));
        const int y = ymin + (int)j;
        wys[tid - 128] = y < ymax ? fmaxf(0.0f, 1.0f - fabsf(((float)y + 0.5f - cy) / fsh)) : 0.0f;
        lrs[tid - 128] = y < ymax ? (y - ylo) * (int)S : (int)(kAaExt * S);
    }
    __syncthreads();
    const uint32_t ox = ox0 + tx, oy = oy0 + ty;
    const bool valid = ox < ow && oy < oh;
    if (!PYR && !valid) return;
    // an invalid lane (PYR only: it must reach the barriers) computes a clamped pixel and stores nothing
    float wx[KM];
    int lc[KM];
#pragma unroll
    for (int j = 0; j < KM; j++) wx[j] = wxs[tx * KM + j], lc[j] = lcs[tx * KM + j];
    constexpr int NC = PYR ? 3 : 4;  // the channels summed: the pyramid's pictures have 3
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, norm = 0.0f;
#pragma unroll
    for (int jy = 0; jy < KM; jy++) {
        const float wy = wys[ty * KM + jy];
        const uint2* lrow = tile + lrs[ty * KM + jy];
#pragma unroll
        for (int jx = 0; jx < KM; jx++) {
            const float wgt = wx[jx] * wy;
            const uint2 q = lrow[lc[jx]];
            const float v[4] = {h2f((uint16_t)q.x), h2f((uint16_t)(q.x >> 16)), h2f((uint16_t)q.y),
                                h2f((uint16_t)(q.y >> 16))};
            // each product as an FMA with +0, which takes the f16 tap as it is (one mixed-precision FMA): the
            // product's value, or +0 for a product of -0, which the sum cannot tell apart (it starts at +0 and a
            // sum of f32 values is -0 only when both are)
#pragma unroll
            for (int i = 0; i < NC; i++) acc[i] = acc[i] + __builtin_fmaf(v[i], wgt, 0.0f);
            norm = norm + wgt;
        }
    }
    float val[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NC; i++) val[i] = acc[i] / norm * x.scale;
    if (valid) st4<false>(out, ((size_t)img * oh + oy) * ow + ox, 0, c, val);
    if constexpr (PYR) {
        if (valid)
#pragma unroll
            for (uint32_t ch = 0; ch < 3; ch++) qt[(ty * kAaT + tx) * 3 + ch] = h2f(f2h(val[ch]));
        __syncthreads();
        const uint32_t h8 = oh / 2, w8 = ow / 2, h16 = h8 / 2, w16 = w8 / 2;
        if (tid < 64) {
            const uint32_t ly = tid / 8, lx = tid % 8, y8 = oy0 / 2 + ly, x8 = ox0 / 2 + lx;
            if (y8 < h8 && x8 < w8) {  // its 2 x 2 block lies in the tile and the picture
                const float* b = qt + ((2 * ly) * kAaT + 2 * lx) * 3;
#pragma unroll
                for (uint32_t ch = 0; ch < 3; ch++) {
                    const float a = ((0.0f + b[ch]) + b[3 + ch]) + b[kAaT * 3 + ch] + b[kAaT * 3 + 3 + ch];
                    const uint16_t hv = f2h(a / 4.0f);
                    q8[tid * 3 + ch] = h2f(hv);
                    pyr.i8.p[(((size_t)img * h8 + y8) * w8 + x8) * pyr.i8.cs + pyr.i8.c0 + ch] = hv;
                }
            }
        }
        __syncthreads();
        if (tid < 16) {
            const uint32_t ly = tid / 4, lx = tid % 4, y16 = oy0 / 4 + ly, x16 = ox0 / 4 + lx;
            if (y16 < h16 && x16 < w16) {
                const float* b = q8 + ((2 * ly) * 8 + 2 * lx) * 3;
                float v[3];
#pragma unroll
                for (uint32_t ch = 0; ch < 3; ch++) {
                    const float a = ((0.0f + b[ch]) + b[3 + ch]) + b[8 * 3 + ch] + b[8 * 3 + 3 + ch];
                    const uint16_t hv = f2h(a / 4.0f);
                    v[ch] = h2f(hv);
                    pyr.i16.p[(((size_t)(img / 2) * h16 + y16) * w16 + x16) * pyr.i16.cs + pyr.i16.c0 + 3 * (img % 2) +
                              ch] = hv;
                }
                st(pyr.l16, ((size_t)(img / 2) * h16 + y16) * w16 + x16, img % 2, lum3(v[0], v[1], v[2]));
            }
        }
    }
}

// Whether interp_aa_lds_kernel's 32-bit byte offsets within a staged window (kAaExt rows of iw pixels) hold.
bool aa_window_offsets_fit(uint32_t iw, uint32_t cs) { return (uint64_t)kAaExt * iw * cs * 2 < (1ull << 32); }

// The largest input extent (rows or columns) of any kAaT-output tile's windows, from the kernel's f32 formulas.
uint32_t aa_tile_extent(uint32_t in, uint32_t outn) {
    const float s = (float)in / (float)outn, f = fmaxf(s, 1.0f);
    int most = 0;
    for (uint32_t o0 = 0; o0 < outn; o0 += kAaT) {
        const uint32_t o1 = std::min(o0 + kAaT, outn) - 1;
        const int lo = std::max(0, (int)floorf(((float)o0 + 0.5f) * s - f + 0.5f));
        const int hi = std::min((int)in, (int)floorf(((float)o1 + 0.5f) * s + f + 0.5f));
        most = std::max(most, hi - lo);
    }
    return (uint32_t)most;
}

// The largest number of taps of any output's antialiased window along one axis (in - 1 rows / columns of the
// output), from the kernel's own f32 formulas.
uint32_t aa_taps(uint32_t in, uint32_t outn) {
    const float s = (float)in / (float)outn, f = fmaxf(s, 1.0f);
    int most = 0;
    for (uint32_t o = 0; o < outn; o++) {
        const float cc = ((float)o + 0.5f) * s;
        const int lo = std::max(0, (int)floorf(cc - f + 0.5f)), hi = std::min((int)in, (int)floorf(cc + f + 0.5f));
        most = std::max(most, hi - lo);
    }
    return (uint32_t)most;
}

// ---- elementwise: binary.wgsl:11-16, unary.wgsl:11-19, chcopy.wgsl:19-22 ------------------------------------
// One lane per (pixel, 4-channel group); VEC: 8-byte accesses (every view 4-channel aligned).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void binary_kernel(View a, View b, OView out, uint32_t c, uint32_t cb,
                                                          int op, uint32_t groups, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t pix = t / groups, ch = (t - pix * groups) * 4;
    float av[4], bv[4], o[4];
    ld4<VEC>(a, pix, ch, c, av);
    if (cb == 1) {  // b's one channel over all of a's
        const float v = ld(b, pix, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) bv[i] = v;
    } else {
        ld4<VEC>(b, pix, ch, c, bv);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float x = av[i] * a.scale, y = bv[i] * b.scale;
        o[i] = op == 1 ? x * y : x + y;
    }
    st4<VEC>(out, pix, ch, c, o);
}

// OP at compile time, one straight-line kernel per op (a run-time choice among the four, written as nested
// conditionals, compiled to code that skipped the negation of op 3)
template <bool VEC, int OP>
__global__ __launch_bounds__(kThreads) void unary_kernel(View x, OView out, uint32_t c, float pa, float pb,
                                                         uint32_t groups, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t pix = t / groups, ch = (t - pix * groups) * 4;
    float v[4], o[4];
    ld4<VEC>(x, pix, ch, c, v);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float u = v[i] * x.scale;
        if constexpr (OP == 0) o[i] = u * pa;
        else if constexpr (OP == 1) o[i] = fminf(fmaxf(u, pa), pb);
        else if constexpr (OP == 2) o[i] = 2.0f / (1.0f + expf(-u)) - 1.0f;
        else o[i] = -u;
    }
    st4<VEC>(out, pix, ch, c, o);
}

// a channel copy: the bits at scale 1 (the reference copies u32 pairs untouched), else f16(x * scale)
__global__ __launch_bounds__(kThreads) void chcopy_kernel(View x, OView out, uint32_t c, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t pix = t / c, ch = t - pix * c;
    const uint16_t v = x.p[(size_t)pix * x.cs + x.c0 + ch];
    out.p[(size_t)pix * out.cs + out.c0 + ch] = x.scale == 1.0f ? v : f2h(h2f(v) * x.scale);
}

// ---- the graph's op chains, fused: each kernel computes what its ops compute one after another, with the same
// f32 operations and the same f16 roundings at the tensors the ops store (bit for bit) ----------------------------------

// The pictures' pyramid of pair() (graph.json ops 14-18, 21-24): avgpool k 2 of the A and B pictures q (batch 2,
// 3 channels) to i8, again to the 1/4 pictures (written into channels 3 * image of i16, the img16 slice of the
// coarse input) and their luma (channel image of l16). One lane per 2 x 2 block of i8 pixels of one picture; the
// second pool reads the first's f16 values and the luma the second's, as the separate ops read stored tensors.
__global__ __launch_bounds__(kThreads) void pair_pyramid_kernel(View q, OView i8, OView i16, OView l16, uint32_t h,
                                                                uint32_t w, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t h8 = h / 2, w8 = w / 2, h16 = h8 / 2, w16 = w8 / 2, hb = (h8 + 1) / 2, wb = (w8 + 1) / 2;
    const uint32_t x2 = t % wb, r = t / wb, y2 = r % hb, img = r / hb;
    float v8[2][2][3];
#pragma unroll
    for (uint32_t dy = 0; dy < 2; dy++)
#pragma unroll
        for (uint32_t dx = 0; dx < 2; dx++) {
            const uint32_t y8 = min(2 * y2 + dy, h8 - 1), x8 = min(2 * x2 + dx, w8 - 1);
            float acc[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t ky = 0; ky < 2; ky++)
#pragma unroll
                for (uint32_t kx = 0; kx < 2; kx++) {
                    const size_t p = ((size_t)img * h + 2 * y8 + ky) * w + 2 * x8 + kx;
#pragma unroll
                    for (uint32_t ch = 0; ch < 3; ch++) acc[ch] = acc[ch] + ld(q, p, ch);
                }
            const size_t p8 = ((size_t)img * h8 + y8) * w8 + x8;
            const bool own = 2 * y2 + dy < h8 && 2 * x2 + dx < w8;
#pragma unroll
            for (uint32_t ch = 0; ch < 3; ch++) {
                const uint16_t hv = f2h(acc[ch] / 4.0f);
                v8[dy][dx][ch] = h2f(hv);
                if (own) i8.p[p8 * i8.cs + i8.c0 + ch] = hv;
            }
        }
    if (y2 >= h16 || x2 >= w16) return;
    const size_t p16 = (size_t)y2 * w16 + x2;
    float v16[3];
#pragma unroll
    for (uint32_t ch = 0; ch < 3; ch++) {
        const float acc = ((0.0f + v8[0][0][ch]) + v8[0][1][ch]) + v8[1][0][ch] + v8[1][1][ch];
        const uint16_t hv = f2h(acc / 4.0f);
        v16[ch] = h2f(hv);
        i16.p[p16 * i16.cs + i16.c0 + 3 * img + ch] = hv;
    }
    st(l16, p16, img, lum3(v16[0], v16[1], v16[2]));
}

// The fine block's input (graph.json op 42, its body up to the concat): both feature maps f8 (batch 2, c channels)
// and both 1/2 pictures i8 (3 channels) warped by the flow (channels 0-1 for A, 2-3 for B, at the view's read scale:
// the flow at 1/8), the warped pictures' luma (channel image of l8) and the scaled flow itself, written into their
// slices of the block's input fx (c0: wa, +c: wb, +2c: ia, +2c+3: ib, +2c+6: flow8). One lane per (pixel, task):
// tasks 0 .. 2G-1 warp 4 feature channels (G groups per map), 2G and 2G+1 a picture with its luma, 2G+2 the flow.
// The coarse head's output resized to the fine grid (coarse_up_kernel's arithmetic): channel ch of out pixel (x, y)
// (h x w) bilinear from o (hi x wi; sh = hi / h, sw = wi / w), times fs for the flow channels 0-3, as the f16
// coarse_up stores.
__device__ __forceinline__ uint16_t coarse_up_at(const View& o, uint32_t hi, uint32_t wi, float sh, float sw,
                                                 float fs, uint32_t x, uint32_t y, uint32_t ch) {
    const float fiy = ((float)y + 0.5f) * sh - 0.5f, fix = ((float)x + 0.5f) * sw - 0.5f;
    const int y0 = (int)floorf(fiy), x0 = (int)floorf(fix);
    const float fy = fiy - (float)y0, fx = fix - (float)x0;
    const size_t r0 = (size_t)clampi(y0, 0, (int)hi - 1) * wi, r1 = (size_t)clampi(y0 + 1, 0, (int)hi - 1) * wi;
    const uint32_t c0 = clampi(x0, 0, (int)wi - 1), c1 = clampi(x0 + 1, 0, (int)wi - 1);
    const float v00 = ld(o, r0 + c0, ch), v01 = ld(o, r0 + c1, ch), v10 = ld(o, r1 + c0, ch), v11 = ld(o, r1 + c1, ch);
    const float val = (v00 * (1.0f - fx) + v01 * fx) * (1.0f - fy) + (v10 * (1.0f - fx) + v11 * fx) * fy;
    return f2h(val * (ch < 4 ? fs : 1.0f));
}

// UP: the flow comes from the coarse head's output o (hi x wi) resized here (coarse_up fused): each lane resizes
// the two flow channels it warps by (read at fl.scale, as the flow view of the fine block reads the stored fv), and
// the flow task also stores all 7 channels into fv (flow times fs, vis) and the flow16 copy into the state (the
// lanes whose pixel index falls in the coarse grid), as coarse_up_kernel does.
// Lanes: a pixel's 2 groups + 3 tasks are consecutive, so the group lanes of a tap pixel read one cache line
// (measured faster than waves of one task over 64 pixels, whose lanes each touch their own line). csh = hi / h and
// csw = wi / w come from the host. blockIdx.y: the pair (its maps and pictures images 2k, 2k + 1 of f8 and i8, its
// image k of every other view).
template <bool VEC, bool UP>
__device__ __forceinline__ void fine_input_at(View f8, View i8, View fl, OView fx, OView l8, uint32_t h, uint32_t w,
                                              uint32_t c, uint32_t groups, View o, OView fv, OView state, uint32_t hi,
                                              uint32_t wi, float fs, float csh, float csw, uint32_t t, uint32_t pair) {
    if (pair) {
        const size_t z = pair, hw = (size_t)h * w;
        f8.p += z * 2 * hw * f8.cs, i8.p += z * 2 * hw * i8.cs, fl.p += z * hw * fl.cs;
        fx.p += z * hw * fx.cs, l8.p += z * hw * l8.cs;
        if constexpr (UP) {
            o.p += z * hi * wi * o.cs, fv.p += z * hw * fv.cs;
            if (state.p) state.p += z * hi * wi * state.cs;
        }
    }
    const uint32_t tasks = 2 * groups + 3, pix = t / tasks, task = t - pix * tasks;
    const uint32_t x = pix % w, y = pix / w;
    if (task < 2 * groups + 2) {
        const uint32_t img = task < 2 * groups ? task / groups : task - 2 * groups;
        float fxv, fyv;
        if constexpr (UP) {
            fxv = h2f(coarse_up_at(o, hi, wi, csh, csw, fs, x, y, 2 * img)) * fl.scale;
            fyv = h2f(coarse_up_at(o, hi, wi, csh, csw, fs, x, y, 2 * img + 1)) * fl.scale;
        } else {
            fxv = ld(fl, pix, 2 * img) * fl.scale, fyv = ld(fl, pix, 2 * img + 1) * fl.scale;
        }
        float o[4];
        if (task < 2 * groups) {
            const uint32_t ch = (task - img * groups) * 4;
            warp4<VEC>(f8, img * h, x, y, h, w, fxv, fyv, ch, c, o);
            OView dst{fx.p, fx.cs, fx.c0 + img * c};
            st4<VEC>(dst, pix, ch, c, o);
        } else {
            warp4<false>(i8, img * h, x, y, h, w, fxv, fyv, 0, 3, o);
            float r[3];
#pragma unroll
            for (uint32_t ch = 0; ch < 3; ch++) {
                const uint16_t hv = f2h(o[ch]);
                r[ch] = h2f(hv);
                fx.p[(size_t)pix * fx.cs + fx.c0 + 2 * c + 3 * img + ch] = hv;
            }
            st(l8, pix, img, lum3(r[0], r[1], r[2]));
        }
    } else {
        uint16_t v[7];
        if constexpr (UP) {
#pragma unroll
            for (uint32_t ch = 0; ch < 7; ch++) {
                v[ch] = coarse_up_at(o, hi, wi, csh, csw, fs, x, y, ch);
                fv.p[(size_t)pix * fv.cs + fv.c0 + ch] = v[ch];
            }
            if (state.p && x < wi && y < hi) {
                const size_t sp = (size_t)y * wi + x;
#pragma unroll
                for (uint32_t ch = 0; ch < 4; ch++) st(state, sp, ch, ld(o, sp, ch) * fs);
            }
        } else {
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) v[i] = fl.p[(size_t)pix * fl.cs + fl.c0 + i];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4; i++)
            fx.p[(size_t)pix * fx.cs + fx.c0 + 2 * c + 6 + i] = fl.scale == 1.0f ? v[i] : f2h(h2f(v[i]) * fl.scale);
    }
}
template <bool VEC, bool UP>
__global__ __launch_bounds__(kThreads) void fine_input_kernel(View f8, View i8, View fl, OView fx, OView l8,
                                                              uint32_t h, uint32_t w, uint32_t c, uint32_t groups,
                                                              uint32_t items, View o, OView fv, OView state,
                                                              uint32_t hi, uint32_t wi, float fs, float csh,
                                                              float csw) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t < items) fine_input_at<VEC, UP>(f8, i8, fl, fx, l8, h, w, c, groups, o, fv, state, hi, wi, fs, csh, csw, t,
                                          blockIdx.y);
}

// The fine block's cost volume (sad_volume of the two lumas fine_input stores, radius R <= kSadRmax) beside
// fine_input in the same launch: a workgroup takes a kSadTX x kSadTY tile of the cost volume and computes the lumas it
// reads itself, A's on the tile and a ring of 1, B's on a ring of 1 + R, at the clamped pixels sad_at reads (so each
// LDS cell holds what sad_at would load for that unclamped position), with fine_input's arithmetic (the flow from
// coarse_up_at at the view's read scale, the picture's warp rounded to f16, its luma rounded to f16). Then sad_at's
// sums from LDS, in its order, one lane per (pixel, displacement). Small tiles (the frame's 60 x 108 grid makes 210
// of them a pair; at radius 2 one luma a lane), loops unrolled so that each lane's luma loads issue together: the
// volume's workgroups then finish within the fine input's.
constexpr uint32_t kSadTX = 8, kSadTY = 4, kSadRmax = 3;
__device__ __forceinline__ float fine_luma_at(const View& i8, const View& o, float fl_scale, uint32_t h, uint32_t w,
                                              uint32_t hi, uint32_t wi, float fs, float csh, float csw, uint32_t img,
                                              uint32_t x, uint32_t y) {
    const float fxv = h2f(coarse_up_at(o, hi, wi, csh, csw, fs, x, y, 2 * img)) * fl_scale;
    const float fyv = h2f(coarse_up_at(o, hi, wi, csh, csw, fs, x, y, 2 * img + 1)) * fl_scale;
    float v[4];
    warp4<false>(i8, img * h, x, y, h, w, fxv, fyv, 0, 3, v);
    return h2f(f2h(lum3(h2f(f2h(v[0])), h2f(f2h(v[1])), h2f(f2h(v[2])))));
}
// tile `tile` (tiles_x per row) of pair `pair`'s cost volume into out (image pair)
template <int R>
__device__ __forceinline__ void fine_sad_tile(View i8, View o, float fl_scale, OView out, uint32_t h, uint32_t w,
                                              uint32_t hi, uint32_t wi, float fs, float csh, float csw, uint32_t tile,
                                              uint32_t tiles_x, uint32_t pair) {
    constexpr uint32_t AW = kSadTX + 2, BW = kSadTX + 2 + 2 * R, NA = AW * (kSadTY + 2),
                       NB = BW * (kSadTY + 2 + 2 * R), SPAN = 2 * R + 1, S2 = SPAN * SPAN;
    __shared__ float la[NA], lb[NB];
    const size_t hw = (size_t)h * w;
    i8.p += (size_t)pair * 2 * hw * i8.cs, o.p += (size_t)pair * hi * wi * o.cs, out.p += (size_t)pair * hw * out.cs;
    const int x0 = (int)((tile % tiles_x) * kSadTX), y0 = (int)((tile / tiles_x) * kSadTY);
    // lanes past the last cell recompute it (unconditional loads)
#pragma unroll
    for (uint32_t k = 0; k < (NA + NB + kThreads - 1) / kThreads; k++) {
        const uint32_t e = min(threadIdx.x + k * kThreads, NA + NB - 1);
        const bool a = e < NA;
        const uint32_t c = a ? e : e - NA, rw = a ? AW : BW, ring = a ? 1 : 1 + R;
        const int yy = y0 - (int)ring + (int)(c / rw), xx = x0 - (int)ring + (int)(c % rw);
        const float v = fine_luma_at(i8, o, fl_scale, h, w, hi, wi, fs, csh, csw, a ? 0 : 1,
                                     (uint32_t)clampi(xx, 0, (int)w - 1), (uint32_t)clampi(yy, 0, (int)h - 1));
        if (a) la[c] = v;
        else lb[c] = v;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < (kSadTX * kSadTY * S2 + kThreads - 1) / kThreads; k++) {
        const uint32_t e = threadIdx.x + k * kThreads;
        const uint32_t p = e / S2, d = e - p * S2, lx = p % kSadTX, ly = p / kSadTX;
        const int x = x0 + (int)lx, y = y0 + (int)ly;
        if (e >= kSadTX * kSadTY * S2 || x >= (int)w || y >= (int)h) continue;
        const int dy = (int)(d / SPAN) - R, dx = (int)(d % SPAN) - R;
        float acc = 0.0f;
#pragma unroll
        for (int wy = -1; wy <= 1; wy++)
#pragma unroll
            for (int wx = -1; wx <= 1; wx++) {
                const int yy = y + wy, xx = x + wx;
                const bool in = yy >= 0 && yy < (int)h && xx >= 0 && xx < (int)w;
                const float lav = la[((int)ly + 1 + wy) * (int)AW + (int)lx + 1 + wx];
                const float lbv = lb[((int)ly + 1 + R + wy + dy) * (int)BW + (int)lx + 1 + R + wx + dx];
                const float dd = fabsf(lav - lbv);
                acc = acc + (in ? dd : 0.0f);
            }
        st(out, (size_t)y * w + x, d, acc / 9.0f);
    }
}
// blocks [0, fine_blocks): fine_input_kernel<VEC, true>; the rest: the cost volume's tiles. blockIdx.y: the pair.
template <bool VEC, int R>
__global__ __launch_bounds__(kThreads) void fine_input_sad_kernel(View f8, View i8, View fl, OView fx, OView l8,
                                                                  uint32_t h, uint32_t w, uint32_t c, uint32_t groups,
                                                                  uint32_t items, View o, OView fv, OView state,
                                                                  uint32_t hi, uint32_t wi, float fs, float csh,
                                                                  float csw, uint32_t fine_blocks, OView sad,
                                                                  uint32_t tiles_x) {
    if (blockIdx.x < fine_blocks) {
        const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
        if (t < items)
            fine_input_at<VEC, true>(f8, i8, fl, fx, l8, h, w, c, groups, o, fv, state, hi, wi, fs, csh, csw, t,
                                     blockIdx.y);
    } else {
        fine_sad_tile<R>(i8, o, fl.scale, sad, h, w, hi, wi, fs, csh, csw, blockIdx.x - fine_blocks, tiles_x,
                         blockIdx.y);
    }
}

// mid()'s flow_t and vis_t (graph.json ops 44-48, 54-60): lin = mul_t(flow) (2t on the forward flow, 2(1 - t) on
// the backward one, stored f16), flow_t = lin + d_flow; dvis = (d_mask, -d_mask, 0) and vis_t = vis + dvis. fv
// holds flow (channels 0-3) and vis (4-6), df the FiLM head's output (d_flow 0-3, d_mask 4), out flow_t | vis_t.
__global__ __launch_bounds__(kThreads) void flow_vis_t_kernel(View fv, View df, OView out, float af, float ab,
                                                              uint32_t items) {
    const uint32_t pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= items) return;
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        const float lin = h2f(f2h(ld(fv, pix, i) * fv.scale * (i < 2 ? af : ab)));
        st(out, pix, i, lin + ld(df, pix, i) * df.scale);
    }
    const uint16_t dm = df.p[(size_t)pix * df.cs + df.c0 + 4];
    const float dv[3] = {h2f(dm), h2f(f2h(h2f(dm) * -1.0f)), 0.0f};
#pragma unroll
    for (uint32_t j = 0; j < 3; j++) st(out, pix, 4 + j, ld(fv, pix, 4 + j) * fv.scale + dv[j]);
}

// The refine head's input (graph.json ops 65-76): both 1/4 pictures q (batch 2, 3 channels) warped by the upsampled
// flow (channels 0-1 A, 2-3 B, at the flow view's read scale), their blend by the upsampled visibility logits
// (blendmix), and the blend's luma gradient, written as the concat rx: c0 rwa, +3 rwb, +6 vis_tq, +9 flow_tq * fs,
// +13 the gradient. The gradient reads the blend at the right and lower neighbours: a lane recomputes those blends
// (from the same warps and weights, so the same values) instead of a second launch.
// f: the flow at pixel (x, y) (A's x, y, then B's), v: its visibility logits, both at their read scales
__device__ __forceinline__ void blend_vals(const View& q, uint32_t x, uint32_t y, uint32_t h, uint32_t w,
                                           const float (&f)[4], const float (&v)[3], float (&ra)[3], float (&rb)[3],
                                           float (&bl)[3]) {
    float oa[4], ob[4];
    warp4<false>(q, 0, x, y, h, w, f[0], f[1], 0, 3, oa);
    warp4<false>(q, h, x, y, h, w, f[2], f[3], 0, 3, ob);
    float ea, eb, ec, s;
    soft3v(v[0], v[1], v[2], ea, eb, ec, s);
    const float pa = h2f(f2h((ea + 0.5f * ec) / s)), pb = h2f(f2h((eb + 0.5f * ec) / s));
#pragma unroll
    for (uint32_t ch = 0; ch < 3; ch++) {
        ra[ch] = h2f(f2h(oa[ch]));
        rb[ch] = h2f(f2h(ob[ch]));
        bl[ch] = h2f(f2h(h2f(f2h(ra[ch] * pa)) + h2f(f2h(rb[ch] * pb))));
    }
}
__device__ __forceinline__ void blend_at(const View& q, const View& fl, const View& vis, uint32_t x, uint32_t y,
                                         uint32_t h, uint32_t w, float (&ra)[3], float (&rb)[3], float (&bl)[3]) {
    const size_t pix = (size_t)y * w + x;
    const float f[4] = {ld(fl, pix, 0) * fl.scale, ld(fl, pix, 1) * fl.scale, ld(fl, pix, 2) * fl.scale,
                        ld(fl, pix, 3) * fl.scale};
    const float v[3] = {ld(vis, pix, 0) * vis.scale, ld(vis, pix, 1) * vis.scale, ld(vis, pix, 2) * vis.scale};
    blend_vals(q, x, y, h, w, f, v, ra, rb, bl);
}

// One wave per 7 x 7 output pixels: each lane computes the blend of one pixel of the 8 x 8 block around them (the
// block's last column and row are the right and lower neighbours of its outputs; clamped to the picture, unused past
// its edge), so no lane computes two; the gradient reads the neighbours' blends from LDS.
constexpr uint32_t kRiT = 7;
// blockIdx.y: image i of flow, vis and rx, whose pictures are pair (i % qmod) of q (images 2p, 2p + 1)
__global__ __launch_bounds__(64) void refine_input_kernel(View q, View fl, View vis, OView rx, uint32_t h, uint32_t w,
                                                          float fs, uint32_t tiles_x, uint32_t qmod) {
    __shared__ float bt[8 * 8 * 3];
    {
        const size_t hw = (size_t)h * w, img = blockIdx.y;
        q.p += (img % qmod) * 2 * hw * q.cs;
        fl.p += img * hw * fl.cs;
        vis.p += img * hw * vis.cs;
        rx.p += img * hw * rx.cs;
    }
    const uint32_t tx = threadIdx.x % 8, ty = threadIdx.x / 8;
    const uint32_t x0 = (blockIdx.x % tiles_x) * kRiT, y0 = (blockIdx.x / tiles_x) * kRiT;
    const uint32_t x = x0 + tx, y = y0 + ty;
    float ra[3], rb[3], bl[3];
    blend_at(q, fl, vis, min(x, w - 1), min(y, h - 1), h, w, ra, rb, bl);
#pragma unroll
    for (uint32_t ch = 0; ch < 3; ch++) bt[(ty * 8 + tx) * 3 + ch] = bl[ch];
    __syncthreads();
    if (tx >= kRiT || ty >= kRiT || x >= w || y >= h) return;
    const float* br = bt + (ty * 8 + tx + 1) * 3;
    const float* bd = bt + ((ty + 1) * 8 + tx) * 3;
    const size_t pix = (size_t)y * w + x;
    uint16_t* o = rx.p + pix * rx.cs + rx.c0;
#pragma unroll
    for (uint32_t ch = 0; ch < 3; ch++) {
        o[ch] = f2h(ra[ch]);
        o[3 + ch] = f2h(rb[ch]);
        o[6 + ch] = vis.p[(size_t)pix * vis.cs + vis.c0 + ch];
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) o[9 + i] = f2h(ld(fl, pix, i) * fs);
    const float cl = lum3(bl[0], bl[1], bl[2]);
    const float gx = x + 1 < w ? lum3(br[0], br[1], br[2]) - cl : 0.0f;
    const float gy = y + 1 < h ? lum3(bd[0], bd[1], bd[2]) - cl : 0.0f;
    o[13] = f2h(fabsf(gx) + fabsf(gy));
}

// ---- mid()'s upsampled flow and the refine head's input in one launch -------------------------------------------
// flow_t / vis_t and the convex upsample (convex_tile_kernel<true>'s arithmetic) computed at every pixel of the
// refine input's 8 x 8 blend block (a 7 x 7 output tile and its right and lower neighbours, clamped to the picture),
// so that refine_input_kernel's warps and blend take the upsampled flow and visibility from the lane's registers as
// they would read them back (rounded to f16): the lanes of the 7 x 7 outputs also store them (the render reads them).
// An 8-pixel span covers at most kMiC input cells; they and their ring of neighbours make the flow_t | vis_t halo.
constexpr uint32_t kMiC = 5, kMiHalo = kMiC + 2;
// h x w: the input grid (the output 2h x 2w). blockIdx.y: image i, phase i / per of pair i % per: image i of df, up
// and rx, image i % per of wt and fv, pair i % per of q. fls: the scale the refine input reads the flow at (the
// visibility: 1); fs: flow_out_scale.
__global__ __launch_bounds__(64) void mid_input_kernel(View wt, View fv, View df, PhaseT ph, uint32_t per, View q,
                                                       OView up, OView rx, uint32_t h, uint32_t w, float fls, float fs,
                                                       uint32_t tiles_x) {
    __shared__ uint16_t lw[kMiC * kMiC * 36];
    __shared__ uint16_t lx[kMiHalo * kMiHalo * 7];
    __shared__ float bt[8 * 8 * 3];
    const uint32_t img = blockIdx.y, pimg = img % per;
    const float af = ph.af[img / per], ab = ph.ab[img / per];
    const uint32_t oh = 2 * h, ow = 2 * w;
    q.p += (size_t)pimg * 2 * oh * ow * q.cs;
    const uint32_t tid = threadIdx.x, tx = tid % 8, ty = tid / 8;
    const uint32_t x0 = (blockIdx.x % tiles_x) * kRiT, y0 = (blockIdx.x / tiles_x) * kRiT;
    const uint32_t x = min(x0 + tx, ow - 1), y = min(y0 + ty, oh - 1);
    const int cx0 = (int)(x0 / 2), cy0 = (int)(y0 / 2);
    // the cells' mask weights (9 quads of 4 channels a cell), coordinates clamped to the grid; every load
    // unconditional, lanes past the last quad rewriting it
#pragma unroll
    for (uint32_t k = 0; k < (kMiC * kMiC * 9 + 63) / 64; k++) {
        const uint32_t e = min(tid + k * 64, kMiC * kMiC * 9 - 1);
        const uint32_t p = e / 9, qd = e - p * 9, py = p / kMiC, px = p % kMiC;
        const int gy = min(cy0 + (int)py, (int)h - 1), gx = min(cx0 + (int)px, (int)w - 1);
        const uint16_t* src = wt.p + (((size_t)pimg * h + gy) * w + gx) * wt.cs + wt.c0 + qd * 4;
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) lw[p * 36 + qd * 4 + i] = src[i];
    }
    if (tid < kMiHalo * kMiHalo) {  // one lane per halo cell: flow_t | vis_t, zero outside the grid
        const uint32_t py = tid / kMiHalo, px = tid % kMiHalo;
        const int gy = cy0 - 1 + (int)py, gx = cx0 - 1 + (int)px;
        const bool in = gy >= 0 && gy < (int)h && gx >= 0 && gx < (int)w;
        uint16_t v[7];
        const size_t pix = (size_t)clampi(gy, 0, (int)h - 1) * w + clampi(gx, 0, (int)w - 1);
        flow_vis_t_at(fv, df, (size_t)pimg * h * w + pix, (size_t)img * h * w + pix, af, ab, v);
#pragma unroll
        for (uint32_t cc = 0; cc < 7; cc++) lx[tid * 7 + cc] = in ? v[cc] : (uint16_t)0;
    }
    __syncthreads();
    // the lane's pixel: cell (lcx, lcy) of the staged ones, sub-pixel sub
    const uint32_t lcx = x / 2 - (uint32_t)cx0, lcy = y / 2 - (uint32_t)cy0, sub = (y % 2) * 2 + x % 2;
    float ws[9];
    convex_weights(lw + (lcy * kMiC + lcx) * 36 + sub, ws);
    uint16_t u[7];
#pragma unroll
    for (uint32_t co = 0; co < 7; co++) {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < 9; k++)
            acc = acc + __builtin_fmaf(h2f(lx[((lcy + k / 3) * kMiHalo + lcx + k % 3) * 7 + co]), ws[k], 0.0f);
        u[co] = f2h(acc);
    }
    const bool own = tx < kRiT && ty < kRiT && x0 + tx < ow && y0 + ty < oh;
    const size_t pix = ((size_t)img * oh + y) * ow + x;
    if (own) {
        uint16_t* o = up.p + pix * up.cs + up.c0;
#pragma unroll
        for (uint32_t co = 0; co < 7; co++) o[co] = u[co];
    }
    // refine_input_kernel from here, on these values
    const float f[4] = {h2f(u[0]) * fls, h2f(u[1]) * fls, h2f(u[2]) * fls, h2f(u[3]) * fls};
    const float v[3] = {h2f(u[4]), h2f(u[5]), h2f(u[6])};
    float ra[3], rb[3], bl[3];
    blend_vals(q, x, y, oh, ow, f, v, ra, rb, bl);
#pragma unroll
    for (uint32_t ch = 0; ch < 3; ch++) bt[(ty * 8 + tx) * 3 + ch] = bl[ch];
    __syncthreads();
    if (!own) return;
    const float* br = bt + (ty * 8 + tx + 1) * 3;
    const float* bd = bt + ((ty + 1) * 8 + tx) * 3;
    uint16_t* o = rx.p + pix * rx.cs + rx.c0;
#pragma unroll
    for (uint32_t ch = 0; ch < 3; ch++) {
        o[ch] = f2h(ra[ch]);
        o[3 + ch] = f2h(rb[ch]);
        o[6 + ch] = u[4 + ch];
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) o[9 + i] = f2h(h2f(u[i]) * fs);
    const float cl = lum3(bl[0], bl[1], bl[2]);
    const float gx = x + 1 < ow ? lum3(br[0], br[1], br[2]) - cl : 0.0f;
    const float gy = y + 1 < oh ? lum3(bd[0], bd[1], bd[2]) - cl : 0.0f;
    o[13] = f2h(fabsf(gx) + fabsf(gy));
}

// ---- the encoders' outputs into their concat slices (graph.json ops 7, 13 and 26's f16a, f16b; 43's f16b) -----
// x holds the two pictures' features as a batch (2, h, w, c); image i goes to channels c0 + i * c of out (batch 1),
// and image 1 also to `also` (the streaming state's f16b), when given. Bits are copied. One lane per (pixel,
// image, 4 channels); VEC: 8-byte copies.
template <bool VEC>
// pair: pair k's two maps are images 2k, 2k + 1 of x, its fold image k of out and also
__device__ __forceinline__ void fold_pair_at(const View& x, const OView& out, const OView& also, uint32_t hw,
                                             uint32_t c, uint32_t groups, uint32_t t, uint32_t pair) {
    const uint32_t g = t % groups, r = t / groups, img = r % 2, pix = r / 2, ch = g * 4;
    const size_t opix = (size_t)pair * hw + pix;
    const uint16_t* src = x.p + ((size_t)(2 * pair + img) * hw + pix) * x.cs + x.c0 + ch;
    uint16_t* dst = out.p + opix * out.cs + out.c0 + img * c + ch;
    uint16_t* dst2 = also.p ? also.p + opix * also.cs + also.c0 + ch : nullptr;
    if constexpr (VEC) {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        *reinterpret_cast<uint2*>(dst) = v;
        if (img == 1 && dst2) *reinterpret_cast<uint2*>(dst2) = v;
    } else {
        for (uint32_t i = 0; i < 4 && ch + i < c; i++) {
            dst[i] = src[i];
            if (img == 1 && dst2) dst2[i] = src[i];
        }
    }
}
template <bool VEC>
__global__ __launch_bounds__(kThreads) void fold_pair_kernel(View x, OView out, OView also, uint32_t hw, uint32_t c,
                                                             uint32_t groups, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t < items) fold_pair_at<VEC>(x, out, also, hw, c, groups, t, 0);
}

// fold_pair and a sad_volume that neither reads what the other writes, side by side in one launch: blocks below
// fold_blocks run the fold of pair blockIdx.y, the rest (of row 0) the cost volume (pair() folds the second encoder
// pair's output while the 1/16 lumas' cost volume, ready since the pyramid, is computed)
struct SadArgs {
    View la, lb;
    OView out;
    uint32_t h, w, r, span2, items;
};
template <bool VEC>
__global__ __launch_bounds__(kThreads) void fold_pair_sad_kernel(View x, OView out, OView also, uint32_t hw,
                                                                 uint32_t c, uint32_t groups, uint32_t items,
                                                                 uint32_t fold_blocks, SadArgs sa) {
    if (blockIdx.x < fold_blocks) {
        const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
        if (t < items) fold_pair_at<VEC>(x, out, also, hw, c, groups, t, blockIdx.y);
    } else if (blockIdx.y == 0) {
        const uint32_t t = (blockIdx.x - fold_blocks) * kThreads + threadIdx.x;
        if (t < sa.items) sad_at(sa.la, sa.lb, sa.out, sa.h, sa.w, sa.r, sa.span2, t);
    }
}

// ---- the coarse head's outputs (graph.json ops 33-40 and 43's flow16) ------------------------------------------
// o (1, hi, wi) holds the coarse flow (channels 0-3, read times fs: flow16) and visibility logits (4-6). Out (1, oh, ow)
// gets both resized bilinearly (interp.wgsl, align_corners false; the scale applies to the result): flow 0-3, vis
// 4-6; `state` (when given) gets the scaled flow itself at the input size (chcopy). One lane per output pixel; the
// lanes of the first hi x wi pixels also write the state.
__global__ __launch_bounds__(kThreads) void coarse_up_kernel(View o, OView out, OView state, uint32_t hi, uint32_t wi,
                                                             uint32_t oh, uint32_t ow, float fs, uint32_t items) {
    const uint32_t pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= items) return;
    const uint32_t ox = pix % ow, oy = pix / ow;
    const float sh = (float)hi / (float)oh, sw = (float)wi / (float)ow;
    const float fiy = ((float)oy + 0.5f) * sh - 0.5f, fix = ((float)ox + 0.5f) * sw - 0.5f;
    const int y0 = (int)floorf(fiy), x0 = (int)floorf(fix);
    const float fy = fiy - (float)y0, fx = fix - (float)x0;
    const size_t r0 = (size_t)clampi(y0, 0, (int)hi - 1) * wi, r1 = (size_t)clampi(y0 + 1, 0, (int)hi - 1) * wi;
    const uint32_t c0 = clampi(x0, 0, (int)wi - 1), c1 = clampi(x0 + 1, 0, (int)wi - 1);
#pragma unroll
    for (uint32_t ch = 0; ch < 7; ch++) {
        const float v00 = ld(o, r0 + c0, ch), v01 = ld(o, r0 + c1, ch), v10 = ld(o, r1 + c0, ch), v11 = ld(o, r1 + c1, ch);
        const float val = (v00 * (1.0f - fx) + v01 * fx) * (1.0f - fy) + (v10 * (1.0f - fx) + v11 * fx) * fy;
        st(out, pix, ch, val * (ch < 4 ? fs : 1.0f));
    }
    if (state.p && ox < wi && oy < hi) {
        const size_t sp = (size_t)oy * wi + ox;
#pragma unroll
        for (uint32_t ch = 0; ch < 4; ch++) st(state, sp, ch, ld(o, sp, ch) * fs);
    }
}

// ---- render_pix: shaders/render.wgsl:83-160 ------------------------------------------------------------------
// One lane per output pixel: flow, visibility logits and residual upsampled bilinearly from the quarter maps, A and
// B sampled at the displaced positions (bilinear, or bicubic: Keys a = -0.75 with every tap clamped to the border),
// blended, + residual, clamped. All taps load from clamped addresses unconditionally (one round of loads).
__device__ __forceinline__ float bil4(float v00, float v01, float v10, float v11, float fx, float fy) {
    return (v00 * (1.0f - fx) + v01 * fx) * (1.0f - fy) + (v10 * (1.0f - fx) + v11 * fx) * fy;
}
// the Keys weights for a = -0.75 in the shader's order ((a + 2) = 1.25, (a + 3) = 2.25, 5a, 8a, 4a)
__device__ __forceinline__ float cub1(float x) { return ((1.25f * x - 2.25f) * x) * x + 1.0f; }
__device__ __forceinline__ float cub2(float x) { return ((-0.75f * x - -3.75f) * x + -6.0f) * x - -3.0f; }

template <bool VEC>
__device__ __forceinline__ void tap3(const View& v, uint32_t h, uint32_t w, int y, int x, float (&o)[4]) {
    ld4<VEC>(v, (size_t)clampi(y, 0, (int)h - 1) * w + clampi(x, 0, (int)w - 1), 0, 3, o);
}

template <bool VEC, bool CUBIC>
__device__ __forceinline__ void sample3(const View& v, uint32_t h, uint32_t w, float gx, float gy, float (&o)[3]) {
    const int px = (int)floorf(gx), py = (int)floorf(gy);
    const float tx = gx - (float)px, ty = gy - (float)py;
    if constexpr (CUBIC) {
        const float cx[4] = {cub2(tx + 1.0f), cub1(tx), cub1(1.0f - tx), cub2(2.0f - tx)};
        const float cy[4] = {cub2(ty + 1.0f), cub1(ty), cub1(1.0f - ty), cub2(2.0f - ty)};
        float t[4][4][4];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) tap3<VEC>(v, h, w, py - 1 + j, px - 1 + i, t[j][i]);
#pragma unroll
        for (int c = 0; c < 3; c++) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float row = t[j][0][c] * cx[0] + t[j][1][c] * cx[1] + t[j][2][c] * cx[2] + t[j][3][c] * cx[3];
                acc = j == 0 ? row * cy[0] : acc + row * cy[j];
            }
            o[c] = acc;
        }
    } else {
        float t00[4], t01[4], t10[4], t11[4];
        tap3<VEC>(v, h, w, py, px, t00);
        tap3<VEC>(v, h, w, py, px + 1, t01);
        tap3<VEC>(v, h, w, py + 1, px, t10);
        tap3<VEC>(v, h, w, py + 1, px + 1, t11);
#pragma unroll
        for (int c = 0; c < 3; c++) o[c] = bil4(t00[c], t01[c], t10[c], t11[c], tx, ty);
    }
}

// the bicubic sum of one picture's 16 raw 8-byte taps (rows j, columns i), in sample3's order
__device__ __forceinline__ void cubic_sum(const uint2* t, float tx, float ty, float (&o)[3]) {
    const float cx[4] = {cub2(tx + 1.0f), cub1(tx), cub1(1.0f - tx), cub2(2.0f - tx)};
    const float cy[4] = {cub2(ty + 1.0f), cub1(ty), cub1(1.0f - ty), cub2(2.0f - ty)};
#pragma unroll
    for (int c = 0; c < 3; c++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint2 q = t[j * 4 + i];
                v[i] = h2f((uint16_t)((c < 2 ? q.x : q.y) >> (c == 1 ? 16 : 0)));
            }
            const float row = v[0] * cx[0] + v[1] * cx[1] + v[2] * cx[2] + v[3] * cx[3];
            acc = j == 0 ? row * cy[0] : acc + row * cy[j];
        }
        o[c] = acc;
    }
}

template <bool VEC, bool CUBIC>
__global__ __launch_bounds__(kThreads) void render_kernel(View a, View b, View fl, View vis, View rt, OView out,
                                                          uint32_t h, uint32_t w, uint32_t hq, uint32_t wq, float fsx,
                                                          float fsy, uint32_t flags, uint32_t items) {
    const uint32_t pix = blockIdx.x * kThreads + threadIdx.x;
    if (pix >= items) return;
    const uint32_t x = pix % w, y = pix / w;
    const float sh = (float)hq / (float)h, sw = (float)wq / (float)w;
    const float iy = ((float)y + 0.5f) * sh - 0.5f, ix = ((float)x + 0.5f) * sw - 0.5f;
    const int qy0 = (int)floorf(iy), qx0 = (int)floorf(ix);
    const float qfy = iy - (float)qy0, qfx = ix - (float)qx0;
    const uint32_t y0 = clampi(qy0, 0, (int)hq - 1), y1 = clampi(qy0 + 1, 0, (int)hq - 1);
    const uint32_t x0 = clampi(qx0, 0, (int)wq - 1), x1 = clampi(qx0 + 1, 0, (int)wq - 1);
    const size_t q00 = (size_t)y0 * wq + x0, q01 = (size_t)y0 * wq + x1, q10 = (size_t)y1 * wq + x0,
                 q11 = (size_t)y1 * wq + x1;
    // every quarter-map value is loaded before any is used: one round of memory latency, not two
    const size_t qs[4] = {q00, q01, q10, q11};
    float fq[4][4], vq[4][3], rq[4][3];
#pragma unroll
    for (int k = 0; k < 4; k++) {
#pragma unroll
        for (uint32_t c = 0; c < 4; c++) fq[k][c] = ld(fl, qs[k], c);
#pragma unroll
        for (uint32_t c = 0; c < 3; c++) vq[k][c] = ld(vis, qs[k], c), rq[k][c] = ld(rt, qs[k], c);
    }
    __builtin_amdgcn_sched_barrier(0);
    float f[4], v[3], r[3];
#pragma unroll
    for (uint32_t c = 0; c < 4; c++)
        f[c] = bil4(fq[0][c], fq[1][c], fq[2][c], fq[3][c], qfx, qfy) * ((c & 1u) == 0 ? fsx : fsy);
#pragma unroll
    for (uint32_t c = 0; c < 3; c++) {
        v[c] = bil4(vq[0][c], vq[1][c], vq[2][c], vq[3][c], qfx, qfy) * vis.scale;
        r[c] = bil4(rq[0][c], rq[1][c], rq[2][c], rq[3][c], qfx, qfy);
    }
    const float m = fmaxf(v[0], fmaxf(v[1], v[2]));
    const float e0 = expf(v[0] - m), e1 = expf(v[1] - m), e2 = expf(v[2] - m), s = e0 + e1 + e2;
    const float wa_w = (e0 + 0.5f * e2) / s, wb_w = (e1 + 0.5f * e2) / s;
    float ca[3], cb[3];
    if constexpr (VEC && CUBIC) {  // both pictures' 32 taps as raw 8-byte values, loaded before any is used
        uint2 t[2][16];
        float tx[2], ty[2];
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const View& src = p == 0 ? a : b;
            const float gx = (float)x + f[2 * p], gy = (float)y + f[2 * p + 1];
            const int px = (int)floorf(gx), py = (int)floorf(gy);
            tx[p] = gx - (float)px, ty[p] = gy - (float)py;
            // 32-bit element offsets from one 24-bit product per row and per column: the launch takes this path
            // only when a row holds fewer than 2^24 elements and a picture fewer than 2^31
            uint32_t col[4], row[4];
#pragma unroll
            for (int i = 0; i < 4; i++) col[i] = __umul24((uint32_t)clampi(px - 1 + i, 0, (int)w - 1), src.cs) + src.c0;
#pragma unroll
            for (int j = 0; j < 4; j++) row[j] = __umul24((uint32_t)clampi(py - 1 + j, 0, (int)h - 1), w * src.cs);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    t[p][j * 4 + i] = *reinterpret_cast<const uint2*>(src.p + (row[j] + col[i]));
        }
        __builtin_amdgcn_sched_barrier(0);
        cubic_sum(t[0], tx[0], ty[0], ca);
        cubic_sum(t[1], tx[1], ty[1], cb);
    } else {
        sample3<VEC, CUBIC>(a, h, w, (float)x + f[0], (float)y + f[1], ca);
        sample3<VEC, CUBIC>(b, h, w, (float)x + f[2], (float)y + f[3], cb);
    }
    float bwa = wa_w, bwb = wb_w, rk = 1.0f, stillw = 0.0f, own[3] = {0.0f, 0.0f, 0.0f};
    const float third = 1.0f / 3.0f;
    const float ef = fabsf(ca[0] - cb[0]) * third + fabsf(ca[1] - cb[1]) * third + fabsf(ca[2] - cb[2]) * third;
    if (flags & 2u) {  // the still test (render.wgsl:134-148)
        float es = 0.0f;
#pragma unroll
        for (int dy = -1; dy <= 1; dy++)
#pragma unroll
            for (int dx = -1; dx <= 1; dx++) {
                float pa[4], pb[4];
                tap3<VEC>(a, h, w, (int)y + dy, (int)x + dx, pa);
                tap3<VEC>(b, h, w, (int)y + dy, (int)x + dx, pb);
#pragma unroll
                for (int c = 0; c < 3; c++) es += fabsf(pa[c] - pb[c]);
            }
        es = es / 27.0f;
        float pa[4], pb[4];
        tap3<VEC>(a, h, w, (int)y, (int)x, pa);
        tap3<VEC>(b, h, w, (int)y, (int)x, pb);
#pragma unroll
        for (int c = 0; c < 3; c++) own[c] = 0.5f * (pa[c] + pb[c]);
        stillw = fminf(fmaxf((ef - es) / 0.04f, 0.0f), 1.0f) * (es < 0.03f ? 1.0f : 0.0f);
    }
    if (flags & 1u) {  // the decisive blend (render.wgsl:149-153)
        const float k = fminf(fmaxf((ef - 0.04f) / 0.08f, 0.0f), 1.0f);
        const float pa = wa_w >= wb_w ? 1.0f : 0.0f;
        bwa = wa_w * (1.0f - k) + pa * k;
        bwb = wb_w * (1.0f - k) + (1.0f - pa) * k;
        rk = 1.0f - k;
    }
#pragma unroll
    for (uint32_t c = 0; c < 3; c++) {
        const float mixed = ca[c] * bwa + cb[c] * bwb + r[c] * rk;
        st(out, pix, c, fminf(fmaxf(mixed * (1.0f - stillw) + own[c] * stillw, 0.0f), 1.0f));
    }
}

// ---- the host's 8-bit frames: rgba_in.wgsl:11-19, rgba_out.wgsl:9-18 -------------------------------------------
// A frame is RGBA8, one 32-bit word per pixel (R | G << 8 | B << 16 | A << 24), rows `pitch` words apart. The network
// reads BGR f16 in [0, 1] replicate-padded to hp x wp: padded pixel (x, y) is frame pixel (min(x, w - 1),
// min(y, h - 1)). A sampler that clamps its coordinates to the padded picture therefore reads exactly what clamping
// them to the frame reads, which the fused kernels below use to sample the 8-bit frame directly.

// BGR channel ch (0 B, 1 G, 2 R) of an RGBA8 word, as f16(f32(byte) / 255): the product with the f32 reciprocal of
// 255 rounds to the same f16 as the quotient for each of the 256 bytes (and both to the f16 of the exact fraction)
__device__ __forceinline__ uint16_t unit_f16(uint32_t v, int ch) {
    return f2h((float)((v >> (16 - 8 * ch)) & 0xffu) * (1.0f / 255.0f));
}
__device__ __forceinline__ float unit_f32(uint32_t v, int ch) { return h2f(unit_f16(v, ch)); }
// rgba_out.wgsl:10: an f16 value in [0, 1] to its byte (v * 255 + 0.5 is exact in f32 for every f16 v)
__device__ __forceinline__ uint32_t byte_of(uint16_t hv) {
    return (uint32_t)(fminf(fmaxf(h2f(hv), 0.0f), 1.0f) * 255.0f + 0.5f);
}

// one lane per padded pixel; VEC4: the output view has 8-byte 4-channel pixels (channel 3 written 0)
template <bool VEC4>
__global__ __launch_bounds__(kThreads) void rgba_in_kernel(const uint32_t* src, uint32_t w, uint32_t h, uint32_t pitch,
                                                           uint64_t fstride, OView out, uint32_t hp, uint32_t wp,
                                                           uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t x = t % wp, r = t / wp, y = r % hp, img = r / hp;
    const uint32_t v = src[img * fstride + (size_t)min(y, h - 1) * pitch + min(x, w - 1)];
    const uint16_t b = unit_f16(v, 0), g = unit_f16(v, 1), rr = unit_f16(v, 2);
    if constexpr (VEC4) {
        *reinterpret_cast<uint2*>(out.p + (size_t)t * out.cs) = uint2{(uint32_t)b | ((uint32_t)g << 16), rr};
    } else {
        uint16_t* o = out.p + (size_t)t * out.cs + out.c0;
        o[0] = b, o[1] = g, o[2] = rr;
    }
}

// one lane per frame pixel: channels 0-2 (B, G, R) of the padded view, cropped to w x h
__global__ __launch_bounds__(kThreads) void rgba_out_kernel(View in, uint32_t hp, uint32_t wp, uint32_t* dst,
                                                            uint32_t w, uint32_t h, uint32_t pitch, uint64_t fstride,
                                                            uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t x = t % w, r = t / w, y = r % h, img = r / h;
    const uint16_t* p = in.p + (((size_t)img * hp + y) * wp + x) * in.cs + in.c0;
    dst[img * fstride + (size_t)y * pitch + x] =
        byte_of(p[2]) | (byte_of(p[1]) << 8) | (byte_of(p[0]) << 16) | 0xff000000u;
}

// 16 and 8 bytes of a frame row at a 4-byte aligned address (global loads need only dword alignment)
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

// The 4 words of frame row y at the clamped columns px - 1 .. px + 2 (w >= 4): one 16-byte load at column
// clamp(px - 1, 0, w - 4), whose 4 words hold every clamped column (each lies 0..3 past it), then a pick per tap.
__device__ __forceinline__ void row_taps4(const uint32_t* f, uint32_t pitch, uint32_t y, int px, uint32_t w,
                                          uint32_t (&t)[4]) {
    const int base = clampi(px - 1, 0, (int)w - 4);
    const u32x4_a4 q = *reinterpret_cast<const u32x4_a4*>(f + (size_t)y * pitch + base);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int off = clampi(px - 1 + i, 0, (int)w - 1) - base;
        t[i] = off == 0 ? q.x : off == 1 ? q.y : off == 2 ? q.z : q.w;
    }
}
// the 2 words of row y at the clamped columns px, px + 1 (w >= 2), the same way
__device__ __forceinline__ void row_taps2(const uint32_t* f, uint32_t pitch, uint32_t y, int px, uint32_t w,
                                          uint32_t (&t)[2]) {
    const int base = clampi(px, 0, (int)w - 2);
    const u32x2_a4 q = *reinterpret_cast<const u32x2_a4*>(f + (size_t)y * pitch + base);
#pragma unroll
    for (int i = 0; i < 2; i++) t[i] = clampi(px + i, 0, (int)w - 1) - base == 0 ? q.x : q.y;
}

// The conversion unit_f32 as a table: entry b is f32(f16(b / 255)), the value rgba_in stores for byte b. A block
// fills its copy (1 KiB of LDS) before any lane reads it; a read costs one VALU op (the byte times 4, a shift with a
// byte select) where the arithmetic takes four.
__device__ __forceinline__ void fill_unit_table(float* tab) {
    for (uint32_t i = threadIdx.x; i < 256; i += kThreads) tab[i] = unit_f32(i << 16, 0);
    __syncthreads();
}
__device__ __forceinline__ float unit_tab(const float* tab, uint32_t v, int ch) {
    return tab[(v >> (16 - 8 * ch)) & 0xffu];
}

// a * b + c: one fused multiply-add (one rounding) with FMA, else the product rounded, then the sum
template <bool FMA>
__device__ __forceinline__ float mac(float a, float b, float c) {
    if constexpr (FMA) return __builtin_fmaf(a, b, c);
    else return a * b + c;
}
// bil4 and the Keys weights in the same expression order, each product feeding a sum fused with it when FMA
template <bool FMA>
__device__ __forceinline__ float bil4m(float v00, float v01, float v10, float v11, float fx, float fy) {
    if constexpr (!FMA) return bil4(v00, v01, v10, v11, fx, fy);
    const float gx = 1.0f - fx;
    return mac<true>(mac<true>(v11, fx, v10 * gx), fy, mac<true>(v01, fx, v00 * gx) * (1.0f - fy));
}
// bil4m<true> with the four taps as f16: each product v * g is written as an FMA with a zero addend (the same value
// up to the sign of a zero product, which no later step can see), so every conversion folds into a mixed-precision
// FMA and no tap needs a conversion instruction of its own
__device__ __forceinline__ float bil4h(_Float16 v00, _Float16 v01, _Float16 v10, _Float16 v11, float fx, float fy) {
    const float gx = 1.0f - fx;
    return __builtin_fmaf(__builtin_fmaf((float)v11, fx, __builtin_fmaf((float)v10, gx, 0.0f)), fy,
                          __builtin_fmaf((float)v01, fx, __builtin_fmaf((float)v00, gx, 0.0f)) * (1.0f - fy));
}
template <bool FMA>
__device__ __forceinline__ float cub1m(float x) {
    if constexpr (!FMA) return cub1(x);
    return mac<true>(mac<true>(1.25f, x, -2.25f) * x, x, 1.0f);
}
template <bool FMA>
__device__ __forceinline__ float cub2m(float x) {
    if constexpr (!FMA) return cub2(x);
    return mac<true>(mac<true>(mac<true>(-0.75f, x, 3.75f), x, -6.0f), x, 3.0f);
}

// Channel c of the bicubic sum over the 4 x 4 taps t (rows j, columns i) with the weights cx, cy (render.wgsl:
// 37-46): each row's four products summed in order, the rows times cy summed in order
template <bool FMA>
__device__ __forceinline__ float cubic_sum(const uint32_t (&t)[4][4], const float (&cx)[4], const float (&cy)[4],
                                           const float* tab, int c) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float row = unit_tab(tab, t[j][0], c) * cx[0];
#pragma unroll
        for (int i = 1; i < 4; i++) row = mac<FMA>(unit_tab(tab, t[j][i], c), cx[i], row);
        acc = j == 0 ? row * cy[0] : mac<FMA>(row, cy[j], acc);
    }
    return acc;
}

// The three channels of one render.wgsl sample (bicubic: :20-47, bilinear: :9-18) of an RGBA8 frame at the sample
// point (px + tx, py + ty), px, py = floor of its coordinates, each tap converted as rgba_in converts it. INNER: the
// columns px - 1 .. px + 2 (bicubic) or px, px + 1 (bilinear) all lie inside the frame for every lane of the wave,
// so one 16- (8-) byte load per row holds the taps in order; otherwise each tap column is clamped to the frame.
template <bool CUBIC, bool INNER, bool FMA = false>
__device__ __forceinline__ void sample_rgba(const uint32_t* src, uint32_t pitch, uint32_t w, uint32_t h, int px,
                                            int py, float tx, float ty, const float* tab, float (&o)[3]) {
    if constexpr (CUBIC) {
        const float cx[4] = {cub2m<FMA>(tx + 1.0f), cub1m<FMA>(tx), cub1m<FMA>(1.0f - tx), cub2m<FMA>(2.0f - tx)};
        const float cy[4] = {cub2m<FMA>(ty + 1.0f), cub1m<FMA>(ty), cub1m<FMA>(1.0f - ty), cub2m<FMA>(2.0f - ty)};
        uint32_t t[4][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t yy = (uint32_t)clampi(py - 1 + j, 0, (int)h - 1);
            if constexpr (INNER) {
                const u32x4_a4 q = *reinterpret_cast<const u32x4_a4*>(src + (size_t)yy * pitch + (px - 1));
                t[j][0] = q.x, t[j][1] = q.y, t[j][2] = q.z, t[j][3] = q.w;
            } else {
                row_taps4(src, pitch, yy, px, w, t[j]);
            }
        }
#pragma unroll
        for (int c = 0; c < 3; c++) o[c] = cubic_sum<FMA>(t, cx, cy, tab, c);
    } else {
        uint32_t t0[2], t1[2];
        const uint32_t ya = (uint32_t)clampi(py, 0, (int)h - 1), yb = (uint32_t)clampi(py + 1, 0, (int)h - 1);
        if constexpr (INNER) {
            const u32x2_a4 q0 = *reinterpret_cast<const u32x2_a4*>(src + (size_t)ya * pitch + px);
            const u32x2_a4 q1 = *reinterpret_cast<const u32x2_a4*>(src + (size_t)yb * pitch + px);
            t0[0] = q0.x, t0[1] = q0.y, t1[0] = q1.x, t1[1] = q1.y;
        } else {
            row_taps2(src, pitch, ya, px, w, t0);
            row_taps2(src, pitch, yb, px, w, t1);
        }
#pragma unroll
        for (int c = 0; c < 3; c++)
            o[c] = bil4m<FMA>(unit_tab(tab, t0[0], c), unit_tab(tab, t0[1], c), unit_tab(tab, t1[0], c),
                              unit_tab(tab, t1[1], c), tx, ty);
    }
}

// A buffer resource over `bytes` bytes at base: loads through it take a 32-bit byte offset (one 24-bit multiply-add
// per row address instead of 64-bit address arithmetic); offsets past `bytes` read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// sample_rgba's INNER case (every tap column inside the frame for the whole wave) through a buffer resource over
// the frame: row y's taps at byte offset y * pitch4 + 4 (px - 1) (bicubic) or y * pitch4 + 4 px (bilinear); the same
// taps, the same arithmetic. ROWS: every tap row inside the frame too for the whole wave, so no row is clamped and
// row j's offset is the first row's plus the wave-uniform j * pitch4 (the load's scalar offset).
template <bool CUBIC, bool FMA, bool ROWS = false>
__device__ __forceinline__ void sample_rgba_inner(__amdgpu_buffer_rsrc_t rs, uint32_t pitch4, int hm1, int px, int py,
                                                  float tx, float ty, const float* tab, float (&o)[3]) {
    if constexpr (CUBIC) {
        const float cx[4] = {cub2m<FMA>(tx + 1.0f), cub1m<FMA>(tx), cub1m<FMA>(1.0f - tx), cub2m<FMA>(2.0f - tx)};
        const float cy[4] = {cub2m<FMA>(ty + 1.0f), cub1m<FMA>(ty), cub1m<FMA>(1.0f - ty), cub2m<FMA>(2.0f - ty)};
        const uint32_t col4 = (uint32_t)(px - 1) * 4u;
        const uint32_t row0 = ROWS ? __umul24((uint32_t)(py - 1), pitch4) + col4 : 0u;
        uint32_t t[4][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint4 q;
            if constexpr (ROWS) {
                q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, row0, (uint32_t)j * pitch4, 0));
            } else {
                const uint32_t yy = (uint32_t)min(max(py - 1 + j, 0), hm1);
                q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, __umul24(yy, pitch4) + col4, 0, 0));
            }
            t[j][0] = q.x, t[j][1] = q.y, t[j][2] = q.z, t[j][3] = q.w;
        }
#pragma unroll
        for (int c = 0; c < 3; c++) o[c] = cubic_sum<FMA>(t, cx, cy, tab, c);
    } else {
        const uint32_t col4 = (uint32_t)px * 4u;
        const uint32_t ya = ROWS ? (uint32_t)py : (uint32_t)min(max(py, 0), hm1);
        const uint32_t yb = ROWS ? (uint32_t)py + 1u : (uint32_t)min(max(py + 1, 0), hm1);
        const uint2 q0 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, __umul24(ya, pitch4) + col4, 0, 0));
        const uint2 q1 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, __umul24(yb, pitch4) + col4, 0, 0));
#pragma unroll
        for (int c = 0; c < 3; c++)
            o[c] = bil4m<FMA>(unit_tab(tab, q0.x, c), unit_tab(tab, q0.y, c), unit_tab(tab, q1.x, c),
                              unit_tab(tab, q1.y, c), tx, ty);
    }
}

// One frame pixel of render_rgba from its upsampled flow f (x, y for A, then for B, in frame pixels), visibility
// logits v and residual r: the blend weights, A and B sampled at the displaced positions, the blend, rgba_out.
template <bool CUBIC, bool FL, bool FMA>
__device__ __forceinline__ void render_rgba_px(uint32_t x, uint32_t y, const float (&f)[4], const float (&v)[3],
                                               const float (&r)[3], const uint32_t* fa, const uint32_t* fb, uint32_t w,
                                               uint32_t h, uint32_t pitch, const float* tab, uint32_t flags,
                                               uint32_t* dst, uint32_t opitch) {
    const float m = fmaxf(v[0], fmaxf(v[1], v[2]));
    float wa_w, wb_w;
    if constexpr (FMA) {  // the hardware exponential and reciprocal (s >= 1: the largest term is exp(0))
        const float e0 = __expf(v[0] - m), e1 = __expf(v[1] - m), e2 = __expf(v[2] - m);
        const float inv = __builtin_amdgcn_rcpf(e0 + e1 + e2);
        wa_w = (e0 + 0.5f * e2) * inv, wb_w = (e1 + 0.5f * e2) * inv;
    } else {
        const float e0 = expf(v[0] - m), e1 = expf(v[1] - m), e2 = expf(v[2] - m), s = e0 + e1 + e2;
        wa_w = (e0 + 0.5f * e2) / s, wb_w = (e1 + 0.5f * e2) / s;
    }
    float ca[3], cb[3];
    const float gxa = (float)x + f[0], gya = (float)y + f[1], gxb = (float)x + f[2], gyb = (float)y + f[3];
    const int pxa = (int)floorf(gxa), pya = (int)floorf(gya), pxb = (int)floorf(gxb), pyb = (int)floorf(gyb);
    const float txa = gxa - (float)pxa, tya = gya - (float)pya, txb = gxb - (float)pxb, tyb = gyb - (float)pyb;
    const int lo = CUBIC ? 1 : 0, hi = (int)w - (CUBIC ? 3 : 2), hir = (int)h - (CUBIC ? 3 : 2);
    const bool inner = pxa >= lo && pxa <= hi && pxb >= lo && pxb <= hi;
    const bool rows = pya >= lo && pya <= hir && pyb >= lo && pyb <= hir;
    const uint32_t fbytes = ((h - 1) * pitch + w) * 4u, pitch4 = pitch * 4u;
    if (__all(inner && rows)) {
        sample_rgba_inner<CUBIC, FMA, true>(buf_rsrc(fa, fbytes), pitch4, (int)h - 1, pxa, pya, txa, tya, tab, ca);
        sample_rgba_inner<CUBIC, FMA, true>(buf_rsrc(fb, fbytes), pitch4, (int)h - 1, pxb, pyb, txb, tyb, tab, cb);
    } else if (__all(inner)) {
        sample_rgba_inner<CUBIC, FMA>(buf_rsrc(fa, fbytes), pitch4, (int)h - 1, pxa, pya, txa, tya, tab, ca);
        sample_rgba_inner<CUBIC, FMA>(buf_rsrc(fb, fbytes), pitch4, (int)h - 1, pxb, pyb, txb, tyb, tab, cb);
    } else {
        sample_rgba<CUBIC, false, FMA>(fa, pitch, w, h, pxa, pya, txa, tya, tab, ca);
        sample_rgba<CUBIC, false, FMA>(fb, pitch, w, h, pxb, pyb, txb, tyb, tab, cb);
    }
    float bwa = wa_w, bwb = wb_w, rk = 1.0f, stillw = 0.0f, own[3] = {0.0f, 0.0f, 0.0f};
    const float third = 1.0f / 3.0f;
    float ef = 0.0f;
    if (FL)
        ef = fabsf(ca[0] - cb[0]) * third + fabsf(ca[1] - cb[1]) * third + fabsf(ca[2] - cb[2]) * third;
    if (FL && (flags & 2u)) {  // the still test (render.wgsl:134-148) on the 3 x 3 neighbourhood, clamped to the frame
        uint32_t ta[3][4], tb[3][4];
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const uint32_t yy = (uint32_t)clampi((int)y - 1 + j, 0, (int)h - 1);
            row_taps4(fa, pitch, yy, (int)x, w, ta[j]);
            row_taps4(fb, pitch, yy, (int)x, w, tb[j]);
        }
        float es = 0.0f;
#pragma unroll
        for (int j = 0; j < 3; j++)
#pragma unroll
            for (int i = 0; i < 3; i++)
#pragma unroll
                for (int c = 0; c < 3; c++) es += fabsf(unit_tab(tab, ta[j][i], c) - unit_tab(tab, tb[j][i], c));
        es = es / 27.0f;
#pragma unroll
        for (int c = 0; c < 3; c++) own[c] = 0.5f * (unit_tab(tab, ta[1][1], c) + unit_tab(tab, tb[1][1], c));
        stillw = fminf(fmaxf((ef - es) / 0.04f, 0.0f), 1.0f) * (es < 0.03f ? 1.0f : 0.0f);
    }
    if (FL && (flags & 1u)) {  // the decisive blend (render.wgsl:149-153)
        const float k = fminf(fmaxf((ef - 0.04f) / 0.08f, 0.0f), 1.0f);
        const float pa = wa_w >= wb_w ? 1.0f : 0.0f;
        bwa = wa_w * (1.0f - k) + pa * k;
        bwb = wb_w * (1.0f - k) + (1.0f - pa) * k;
        rk = 1.0f - k;
    }
    uint32_t bytes[3];
#pragma unroll
    for (int c = 0; c < 3; c++) {
        if constexpr (FL) {
            const float mixed = mac<FMA>(r[c], rk, mac<FMA>(cb[c], bwb, ca[c] * bwa));
            bytes[c] = byte_of(f2h(fminf(fmaxf(mac<FMA>(own[c], stillw, mixed * (1.0f - stillw)), 0.0f), 1.0f)));
        } else {
            bytes[c] = byte_of(f2h(fminf(fmaxf(mac<FMA>(cb[c], bwb, ca[c] * bwa) + r[c], 0.0f), 1.0f)));
        }
    }
    dst[(size_t)y * opitch + x] = bytes[2] | (bytes[1] << 8) | (bytes[0] << 16) | 0xff000000u;
}

// render_pix of the padded frame (hp x wp) from the two RGBA8 frames, written as RGBA8 (rgba_out of the f16 result),
// cropped to w x h: render.wgsl:83-160 with its sources replaced by rgba_in.wgsl's conversion of the frames, then
// rgba_out.wgsl. One lane per frame pixel. QV: flow and vis are channels 0-3 and 4-6 of one 8-channel view (16-byte
// pixels) and rt has 8-byte pixels, so each quarter-map tap is two loads. A wave whose sample windows all lie inside
// the frame takes the unclamped tap loads (the same values: clamping changes no column there).
// A block is 64 x 4 pixels (a wave per row segment); sh = hq / hp and sw = wq / wp come from the host (the same f32
// quotients the reference forms per pixel). FL: flags may be nonzero. Without flags (the engine's default) stillw = 0
// and rk = 1, so r * rk is r and mixed * (1 - stillw) + own * stillw is mixed (or +0 for a mixed of -0, which the
// clamp and the byte conversion turn into the same byte 0): that variant leaves those terms out.
template <bool CUBIC, bool QV, bool FL, bool FMA>
// blockIdx.z: generated frame z of `phases` per pair, pair-major (pair p = z / phases, phase j): its frames at
// p * pstride words past fa and fb, its maps image j * per + p of fl, vis and rt, its output frame j * per + p,
// ostride words apart (one frame: z = 0)
__global__ __launch_bounds__(kThreads) void render_rgba_kernel(const uint32_t* fa, const uint32_t* fb, uint32_t w,
                                                               uint32_t h, uint32_t pitch, float sh, float sw,
                                                               View fl, View vis, View rt, uint32_t hq, uint32_t wq,
                                                               float fsx, float fsy, uint32_t flags, uint32_t* dst,
                                                               uint32_t opitch, uint64_t pstride, uint32_t per,
                                                               uint32_t phases, uint64_t ostride) {
    __shared__ float tab[256];
    if (blockIdx.z) {
        const uint32_t p = blockIdx.z / phases, img = (blockIdx.z - p * phases) * per + p;
        fa += p * pstride, fb += p * pstride, dst += img * ostride;
        const size_t q = (size_t)img * hq * wq;
        fl.p += q * fl.cs, vis.p += q * vis.cs, rt.p += q * rt.cs;
    }
    fill_unit_table(tab);
    const uint32_t x = blockIdx.x * 64 + (threadIdx.x & 63u), y = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (x >= w || y >= h) return;
    const float iy = ((float)y + 0.5f) * sh - 0.5f, ix = ((float)x + 0.5f) * sw - 0.5f;
    const int qy0 = (int)floorf(iy), qx0 = (int)floorf(ix);
    const float qfy = iy - (float)qy0, qfx = ix - (float)qx0;
    const uint32_t y0 = clampi(qy0, 0, (int)hq - 1), y1 = clampi(qy0 + 1, 0, (int)hq - 1);
    const uint32_t x0 = clampi(qx0, 0, (int)wq - 1), x1 = clampi(qx0 + 1, 0, (int)wq - 1);
    const uint32_t r0 = __umul24(y0, wq), r1 = __umul24(y1, wq);
    const uint32_t qs[4] = {r0 + x0, r0 + x1, r1 + x0, r1 + x1};
    float fq[4][4], vq[4][3], rq[4][3];
    const uint32_t nq = hq * wq;
    const auto rfl = buf_rsrc(fl.p, QV ? nq * 16u : 0u), rrt = buf_rsrc(rt.p, QV ? nq * rt.cs * 2u : 0u);
    float f[4], v[3], r[3];
    if constexpr (QV && FMA) {  // the taps stay f16 and feed bil4h
        _Float16 hq4[4][8], hr4[4][4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rfl, qs[k] * 16u, 0, 0));
            const uint2 b =
                __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rrt, (qs[k] * rt.cs + rt.c0) * 2u, 0, 0));
            const uint32_t wv[6] = {a.x, a.y, a.z, a.w, b.x, b.y};
#pragma unroll
            for (int c = 0; c < 8; c++) hq4[k][c] = __builtin_bit_cast(_Float16, (uint16_t)(wv[c >> 1] >> (16 * (c & 1))));
#pragma unroll
            for (int c = 0; c < 4; c++)
                hr4[k][c] = __builtin_bit_cast(_Float16, (uint16_t)(wv[4 + (c >> 1)] >> (16 * (c & 1))));
        }
#pragma unroll
        for (uint32_t c = 0; c < 4; c++)
            f[c] = bil4h(hq4[0][c], hq4[1][c], hq4[2][c], hq4[3][c], qfx, qfy) * ((c & 1u) == 0 ? fsx : fsy);
#pragma unroll
        for (uint32_t c = 0; c < 3; c++) {
            v[c] = bil4h(hq4[0][4 + c], hq4[1][4 + c], hq4[2][4 + c], hq4[3][4 + c], qfx, qfy) * vis.scale;
            r[c] = bil4h(hr4[0][c], hr4[1][c], hr4[2][c], hr4[3][c], qfx, qfy);
        }
        render_rgba_px<CUBIC, FL, FMA>(x, y, f, v, r, fa, fb, w, h, pitch, tab, flags, dst, opitch);
        return;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if constexpr (QV) {
            const uint4 a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rfl, qs[k] * 16u, 0, 0));
            const uint2 r =
                __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rrt, (qs[k] * rt.cs + rt.c0) * 2u, 0, 0));
            const uint32_t wv[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int c = 0; c < 4; c++) fq[k][c] = h2f((uint16_t)(wv[c >> 1] >> (16 * (c & 1))));
#pragma unroll
            for (int c = 0; c < 3; c++) vq[k][c] = h2f((uint16_t)(wv[2 + (c >> 1)] >> (16 * (c & 1))));
            rq[k][0] = h2f((uint16_t)r.x), rq[k][1] = h2f((uint16_t)(r.x >> 16)), rq[k][2] = h2f((uint16_t)r.y);
        } else {
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) fq[k][c] = ld(fl, qs[k], c);
#pragma unroll
            for (uint32_t c = 0; c < 3; c++) vq[k][c] = ld(vis, qs[k], c), rq[k][c] = ld(rt, qs[k], c);
        }
    }
#pragma unroll
    for (uint32_t c = 0; c < 4; c++)
        f[c] = bil4m<FMA>(fq[0][c], fq[1][c], fq[2][c], fq[3][c], qfx, qfy) * ((c & 1u) == 0 ? fsx : fsy);
#pragma unroll
    for (uint32_t c = 0; c < 3; c++) {
        v[c] = bil4m<FMA>(vq[0][c], vq[1][c], vq[2][c], vq[3][c], qfx, qfy) * vis.scale;
        r[c] = bil4m<FMA>(rq[0][c], rq[1][c], rq[2][c], rq[3][c], qfx, qfy);
    }
    render_rgba_px<CUBIC, FL, FMA>(x, y, f, v, r, fa, fb, w, h, pitch, tab, flags, dst, opitch);
}

// The antialiased resize of n padded RGBA8 frames (hp x wp, rgba_in's BGR f16) to oh x ow, into a view of 8-byte
// 4-channel pixels (channel 3 written 0): rgba_in.wgsl then interp.wgsl:11-45 with antialias, as
// interp_aa_lds_kernel computes it. A workgroup stages the union of its 16 x 16 outputs' windows, at most
// EXT x EXT padded pixels (EXT <= 16 * R, the lanes' R x R load stripes covering it), each converted once; the
// values are those of the f16 picture rgba_in writes, held in LDS as f16: each tap's product is one mixed-precision
// FMA that takes the f16 value as it is. SPLIT: a staged pixel's B, G in a 4-byte cell and its R in a 2-byte cell of
// a second array (6 bytes, two reads a tap) rather than one 8-byte cell (one read). The LDS a workgroup holds sets
// how many share a CU: the 6-byte cells let four 78 x 78 windows share one where three 80 x 80 8-byte windows do
// not fit. Measured warm: sixteen 2160p frames (10 taps, a 78-pixel window) 334 us in 8-byte cells, 310 us split;
// two 1080p frames (40 x 40 cells, occupancy bound by waves either way) 12.9 us in 8-byte cells against 14.8 us
// for an f32 pair plus an f32 (12 bytes, all-f32 arithmetic); with each tap widened one instruction at a time the
// 8-byte cells were the slower layout (13.1 against 12.8 us, and 379 us at 2160p).
template <int KM, int R, int EXT, bool SPLIT>
__global__ __launch_bounds__(kThreads) void rgba_resize_kernel(const uint32_t* src, uint32_t w, uint32_t h,
                                                               uint32_t pitch, uint64_t fstride, uint32_t ih,
                                                               uint32_t iw, OView out, uint32_t oh, uint32_t ow,
                                                               uint32_t tiles_x, uint32_t tiles_y, float sh, float sw) {
    static_assert(EXT <= kAaT * R, "the load stripes cover the window");
    using Cell = typename std::conditional<SPLIT, uint32_t, uint2>::type;
    __shared__ Cell tile[EXT * EXT];
    __shared__ uint16_t tileb[SPLIT ? EXT * EXT : 1];
    __shared__ uint16_t tab[256];  // entry b: the f16 bits rgba_in stores for byte b
    __shared__ float wxs[kAaT * KM], wys[kAaT * KM];
    __shared__ int lcs[kAaT * KM], lrs[kAaT * KM];
    const uint32_t tid = threadIdx.x, tx = tid % kAaT, ty = tid / kAaT;
    const uint32_t bt = blockIdx.x, txi = bt % tiles_x, rr = bt / tiles_x, tyi = rr % tiles_y, img = rr / tiles_y;
    const uint32_t ox0 = txi * kAaT, oy0 = tyi * kAaT;
    const uint32_t ox_last = min(ox0 + kAaT, ow) - 1, oy_last = min(oy0 + kAaT, oh) - 1;
    const float fsh = fmaxf(sh, 1.0f), fsw = fmaxf(sw, 1.0f);  // sh = ih / oh, sw = iw / ow from the host
    const int ylo = max(0, (int)floorf(((float)oy0 + 0.5f) * sh - fsh + 0.5f));
    const int yhi = min((int)ih, (int)floorf(((float)oy_last + 0.5f) * sh + fsh + 0.5f));
    const int xlo = max(0, (int)floorf(((float)ox0 + 0.5f) * sw - fsw + 0.5f));
    const int xhi = min((int)iw, (int)floorf(((float)ox_last + 0.5f) * sw + fsw + 0.5f));
    const int ny = max(1, min(yhi - ylo, (int)EXT)), nx = max(1, min(xhi - xlo, (int)EXT));
    // the tap weights and window indices of the block's 16 columns (entries 0 .. kAaT KM - 1) and 16 rows (the next
    // kAaT KM): interp_aa.wgsl's per-tap weight, which depends on the output column (row) alone, once per block
    tab[tid] = unit_f16(tid << 16, 0);
    for (uint32_t e = tid; e < 2 * kAaT * KM; e += kThreads) {
        const bool rows = e >= kAaT * KM;
        const uint32_t k = rows ? e - kAaT * KM : e;
        const uint32_t o = (rows ? oy0 : ox0) + k / KM;
        const float sc = rows ? sh : sw, fs = rows ? fsh : fsw;
        const int n = rows ? (int)ih : (int)iw, lo = rows ? ylo : xlo, nn = rows ? ny : nx;
        const float c = ((float)o + 0.5f) * sc;
        const int tmin = max(0, (int)floorf(c - fs + 0.5f)), tmax = min(n, (int)floorf(c + fs + 0.5f));
        const int tt = tmin + (int)(k % KM);
        const float wgt = tt < tmax ? fmaxf(0.0f, 1.0f - fabsf(((float)tt + 0.5f - c) / fs)) : 0.0f;
        const int li = min(max(tt - lo, 0), nn - 1);
        if (rows) wys[k] = wgt, lrs[k] = li;
        else wxs[k] = wgt, lcs[k] = li;
    }
    __syncthreads();
    // the frame through a buffer resource: a tap's byte offset is one 24-bit multiply-add
    const auto rf = buf_rsrc(src + img * fstride, ((h - 1) * pitch + w) * 4u);
    const uint32_t pitch4 = pitch * 4u;
#pragma unroll
    for (uint32_t i = 0; i < R; i++)
#pragma unroll
        for (uint32_t j = 0; j < R; j++) {
            const int row = min((int)(ty + kAaT * i), ny - 1), col = min((int)(tx + kAaT * j), nx - 1);
            const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(
                rf, __umul24((uint32_t)min(ylo + row, (int)h - 1), pitch4) + (uint32_t)min(xlo + col, (int)w - 1) * 4u,
                0, 0);
            const uint32_t c01 = (uint32_t)tab[(v >> 16) & 0xffu] | ((uint32_t)tab[(v >> 8) & 0xffu] << 16);
            if constexpr (SPLIT)
                tile[row * EXT + col] = c01, tileb[row * EXT + col] = tab[v & 0xffu];
            else
                tile[row * EXT + col] = uint2{c01, (uint32_t)tab[v & 0xffu]};
        }
    __syncthreads();
    const uint32_t ox = ox0 + tx, oy = oy0 + ty;
    if (ox >= ow || oy >= oh) return;
    float wx[KM];
    int lc[KM];
#pragma unroll
    for (int j = 0; j < KM; j++) wx[j] = wxs[tx * KM + j], lc[j] = lcs[tx * KM + j];
    float acc[3] = {0.0f, 0.0f, 0.0f}, norm = 0.0f;
#pragma unroll
    for (int jy = 0; jy < KM; jy++) {
        const float wy = wys[ty * KM + jy];
        const uint32_t lrow = lrs[ty * KM + jy] * EXT;
#pragma unroll
        for (int jx = 0; jx < KM; jx++) {
            // a tap outside the window has weight +0 and a value in [0, 1]: it adds +0, leaving acc and norm as the
            // reference's skipped tap leaves them (interp_aa_lds_kernel, whose views may hold any value, points such
            // taps at a zero cell instead)
            const float wgt = wx[jx] * wy;
            const Cell q = tile[lrow + lc[jx]];
            float vv[3];
            if constexpr (SPLIT) vv[0] = h2f((uint16_t)q), vv[1] = h2f((uint16_t)(q >> 16)), vv[2] = h2f(tileb[lrow + lc[jx]]);
            else vv[0] = h2f((uint16_t)q.x), vv[1] = h2f((uint16_t)(q.x >> 16)), vv[2] = h2f((uint16_t)q.y);
            // each product as an FMA with +0, which takes the f16 tap as it is (one mixed-precision FMA, no
            // widening) and rounds as the product does (taps and weights are >= 0, so no product is -0)
#pragma unroll
            for (int i = 0; i < 3; i++) acc[i] = acc[i] + __builtin_fmaf(vv[i], wgt, 0.0f);
            norm = norm + wgt;
        }
    }
    *reinterpret_cast<uint2*>(out.p + (((size_t)img * oh + oy) * ow + ox) * out.cs) =
        uint2{(uint32_t)f2h(acc[0] / norm) | ((uint32_t)f2h(acc[1] / norm) << 16), (uint32_t)f2h(acc[2] / norm)};
}

// ---- GMHS: the periodic-structure repair of the pair's E8 flow (gmhs.rs:149-206) ----------------------------------
// Eight launches where the reference records fourteen dispatches: four fit rounds (gm_fit_reduce.wgsl, each round
// solving the previous one's normal equations first, gm_fit_solve.wgsl), the cost maps (gm_cost.wgsl, solving the
// last round), the texture window (box_h + box_v fused, gm_box.wgsl), and the decision window at the cells the select
// reads (its box_h at their columns, then its box_v at their rows with the select, gm_select.wgsl). Every value is
// the reference kernels' arithmetic in their order: the fit keeps gm_fit_reduce's 32 workgroups of 256 lanes with
// their strided per-lane sums and pairwise lane tree (its last levels as in-wave shuffles, the same pairs), so the
// sums round as there; a box sums its clamped taps in order. The stage is latency-bound (a few MB of L2-resident
// maps, 6480 flow cells at 1080p): the kernels are shaped for waves in flight, with every tap load of a sum issued
// before its in-order additions.
constexpr uint32_t kGmNwg = gmfit::kNwg, kGmWg = gmfit::kWg;  // gm_fit_reduce's workgroups and their size
constexpr uint32_t kGmPart = gmfit::kPart;                     // one round's partial sums [workgroup][channel][9]
constexpr uint32_t kGmT = 16;                 // the box tile's edge and the cost block's width, in cells
constexpr uint32_t kGmRmax = 32;              // largest box radius: r_dwin = round(16 s), s <= 2

// The repair of several pairs at once: every kernel below takes the pair from one grid dimension (pair k: pictures
// 2k images past a and b, flow image k, workspace k at wsf floats past workspace 0); one pair is pair 0.

// one fit round (gm_fit_reduce.wgsl:15-44, the round before solved first) for workgroup blockIdx.x of channel
// blockIdx.y of pair blockIdx.z: the shared round body (gm_fit.h) at 256 threads
__global__ __launch_bounds__(kGmWg) void gm_fit_kernel(View flow, uint32_t h8, uint32_t w8, float delta, uint32_t round,
                                                       const float* part_in, float* part_out, size_t wsf) {
    __shared__ gmfit::RoundLds lds;
    const size_t z = blockIdx.z;
    gmfit::round_body<kGmWg>(flow.p + z * h8 * w8 * flow.cs, flow.cs, flow.c0, h8, w8, delta, round, part_in + z * wsf,
                             part_out + z * wsf, blockIdx.x, blockIdx.y, lds);
}

// the B, G, R of pixel pix of a picture view (VEC: one 8-byte load, 4-channel aligned views)
template <bool VEC>
__device__ __forceinline__ void bgr(const View& v, size_t pix, float (&o)[3]) {
    if constexpr (VEC) {
        const uint2 q = *reinterpret_cast<const uint2*>(v.p + pix * v.cs + v.c0);
        o[0] = h2f((uint16_t)q.x), o[1] = h2f((uint16_t)(q.x >> 16)), o[2] = h2f((uint16_t)q.y);
    } else {
        o[0] = ld(v, pix, 0), o[1] = ld(v, pix, 1), o[2] = ld(v, pix, 2);
    }
}
template <bool VEC>
__device__ __forceinline__ float gm_lum(const View& v, uint32_t w, int y, int x) {
    float p[3];
    bgr<VEC>(v, (size_t)y * w + x, p);
    return lum3(p[0], p[1], p[2]);
}
// gm_cost.wgsl:23-29: bilinear luma, coordinates clamped
template <bool VEC>
__device__ float gm_samp(const View& v, uint32_t h, uint32_t w, float gx, float gy) {
    const int x0 = (int)floorf(gx), y0 = (int)floorf(gy);
    const float ax = gx - (float)x0, ay = gy - (float)y0;
    const int x0c = clampi(x0, 0, (int)w - 1), x1c = clampi(x0 + 1, 0, (int)w - 1);
    const int y0c = clampi(y0, 0, (int)h - 1), y1c = clampi(y0 + 1, 0, (int)h - 1);
    const float top = gm_lum<VEC>(v, w, y0c, x0c) * (1.0f - ax) + gm_lum<VEC>(v, w, y0c, x1c) * ax;
    const float bot = gm_lum<VEC>(v, w, y1c, x0c) * (1.0f - ax) + gm_lum<VEC>(v, w, y1c, x1c) * ax;
    return top * (1.0f - ay) + bot * ay;
}

// gm_cost.wgsl:55-75, maps 0-4 (planar [5][hc][wc]) for a 16 x 8 block of cells, the block solving the last fit
// round first (block 0 also stores the coefficients, [4][4], for the select and the caller). Two lanes per cell,
// in different waves: threads 0-127 sample for cm and l (maps 0, 3, 4), threads 128-255 for ca and dv (maps 1, 2);
// ca outside the pictures is cm, handed over through LDS. VEC: the pictures and the flow are 4-channel aligned
// views (one 8-byte load per pixel). blockIdx.z: the pair.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void gm_cost_kernel(View a, View b, uint32_t h, uint32_t w, View flow,
                                                           uint32_t h8, uint32_t w8, const float* part, float* coef,
                                                           float* maps, uint32_t hc, uint32_t wc, size_t wsf) {
    __shared__ float ss[4][9], cf[4][3], cms[128];
    {
        const size_t z = blockIdx.z;
        a.p += z * 2 * h * w * a.cs, b.p += z * 2 * h * w * b.cs, flow.p += z * h8 * w8 * flow.cs;
        part += z * wsf, coef += z * wsf, maps += z * wsf;
    }
    const uint32_t t = threadIdx.x, cl = t % 128;
    const bool second = t >= 128;  // uniform over each wave
    const uint32_t x = blockIdx.x * 16 + cl % 16, y = blockIdx.y * 8 + cl / 16;
    const bool valid = x < wc && y < hc;
    const float rx = ((float)x + 0.5f) * 2.0f - 0.5f, ry = ((float)y + 0.5f) * 2.0f - 0.5f;
    // the E8 flow at (rx, ry), bilinear (gm_cost.wgsl:38-48), loaded before the block's solve
    const float ix = (rx + 0.5f) * (float)w8 / (float)w - 0.5f, iy = (ry + 0.5f) * (float)h8 / (float)h - 0.5f;
    const int qx0 = (int)floorf(ix), qy0 = (int)floorf(iy);
    const float fx = ix - (float)qx0, fy = iy - (float)qy0;
    const uint32_t x0 = clampi(qx0, 0, (int)w8 - 1), x1 = clampi(qx0 + 1, 0, (int)w8 - 1);
    const uint32_t y0 = clampi(qy0, 0, (int)h8 - 1), y1 = clampi(qy0 + 1, 0, (int)h8 - 1);
    float q[4][4] = {};
    if (valid) {
        const size_t taps[4] = {(size_t)y0 * w8 + x0, (size_t)y0 * w8 + x1, (size_t)y1 * w8 + x0, (size_t)y1 * w8 + x1};
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            if constexpr (VEC) {
                const uint2 v = *reinterpret_cast<const uint2*>(flow.p + taps[k] * flow.cs + flow.c0);
                q[k][0] = h2f((uint16_t)v.x), q[k][1] = h2f((uint16_t)(v.x >> 16));
                q[k][2] = h2f((uint16_t)v.y), q[k][3] = h2f((uint16_t)(v.y >> 16));
            } else {
#pragma unroll
                for (uint32_t c = 0; c < 4; c++) q[k][c] = ld(flow, taps[k], c);
            }
        }
    }
    gmfit::solve_block(part, 0xfu, ss, cf);
    if (blockIdx.x == 0 && blockIdx.y == 0 && t < 16) coef[t] = (t & 3u) == 3u ? 0.0f : cf[t >> 2][t & 3u];
    const size_t n = (size_t)hc * wc, i = (size_t)y * wc + x;
    const float xn = -1.0f + 2.0f * ix / (float)max(w8 - 1, 1u), yn = -1.0f + 2.0f * iy / (float)max(h8 - 1, 1u);
    float f[4], gh[4];
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {
        const float top = q[0][c] * (1.0f - fx) + q[1][c] * fx, bot = q[2][c] * (1.0f - fx) + q[3][c] * fx;
        f[c] = top * (1.0f - fy) + bot * fy;
        gh[c] = cf[c][0] + cf[c][1] * xn + cf[c][2] * yn;
    }
    float ca = 0.0f;
    bool inside = false;
    if (!second) {
        float cm = 0.0f;
        if (valid) {
            cm = fabsf(gm_samp<VEC>(a, h, w, rx + f[0], ry + f[1]) - gm_samp<VEC>(b, h, w, rx + f[2], ry + f[3]));
            const float l = gm_samp<VEC>(a, h, w, rx, ry);
            maps[i] = cm, maps[3 * n + i] = l, maps[4 * n + i] = l * l;
        }
        cms[cl] = cm;
    } else if (valid) {
        const float wm = (float)w - 1.0f, hm = (float)h - 1.0f;
        const float ax = rx + gh[0], ay = ry + gh[1], bx = rx + gh[2], by = ry + gh[3];
        inside = ax >= 0.0f && ax <= wm && ay >= 0.0f && ay <= hm && bx >= 0.0f && bx <= wm && by >= 0.0f && by <= hm;
        if (inside) ca = fabsf(gm_samp<VEC>(a, h, w, ax, ay) - gm_samp<VEC>(b, h, w, bx, by));
        const float dvx = (gh[2] - gh[0]) - (f[2] - f[0]), dvy = (gh[3] - gh[1]) - (f[3] - f[1]);
        maps[2 * n + i] = sqrtf(dvx * dvx + dvy * dvy);
    }
    __syncthreads();
    if (second && valid) maps[n + i] = inside ? ca : cms[cl];
}

// box_h then box_v of radius r (gm_box.wgsl:8-25) on map channel blockIdx.z % 5 of src ([5][hc][wc]) into the same
// channel of dst, for the block's 16 x 16 tile of cells, pair blockIdx.z / 5. The window of clamped rows and columns
// the tile's taps reach ((16 + 2r)^2 cells, NB x NB blocks of 16 x 16, dynamic LDS) is staged with every load issued
// before the first store; box_h runs on every window row (a window row is a clamped map row, so its sums are the
// map's own), box_v on the tile, each sum over its taps in order.
template <uint32_t NB>
__global__ __launch_bounds__(kThreads) void gm_box_kernel(const float* src, float* dst, uint32_t hc, uint32_t wc,
                                                          uint32_t r, size_t wsf) {
    extern __shared__ float glds[];
    const uint32_t t = threadIdx.x, x0 = blockIdx.x * kGmT, y0 = blockIdx.y * kGmT, ch = blockIdx.z % 5;
    src += (size_t)(blockIdx.z / 5) * wsf, dst += (size_t)(blockIdx.z / 5) * wsf;
    const uint32_t ty = t / kGmT, tx = t % kGmT;
    const uint32_t span = 2 * r + 1, rows = kGmT + 2 * r;
    float* win = glds;                // [rows][rows]
    float* hs = glds + rows * rows;   // [rows][16]
    const size_t n = (size_t)hc * wc;
    const float* plane = src + ch * n;
    const float den = (float)span;
    float v[NB][NB];
#pragma unroll
    for (uint32_t bj = 0; bj < NB; bj++)
#pragma unroll
        for (uint32_t bi = 0; bi < NB; bi++) {
            const uint32_t j = min(ty + kGmT * bj, rows - 1), i = min(tx + kGmT * bi, rows - 1);
            const int yy = clampi((int)y0 - (int)r + (int)j, 0, (int)hc - 1);
            const int xx = clampi((int)x0 - (int)r + (int)i, 0, (int)wc - 1);
            v[bj][bi] = plane[(size_t)yy * wc + xx];
        }
#pragma unroll
    for (uint32_t bj = 0; bj < NB; bj++)
#pragma unroll
        for (uint32_t bi = 0; bi < NB; bi++) {
            const uint32_t j = ty + kGmT * bj, i = tx + kGmT * bi;
            if (j < rows && i < rows) win[j * rows + i] = v[bj][bi];
        }
    __syncthreads();
#pragma unroll
    for (uint32_t bj = 0; bj < NB; bj++) {
        const uint32_t j = ty + kGmT * bj;
        if (j < rows) {
            const float* row = win + j * rows + tx;
            float acc = 0.0f;
#pragma unroll 8
            for (uint32_t d = 0; d < span; d++) acc = acc + row[d];
            hs[j * kGmT + tx] = acc / den;
        }
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll 8
    for (uint32_t d = 0; d < span; d++) acc = acc + hs[(ty + d) * kGmT + tx];
    if (x0 + tx < wc && y0 + ty < hc) dst[ch * n + (size_t)(y0 + ty) * wc + x0 + tx] = acc / den;
}

// the cost cell the select reads for E8 row i (column j): gm_select.wgsl:17-18
__host__ __device__ __forceinline__ int gm_sel_row(uint32_t i, uint32_t hc, uint32_t h8) {
    const int v = (int)floorf(((float)i + 0.5f) * (float)hc / (float)h8);
    return v < 0 ? 0 : v > (int)hc - 1 ? (int)hc - 1 : v;
}

// The decision window (box_h then box_v of radius r on maps 0-2, gm_box.wgsl:8-25) is needed only at the cost
// cells the select reads: box_h at their columns (every row), then box_v at their rows, the same sums in the same
// order as the full windows there. NT >= 2r + 1: a sum's taps are loaded together (clamped addresses; the loads
// past the window repeat its last tap and are not added), then added in order.
// box_h of maps 0-2 of tex ([5][hc][wc], after the texture window) at the select's columns: hs [3][hc][w8];
// blockIdx.y: the pair
template <uint32_t NT>
__global__ __launch_bounds__(kThreads) void gm_dwin_h_kernel(const float* tex, float* hs, uint32_t hc, uint32_t wc,
                                                             uint32_t w8, uint32_t r, uint32_t items, size_t wsf) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    tex += blockIdx.y * wsf, hs += blockIdx.y * wsf;
    const uint32_t j = t % w8, rr = t / w8, row = rr % hc, m = rr / hc, span = 2 * r + 1;
    const int x = gm_sel_row(j, wc, w8);
    const float* src = tex + m * (size_t)hc * wc + (size_t)row * wc;
    float v[NT];
#pragma unroll
    for (uint32_t d = 0; d < NT; d++) v[d] = src[clampi(x - (int)r + (int)min(d, span - 1), 0, (int)wc - 1)];
    float acc = 0.0f;
#pragma unroll
    for (uint32_t d = 0; d < NT; d++)
        if (d < span) acc = acc + v[d];
    hs[t] = acc / (float)span;
}

// v of lane K of each aligned group of four lanes, in all four (a DPP quad permutation)
template <int K>
__device__ __forceinline__ float quad_lane(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), K * 0x55, 0xf, 0xf, false));
}

// box_v of hs at the select's rows, then the select (gm_select.wgsl:14-27); dec [5][h8][w8] receives the five values
// an E8 cell decides on (maps 0-2 after both windows, maps 3-4 after the texture window). Four consecutive lanes per
// cell: lane m < 3 sums map m's window (its NT loads in one batch), lane 3 loads maps 3-4, and every lane of the
// four gathers the five values (quad broadcasts), decides as the select does and stores flow channel m. The lanes
// past the last cell shadow it (in-bounds loads, so that every lane of a wave takes part in the shuffles) and store
// nothing. items: cells. blockIdx.y: the pair.
template <uint32_t NT>
__global__ __launch_bounds__(kThreads) void gm_dwin_v_select_kernel(const float* hs, const float* tex,
                                                                    const float* coef, OView flow, float* dec,
                                                                    uint32_t h8, uint32_t w8, uint32_t hc, uint32_t wc,
                                                                    uint32_t r, float eps, float dmin, float texf,
                                                                    uint32_t items, size_t wsf) {
    {
        const size_t z = blockIdx.y;
        hs += z * wsf, tex += z * wsf, coef += z * wsf, dec += z * wsf, flow.p += z * h8 * w8 * flow.cs;
    }
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x, cell = t / 4, m = t % 4;
    const bool live = cell < items;
    const uint32_t cl = live ? cell : items - 1;
    const uint32_t i = cl / w8, j = cl % w8, span = 2 * r + 1;
    const int y = gm_sel_row(i, hc, h8), x = gm_sel_row(j, wc, w8);
    const size_t n = (size_t)hc * wc, idx = (size_t)y * wc + x;
    float own, own2 = 0.0f;
    if (m < 3) {
        const float* col = hs + (size_t)m * hc * w8 + j;
        float v[NT];
#pragma unroll
        for (uint32_t d = 0; d < NT; d++)
            v[d] = col[(size_t)clampi(y - (int)r + (int)min(d, span - 1), 0, (int)hc - 1) * w8];
        float acc = 0.0f;
#pragma unroll
        for (uint32_t d = 0; d < NT; d++)
            if (d < span) acc = acc + v[d];
        own = acc / (float)span;
    } else {
        own = tex[3 * n + idx], own2 = tex[4 * n + idx];
    }
    // lane m of the cell's quad of lanes broadcast to the quad (DPP quad_perm(m, m, m, m))
    const float cm = quad_lane<0>(own), ca = quad_lane<1>(own), dv = quad_lane<2>(own);
    const float lm = quad_lane<3>(own), l2 = quad_lane<3>(own2);
    if (!live) return;
    const size_t n8 = (size_t)h8 * w8;
    dec[m * n8 + cell] = own;
    if (m == 3) dec[4 * n8 + cell] = own2;
    const float sd = sqrtf(fmaxf(l2 - lm * lm, 0.0f));
    if (ca + eps < cm && dv > dmin && sd > texf) {
        const float xn = -1.0f + 2.0f * (float)j / (float)max(w8 - 1, 1u);
        const float yn = -1.0f + 2.0f * (float)i / (float)max(h8 - 1, 1u);
        st(flow, cell, m, coef[m * 4] + coef[m * 4 + 1] * xn + coef[m * 4 + 2] * yn);
    }
}

// ---- host side ----------------------------------------------------------------------------------------------------

constexpr uint64_t kMaxItems = 1ull << 31;

// validates a view that `channels` channels are read from / written to; scaled: the op applies the view's scale
int check(const fhc_tensor* t, const char* name, uint32_t channels, bool scaled, bool output = false) {
    if (!t) return fail(-1, "%s: null view", name);
    if (!t->p) return fail(-1, "%s: null pointer", name);
    if ((uint64_t)t->c0 + channels > t->cstride)
        return fail(-1, "%s: view (cstride %u, c0 %u) does not hold %u channels", name, t->cstride, t->c0, channels);
    if (!output && !scaled && t->scale != 1.0f)
        return fail(-1, "%s: this op reads the view unscaled (scale %g given; materialise it first)", name,
                    (double)t->scale);
    if (!output && !std::isfinite(t->scale)) return fail(-1, "%s: scale is not finite", name);
    return 0;
}

// whether the 8-byte path serves these views for channel groups of 4 over c channels
bool vec4(uint32_t c, std::initializer_list<const fhc_tensor*> views) {
    if (c % 4) return false;
    for (const fhc_tensor* v : views)
        if (v->cstride % 4 || v->c0 % 4 || reinterpret_cast<uintptr_t>(v->p) % 8) return false;
    return true;
}

View in(const fhc_tensor* t) { return View{static_cast<const uint16_t*>(t->p), t->cstride, t->c0, t->scale}; }
OView outv(const fhc_tensor* t) { return OView{static_cast<uint16_t*>(t->p), t->cstride, t->c0}; }

template <class F>
int launch(const char* op, uint64_t items, F&& f) {
    if (items >= kMaxItems) return fail(-1, "%s: %llu work items exceed the 2^31 limit", op, (unsigned long long)items);
    const dim3 grid((uint32_t)((items + kThreads - 1) / kThreads));
    f(grid, (uint32_t)items);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-2, "%s: launch failed: %s", op, hipGetErrorString(e));
    return 0;
}

#define FHC_TRY(x)              \
    do {                        \
        const int rc_ = (x);    \
        if (rc_ < 0) return rc_; \
    } while (0)

// gmhs.rs:149-160: the cost grid (DS = 2), the two box radii, the jump and Huber thresholds; eps 0, tex 0.015
// (gmhs.rs:195). The workspace: the coefficients [4][4] at byte 0, two rounds of fit partials, then the decision
// maps [5][hc][wc] and their box-filtered copy, 256-byte aligned.
int gm_params(uint32_t h, uint32_t w, uint32_t full_w, uint32_t level, fhc_gmhs_par* p) {
    if (!p) return fail(-1, "gmhs: null parameter block");
    if (h == 0 || w == 0) return fail(-1, "gmhs: empty network (%u x %u)", w, h);
    if (level < 1 || level > 2) return fail(-1, "gmhs: repair level %u (1 safe, 2 aggressive)", level);
    if (full_w < w) return fail(-1, "gmhs: the network (%u wide) is wider than the padded frame (%u)", w, full_w);
    p->hc = (h + 1) / 2, p->wc = (w + 1) / 2;
    const float s = (float)w / ((float)full_w / 2.0f);
    const float rb = std::round(20.0f * s / 2.0f), rw = std::round(32.0f * s / 2.0f);
    p->s = s;
    p->r_blk = rb < 1.0f ? 1u : (uint32_t)rb;
    p->r_dwin = rw < 1.0f ? 1u : (uint32_t)rw;
    p->dmin = level >= 2 ? 0.0f : 8.0f * s;
    p->delta = 1.5f * s;
    p->eps = 0.0f, p->tex = 0.015f;
    const uint64_t head = (16 + 2 * (uint64_t)kGmPart) * sizeof(float), cells = (uint64_t)p->hc * p->wc;
    p->maps_offset = (head + 255) / 256 * 256;
    p->dec_offset = p->maps_offset + 5 * cells * sizeof(float);
    p->ws_bytes = p->dec_offset + 5 * cells * sizeof(float);
    return 0;
}

}  // namespace

}  // namespace fhc

using namespace fhc;

extern "C" int fhc_warp(const fhc_tensor* img, const fhc_tensor* flow, const fhc_tensor* out, uint32_t n, uint32_t h,
                        uint32_t w, uint32_t c, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w * c == 0) return 0;
        FHC_TRY(check(img, "warp img", c, true));
        FHC_TRY(check(flow, "warp flow", 2, true));
        FHC_TRY(check(out, "warp out", c, false, true));
        const uint32_t groups = (c + 3) / 4;
        const bool v = vec4(c, {img, out});
        return launch("warp", (uint64_t)n * h * w * groups, [&](dim3 g, uint32_t items) {
            auto k = v ? warp_kernel<true> : warp_kernel<false>;
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(img), in(flow), outv(out), h, w, c,
                               groups, items);
        });
    });
}

extern "C" int fhc_luma(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, int grad,
                        void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w == 0) return 0;
        FHC_TRY(check(x, "luma x", 3, true));
        FHC_TRY(check(out, "luma out", 1, false, true));
        return launch("luma", (uint64_t)n * h * w, [&](dim3 g, uint32_t items) {
            auto k = grad ? luma_kernel<true> : luma_kernel<false>;
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), h, w, items);
        });
    });
}

extern "C" int fhc_sad_volume(const fhc_tensor* la, const fhc_tensor* lb, const fhc_tensor* out, uint32_t n,
                              uint32_t h, uint32_t w, uint32_t radius, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if (radius > 7) return fail(-1, "sad_volume: radius %u above 7", radius);
        const uint32_t span2 = (2 * radius + 1) * (2 * radius + 1);
        if ((uint64_t)n * h * w == 0) return 0;
        FHC_TRY(check(la, "sad_volume la", 1, false));
        FHC_TRY(check(lb, "sad_volume lb", 1, false));
        FHC_TRY(check(out, "sad_volume out", span2, false, true));
        return launch("sad_volume", (uint64_t)n * h * w * span2, [&](dim3 g, uint32_t items) {
            hipLaunchKernelGGL(sad_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(la), in(lb), outv(out), h, w,
                               radius, span2, items);
        });
    });
}

extern "C" int fhc_convex_upsample(const fhc_tensor* wt, const fhc_tensor* x, const fhc_tensor* out, uint32_t n,
                                   uint32_t h, uint32_t w, uint32_t c, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w * c == 0) return 0;
        FHC_TRY(check(wt, "convex_upsample wt", 36, false));
        FHC_TRY(check(x, "convex_upsample x", c, false));
        FHC_TRY(check(out, "convex_upsample out", c, false, true));
        if (c > 256) return fail(-1, "convex_upsample: %u channels above 256", c);
        const uint32_t tx = (w + kCvIn - 1) / kCvIn, ty = (h + kCvIn - 1) / kCvIn;
        if ((uint64_t)n * tx * ty >= kMaxItems) return fail(-1, "convex_upsample: too many tiles");
        const size_t lds = (kCvIn * kCvIn * 36 + kCvHalo * kCvHalo * c) * 2;
        const View none{nullptr, 0, 0, 1.0f};
        hipLaunchKernelGGL(convex_tile_kernel<false>, dim3(n * tx * ty), dim3(kCvThreads), lds, (hipStream_t)stream,
                           in(wt), in(x), outv(out), h, w, c, tx, ty, none, none, PhaseT{}, n);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "convex_upsample: launch failed: %s", hipGetErrorString(e));
    });
}

extern "C" int fhc_film_modulate(const fhc_tensor* hv, const void* gvec, const fhc_tensor* out, uint32_t n,
                                 uint32_t h, uint32_t w, uint32_t c, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w * c == 0) return 0;
        if (!gvec) return fail(-1, "film_modulate: null g");
        FHC_TRY(check(hv, "film_modulate h", c, false));
        FHC_TRY(check(out, "film_modulate out", c, false, true));
        const uint32_t groups = (c + 3) / 4;
        const bool v = vec4(c, {hv, out});
        return launch("film_modulate", (uint64_t)n * h * w * groups, [&](dim3 g, uint32_t items) {
            auto k = v ? film_kernel<true> : film_kernel<false>;
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(hv),
                               static_cast<const uint16_t*>(gvec), outv(out), h * w, c, groups, items);
        });
    });
}

extern "C" int fhc_blend_weights(const fhc_tensor* vis, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w,
                                 void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w == 0) return 0;
        FHC_TRY(check(vis, "blend_weights vis", 3, true));
        FHC_TRY(check(out, "blend_weights out", 2, false, true));
        return launch("blend_weights", (uint64_t)n * h * w, [&](dim3 g, uint32_t items) {
            hipLaunchKernelGGL(blend_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(vis), outv(out), items);
        });
    });
}

extern "C" int fhc_blendmix(const fhc_tensor* wa, const fhc_tensor* wb, const fhc_tensor* vis, const fhc_tensor* out,
                            uint32_t n, uint32_t h, uint32_t w, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w == 0) return 0;
        FHC_TRY(check(wa, "blendmix wa", 3, false));
        FHC_TRY(check(wb, "blendmix wb", 3, false));
        FHC_TRY(check(vis, "blendmix vis", 3, true));
        FHC_TRY(check(out, "blendmix out", 3, false, true));
        return launch("blendmix", (uint64_t)n * h * w, [&](dim3 g, uint32_t items) {
            hipLaunchKernelGGL(blendmix_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(wa), in(wb), in(vis),
                               outv(out), items);
        });
    });
}

extern "C" int fhc_avgpool(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w,
                           uint32_t c, uint32_t k, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if (k == 0) return fail(-1, "avgpool: k is 0");
        const uint32_t oh = h / k, ow = w / k;
        if ((uint64_t)n * oh * ow * c == 0) return 0;
        FHC_TRY(check(x, "avgpool x", c, false));
        FHC_TRY(check(out, "avgpool out", c, false, true));
        const uint32_t groups = (c + 3) / 4;
        const bool v = vec4(c, {x, out});
        return launch("avgpool", (uint64_t)n * oh * ow * groups, [&](dim3 g, uint32_t items) {
            auto kern = k == 2 ? (v ? avgpool_kernel<true, 2> : avgpool_kernel<false, 2>)
                               : (v ? avgpool_kernel<true, 0> : avgpool_kernel<false, 0>);
            hipLaunchKernelGGL(kern, g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), h, w, oh, ow, c, k,
                               groups, items);
        });
    });
}

extern "C" int fhc_interpolate(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t c, uint32_t ih,
                               uint32_t iw, uint32_t oh, uint32_t ow, int antialias, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * oh * ow * c == 0) return 0;
        if (ih == 0 || iw == 0) return fail(-1, "interpolate: empty input (%u x %u) for a %u x %u output", ih, iw, oh, ow);
        FHC_TRY(check(x, "interpolate x", c, true));
        FHC_TRY(check(out, "interpolate out", c, false, true));
        const uint32_t groups = (c + 3) / 4;
        if (antialias) {
            const uint32_t taps = std::max(aa_taps(ih, oh), aa_taps(iw, ow));
            if (c <= 4 && taps <= 8 && aa_tile_extent(ih, oh) <= kAaExt && aa_tile_extent(iw, ow) <= kAaExt &&
                aa_window_offsets_fit(iw, x->cstride)) {
                const uint32_t tx = (ow + kAaT - 1) / kAaT, ty = (oh + kAaT - 1) / kAaT;
                if ((uint64_t)n * tx * ty >= kMaxItems) return fail(-1, "interpolate: too many tiles");
                const bool v4 = vec4(4, {x});
                auto kl = taps <= 4 ? (v4 ? interp_aa_lds_kernel<4, false, true> : interp_aa_lds_kernel<4, false, false>)
                                    : (v4 ? interp_aa_lds_kernel<8, false, true> : interp_aa_lds_kernel<8, false, false>);
                hipLaunchKernelGGL(kl, dim3(n * tx * ty), dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out),
                                   ih, iw, oh, ow, c, tx, ty, PyrOut{});
                const hipError_t e = hipGetLastError();
                return e == hipSuccess ? 0 : fail(-2, "interpolate: launch failed: %s", hipGetErrorString(e));
            }
            decltype(&interp_aa_kernel<3>) k = nullptr;
            if (taps <= 3) k = interp_aa_kernel<3>;
            else if (taps <= 4) k = interp_aa_kernel<4>;
            else if (taps <= 6) k = interp_aa_kernel<6>;
            else if (taps <= 8) k = interp_aa_kernel<8>;
            else if (taps <= 12) k = interp_aa_kernel<12>;
            else if (taps <= 16) k = interp_aa_kernel<16>;
            if (k)
                return launch("interpolate", (uint64_t)n * oh * ow * groups, [&](dim3 g, uint32_t items) {
                    hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), ih, iw, oh, ow,
                                       c, groups, items);
                });
        }
        const bool v = vec4(c, {x, out});
        return launch("interpolate", (uint64_t)n * oh * ow * groups, [&](dim3 g, uint32_t items) {
            auto k = antialias ? (v ? interp_kernel<true, true> : interp_kernel<false, true>)
                               : (v ? interp_kernel<true, false> : interp_kernel<false, false>);
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), ih, iw, oh, ow, c,
                               groups, items);
        });
    });
}

extern "C" int fhc_binary(const fhc_tensor* a, const fhc_tensor* b, const fhc_tensor* out, uint32_t n, uint32_t h,
                          uint32_t w, uint32_t c, uint32_t cb, int op, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if (op != 0 && op != 1) return fail(-1, "binary: op %d is neither 0 (add) nor 1 (mul)", op);
        if (cb != 1 && cb != c) return fail(-1, "binary: b has %u channels, neither 1 nor %u", cb, c);
        if ((uint64_t)n * h * w * c == 0) return 0;
        FHC_TRY(check(a, "binary a", c, true));
        FHC_TRY(check(b, "binary b", cb, true));
        FHC_TRY(check(out, "binary out", c, false, true));
        const uint32_t groups = (c + 3) / 4;
        const bool v = vec4(c, {a, out}) && (cb == 1 || vec4(c, {b}));
        return launch("binary", (uint64_t)n * h * w * groups, [&](dim3 g, uint32_t items) {
            auto k = v ? binary_kernel<true> : binary_kernel<false>;
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(a), in(b), outv(out), c, cb, op,
                               groups, items);
        });
    });
}

extern "C" int fhc_unary(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                         int op, float a, float b, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if (op < 0 || op > 3) return fail(-1, "unary: op %d outside 0..3", op);
        if ((uint64_t)n * h * w * c == 0) return 0;
        FHC_TRY(check(x, "unary x", c, true));
        FHC_TRY(check(out, "unary out", c, false, true));
        const uint32_t groups = (c + 3) / 4;
        const bool v = vec4(c, {x, out});
        return launch("unary", (uint64_t)n * h * w * groups, [&](dim3 g, uint32_t items) {
            using K = decltype(&unary_kernel<true, 0>);
            static const K table[2][4] = {
                {unary_kernel<false, 0>, unary_kernel<false, 1>, unary_kernel<false, 2>, unary_kernel<false, 3>},
                {unary_kernel<true, 0>, unary_kernel<true, 1>, unary_kernel<true, 2>, unary_kernel<true, 3>}};
            hipLaunchKernelGGL(table[v][op], g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), c, a, b,
                               groups, items);
        });
    });
}

extern "C" int fhc_chcopy(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                          void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w * c == 0) return 0;
        FHC_TRY(check(x, "chcopy x", c, true));
        FHC_TRY(check(out, "chcopy out", c, false, true));
        return launch("chcopy", (uint64_t)n * h * w * c, [&](dim3 g, uint32_t items) {
            hipLaunchKernelGGL(chcopy_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), c, items);
        });
    });
}

extern "C" int fhc_pair_pyramid(const fhc_tensor* q, const fhc_tensor* i8, const fhc_tensor* i16,
                                const fhc_tensor* l16, uint32_t h, uint32_t w, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if (h < 4 || w < 4) return h == 0 || w == 0 ? 0 : fail(-1, "pair_pyramid: %u x %u is below 4 x 4", h, w);
        FHC_TRY(check(q, "pair_pyramid q", 3, false));
        FHC_TRY(check(i8, "pair_pyramid i8", 3, false, true));
        FHC_TRY(check(i16, "pair_pyramid i16", 6, false, true));
        FHC_TRY(check(l16, "pair_pyramid l16", 2, false, true));
        const uint64_t items = 2ull * ((h / 2 + 1) / 2) * ((w / 2 + 1) / 2);
        return launch("pair_pyramid", items, [&](dim3 g, uint32_t n) {
            hipLaunchKernelGGL(pair_pyramid_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(q), outv(i8),
                               outv(i16), outv(l16), h, w, n);
        });
    });
}

extern "C" int fhc_fine_input(const fhc_tensor* f8, const fhc_tensor* i8, const fhc_tensor* flow,
                              const fhc_tensor* fx, const fhc_tensor* l8, uint32_t h, uint32_t w, uint32_t c,
                              void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)h * w * c == 0) return 0;
        FHC_TRY(check(f8, "fine_input f8", c, true));
        FHC_TRY(check(i8, "fine_input i8", 3, true));
        FHC_TRY(check(flow, "fine_input flow", 4, true));
        FHC_TRY(check(fx, "fine_input fx", 2 * c + 10, false, true));
        FHC_TRY(check(l8, "fine_input l8", 2, false, true));
        const uint32_t groups = (c + 3) / 4;
        fhc_tensor fxb = *fx;  // the second map's slice must be 8-byte aligned too for the vector path
        fxb.c0 += c;
        const bool v = vec4(c, {f8, fx, &fxb});
        const View none{nullptr, 0, 0, 1.0f};
        const OView onone{nullptr, 0, 0};
        return launch("fine_input", (uint64_t)h * w * (2 * groups + 3), [&](dim3 g, uint32_t n) {
            auto k = v ? fine_input_kernel<true, false> : fine_input_kernel<false, false>;
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(f8), in(i8), in(flow), outv(fx),
                               outv(l8), h, w, c, groups, n, none, onone, onone, 0u, 0u, 0.0f, 0.0f, 0.0f);
        });
    });
}

extern "C" int fhc_flow_vis_t(const fhc_tensor* fv, const fhc_tensor* dfilm, const fhc_tensor* out, uint32_t n,
                              uint32_t h, uint32_t w, float t, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w == 0) return 0;
        FHC_TRY(check(fv, "flow_vis_t fv", 7, true));
        FHC_TRY(check(dfilm, "flow_vis_t dfilm", 5, true));
        FHC_TRY(check(out, "flow_vis_t out", 7, false, true));
        const float af = 2.0f * t, ab = 2.0f * (1.0f - t);  // the mul_t factors (net/build.rs:293)
        return launch("flow_vis_t", (uint64_t)n * h * w, [&](dim3 g, uint32_t items) {
            hipLaunchKernelGGL(flow_vis_t_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(fv), in(dfilm),
                               outv(out), af, ab, items);
        });
    });
}

extern "C" int fhc_refine_input(const fhc_tensor* q, const fhc_tensor* flow, const fhc_tensor* vis,
                                const fhc_tensor* rx, uint32_t h, uint32_t w, float flow_out_scale, void* stream) {
    return fhc_refine_input_n(q, flow, vis, rx, h, w, flow_out_scale, 1, 1, stream);
}

extern "C" int fhc_refine_input_n(const fhc_tensor* q, const fhc_tensor* flow, const fhc_tensor* vis,
                                  const fhc_tensor* rx, uint32_t h, uint32_t w, float flow_out_scale, uint32_t n,
                                  uint32_t qmod, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)h * w * n == 0) return 0;
        if (qmod == 0 || qmod > n) return fail(-1, "refine_input: %u picture pairs for %u images", qmod, n);
        if (n > 65535) return fail(-1, "refine_input: %u images exceed the launch limit", n);
        FHC_TRY(check(q, "refine_input q", 3, true));
        FHC_TRY(check(flow, "refine_input flow", 4, true));
        FHC_TRY(check(vis, "refine_input vis", 3, true));
        FHC_TRY(check(rx, "refine_input rx", 14, false, true));
        const uint32_t tx = (w + kRiT - 1) / kRiT, ty = (h + kRiT - 1) / kRiT;
        if ((uint64_t)tx * ty >= kMaxItems / 64) return fail(-1, "refine_input: %u x %u is too large", w, h);
        hipLaunchKernelGGL(refine_input_kernel, dim3(tx * ty, n), dim3(64), 0, (hipStream_t)stream, in(q), in(flow),
                           in(vis), outv(rx), h, w, flow_out_scale, tx, qmod);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "refine_input: launch failed: %s", hipGetErrorString(e));
    });
}

extern "C" int fhc_pair_input(const fhc_tensor* ab, const fhc_tensor* q, const fhc_tensor* i8, const fhc_tensor* i16,
                              const fhc_tensor* l16, uint32_t ih, uint32_t iw, uint32_t oh, uint32_t ow,
                              void* stream) {
    return fhc_pair_input_n(ab, q, i8, i16, l16, ih, iw, oh, ow, 1, stream);
}

extern "C" int fhc_pair_input_n(const fhc_tensor* ab, const fhc_tensor* q, const fhc_tensor* i8,
                                const fhc_tensor* i16, const fhc_tensor* l16, uint32_t ih, uint32_t iw, uint32_t oh,
                                uint32_t ow, uint32_t pairs, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)ih * iw * oh * ow * pairs == 0) return 0;
        FHC_TRY(check(ab, "pair_input ab", 3, true));
        FHC_TRY(check(q, "pair_input q", 3, false, true));
        FHC_TRY(check(i8, "pair_input i8", 3, false, true));
        FHC_TRY(check(i16, "pair_input i16", 6, false, true));
        FHC_TRY(check(l16, "pair_input l16", 2, false, true));
        const uint32_t taps = std::max(aa_taps(ih, oh), aa_taps(iw, ow));
        if (!(taps <= 8 && aa_tile_extent(ih, oh) <= kAaExt && aa_tile_extent(iw, ow) <= kAaExt &&
              aa_window_offsets_fit(iw, ab->cstride))) {
            // no one-launch form for this scale: the resize of every picture, then each pair's pyramid
            FHC_TRY(fhc_interpolate(ab, q, 2 * pairs, 3, ih, iw, oh, ow, 1, stream));
            for (uint32_t k = 0; k < pairs; k++) {
                const auto at = [k](const fhc_tensor* t, uint64_t image) {
                    fhc_tensor v = *t;
                    v.p = static_cast<uint16_t*>(v.p) + k * image * v.cstride;
                    return v;
                };
                const fhc_tensor qk = at(q, 2ull * oh * ow), i8k = at(i8, 2ull * (oh / 2) * (ow / 2)),
                                 i16k = at(i16, (uint64_t)(oh / 4) * (ow / 4)), l16k = at(l16, (uint64_t)(oh / 4) * (ow / 4));
                FHC_TRY(fhc_pair_pyramid(&qk, &i8k, &i16k, &l16k, oh, ow, stream));
            }
            return 0;
        }
        if (oh < 4 || ow < 4) return fail(-1, "pair_input: %u x %u is below 4 x 4", oh, ow);
        const uint32_t tx = (ow + kAaT - 1) / kAaT, ty = (oh + kAaT - 1) / kAaT;
        const bool v4 = vec4(4, {ab});
        auto kl = taps <= 4 ? (v4 ? interp_aa_lds_kernel<4, true, true> : interp_aa_lds_kernel<4, true, false>)
                            : (v4 ? interp_aa_lds_kernel<8, true, true> : interp_aa_lds_kernel<8, true, false>);
        if ((uint64_t)2 * pairs * tx * ty >= kMaxItems / kThreads) return fail(-1, "pair_input: too many tiles");
        hipLaunchKernelGGL(kl, dim3(2 * pairs * tx * ty), dim3(kThreads), 0, (hipStream_t)stream, in(ab), outv(q), ih,
                           iw, oh, ow, 3u, tx, ty, PyrOut{outv(i8), outv(i16), outv(l16)});
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "pair_input: launch failed: %s", hipGetErrorString(e));
    });
}

extern "C" int fhc_render(const fhc_tensor* a, const fhc_tensor* b, const fhc_tensor* flow, const fhc_tensor* vis,
                          const fhc_tensor* rt, const fhc_tensor* out, uint32_t h, uint32_t w, uint32_t hq, uint32_t wq,
                          float fsx, float fsy, int cubic, uint32_t flags, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)h * w == 0) return 0;
        if (hq == 0 || wq == 0) return fail(-1, "render: empty quarter maps (%u x %u)", hq, wq);
        if (flags > 3) return fail(-1, "render: flags %u (bit 0 decisive, bit 1 still)", flags);
        FHC_TRY(check(a, "render a", 3, false));
        FHC_TRY(check(b, "render b", 3, false));
        FHC_TRY(check(flow, "render flow", 4, false));
        FHC_TRY(check(vis, "render vis", 3, true));
        FHC_TRY(check(rt, "render rt", 3, false));
        FHC_TRY(check(out, "render out", 3, false, true));
        // the bicubic 8-byte path addresses its taps with 32-bit element offsets
        const auto fits32 = [&](const fhc_tensor* t) {
            return (uint64_t)w * t->cstride < (1u << 24) && (uint64_t)h * w * t->cstride + t->c0 < (1u << 31);
        };
        const bool v = vec4(4, {a, b}) && (!cubic || (fits32(a) && fits32(b)));
        return launch("render", (uint64_t)h * w, [&](dim3 g, uint32_t items) {
            auto k = cubic ? (v ? render_kernel<true, true> : render_kernel<false, true>)
                           : (v ? render_kernel<true, false> : render_kernel<false, false>);
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(a), in(b), in(flow), in(vis), in(rt),
                               outv(out), h, w, hq, wq, fsx, fsy, flags, items);
        });
    });
}

extern "C" int fhc_fold_pair(const fhc_tensor* x, const fhc_tensor* out, const fhc_tensor* also, uint32_t h,
                             uint32_t w, uint32_t c, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)h * w * c == 0) return 0;
        FHC_TRY(check(x, "fold_pair x", c, false));
        FHC_TRY(check(out, "fold_pair out", 2 * c, false, true));
        if (also) FHC_TRY(check(also, "fold_pair also", c, false, true));
        fhc_tensor out1 = *out;  // image 1's slice must be aligned too for the vector path
        out1.c0 += c;
        const bool v = also ? vec4(c, {x, out, &out1, also}) : vec4(c, {x, out, &out1});
        const uint32_t groups = (c + 3) / 4;
        const OView a2 = also ? outv(also) : OView{nullptr, 0, 0};
        return launch("fold_pair", (uint64_t)h * w * 2 * groups, [&](dim3 g, uint32_t items) {
            auto k = v ? fold_pair_kernel<true> : fold_pair_kernel<false>;
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), a2, h * w, c, groups,
                               items);
        });
    });
}

extern "C" int fhc_coarse_up(const fhc_tensor* o, const fhc_tensor* out, const fhc_tensor* state, uint32_t hi,
                             uint32_t wi, uint32_t oh, uint32_t ow, float flow_scale, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)oh * ow == 0) return 0;
        if (hi == 0 || wi == 0) return fail(-1, "coarse_up: empty input (%u x %u)", hi, wi);
        if (state && (hi > oh || wi > ow)) return fail(-1, "coarse_up: the state is larger than the output");
        FHC_TRY(check(o, "coarse_up o", 7, false));
        FHC_TRY(check(out, "coarse_up out", 7, false, true));
        if (state) FHC_TRY(check(state, "coarse_up state", 4, false, true));
        const OView sv = state ? outv(state) : OView{nullptr, 0, 0};
        return launch("coarse_up", (uint64_t)oh * ow, [&](dim3 g, uint32_t items) {
            hipLaunchKernelGGL(coarse_up_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(o), outv(out), sv, hi,
                               wi, oh, ow, flow_scale, items);
        });
    });
}

// ---- the host's 8-bit frames -----------------------------------------------------------------------------------

namespace {
int check_frames(const char* op, const void* p, uint32_t n, uint32_t w, uint32_t h, uint32_t pitch, uint64_t fstride,
                 uint32_t hp, uint32_t wp) {
    if (!p) return fail(-1, "%s: null frame pointer", op);
    if (reinterpret_cast<uintptr_t>(p) % 4) return fail(-1, "%s: frames must be 4-byte aligned", op);
    if (pitch < w) return fail(-1, "%s: row pitch %u is below the width %u", op, pitch, w);
    if (n > 1 && fstride < (uint64_t)pitch * h) return fail(-1, "%s: frame stride below pitch * h", op);
    if (hp < h || wp < w) return fail(-1, "%s: padded size %u x %u below the frame's %u x %u", op, wp, hp, w, h);
    if ((uint64_t)n * hp * wp >= kMaxItems) return fail(-1, "%s: too many pixels", op);
    return 0;
}
}  // namespace

extern "C" int fhc_rgba_in(const void* rgba, uint32_t n, uint32_t w, uint32_t h, uint32_t pitch, uint64_t fstride,
                           const fhc_tensor* out, uint32_t hp, uint32_t wp, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * w * h == 0) return 0;
        FHC_TRY(check_frames("rgba_in", rgba, n, w, h, pitch, fstride, hp, wp));
        FHC_TRY(check(out, "rgba_in out", 3, false, true));
        const bool v4 = out->cstride == 4 && out->c0 == 0 && reinterpret_cast<uintptr_t>(out->p) % 8 == 0;
        return launch("rgba_in", (uint64_t)n * hp * wp, [&](dim3 g, uint32_t items) {
            auto k = v4 ? rgba_in_kernel<true> : rgba_in_kernel<false>;
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, static_cast<const uint32_t*>(rgba), w, h,
                               pitch, fstride, outv(out), hp, wp, items);
        });
    });
}

extern "C" int fhc_rgba_out(const fhc_tensor* in_, uint32_t n, uint32_t hp, uint32_t wp, void* rgba, uint32_t w,
                            uint32_t h, uint32_t pitch, uint64_t fstride, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * w * h == 0) return 0;
        FHC_TRY(check_frames("rgba_out", rgba, n, w, h, pitch, fstride, hp, wp));
        FHC_TRY(check(in_, "rgba_out in", 3, false));
        return launch("rgba_out", (uint64_t)n * h * w, [&](dim3 g, uint32_t items) {
            hipLaunchKernelGGL(rgba_out_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(in_), hp, wp,
                               static_cast<uint32_t*>(rgba), w, h, pitch, fstride, items);
        });
    });
}

extern "C" int fhc_rgba_resize(const void* rgba, uint32_t n, uint32_t w, uint32_t h, uint32_t pitch, uint64_t fstride,
                               uint32_t hp, uint32_t wp, const fhc_tensor* out, uint32_t oh, uint32_t ow,
                               void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * oh * ow == 0) return 0;
        FHC_TRY(check_frames("rgba_resize", rgba, n, w, h, pitch, fstride, hp, wp));
        FHC_TRY(check(out, "rgba_resize out", 3, false, true));
        if (out->cstride != 4 || out->c0 != 0 || reinterpret_cast<uintptr_t>(out->p) % 8)
            return fail(-1, "rgba_resize: the output must have 8-byte 4-channel pixels (cstride 4, c0 0)");
        if (oh > hp || ow > wp) return fail(-1, "rgba_resize: %u x %u is not a downscale of %u x %u", ow, oh, wp, hp);
        const uint32_t taps = std::max(aa_taps(hp, oh), aa_taps(wp, ow));
        const uint32_t ext = std::max(aa_tile_extent(hp, oh), aa_tile_extent(wp, ow));
        if (taps > 10 || ext > 84)
            return fail(-1, "rgba_resize: %u x %u -> %u x %u needs %u taps, a %u-pixel tile window (at most 10 and 84)",
                        wp, hp, ow, oh, taps, ext);
        const uint32_t tx = (ow + kAaT - 1) / kAaT, ty = (oh + kAaT - 1) / kAaT;
        // the 40-pixel window covers the common downscales (1080p to 864 x 480: 39 x 38); 2160p to 864 x 480 takes
        // 10 taps and a 78 x 76 window (4096 x 2176: 81 columns); the windows above 48 pixels hold 6-byte cells
        // (78 x 78: 40,096 bytes of LDS with the tables, four workgroups a CU)
        auto k = ext <= 40 && taps <= 5 ? rgba_resize_kernel<5, 3, 40, false>
                 : ext <= 3 * kAaT
                     ? (taps <= 5 ? rgba_resize_kernel<5, 3, 48, false> : taps <= 6 ? rgba_resize_kernel<6, 3, 48, false>
                                                                        : rgba_resize_kernel<8, 3, 48, false>)
                 : ext <= 5 * kAaT && taps <= 8
                     ? (taps <= 6 ? rgba_resize_kernel<6, 5, 80, true> : rgba_resize_kernel<8, 5, 80, true>)
                 : ext <= 78 ? rgba_resize_kernel<10, 5, 78, true> : rgba_resize_kernel<10, 6, 84, true>;
        if ((uint64_t)pitch * 4 >= (1u << 24) || (uint64_t)h * pitch * 4 >= (1u << 31))
            return fail(-1, "rgba_resize: frames of pitch %u and %u rows are too large", pitch, h);
        hipLaunchKernelGGL(k, dim3(n * tx * ty), dim3(kThreads), 0, (hipStream_t)stream,
                           static_cast<const uint32_t*>(rgba), w, h, pitch, fstride, hp, wp, outv(out), oh, ow, tx, ty,
                           (float)hp / (float)oh, (float)wp / (float)ow);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "rgba_resize: launch failed: %s", hipGetErrorString(e));
    });
}

namespace {
// fhc_render_rgba over pairs x phases generated frames (the pair's frames at p * pstride words past a and b)
int render_rgba_run(const void* a, const void* b, uint64_t pstride, uint32_t pairs, uint32_t phases, uint32_t w,
                    uint32_t h, uint32_t pitch, uint32_t hp, uint32_t wp, const fhc_tensor* flow, const fhc_tensor* vis,
                    const fhc_tensor* rt, uint32_t hq, uint32_t wq, float fsx, float fsy, int cubic, uint32_t flags,
                    void* out, uint32_t opitch, uint64_t ostride, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)h * w * pairs * phases == 0) return 0;
        if ((uint64_t)pairs * phases > 65535)
            return fail(-1, "render_rgba: %u generated frames exceed the launch limit", pairs * phases);
        if (hq == 0 || wq == 0) return fail(-1, "render_rgba: empty quarter maps (%u x %u)", hq, wq);
        if (flags > 7)
            return fail(-1, "render_rgba: flags %u (bit 0 decisive, bit 1 still, bit 2 exact f32 order)", flags);
        if (w < 4) return fail(-1, "render_rgba: frames narrower than 4 pixels");
        if (pairs > 1 && pstride < (uint64_t)pitch * h) return fail(-1, "render_rgba: pair stride below pitch * h");
        FHC_TRY(check_frames("render_rgba a", a, 1, w, h, pitch, 0, hp, wp));
        FHC_TRY(check_frames("render_rgba b", b, 1, w, h, pitch, 0, hp, wp));
        FHC_TRY(check_frames("render_rgba out", out, pairs * phases, w, h, opitch, ostride, hp, wp));
        FHC_TRY(check(flow, "render_rgba flow", 4, false));
        FHC_TRY(check(vis, "render_rgba vis", 3, true));
        FHC_TRY(check(rt, "render_rgba rt", 3, false));
        // the tap rows' 32-bit byte offsets (24-bit row multiply) and the quarter maps' buffer sizes
        if ((uint64_t)pitch * 4 >= (1u << 24) || (uint64_t)h * pitch * 4 >= (1u << 31) ||
            (uint64_t)hq * wq * std::max(16u, 2 * rt->cstride) >= (1u << 31) || hq >= (1u << 24) || wq >= (1u << 24))
            return fail(-1, "render_rgba: frame (pitch %u, %u rows) or quarter maps (%u x %u) too large", pitch, h, wq, hq);
        const bool qv = flow->p == vis->p && flow->cstride == 8 && vis->cstride == 8 && flow->c0 == 0 &&
                        vis->c0 == 4 && reinterpret_cast<uintptr_t>(flow->p) % 16 == 0 && vec4(4, {rt});
        if ((uint64_t)h * w >= kMaxItems || h > 4u * 65535u)
            return fail(-1, "render_rgba: %u x %u pixels exceed the launch limits", w, h);
        using K = decltype(&render_rgba_kernel<true, true, true, true>);
        // [exact order][cubic][quarter-map vectors][mode flags]
        static const K ks[2][2][2][2] = {
            {{{render_rgba_kernel<false, false, false, true>, render_rgba_kernel<false, false, true, true>},
              {render_rgba_kernel<false, true, false, true>, render_rgba_kernel<false, true, true, true>}},
             {{render_rgba_kernel<true, false, false, true>, render_rgba_kernel<true, false, true, true>},
              {render_rgba_kernel<true, true, false, true>, render_rgba_kernel<true, true, true, true>}}},
            {{{render_rgba_kernel<false, false, false, false>, render_rgba_kernel<false, false, true, false>},
              {render_rgba_kernel<false, true, false, false>, render_rgba_kernel<false, true, true, false>}},
             {{render_rgba_kernel<true, false, false, false>, render_rgba_kernel<true, false, true, false>},
              {render_rgba_kernel<true, true, false, false>, render_rgba_kernel<true, true, true, false>}}}};
        const uint32_t modes = flags & 3u;
        hipLaunchKernelGGL(ks[(flags >> 2) & 1u][cubic ? 1 : 0][qv ? 1 : 0][modes ? 1 : 0],
                           dim3((w + 63) / 64, (h + 3) / 4, pairs * phases), dim3(kThreads), 0, (hipStream_t)stream,
                           static_cast<const uint32_t*>(a), static_cast<const uint32_t*>(b), w, h, pitch,
                           (float)hq / (float)hp, (float)wq / (float)wp, in(flow), in(vis), in(rt), hq, wq, fsx, fsy,
                           modes, static_cast<uint32_t*>(out), opitch, pstride, pairs, phases, ostride);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "render_rgba: launch failed: %s", hipGetErrorString(e));
    });
}
}  // namespace

extern "C" int fhc_render_rgba(const void* a, const void* b, uint32_t w, uint32_t h, uint32_t pitch, uint32_t hp,
                               uint32_t wp, const fhc_tensor* flow, const fhc_tensor* vis, const fhc_tensor* rt,
                               uint32_t hq, uint32_t wq, float fsx, float fsy, int cubic, uint32_t flags, void* out,
                               uint32_t opitch, void* stream) {
    return render_rgba_run(a, b, 0, 1, 1, w, h, pitch, hp, wp, flow, vis, rt, hq, wq, fsx, fsy, cubic, flags, out,
                           opitch, 0, stream);
}

extern "C" int fhc_render_rgba_n(const void* frames, uint32_t pairs, uint32_t phases, uint32_t w, uint32_t h,
                                 uint32_t pitch, uint64_t fstride, uint32_t hp, uint32_t wp, const fhc_tensor* flow,
                                 const fhc_tensor* vis, const fhc_tensor* rt, uint32_t hq, uint32_t wq, float fsx,
                                 float fsy, int cubic, uint32_t flags, void* out, uint32_t opitch, uint64_t ostride,
                                 void* stream) {
    if (pairs && fstride < (uint64_t)pitch * h) {
        clear_error();
        return fail(-1, "render_rgba: frame stride below pitch * h");
    }
    const void* b = frames ? static_cast<const uint32_t*>(frames) + fstride : nullptr;
    return render_rgba_run(frames, b, 2 * fstride, pairs, phases, w, h, pitch, hp, wp, flow, vis, rt, hq, wq, fsx, fsy,
                           cubic, flags, out, opitch, ostride, stream);
}

extern "C" int fhc_gmhs_params(uint32_t h, uint32_t w, uint32_t full_w, uint32_t level, fhc_gmhs_par* out) {
    return guard(-3, [&]() -> int {
        clear_error();
        return gm_params(h, w, full_w, level, out);
    });
}

int fhc::gmhs_run(const fhc_tensor* a, const fhc_tensor* b, uint32_t h, uint32_t w, const fhc_tensor* flow,
                  uint32_t h8, uint32_t w8, uint32_t full_w, uint32_t level, void* ws, size_t ws_bytes,
                  const GmCoRun* co, void* stream, uint32_t pairs) {
    return guard(-3, [&]() -> int {
        clear_error();
        if (level == 0 || pairs == 0) return 0;
        if (co && pairs != 1) return fail(-1, "gmhs: a co-runner goes with one pair, %u given", pairs);
        if (pairs > 65535 / 5) return fail(-1, "gmhs: %u pairs exceed the launch limit", pairs);
        fhc_gmhs_par p;
        FHC_TRY(gm_params(h, w, full_w, level, &p));
        if (h8 == 0 || w8 == 0) return fail(-1, "gmhs: empty E8 flow (%u x %u)", w8, h8);
        FHC_TRY(check(a, "gmhs a", 3, false));
        FHC_TRY(check(b, "gmhs b", 3, false));
        FHC_TRY(check(flow, "gmhs flow", 4, false));
        if (!ws) return fail(-1, "gmhs: null workspace");
        // pair k's workspace starts at k * stride bytes (the last pair's needs only ws_bytes)
        const uint64_t stride = (p.ws_bytes + 255) / 256 * 256, need = (pairs - 1) * stride + p.ws_bytes;
        const size_t wsf = stride / sizeof(float);
        if (ws_bytes < need)
            return fail(-1, "gmhs: workspace of %zu bytes, %llu needed", ws_bytes, (unsigned long long)need);
        if (reinterpret_cast<uintptr_t>(ws) % 256) return fail(-1, "gmhs: the workspace must be 256-byte aligned");
        if (p.r_blk > kGmRmax || p.r_dwin > kGmRmax)
            return fail(-1, "gmhs: box radii %u, %u exceed %u", p.r_blk, p.r_dwin, kGmRmax);
        if ((uint64_t)h8 * w8 >= kMaxItems || (uint64_t)h * w >= kMaxItems)
            return fail(-1, "gmhs: %u x %u network, %u x %u flow: too large", w, h, w8, h8);
        // the raw cost maps' region, once the texture window has read them, holds dec [5][h8][w8] then hs [3][hc][w8]
        const uint64_t cells = (uint64_t)p.hc * p.wc, hs_off = ((uint64_t)5 * h8 * w8 + 63) / 64 * 64;
        if (h8 > p.hc || w8 > p.wc || hs_off + (uint64_t)3 * p.hc * w8 > 5 * cells)
            return fail(-1, "gmhs: the E8 flow (%u x %u) is too large for the cost grid (%u x %u)", w8, h8, p.wc, p.hc);
        float* coef = static_cast<float*>(ws);
        float* part[2] = {coef + 16, coef + 16 + kGmPart};
        float* maps = reinterpret_cast<float*>(static_cast<char*>(ws) + p.maps_offset);  // after the texture window
        float* raw = reinterpret_cast<float*>(static_cast<char*>(ws) + p.dec_offset);    // the cost maps, then dec
        float* hs = raw + hs_off;
        const hipStream_t st = (hipStream_t)stream;
        for (uint32_t round = 0; round < 4; round++) {
            const FitRoundArgs fa{static_cast<const uint16_t*>(flow->p), flow->cstride, flow->c0, h8, w8, p.delta,
                                  round, part[(round + 1) & 1u], part[round & 1u]};
            if (co && round == 0) {  // the co-runner's pair beside the first round's workgroups
                const hipError_t ce = co->fn(fa, co->pk, co->tiles, st);
                if (ce != hipSuccess) return fail(-2, "gmhs: launch failed: %s", hipGetErrorString(ce));
                continue;
            }
            if (co && co->cfn && round == 1) {  // its conv beside the second round's
                const hipError_t ce = co->cfn(fa, co->ca, co->cgrid, st);
                if (ce != hipSuccess) return fail(-2, "gmhs: launch failed: %s", hipGetErrorString(ce));
                continue;
            }
            hipLaunchKernelGGL(gm_fit_kernel, dim3(kGmNwg, 4, pairs), dim3(kGmWg), 0, st, in(flow), h8, w8, p.delta,
                               round, part[(round + 1) & 1u], part[round & 1u], wsf);
        }
        const bool v = vec4(4, {a, b, flow});
        const dim3 tiles((p.wc + kGmT - 1) / kGmT, (p.hc + kGmT - 1) / kGmT);
        const dim3 ctiles(tiles.x, (p.hc + 7) / 8, pairs);  // the cost kernel's 16 x 8 blocks
        hipLaunchKernelGGL(v ? gm_cost_kernel<true> : gm_cost_kernel<false>, ctiles, dim3(kThreads), 0, st, in(a), in(b),
                           h, w, in(flow), h8, w8, part[1], coef, raw, p.hc, p.wc, wsf);
        // the texture window over the 5 maps (raw -> maps), then the decision window at the cells the select reads
        // (its rows at their columns, its columns at their rows) and the select (maps -> dec, flow)
        const uint32_t rows = kGmT + 2 * p.r_blk, nb = (rows + kGmT - 1) / kGmT;  // r <= 32: 2 .. 5 blocks a side
        auto box = nb <= 2 ? gm_box_kernel<2> : nb == 3 ? gm_box_kernel<3> : nb == 4 ? gm_box_kernel<4> : gm_box_kernel<5>;
        hipLaunchKernelGGL(box, dim3(tiles.x, tiles.y, 5 * pairs), dim3(kThreads), (rows * rows + rows * kGmT) * 4, st,
                           raw, maps, p.hc, p.wc, p.r_blk, wsf);
        const bool wide = 2 * p.r_dwin + 1 > 33;
        const uint32_t nh = 3 * p.hc * w8, ne = h8 * w8;
        hipLaunchKernelGGL(wide ? gm_dwin_h_kernel<65> : gm_dwin_h_kernel<33>,
                           dim3((nh + kThreads - 1) / kThreads, pairs), dim3(kThreads), 0, st, maps, hs, p.hc, p.wc, w8,
                           p.r_dwin, nh, wsf);
        hipLaunchKernelGGL(wide ? gm_dwin_v_select_kernel<65> : gm_dwin_v_select_kernel<33>,
                           dim3((4 * ne + kThreads - 1) / kThreads, pairs), dim3(kThreads), 0, st, hs, maps, coef,
                           outv(flow), raw, h8, w8, p.hc, p.wc, p.r_dwin, p.eps, p.dmin, p.tex, ne, wsf);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "gmhs: launch failed: %s", hipGetErrorString(e));
    });
}

extern "C" int fhc_gmhs(const fhc_tensor* a, const fhc_tensor* b, uint32_t h, uint32_t w, const fhc_tensor* flow,
                        uint32_t h8, uint32_t w8, uint32_t full_w, uint32_t level, void* ws, size_t ws_bytes,
                        void* stream) {
    return gmhs_run(a, b, h, w, flow, h8, w8, full_w, level, ws, ws_bytes, nullptr, stream);
}

extern "C" int fhc_gmhs_n(const fhc_tensor* a, const fhc_tensor* b, uint32_t h, uint32_t w, const fhc_tensor* flow,
                          uint32_t h8, uint32_t w8, uint32_t full_w, uint32_t level, uint32_t pairs, void* ws,
                          size_t ws_bytes, void* stream) {
    return gmhs_run(a, b, h, w, flow, h8, w8, full_w, level, ws, ws_bytes, nullptr, stream, pairs);
}

extern "C" int fhc_coarse_fine_input(const fhc_tensor* o, const fhc_tensor* fv, const fhc_tensor* state,
                                     uint32_t hi, uint32_t wi, float flow_scale, const fhc_tensor* f8,
                                     const fhc_tensor* i8, float fine_scale, const fhc_tensor* fx,
                                     const fhc_tensor* l8, uint32_t h, uint32_t w, uint32_t c, void* stream) {
    return fhc_coarse_fine_input_n(o, fv, state, hi, wi, flow_scale, f8, i8, fine_scale, fx, l8, h, w, c, 1, stream);
}

extern "C" int fhc_coarse_fine_input_n(const fhc_tensor* o, const fhc_tensor* fv, const fhc_tensor* state,
                                       uint32_t hi, uint32_t wi, float flow_scale, const fhc_tensor* f8,
                                       const fhc_tensor* i8, float fine_scale, const fhc_tensor* fx,
                                       const fhc_tensor* l8, uint32_t h, uint32_t w, uint32_t c, uint32_t pairs,
                                       void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)h * w * c * pairs == 0) return 0;
        if (pairs > 65535) return fail(-1, "coarse_fine_input: %u pairs exceed the launch limit", pairs);
        if (hi == 0 || wi == 0) return fail(-1, "coarse_fine_input: empty coarse output (%u x %u)", hi, wi);
        if (state && (hi > h || wi > w)) return fail(-1, "coarse_fine_input: the state is larger than the fine grid");
        FHC_TRY(check(o, "coarse_fine_input o", 7, false));
        FHC_TRY(check(fv, "coarse_fine_input fv", 7, false, true));
        if (state) FHC_TRY(check(state, "coarse_fine_input state", 4, false, true));
        FHC_TRY(check(f8, "coarse_fine_input f8", c, true));
        FHC_TRY(check(i8, "coarse_fine_input i8", 3, true));
        FHC_TRY(check(fx, "coarse_fine_input fx", 2 * c + 10, false, true));
        FHC_TRY(check(l8, "coarse_fine_input l8", 2, false, true));
        if (!std::isfinite(fine_scale)) return fail(-1, "coarse_fine_input: the flow's read scale is not finite");
        const uint32_t groups = (c + 3) / 4;
        fhc_tensor fxb = *fx;
        fxb.c0 += c;
        const bool v = vec4(c, {f8, fx, &fxb});
        const View fl{static_cast<const uint16_t*>(fv->p), fv->cstride, fv->c0, fine_scale};
        const OView sv = state ? outv(state) : OView{nullptr, 0, 0};
        return launch("coarse_fine_input", (uint64_t)h * w * (2 * groups + 3), [&](dim3 g, uint32_t n) {
            auto k = v ? fine_input_kernel<true, true> : fine_input_kernel<false, true>;
            hipLaunchKernelGGL(k, dim3(g.x, pairs), dim3(kThreads), 0, (hipStream_t)stream, in(f8), in(i8), fl,
                               outv(fx), outv(l8), h, w, c, groups, n, in(o), outv(fv), sv, hi, wi, flow_scale,
                               (float)hi / (float)h, (float)wi / (float)w);
        });
    });
}

extern "C" int fhc_coarse_fine_input_sad_n(const fhc_tensor* o, const fhc_tensor* fv, const fhc_tensor* state,
                                           uint32_t hi, uint32_t wi, float flow_scale, const fhc_tensor* f8,
                                           const fhc_tensor* i8, float fine_scale, const fhc_tensor* fx,
                                           const fhc_tensor* l8, uint32_t h, uint32_t w, uint32_t c, uint32_t pairs,
                                           const fhc_tensor* sad_out, uint32_t radius, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)h * w * c * pairs == 0) return 0;
        if (pairs > 65535) return fail(-1, "coarse_fine_input_sad: %u pairs exceed the launch limit", pairs);
        if (hi == 0 || wi == 0) return fail(-1, "coarse_fine_input_sad: empty coarse output (%u x %u)", hi, wi);
        if (state && (hi > h || wi > w))
            return fail(-1, "coarse_fine_input_sad: the state is larger than the fine grid");
        if (radius > kSadRmax) return fail(-1, "coarse_fine_input_sad: radius %u above %u", radius, kSadRmax);
        const uint32_t span2 = (2 * radius + 1) * (2 * radius + 1);
        FHC_TRY(check(o, "coarse_fine_input_sad o", 7, false));
        FHC_TRY(check(fv, "coarse_fine_input_sad fv", 7, false, true));
        if (state) FHC_TRY(check(state, "coarse_fine_input_sad state", 4, false, true));
        FHC_TRY(check(f8, "coarse_fine_input_sad f8", c, true));
        FHC_TRY(check(i8, "coarse_fine_input_sad i8", 3, true));
        FHC_TRY(check(fx, "coarse_fine_input_sad fx", 2 * c + 10, false, true));
        FHC_TRY(check(l8, "coarse_fine_input_sad l8", 2, false, true));
        FHC_TRY(check(sad_out, "coarse_fine_input_sad sad out", span2, false, true));
        if (!std::isfinite(fine_scale)) return fail(-1, "coarse_fine_input_sad: the flow's read scale is not finite");
        const uint32_t groups = (c + 3) / 4;
        const uint64_t items = (uint64_t)h * w * (2 * groups + 3);
        const uint32_t tiles_x = (w + kSadTX - 1) / kSadTX, tiles = tiles_x * ((h + kSadTY - 1) / kSadTY);
        if (items + (uint64_t)tiles * kThreads >= kMaxItems)
            return fail(-1, "coarse_fine_input_sad: %u x %u is too large", w, h);
        fhc_tensor fxb = *fx;
        fxb.c0 += c;
        const bool v = vec4(c, {f8, fx, &fxb});
        const View fl{static_cast<const uint16_t*>(fv->p), fv->cstride, fv->c0, fine_scale};
        const OView sv = state ? outv(state) : OView{nullptr, 0, 0};
        const uint32_t fine_blocks = (uint32_t)((items + kThreads - 1) / kThreads);
        decltype(&fine_input_sad_kernel<true, 1>) k;
        if (radius == 0) k = v ? fine_input_sad_kernel<true, 0> : fine_input_sad_kernel<false, 0>;
        else if (radius == 1) k = v ? fine_input_sad_kernel<true, 1> : fine_input_sad_kernel<false, 1>;
        else if (radius == 2) k = v ? fine_input_sad_kernel<true, 2> : fine_input_sad_kernel<false, 2>;
        else k = v ? fine_input_sad_kernel<true, 3> : fine_input_sad_kernel<false, 3>;
        hipLaunchKernelGGL(k, dim3(fine_blocks + tiles, pairs), dim3(kThreads), 0, (hipStream_t)stream, in(f8), in(i8),
                           fl, outv(fx), outv(l8), h, w, c, groups, (uint32_t)items, in(o), outv(fv), sv, hi, wi,
                           flow_scale, (float)hi / (float)h, (float)wi / (float)w, fine_blocks, outv(sad_out),
                           tiles_x);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "coarse_fine_input_sad: launch failed: %s", hipGetErrorString(e));
    });
}

extern "C" int fhc_flow_vis_t_convex(const fhc_tensor* wt, const fhc_tensor* fv, const fhc_tensor* dfilm, float t,
                                     const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, void* stream) {
    return fhc_flow_vis_t_convex_n(wt, fv, dfilm, &t, 1, out, n, h, w, stream);
}

extern "C" int fhc_flow_vis_t_convex_n(const fhc_tensor* wt, const fhc_tensor* fv, const fhc_tensor* dfilm,
                                       const float* ts, uint32_t phases, const fhc_tensor* out, uint32_t n, uint32_t h,
                                       uint32_t w, void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w * phases == 0) return 0;
        if (!ts) return fail(-1, "flow_vis_t_convex: null phases");
        if (phases > kMaxPhases) return fail(-1, "flow_vis_t_convex: %u phases (at most %u)", phases, kMaxPhases);
        PhaseT ph{};
        for (uint32_t j = 0; j < phases; j++)  // the mul_t factors (net/build.rs:293)
            ph.af[j] = 2.0f * ts[j], ph.ab[j] = 2.0f * (1.0f - ts[j]);
        FHC_TRY(check(wt, "flow_vis_t_convex wt", 36, false));
        FHC_TRY(check(fv, "flow_vis_t_convex fv", 7, true));
        FHC_TRY(check(dfilm, "flow_vis_t_convex dfilm", 5, true));
        FHC_TRY(check(out, "flow_vis_t_convex out", 7, false, true));
        const uint32_t tx = (w + kCvIn - 1) / kCvIn, ty = (h + kCvIn - 1) / kCvIn;
        if ((uint64_t)phases * n * tx * ty >= kMaxItems) return fail(-1, "flow_vis_t_convex: too many tiles");
        const size_t lds = (kCvIn * kCvIn * 36 + kCvHalo * kCvHalo * 7) * 2;
        const View none{nullptr, 0, 0, 1.0f};
        hipLaunchKernelGGL(convex_tile_kernel<true>, dim3(phases * n * tx * ty), dim3(kCvThreads), lds,
                           (hipStream_t)stream, in(wt), none, outv(out), h, w, 7u, tx, ty, in(fv), in(dfilm), ph, n);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "flow_vis_t_convex: launch failed: %s", hipGetErrorString(e));
    });
}

extern "C" int fhc_mid_input_n(const fhc_tensor* wt, const fhc_tensor* fv, const fhc_tensor* dfilm, const float* ts,
                               uint32_t phases, const fhc_tensor* up, const fhc_tensor* q, const fhc_tensor* rx,
                               uint32_t n, uint32_t h, uint32_t w, float flow_scale, float flow_out_scale,
                               void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        if ((uint64_t)n * h * w * phases == 0) return 0;
        if (!ts) return fail(-1, "mid_input: null phases");
        if (phases > kMaxPhases) return fail(-1, "mid_input: %u phases (at most %u)", phases, kMaxPhases);
        if ((uint64_t)phases * n > 65535) return fail(-1, "mid_input: %u images exceed the launch limit", phases * n);
        if (!std::isfinite(flow_scale)) return fail(-1, "mid_input: the flow's read scale is not finite");
        PhaseT ph{};
        for (uint32_t j = 0; j < phases; j++)  // the mul_t factors (net/build.rs:293)
            ph.af[j] = 2.0f * ts[j], ph.ab[j] = 2.0f * (1.0f - ts[j]);
        FHC_TRY(check(wt, "mid_input wt", 36, false));
        FHC_TRY(check(fv, "mid_input fv", 7, true));
        FHC_TRY(check(dfilm, "mid_input dfilm", 5, true));
        FHC_TRY(check(up, "mid_input up", 7, false, true));
        FHC_TRY(check(q, "mid_input q", 3, true));
        FHC_TRY(check(rx, "mid_input rx", 14, false, true));
        const uint32_t tx = (2 * w + kRiT - 1) / kRiT, ty = (2 * h + kRiT - 1) / kRiT;
        if ((uint64_t)tx * ty >= kMaxItems / 64) return fail(-1, "mid_input: %u x %u is too large", w, h);
        hipLaunchKernelGGL(mid_input_kernel, dim3(tx * ty, phases * n), dim3(64), 0, (hipStream_t)stream, in(wt),
                           in(fv), in(dfilm), ph, n, in(q), outv(up), outv(rx), h, w, flow_scale, flow_out_scale, tx);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "mid_input: launch failed: %s", hipGetErrorString(e));
    });
}

extern "C" int fhc_fold_pair_sad(const fhc_tensor* x, const fhc_tensor* out, const fhc_tensor* also, uint32_t h,
                                 uint32_t w, uint32_t c, const fhc_tensor* la, const fhc_tensor* lb,
                                 const fhc_tensor* sad_out, uint32_t sn, uint32_t sh, uint32_t sw, uint32_t radius,
                                 void* stream) {
    return fhc_fold_pair_sad_n(x, out, also, h, w, c, 1, la, lb, sad_out, sn, sh, sw, radius, stream);
}

extern "C" int fhc_fold_pair_sad_n(const fhc_tensor* x, const fhc_tensor* out, const fhc_tensor* also, uint32_t h,
                                   uint32_t w, uint32_t c, uint32_t pairs, const fhc_tensor* la, const fhc_tensor* lb,
                                   const fhc_tensor* sad_out, uint32_t sn, uint32_t sh, uint32_t sw, uint32_t radius,
                                   void* stream) {
    return guard(-3, [&]() -> int {
        clear_error();
        const uint64_t fold_items = (uint64_t)pairs * h * w * 2 * ((c + 3) / 4);  // all pairs'
        if (radius > 7) return fail(-1, "fold_pair_sad: radius %u above 7", radius);
        if (pairs > 65535) return fail(-1, "fold_pair_sad: %u pairs exceed the launch limit", pairs);
        const uint32_t span2 = (2 * radius + 1) * (2 * radius + 1);
        const uint64_t sad_items = (uint64_t)sn * sh * sw * span2;
        if (fold_items == 0 && sad_items == 0) return 0;
        if (fold_items) {
            FHC_TRY(check(x, "fold_pair_sad x", c, false));
            FHC_TRY(check(out, "fold_pair_sad out", 2 * c, false, true));
            if (also) FHC_TRY(check(also, "fold_pair_sad also", c, false, true));
        }
        if (sad_items) {
            FHC_TRY(check(la, "fold_pair_sad la", 1, false));
            FHC_TRY(check(lb, "fold_pair_sad lb", 1, false));
            FHC_TRY(check(sad_out, "fold_pair_sad sad out", span2, false, true));
        }
        const uint64_t fold1 = fold_items ? fold_items / pairs : 0;  // one pair's
        const uint64_t fb = (fold1 + kThreads - 1) / kThreads, sb = (sad_items + kThreads - 1) / kThreads;
        if (fold_items >= kMaxItems || sad_items >= kMaxItems || fb + sb >= (1u << 31))
            return fail(-1, "fold_pair_sad: too many work items");
        bool v = false;
        OView a2{nullptr, 0, 0};
        View xv{nullptr, 0, 0, 1.0f};
        OView ov{nullptr, 0, 0};
        if (fold_items) {
            fhc_tensor out1 = *out;  // image 1's slice must be aligned too for the vector path
            out1.c0 += c;
            v = also ? vec4(c, {x, out, &out1, also}) : vec4(c, {x, out, &out1});
            a2 = also ? outv(also) : a2;
            xv = in(x), ov = outv(out);
        }
        const View none{nullptr, 0, 0, 1.0f};
        const SadArgs sa{sad_items ? in(la) : none, sad_items ? in(lb) : none,
                         sad_items ? outv(sad_out) : OView{nullptr, 0, 0}, sh, sw, radius, span2, (uint32_t)sad_items};
        auto k = v ? fold_pair_sad_kernel<true> : fold_pair_sad_kernel<false>;
        hipLaunchKernelGGL(k, dim3((uint32_t)(fb + sb), fold_items ? pairs : 1u), dim3(kThreads), 0,
                           (hipStream_t)stream, xv, ov, a2, h * w, c, (c + 3) / 4, (uint32_t)fold1, (uint32_t)fb, sa);
        const hipError_t e = hipGetLastError();
        return e == hipSuccess ? 0 : fail(-2, "fold_pair_sad: launch failed: %s", hipGetErrorString(e));
    });
}
