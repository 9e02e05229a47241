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
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float ld(const View& v, size_t pix, uint32_t ch) { return h2f(v.p[pix * v.cs + v.c0 + ch]); }
__device__ __forceinline__ void st(const OView& v, size_t pix, uint32_t ch, float x) {
    v.p[pix * v.cs + v.c0 + ch] = f2h(x);
}
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

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
template <bool VEC>
__global__ __launch_bounds__(kThreads) void warp_kernel(View img, View flow, OView out, uint32_t h, uint32_t w,
                                                        uint32_t c, uint32_t groups, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t pix = t / groups, ch = (t - pix * groups) * 4;
    const uint32_t x = pix % w, row = pix / w, y = row % h, img0 = row - y;  // img0 = image * h
    const float fx = ld(flow, pix, 0) * flow.scale, fy = ld(flow, pix, 1) * flow.scale;
    const float gx = (float)x + fx, gy = (float)y + fy;
    const int x0 = (int)floorf(gx), y0 = (int)floorf(gy);
    const float ax = gx - (float)x0, ay = gy - (float)y0;
    const int x0c = clampi(x0, 0, (int)w - 1), x1c = clampi(x0 + 1, 0, (int)w - 1);
    const int y0c = clampi(y0, 0, (int)h - 1), y1c = clampi(y0 + 1, 0, (int)h - 1);
    const size_t r0 = (size_t)(img0 + y0c) * w, r1 = (size_t)(img0 + y1c) * w;
    float v00[4], v01[4], v10[4], v11[4], o[4];
    ld4<VEC>(img, r0 + x0c, ch, c, v00);
    ld4<VEC>(img, r0 + x1c, ch, c, v01);
    ld4<VEC>(img, r1 + x0c, ch, c, v10);
    ld4<VEC>(img, r1 + x1c, ch, c, v11);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float top = v00[i] * (1.0f - ax) + v01[i] * ax, bot = v10[i] * (1.0f - ax) + v11[i] * ax;
        o[i] = (top * (1.0f - ay) + bot * ay) * img.scale;
    }
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
__global__ __launch_bounds__(kThreads) void sad_kernel(View la, View lb, OView out, uint32_t h, uint32_t w,
                                                       uint32_t r, uint32_t span2, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
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

// ---- convex upsample: shaders/convex.wgsl:12-34 ------------------------------------------------------------------
// A workgroup computes 16 x 16 output pixels (8 x 8 input pixels, 4 sub-pixels each): it stages the 36 weight
// channels of its input pixels and the 10 x 10 neighbourhood of x (zeros outside the image: adding 0 * weight is
// what the reference's zero branch adds) in LDS with coalesced reads, then one lane per output pixel computes its
// softmax once and every channel from LDS, in the reference's order.
constexpr uint32_t kCvIn = 8, kCvHalo = kCvIn + 2;

__global__ __launch_bounds__(kThreads) void convex_tile_kernel(View wt, View x, OView out, uint32_t h, uint32_t w,
                                                               uint32_t c, uint32_t tiles_x, uint32_t tiles_y) {
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t* lw = lds;                       // [kCvIn * kCvIn][36]
    uint16_t* lx = lds + kCvIn * kCvIn * 36;  // [kCvHalo * kCvHalo][c]
    const uint32_t tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    const uint32_t bt = blockIdx.x, txi = bt % tiles_x, r = bt / tiles_x, tyi = r % tiles_y, img = r / tiles_y;
    const int ix0 = (int)(txi * kCvIn), iy0 = (int)(tyi * kCvIn);
    // staging with every load unconditional (clamped to the image / the view) and unrolled, so they issue together
#pragma unroll
    for (uint32_t k = 0; k < (kCvIn * kCvIn * 9 + kThreads - 1) / kThreads; k++) {  // 9 quads of 4 channels a pixel
        const uint32_t e = min(tid + k * kThreads, kCvIn * kCvIn * 9 - 1);
        const uint32_t p = e / 9, q = e - p * 9, py = p / kCvIn, px = p % kCvIn;
        const int gy = min(iy0 + (int)py, (int)h - 1), gx = min(ix0 + (int)px, (int)w - 1);
        const uint16_t* src = wt.p + (((size_t)img * h + gy) * w + gx) * wt.cs + wt.c0 + q * 4;
        // lanes past the last quad rewrite that quad with its own value (a conditional store would pull the load
        // into the branch and serialise the loads again)
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) lw[p * 36 + q * 4 + i] = src[i];
    }
    if (tid < kCvHalo * kCvHalo) {  // one lane per halo pixel, channels 8 at a time
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
    const uint16_t* pw = lw + (liy * kCvIn + lix) * 36 + sub;
    float m = -3.0e38f, ws[9];
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
    const size_t opix = ((size_t)img * 2 * h + oy) * 2 * w + ox;
    for (uint32_t co = 0; co < c; co++) {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < 9; k++)
            acc = acc + ws[k] * h2f(lx[((liy + k / 3) * kCvHalo + lix + k % 3) * c + co]);
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
__device__ __forceinline__ void soft3(const View& vis, size_t pix, float& ea, float& eb, float& ec, float& s) {
    const float a = ld(vis, pix, 0) * vis.scale, b = ld(vis, pix, 1) * vis.scale, c = ld(vis, pix, 2) * vis.scale;
    const float m = fmaxf(a, fmaxf(b, c));
    ea = expf(a - m), eb = expf(b - m), ec = expf(c - m);
    s = ea + eb + ec;
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

template <int KM>
__global__ __launch_bounds__(kThreads) void interp_aa_lds_kernel(View x, OView out, uint32_t ih, uint32_t iw,
                                                                 uint32_t oh, uint32_t ow, uint32_t c,
                                                                 uint32_t tiles_x, uint32_t tiles_y) {
    __shared__ uint2 tile[kAaExt * kAaExt];
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
    const size_t rowbase = (size_t)img * ih + ylo;
#pragma unroll
    for (uint32_t i = 0; i < kAaR; i++)
#pragma unroll
        for (uint32_t j = 0; j < kAaR; j++) {
            const int row = min((int)(ty + kAaT * i), ny - 1), col = min((int)(tx + kAaT * j), nx - 1);
            const uint16_t* src = x.p + ((rowbase + row) * iw + xlo + col) * x.cs + x.c0;
            uint16_t v[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; k++) v[k] = src[min(k, c - 1)];
            tile[row * kAaExt + col] = uint2{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16)};
        }
    __syncthreads();
    const uint32_t ox = ox0 + tx, oy = oy0 + ty;
    if (ox >= ow || oy >= oh) return;
    const float cy = ((float)oy + 0.5f) * sh, cx = ((float)ox + 0.5f) * sw;
    const int ymin = max(0, (int)floorf(cy - fsh + 0.5f)), ymax = min((int)ih, (int)floorf(cy + fsh + 0.5f));
    const int xmin = max(0, (int)floorf(cx - fsw + 0.5f)), xmax = min((int)iw, (int)floorf(cx + fsw + 0.5f));
    float wx[KM];
    int lc[KM];
#pragma unroll
    for (int j = 0; j < KM; j++) {
        const int xx = xmin + j;
        wx[j] = xx < xmax ? fmaxf(0.0f, 1.0f - fabsf(((float)xx + 0.5f - cx) / fsw)) : 0.0f;
        lc[j] = min(max(xx - xlo, 0), nx - 1);
    }
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, norm = 0.0f;
#pragma unroll
    for (int jy = 0; jy < KM; jy++) {
        const int y = ymin + jy;
        const float wy = y < ymax ? fmaxf(0.0f, 1.0f - fabsf(((float)y + 0.5f - cy) / fsh)) : 0.0f;
        const uint2* lrow = tile + min(max(y - ylo, 0), ny - 1) * kAaExt;
#pragma unroll
        for (int jx = 0; jx < KM; jx++) {
            const bool in = (y < ymax) & (xmin + jx < xmax);
            const float wgt = wx[jx] * wy;
            const uint2 q = lrow[lc[jx]];
            const float v[4] = {h2f((uint16_t)q.x), h2f((uint16_t)(q.x >> 16)), h2f((uint16_t)q.y),
                                h2f((uint16_t)(q.y >> 16))};
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = acc[i] + (in ? v[i] : 0.0f) * wgt;
            norm = norm + wgt;
        }
    }
    float val[4];
#pragma unroll
    for (int i = 0; i < 4; i++) val[i] = acc[i] / norm * x.scale;
    st4<false>(out, ((size_t)img * oh + oy) * ow + ox, 0, c, val);
}

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

template <bool VEC>
__global__ __launch_bounds__(kThreads) void unary_kernel(View x, OView out, uint32_t c, int op, float pa, float pb,
                                                         uint32_t groups, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t pix = t / groups, ch = (t - pix * groups) * 4;
    float v[4], o[4];
    ld4<VEC>(x, pix, ch, c, v);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float u = v[i] * x.scale;
        o[i] = op == 0 ? u * pa : op == 1 ? fminf(fmaxf(u, pa), pb) : op == 2 ? 2.0f / (1.0f + expf(-u)) - 1.0f : -u;
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
        hipLaunchKernelGGL(convex_tile_kernel, dim3(n * tx * ty), dim3(kThreads), lds, (hipStream_t)stream, in(wt),
                           in(x), outv(out), h, w, c, tx, ty);
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
            if (c <= 4 && taps <= 8 && aa_tile_extent(ih, oh) <= kAaExt && aa_tile_extent(iw, ow) <= kAaExt) {
                const uint32_t tx = (ow + kAaT - 1) / kAaT, ty = (oh + kAaT - 1) / kAaT;
                if ((uint64_t)n * tx * ty >= kMaxItems) return fail(-1, "interpolate: too many tiles");
                auto kl = taps <= 4 ? interp_aa_lds_kernel<4> : interp_aa_lds_kernel<8>;
                hipLaunchKernelGGL(kl, dim3(n * tx * ty), dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out),
                                   ih, iw, oh, ow, c, tx, ty);
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
            auto k = v ? unary_kernel<true> : unary_kernel<false>;
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), c, op, a, b, groups,
                               items);
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
