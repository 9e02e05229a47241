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
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) o[i] = ch + i < c ? ld(v, pix, ch + i) : 0.0f;
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
            const int yy = (int)y + wy, xx = (int)x + wx;
            if (yy >= 0 && yy < (int)h && xx >= 0 && xx < (int)w) {
                const float lav = ld(la, (size_t)(img0 + yy) * w + xx, 0);
                const int syy = clampi(yy + dy, 0, (int)h - 1), sxx = clampi(xx + dx, 0, (int)w - 1);
                acc = acc + fabsf(lav - ld(lb, (size_t)(img0 + syy) * w + sxx, 0));
            }
        }
    st(out, pix, d, acc / 9.0f);
}

// ---- convex upsample: shaders/convex.wgsl:12-34; one lane per output pixel, all channels ------------------------
__global__ __launch_bounds__(kThreads) void convex_kernel(View wt, View x, OView out, uint32_t h, uint32_t w,
                                                          uint32_t c, uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t ow = 2 * w, oh = 2 * h;
    const uint32_t ox = t % ow, row = t / ow, oy = row % oh, img = row / oh;
    const uint32_t ih = oy / 2, iw = ox / 2, sub = (oy % 2) * 2 + ox % 2;
    const size_t ipix = ((size_t)img * h + ih) * w + iw;
    float m = -3.0e38f, ws[9];
#pragma unroll
    for (uint32_t k = 0; k < 9; k++) {
        ws[k] = ld(wt, ipix, k * 4 + sub);
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
    for (uint32_t co = 0; co < c; co++) {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < 9; k++) {
            const int ny = (int)ih - 1 + (int)(k / 3), nx = (int)iw - 1 + (int)(k % 3);
            const bool in = ny >= 0 && ny < (int)h && nx >= 0 && nx < (int)w;
            const float xv = in ? ld(x, ((size_t)img * h + ny) * w + nx, co) : 0.0f;
            acc = acc + ws[k] * xv;
        }
        st(out, t, co, acc);
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
template <bool VEC>
__global__ __launch_bounds__(kThreads) void avgpool_kernel(View x, OView out, uint32_t h, uint32_t w, uint32_t oh,
                                                           uint32_t ow, uint32_t c, uint32_t k, uint32_t groups,
                                                           uint32_t items) {
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= items) return;
    const uint32_t opix = t / groups, ch = (t - opix * groups) * 4;
    const uint32_t ox = opix % ow, row = opix / ow, oy = row % oh, img = row / oh;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, v[4];
    for (uint32_t ky = 0; ky < k; ky++)
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
        return launch("convex_upsample", (uint64_t)n * 4 * h * w, [&](dim3 g, uint32_t items) {
            hipLaunchKernelGGL(convex_kernel, g, dim3(kThreads), 0, (hipStream_t)stream, in(wt), in(x), outv(out), h,
                               w, c, items);
        });
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
            auto kern = v ? avgpool_kernel<true> : avgpool_kernel<false>;
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
        const bool v = vec4(c, {x, out});
        return launch("interpolate", (uint64_t)n * oh * ow * groups, [&](dim3 g, uint32_t items) {
            auto k = antialias ? (v ? interp_kernel<true, true> : interp_kernel<false, true>)
                               : (v ? interp_kernel<true, false> : interp_kernel<false, false>);
            hipLaunchKernelGGL(k, g, dim3(kThreads), 0, (hipStream_t)stream, in(x), outv(out), ih, iw, oh, ow, c,
                               groups, items);
        });
    });
}
