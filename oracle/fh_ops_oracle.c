/* CPU oracle of the FlyHighFG network ops: TEST INFRASTRUCTURE ONLY (see fh_ops_oracle.h).
 * Each function follows its WGSL kernel's arithmetic in f32, in the kernel's order; f16 rounding is
 * round-to-nearest-even (fho_f32_to_f16). Built with -ffp-contract=off so no product is fused into a sum. */
#include "fh_ops_oracle.h"

#include <math.h>
#include <stddef.h>

#include "fh_oracle.h"

static float rd(const fho_view* v, uint32_t h, uint32_t w, uint32_t img, int y, int x, uint32_t ch) {
    const uint16_t* p = (const uint16_t*)v->p;
    return fho_f16_to_f32(p[(((size_t)img * h + (size_t)y) * w + (size_t)x) * v->cs + v->c0 + ch]);
}

static void wr(const fho_view* v, uint32_t h, uint32_t w, uint32_t img, uint32_t y, uint32_t x, uint32_t ch,
               float val) {
    uint16_t* p = (uint16_t*)v->p;
    p[(((size_t)img * h + y) * w + x) * v->cs + v->c0 + ch] = fho_f32_to_f16(val);
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* shaders/warp.wgsl:14-28 */
void fho_warp(const fho_view* img, const fho_view* flow, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
              uint32_t c) {
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t x = 0; x < w; x++) {
                const float fx = rd(flow, h, w, b, (int)y, (int)x, 0) * flow->scale;
                const float fy = rd(flow, h, w, b, (int)y, (int)x, 1) * flow->scale;
                const float gx = (float)x + fx, gy = (float)y + fy;
                const int x0 = (int)floorf(gx), y0 = (int)floorf(gy);
                const float ax = gx - (float)x0, ay = gy - (float)y0;
                const int x0c = clampi(x0, 0, (int)w - 1), x1c = clampi(x0 + 1, 0, (int)w - 1);
                const int y0c = clampi(y0, 0, (int)h - 1), y1c = clampi(y0 + 1, 0, (int)h - 1);
                for (uint32_t ch = 0; ch < c; ch++) {
                    const float v00 = rd(img, h, w, b, y0c, x0c, ch), v01 = rd(img, h, w, b, y0c, x1c, ch);
                    const float v10 = rd(img, h, w, b, y1c, x0c, ch), v11 = rd(img, h, w, b, y1c, x1c, ch);
                    const float top = v00 * (1.0f - ax) + v01 * ax, bot = v10 * (1.0f - ax) + v11 * ax;
                    wr(out, h, w, b, y, x, ch, (top * (1.0f - ay) + bot * ay) * img->scale);
                }
            }
}

/* shaders/luma.wgsl:9-12 (channel 2 is R, 1 G, 0 B) */
static float lum(const fho_view* x, uint32_t h, uint32_t w, uint32_t b, int yy, int xx) {
    return (0.299f * rd(x, h, w, b, yy, xx, 2) + 0.587f * rd(x, h, w, b, yy, xx, 1) +
            0.114f * rd(x, h, w, b, yy, xx, 0)) *
           x->scale;
}

/* shaders/luma.wgsl:14-28 */
void fho_luma(const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w, int grad) {
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t xx = 0; xx < w; xx++) {
                const float c = lum(x, h, w, b, (int)y, (int)xx);
                if (!grad) {
                    wr(out, h, w, b, y, xx, 0, c);
                    continue;
                }
                const float gx = xx + 1 < w ? lum(x, h, w, b, (int)y, (int)xx + 1) - c : 0.0f;
                const float gy = y + 1 < h ? lum(x, h, w, b, (int)y + 1, (int)xx) - c : 0.0f;
                wr(out, h, w, b, y, xx, 0, fabsf(gx) + fabsf(gy));
            }
}

/* shaders/sad.wgsl:12-28 */
void fho_sad(const fho_view* la, const fho_view* lb, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
             uint32_t r) {
    const uint32_t span = 2 * r + 1;
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t x = 0; x < w; x++)
                for (uint32_t c = 0; c < span * span; c++) {
                    const int dy = (int)(c / span) - (int)r, dx = (int)(c % span) - (int)r;
                    float acc = 0.0f;
                    for (int wy = -1; wy <= 1; wy++)
                        for (int wx = -1; wx <= 1; wx++) {
                            const int yy = (int)y + wy, xx = (int)x + wx;
                            if (yy >= 0 && yy < (int)h && xx >= 0 && xx < (int)w) {
                                const float lav = rd(la, h, w, b, yy, xx, 0);
                                const int syy = clampi(yy + dy, 0, (int)h - 1), sxx = clampi(xx + dx, 0, (int)w - 1);
                                acc = acc + fabsf(lav - rd(lb, h, w, b, syy, sxx, 0));
                            }
                        }
                    wr(out, h, w, b, y, x, c, acc / 9.0f);
                }
}

/* shaders/convex.wgsl:12-34 */
void fho_convex(const fho_view* wt, const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
                uint32_t c) {
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t oy = 0; oy < 2 * h; oy++)
            for (uint32_t ox = 0; ox < 2 * w; ox++) {
                const uint32_t ih = oy / 2, iw = ox / 2, sy = oy % 2, sx = ox % 2;
                float m = -3.0e38f, ws[9];
                for (uint32_t k = 0; k < 9; k++) {
                    ws[k] = rd(wt, h, w, b, (int)ih, (int)iw, k * 4 + sy * 2 + sx);
                    m = fmaxf(m, ws[k]);
                }
                float denom = 0.0f;
                for (uint32_t k = 0; k < 9; k++) {
                    ws[k] = expf(ws[k] - m);
                    denom = denom + ws[k];
                }
                for (uint32_t co = 0; co < c; co++) {
                    float acc = 0.0f;
                    for (uint32_t k = 0; k < 9; k++) {
                        const int ny = (int)ih - 1 + (int)(k / 3), nx = (int)iw - 1 + (int)(k % 3);
                        const float xv =
                            (ny >= 0 && ny < (int)h && nx >= 0 && nx < (int)w) ? rd(x, h, w, b, ny, nx, co) : 0.0f;
                        acc = acc + (ws[k] / denom) * xv;
                    }
                    wr(out, 2 * h, 2 * w, b, oy, ox, co, acc);
                }
            }
}

/* shaders/film.wgsl:11-14 */
void fho_film(const fho_view* hv, const uint16_t* g, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
              uint32_t c) {
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t x = 0; x < w; x++)
                for (uint32_t ch = 0; ch < c; ch++) {
                    const float sc = fho_f16_to_f32(g[(size_t)b * 2 * c + ch]);
                    const float bi = fho_f16_to_f32(g[(size_t)b * 2 * c + c + ch]);
                    wr(out, h, w, b, y, x, ch, rd(hv, h, w, b, (int)y, (int)x, ch) * (1.0f + sc) + bi);
                }
}

/* the softmax of the three visibility logits: shaders/blend.wgsl:15-19, blendmix.wgsl:18-21 */
static void soft3(const fho_view* vis, uint32_t h, uint32_t w, uint32_t b, uint32_t y, uint32_t x, float* ea,
                  float* eb, float* ec, float* s) {
    const float a = rd(vis, h, w, b, (int)y, (int)x, 0) * vis->scale;
    const float bb = rd(vis, h, w, b, (int)y, (int)x, 1) * vis->scale;
    const float c = rd(vis, h, w, b, (int)y, (int)x, 2) * vis->scale;
    const float m = fmaxf(a, fmaxf(bb, c));
    *ea = expf(a - m);
    *eb = expf(bb - m);
    *ec = expf(c - m);
    *s = *ea + *eb + *ec;
}

/* shaders/blend.wgsl:11-20 */
void fho_blend(const fho_view* vis, const fho_view* out, uint32_t n, uint32_t h, uint32_t w) {
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t x = 0; x < w; x++) {
                float ea, eb, ec, s;
                soft3(vis, h, w, b, y, x, &ea, &eb, &ec, &s);
                const float p0 = ea / s, p1 = eb / s, p2 = ec / s;
                wr(out, h, w, b, y, x, 0, p0 + 0.5f * p2);
                wr(out, h, w, b, y, x, 1, p1 + 0.5f * p2);
            }
}

/* shaders/blendmix.wgsl:14-27 */
void fho_blendmix(const fho_view* wa, const fho_view* wb, const fho_view* vis, const fho_view* out, uint32_t n,
                  uint32_t h, uint32_t w) {
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t x = 0; x < w; x++) {
                float ea, eb, ec, s;
                soft3(vis, h, w, b, y, x, &ea, &eb, &ec, &s);
                const float pa = fho_f16_to_f32(fho_f32_to_f16((ea + 0.5f * ec) / s));
                const float pb = fho_f16_to_f32(fho_f32_to_f16((eb + 0.5f * ec) / s));
                for (uint32_t ch = 0; ch < 3; ch++) {
                    const float t1 = fho_f16_to_f32(fho_f32_to_f16(rd(wa, h, w, b, (int)y, (int)x, ch) * pa));
                    const float t2 = fho_f16_to_f32(fho_f32_to_f16(rd(wb, h, w, b, (int)y, (int)x, ch) * pb));
                    wr(out, h, w, b, y, x, ch, t1 + t2);
                }
            }
}

/* shaders/avgpool.wgsl:10-18 */
void fho_avgpool(const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c, uint32_t k) {
    const uint32_t oh = h / k, ow = w / k;
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t oy = 0; oy < oh; oy++)
            for (uint32_t ox = 0; ox < ow; ox++)
                for (uint32_t ch = 0; ch < c; ch++) {
                    float acc = 0.0f;
                    for (uint32_t ky = 0; ky < k; ky++)
                        for (uint32_t kx = 0; kx < k; kx++)
                            acc = acc + rd(x, h, w, b, (int)(oy * k + ky), (int)(ox * k + kx), ch);
                    wr(out, oh, ow, b, oy, ox, ch, acc / (float)(k * k));
                }
}

/* shaders/interp.wgsl:13-44 */
void fho_interp(const fho_view* x, const fho_view* out, uint32_t n, uint32_t c, uint32_t ih, uint32_t iw,
                uint32_t oh, uint32_t ow, int aa) {
    const float sh = (float)ih / (float)oh, sw = (float)iw / (float)ow;
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t oy = 0; oy < oh; oy++)
            for (uint32_t ox = 0; ox < ow; ox++)
                for (uint32_t ch = 0; ch < c; ch++) {
                    float val;
                    if (!aa) {
                        const float iy = ((float)oy + 0.5f) * sh - 0.5f, ix = ((float)ox + 0.5f) * sw - 0.5f;
                        const int y0 = (int)floorf(iy), x0 = (int)floorf(ix);
                        const float fy = iy - (float)y0, fx = ix - (float)x0;
                        const int y0c = clampi(y0, 0, (int)ih - 1), y1c = clampi(y0 + 1, 0, (int)ih - 1);
                        const int x0c = clampi(x0, 0, (int)iw - 1), x1c = clampi(x0 + 1, 0, (int)iw - 1);
                        const float v00 = rd(x, ih, iw, b, y0c, x0c, ch), v01 = rd(x, ih, iw, b, y0c, x1c, ch);
                        const float v10 = rd(x, ih, iw, b, y1c, x0c, ch), v11 = rd(x, ih, iw, b, y1c, x1c, ch);
                        val = (v00 * (1.0f - fx) + v01 * fx) * (1.0f - fy) + (v10 * (1.0f - fx) + v11 * fx) * fy;
                    } else {
                        const float fsh = fmaxf(sh, 1.0f), fsw = fmaxf(sw, 1.0f);
                        const float cy = ((float)oy + 0.5f) * sh, cx = ((float)ox + 0.5f) * sw;
                        int ymin = (int)floorf(cy - fsh + 0.5f), ymax = (int)floorf(cy + fsh + 0.5f);
                        int xmin = (int)floorf(cx - fsw + 0.5f), xmax = (int)floorf(cx + fsw + 0.5f);
                        ymin = ymin < 0 ? 0 : ymin;
                        xmin = xmin < 0 ? 0 : xmin;
                        ymax = ymax > (int)ih ? (int)ih : ymax;
                        xmax = xmax > (int)iw ? (int)iw : xmax;
                        float acc = 0.0f, norm = 0.0f;
                        for (int y = ymin; y < ymax; y++) {
                            const float wy = fmaxf(0.0f, 1.0f - fabsf(((float)y + 0.5f - cy) / fsh));
                            for (int xx = xmin; xx < xmax; xx++) {
                                const float wx = fmaxf(0.0f, 1.0f - fabsf(((float)xx + 0.5f - cx) / fsw));
                                const float wgt = wx * wy;
                                acc = acc + rd(x, ih, iw, b, y, xx, ch) * wgt;
                                norm = norm + wgt;
                            }
                        }
                        val = acc / norm;
                    }
                    wr(out, oh, ow, b, oy, ox, ch, val * x->scale);
                }
}

/* shaders/binary.wgsl:11-16 */
void fho_binary(const fho_view* a, const fho_view* b, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
                uint32_t c, uint32_t cb, int op) {
    for (uint32_t i = 0; i < n; i++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t x = 0; x < w; x++)
                for (uint32_t ch = 0; ch < c; ch++) {
                    const float av = rd(a, h, w, i, (int)y, (int)x, ch) * a->scale;
                    const float bv = rd(b, h, w, i, (int)y, (int)x, cb == 1 ? 0 : ch) * b->scale;
                    wr(out, h, w, i, y, x, ch, op == 1 ? av * bv : av + bv);
                }
}

/* shaders/unary.wgsl:11-19 */
void fho_unary(const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int op,
               float a, float b) {
    for (uint32_t i = 0; i < n; i++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t xx = 0; xx < w; xx++)
                for (uint32_t ch = 0; ch < c; ch++) {
                    const float v = rd(x, h, w, i, (int)y, (int)xx, ch) * x->scale;
                    float r;
                    if (op == 0) r = v * a;
                    else if (op == 1) r = fminf(fmaxf(v, a), b);
                    else if (op == 2) r = 2.0f / (1.0f + expf(-v)) - 1.0f;
                    else r = -v;
                    wr(out, h, w, i, y, xx, ch, r);
                }
}

/* shaders/chcopy.wgsl:19-22 (scl) for one input */
void fho_chcopy(const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c) {
    const uint16_t* src = (const uint16_t*)x->p;
    uint16_t* dst = (uint16_t*)out->p;
    for (size_t pix = 0; pix < (size_t)n * h * w; pix++)
        for (uint32_t ch = 0; ch < c; ch++) {
            const uint16_t v = src[pix * x->cs + x->c0 + ch];
            dst[pix * out->cs + out->c0 + ch] =
                x->scale == 1.0f ? v : fho_f32_to_f16(fho_f16_to_f32(v) * x->scale);
        }
}

/* ---- render_pix: shaders/render.wgsl ---------------------------------------------------------------------- */

/* bil4 (render.wgsl:29-31) */
static float bil4(float v00, float v01, float v10, float v11, float fx, float fy) {
    return (v00 * (1.0f - fx) + v01 * fx) * (1.0f - fy) + (v10 * (1.0f - fx) + v11 * fx) * fy;
}
/* Keys cubic convolution, a = -0.75 (render.wgsl:50-53): (a + 2) = 1.25, (a + 3) = 2.25, 5a = -3.75, 8a = -6,
 * 4a = -3, in the shader's order */
static float cub1(float x) { return ((1.25f * x - 2.25f) * x) * x + 1.0f; }
static float cub2(float x) { return ((-0.75f * x - -3.75f) * x + -6.0f) * x - -3.0f; }
static float rpx(const fho_view* v, uint32_t h, uint32_t w, int y, int x, uint32_t ch) {
    return rd(v, h, w, 0, clampi(y, 0, (int)h - 1), clampi(x, 0, (int)w - 1), ch);
}
/* one bicubic sample (render.wgsl:54-81) */
static float cubic_at(const fho_view* v, uint32_t h, uint32_t w, uint32_t ch, float gx, float gy) {
    const int px = (int)floorf(gx), py = (int)floorf(gy);
    const float tx = gx - (float)px, ty = gy - (float)py;
    const float cx[4] = {cub2(tx + 1.0f), cub1(tx), cub1(1.0f - tx), cub2(2.0f - tx)};
    const float cy[4] = {cub2(ty + 1.0f), cub1(ty), cub1(1.0f - ty), cub2(2.0f - ty)};
    float acc = 0.0f;
    for (int j = 0; j < 4; j++) {
        const int yy = py - 1 + j;
        const float row = rpx(v, h, w, yy, px - 1, ch) * cx[0] + rpx(v, h, w, yy, px, ch) * cx[1] +
                          rpx(v, h, w, yy, px + 1, ch) * cx[2] + rpx(v, h, w, yy, px + 2, ch) * cx[3];
        acc = j == 0 ? row * cy[0] : acc + row * cy[j];
    }
    return acc;
}
/* one bilinear sample with clamped corners (render.wgsl:43-48, 105-114) */
static float bil_at(const fho_view* v, uint32_t h, uint32_t w, uint32_t ch, float gx, float gy) {
    const int x0 = (int)floorf(gx), y0 = (int)floorf(gy);
    const float ax = gx - (float)x0, ay = gy - (float)y0;
    return bil4(rpx(v, h, w, y0, x0, ch), rpx(v, h, w, y0, x0 + 1, ch), rpx(v, h, w, y0 + 1, x0, ch),
                rpx(v, h, w, y0 + 1, x0 + 1, ch), ax, ay);
}
static float clampf01(float v) { return fminf(fmaxf(v, 0.0f), 1.0f); }

/* rows y0 .. y1 - 1 of the render; every output pixel is independent of the others */
void fho_render_rows(const fho_view* a, const fho_view* b, const fho_view* flow, const fho_view* vis,
                     const fho_view* rt, const fho_view* out, uint32_t h, uint32_t w, uint32_t hq, uint32_t wq,
                     float fsx, float fsy, int cubic, uint32_t flags, uint32_t y0_, uint32_t y1_) {
    const float sh = (float)hq / (float)h, sw = (float)wq / (float)w;
    for (uint32_t y = y0_; y < y1_ && y < h; y++)
        for (uint32_t x = 0; x < w; x++) {
            const float iy = ((float)y + 0.5f) * sh - 0.5f, ix = ((float)x + 0.5f) * sw - 0.5f;
            const int qy0 = (int)floorf(iy), qx0 = (int)floorf(ix);
            const float qfy = iy - (float)qy0, qfx = ix - (float)qx0;
            const int y0 = clampi(qy0, 0, (int)hq - 1), y1 = clampi(qy0 + 1, 0, (int)hq - 1);
            const int x0 = clampi(qx0, 0, (int)wq - 1), x1 = clampi(qx0 + 1, 0, (int)wq - 1);
            float f[4], v[3], r[3];
            for (uint32_t c = 0; c < 4; c++)
                f[c] = bil4(rd(flow, hq, wq, 0, y0, x0, c), rd(flow, hq, wq, 0, y0, x1, c), rd(flow, hq, wq, 0, y1, x0, c),
                            rd(flow, hq, wq, 0, y1, x1, c), qfx, qfy) *
                       ((c & 1u) == 0 ? fsx : fsy);
            for (uint32_t c = 0; c < 3; c++) {
                v[c] = bil4(rd(vis, hq, wq, 0, y0, x0, c), rd(vis, hq, wq, 0, y0, x1, c), rd(vis, hq, wq, 0, y1, x0, c),
                            rd(vis, hq, wq, 0, y1, x1, c), qfx, qfy) *
                       vis->scale;
                r[c] = bil4(rd(rt, hq, wq, 0, y0, x0, c), rd(rt, hq, wq, 0, y0, x1, c), rd(rt, hq, wq, 0, y1, x0, c),
                            rd(rt, hq, wq, 0, y1, x1, c), qfx, qfy);
            }
            const float m = fmaxf(v[0], fmaxf(v[1], v[2]));
            const float e0 = expf(v[0] - m), e1 = expf(v[1] - m), e2 = expf(v[2] - m), s = e0 + e1 + e2;
            const float wa_w = (e0 + 0.5f * e2) / s, wb_w = (e1 + 0.5f * e2) / s;
            const float gxa = (float)x + f[0], gya = (float)y + f[1], gxb = (float)x + f[2], gyb = (float)y + f[3];
            float ca[3], cb[3];
            for (uint32_t c = 0; c < 3; c++) {
                ca[c] = cubic ? cubic_at(a, h, w, c, gxa, gya) : bil_at(a, h, w, c, gxa, gya);
                cb[c] = cubic ? cubic_at(b, h, w, c, gxb, gyb) : bil_at(b, h, w, c, gxb, gyb);
            }
            float bwa = wa_w, bwb = wb_w, rk = 1.0f, stillw = 0.0f, own[3] = {0.0f, 0.0f, 0.0f};
            const float third = 1.0f / 3.0f;
            const float ef = fabsf(ca[0] - cb[0]) * third + fabsf(ca[1] - cb[1]) * third + fabsf(ca[2] - cb[2]) * third;
            if (flags & 2u) { /* render.wgsl:134-148 */
                float es = 0.0f;
                for (int dy = -1; dy <= 1; dy++)
                    for (int dx = -1; dx <= 1; dx++)
                        for (uint32_t c = 0; c < 3; c++)
                            es += fabsf(rpx(a, h, w, (int)y + dy, (int)x + dx, c) - rpx(b, h, w, (int)y + dy, (int)x + dx, c));
                es = es / 27.0f;
                for (uint32_t c = 0; c < 3; c++)
                    own[c] = 0.5f * (rd(a, h, w, 0, (int)y, (int)x, c) + rd(b, h, w, 0, (int)y, (int)x, c));
                stillw = fminf(fmaxf((ef - es) / 0.04f, 0.0f), 1.0f) * (es < 0.03f ? 1.0f : 0.0f);
            }
            if (flags & 1u) { /* render.wgsl:149-153 */
                const float k = fminf(fmaxf((ef - 0.04f) / 0.08f, 0.0f), 1.0f);
                const float pa = wa_w >= wb_w ? 1.0f : 0.0f;
                bwa = wa_w * (1.0f - k) + pa * k;
                bwb = wb_w * (1.0f - k) + (1.0f - pa) * k;
                rk = 1.0f - k;
            }
            for (uint32_t c = 0; c < 3; c++) {
                const float mixed = ca[c] * bwa + cb[c] * bwb + r[c] * rk;
                wr(out, h, w, 0, y, x, c, clampf01(mixed * (1.0f - stillw) + own[c] * stillw));
            }
        }
}

void fho_render(const fho_view* a, const fho_view* b, const fho_view* flow, const fho_view* vis, const fho_view* rt,
                const fho_view* out, uint32_t h, uint32_t w, uint32_t hq, uint32_t wq, float fsx, float fsy,
                int cubic, uint32_t flags) {
    fho_render_rows(a, b, flow, vis, rt, out, h, w, hq, wq, fsx, fsy, cubic, flags, 0, h);
}

/* shaders/rgba_in.wgsl:11-19 (the planar output [3][hp][wp] written as channels 0-2 of an NHWC view) */
void fho_rgba_in(const uint32_t* rgba, uint32_t n, uint32_t w, uint32_t h, uint32_t pitch, uint64_t fstride,
                 const fho_view* out, uint32_t hp, uint32_t wp) {
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t y = 0; y < hp; y++)
            for (uint32_t x = 0; x < wp; x++) {
                const uint32_t v = rgba[b * fstride + (size_t)(y < h ? y : h - 1) * pitch + (x < w ? x : w - 1)];
                wr(out, hp, wp, b, y, x, 0, (float)((v >> 16) & 0xffu) / 255.0f);
                wr(out, hp, wp, b, y, x, 1, (float)((v >> 8) & 0xffu) / 255.0f);
                wr(out, hp, wp, b, y, x, 2, (float)(v & 0xffu) / 255.0f);
            }
}

/* rgba_out.wgsl:10: q(v) = u32(clamp(f32(v), 0, 1) * 255 + 0.5) */
static uint32_t q8(float v) { return (uint32_t)(fminf(fmaxf(v, 0.0f), 1.0f) * 255.0f + 0.5f); }

/* shaders/rgba_out.wgsl:12-18 (channels 0-2 of an NHWC view of hp x wp, cropped to w x h) */
void fho_rgba_out(const fho_view* in, uint32_t n, uint32_t hp, uint32_t wp, uint32_t* rgba, uint32_t w, uint32_t h,
                  uint32_t pitch, uint64_t fstride) {
    for (uint32_t b = 0; b < n; b++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t x = 0; x < w; x++)
                rgba[b * fstride + (size_t)y * pitch + x] = q8(rd(in, hp, wp, b, (int)y, (int)x, 2)) |
                                                            (q8(rd(in, hp, wp, b, (int)y, (int)x, 1)) << 8) |
                                                            (q8(rd(in, hp, wp, b, (int)y, (int)x, 0)) << 16) |
                                                            0xff000000u;
}

/* ---- GMHS: the periodic-structure repair of the pair's E8 flow (crates/flyhigh-engine/src/gmhs.rs) ------------ */

#define GM_NWG 32u  /* gm_fit_reduce's workgroups (gmhs.rs:160) */
#define GM_WG 256u  /* its workgroup size (gm_fit_reduce.wgsl:13) */

/* gmhs.rs:149-160, :195 (DS = 2, gmhs.rs:129; eps 0, tex 0.015) */
void fho_gm_params(uint32_t h, uint32_t w, uint32_t full_w, uint32_t level, fho_gm_par* p) {
    p->hc = (h + 1) / 2;
    p->wc = (w + 1) / 2;
    const float s = (float)w / ((float)full_w / 2.0f);
    const float rb = roundf(20.0f * s / 2.0f), rw = roundf(32.0f * s / 2.0f);
    p->s = s;
    p->r_blk = rb < 1.0f ? 1u : (uint32_t)rb;
    p->r_dwin = rw < 1.0f ? 1u : (uint32_t)rw;
    p->dmin = level >= 2 ? 0.0f : 8.0f * s;
    p->delta = 1.5f * s;
    p->eps = 0.0f;
    p->tex = 0.015f;
}

/* gm_fit_reduce.wgsl:15-44: GM_NWG workgroups of GM_WG lanes; lane t of workgroup g sums the elements g * 256 + t +
 * k * 8192 in order, then the workgroup adds its lanes pairwise (t, t + off) for off = 128 .. 1 */
static void gm_fit_reduce(const fho_view* flow, uint32_t h8, uint32_t w8, const float* coef, int use_w, float delta,
                          float* part) {
    const uint32_t n = h8 * w8, stride = GM_WG * GM_NWG;
    const float sx = 2.0f / (float)(w8 - 1 > 1 ? w8 - 1 : 1), sy = 2.0f / (float)(h8 - 1 > 1 ? h8 - 1 : 1);
    float sh[9][GM_WG];
    for (uint32_t g = 0; g < GM_NWG; g++)
        for (uint32_t c = 0; c < 4; c++) {
            for (uint32_t t = 0; t < GM_WG; t++) {
                float s[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
                for (uint32_t i = g * GM_WG + t; i < n; i += stride) {
                    const uint32_t yy = i / w8, xx = i - yy * w8;
                    const float x = -1.0f + sx * (float)xx, y = -1.0f + sy * (float)yy;
                    const float f = rd(flow, h8, w8, 0, (int)yy, (int)xx, c);
                    float w2 = 1.0f;
                    if (use_w) {
                        const float r = fabsf(f - (coef[c * 4] + coef[c * 4 + 1] * x + coef[c * 4 + 2] * y));
                        w2 = delta / fmaxf(delta, r);
                    }
                    s[0] = s[0] + w2, s[1] = s[1] + w2 * x, s[2] = s[2] + w2 * y;
                    s[3] = s[3] + w2 * x * x, s[4] = s[4] + w2 * x * y, s[5] = s[5] + w2 * y * y;
                    s[6] = s[6] + w2 * f, s[7] = s[7] + w2 * x * f, s[8] = s[8] + w2 * y * f;
                }
                for (uint32_t k = 0; k < 9; k++) sh[k][t] = s[k];
            }
            for (uint32_t off = GM_WG / 2; off > 0; off >>= 1)
                for (uint32_t t = 0; t < off; t++)
                    for (uint32_t k = 0; k < 9; k++) sh[k][t] = sh[k][t] + sh[k][t + off];
            for (uint32_t k = 0; k < 9; k++) part[(g * 4 + c) * 9 + k] = sh[k][0];
        }
}

/* gm_fit_solve.wgsl:8-25: the partials summed in workgroup order, the 3 x 3 normal equations inverted by cofactors */
static void gm_fit_solve(const float* part, float* coef) {
    for (uint32_t c = 0; c < 4; c++) {
        float s[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t g = 0; g < GM_NWG; g++)
            for (uint32_t k = 0; k < 9; k++) s[k] = s[k] + part[(g * 4 + c) * 9 + k];
        const float m00 = s[0] + 1e-6f, m01 = s[1], m02 = s[2], m11 = s[3] + 1e-6f, m12 = s[4], m22 = s[5] + 1e-6f;
        const float det = m00 * (m11 * m22 - m12 * m12) - m01 * (m01 * m22 - m12 * m02) + m02 * (m01 * m12 - m11 * m02);
        float* o = coef + c * 4;
        if (fabsf(det) < 1e-12f) {
            o[0] = s[6] / fmaxf(s[0], 1e-6f), o[1] = 0.0f, o[2] = 0.0f, o[3] = 0.0f;
            continue;
        }
        const float i00 = (m11 * m22 - m12 * m12) / det, i01 = (m02 * m12 - m01 * m22) / det;
        const float i02 = (m01 * m12 - m02 * m11) / det, i11 = (m00 * m22 - m02 * m02) / det;
        const float i12 = (m01 * m02 - m00 * m12) / det, i22 = (m00 * m11 - m01 * m01) / det;
        o[0] = i00 * s[6] + i01 * s[7] + i02 * s[8];
        o[1] = i01 * s[6] + i11 * s[7] + i12 * s[8];
        o[2] = i02 * s[6] + i12 * s[7] + i22 * s[8];
        o[3] = 0.0f;
    }
}

/* the fit of gmhs.rs:161-171: `iters` rounds of reduce + solve, the first unweighted */
void fho_gm_fit(const fho_view* flow, uint32_t h8, uint32_t w8, float delta, uint32_t iters, float* coef) {
    float part[GM_NWG * 4 * 9];
    for (uint32_t k = 0; k < 16; k++) coef[k] = 0.0f;
    for (uint32_t it = 0; it < iters; it++) {
        gm_fit_reduce(flow, h8, w8, coef, it > 0, delta, part);
        gm_fit_solve(part, coef);
    }
}

/* gm_cost.wgsl:14-17: luma of a BGR view, no read scale */
static float gm_lum(const fho_view* v, uint32_t h, uint32_t w, int y, int x) {
    return 0.299f * rd(v, h, w, 0, y, x, 2) + 0.587f * rd(v, h, w, 0, y, x, 1) + 0.114f * rd(v, h, w, 0, y, x, 0);
}

/* gm_cost.wgsl:23-29: bilinear luma, coordinates clamped */
static float gm_samp(const fho_view* v, uint32_t h, uint32_t w, float gx, float gy) {
    const int x0 = (int)floorf(gx), y0 = (int)floorf(gy);
    const float ax = gx - (float)x0, ay = gy - (float)y0;
    const int x0c = clampi(x0, 0, (int)w - 1), x1c = clampi(x0 + 1, 0, (int)w - 1);
    const int y0c = clampi(y0, 0, (int)h - 1), y1c = clampi(y0 + 1, 0, (int)h - 1);
    const float top = gm_lum(v, h, w, y0c, x0c) * (1.0f - ax) + gm_lum(v, h, w, y0c, x1c) * ax;
    const float bot = gm_lum(v, h, w, y1c, x0c) * (1.0f - ax) + gm_lum(v, h, w, y1c, x1c) * ax;
    return top * (1.0f - ay) + bot * ay;
}

/* gm_cost.wgsl:38-48: the E8 flow at a network position, bilinear, align_corners false */
static float gm_flow8(const fho_view* fl, uint32_t h8, uint32_t w8, uint32_t h, uint32_t w, uint32_t c, float rx,
                      float ry) {
    const float ix = (rx + 0.5f) * (float)w8 / (float)w - 0.5f, iy = (ry + 0.5f) * (float)h8 / (float)h - 0.5f;
    const int x0 = (int)floorf(ix), y0 = (int)floorf(iy);
    const float fx = ix - (float)x0, fy = iy - (float)y0;
    const int x0c = clampi(x0, 0, (int)w8 - 1), x1c = clampi(x0 + 1, 0, (int)w8 - 1);
    const int y0c = clampi(y0, 0, (int)h8 - 1), y1c = clampi(y0 + 1, 0, (int)h8 - 1);
    const float top = rd(fl, h8, w8, 0, y0c, x0c, c) * (1.0f - fx) + rd(fl, h8, w8, 0, y0c, x1c, c) * fx;
    const float bot = rd(fl, h8, w8, 0, y1c, x0c, c) * (1.0f - fx) + rd(fl, h8, w8, 0, y1c, x1c, c) * fx;
    return top * (1.0f - fy) + bot * fy;
}

/* gm_cost.wgsl:49-53: the affine hypothesis at a network position */
static float gm_aff(const float* coef, uint32_t c, uint32_t h8, uint32_t w8, uint32_t h, uint32_t w, float rx,
                    float ry) {
    const float ix = (rx + 0.5f) * (float)w8 / (float)w - 0.5f, iy = (ry + 0.5f) * (float)h8 / (float)h - 0.5f;
    const float xn = -1.0f + 2.0f * ix / (float)(w8 - 1 > 1 ? w8 - 1 : 1);
    const float yn = -1.0f + 2.0f * iy / (float)(h8 - 1 > 1 ? h8 - 1 : 1);
    return coef[c * 4] + coef[c * 4 + 1] * xn + coef[c * 4 + 2] * yn;
}

/* gm_cost.wgsl:55-75, channels 0-4 (channel 5, the plain frame change, feeds cadence smoothing only) */
void fho_gm_cost(const fho_view* a, const fho_view* b, uint32_t h, uint32_t w, const fho_view* flow, uint32_t h8,
                 uint32_t w8, const float* coef, uint32_t hc, uint32_t wc, float* maps) {
    const size_t n = (size_t)hc * wc;
    const float ds = 2.0f;
    for (uint32_t y = 0; y < hc; y++)
        for (uint32_t x = 0; x < wc; x++) {
            const size_t i = (size_t)y * wc + x;
            const float rx = ((float)x + 0.5f) * ds - 0.5f, ry = ((float)y + 0.5f) * ds - 0.5f;
            const float f0x = gm_flow8(flow, h8, w8, h, w, 0, rx, ry), f0y = gm_flow8(flow, h8, w8, h, w, 1, rx, ry);
            const float f1x = gm_flow8(flow, h8, w8, h, w, 2, rx, ry), f1y = gm_flow8(flow, h8, w8, h, w, 3, rx, ry);
            const float cm = fabsf(gm_samp(a, h, w, rx + f0x, ry + f0y) - gm_samp(b, h, w, rx + f1x, ry + f1y));
            const float g0x = gm_aff(coef, 0, h8, w8, h, w, rx, ry), g0y = gm_aff(coef, 1, h8, w8, h, w, rx, ry);
            const float g1x = gm_aff(coef, 2, h8, w8, h, w, rx, ry), g1y = gm_aff(coef, 3, h8, w8, h, w, rx, ry);
            const float wm = (float)w - 1.0f, hm = (float)h - 1.0f;
            const float ax = rx + g0x, ay = ry + g0y, bx = rx + g1x, by = ry + g1y;
            const int inside = ax >= 0.0f && ax <= wm && ay >= 0.0f && ay <= hm && bx >= 0.0f && bx <= wm &&
                               by >= 0.0f && by <= hm;
            const float ca = inside ? fabsf(gm_samp(a, h, w, ax, ay) - gm_samp(b, h, w, bx, by)) : cm;
            const float l = gm_samp(a, h, w, rx, ry);
            const float dvx = (g1x - g0x) - (f1x - f0x), dvy = (g1y - g0y) - (f1y - f0y);
            maps[i] = cm, maps[n + i] = ca, maps[2 * n + i] = sqrtf(dvx * dvx + dvy * dvy);
            maps[3 * n + i] = l, maps[4 * n + i] = l * l;
        }
}

/* gm_box.wgsl:8-25: box mean of radius r along x (vert 0) or y, edges replicated, over c planes [c][h][w] */
void fho_gm_box(const float* src, float* dst, uint32_t c, uint32_t h, uint32_t w, uint32_t r, int vert) {
    for (uint32_t ch = 0; ch < c; ch++)
        for (uint32_t y = 0; y < h; y++)
            for (uint32_t x = 0; x < w; x++) {
                const size_t plane = (size_t)ch * h * w;
                float acc = 0.0f;
                for (int d = -(int)r; d <= (int)r; d++) {
                    const size_t at = vert ? (size_t)clampi((int)y + d, 0, (int)h - 1) * w + x
                                           : (size_t)y * w + (size_t)clampi((int)x + d, 0, (int)w - 1);
                    acc = acc + src[plane + at];
                }
                dst[plane + (size_t)y * w + x] = acc / (float)(2 * r + 1);
            }
}

/* gm_select.wgsl:14-27: the cells that adopt the affine hypothesis, rewritten in the E8 flow */
void fho_gm_select(const float* maps, const float* coef, const fho_view* flow, uint32_t h8, uint32_t w8, uint32_t hc,
                   uint32_t wc, float eps, float dmin, float tex) {
    const size_t n = (size_t)hc * wc;
    for (uint32_t i = 0; i < h8; i++)
        for (uint32_t j = 0; j < w8; j++) {
            const int x = clampi((int)floorf(((float)j + 0.5f) * (float)wc / (float)w8), 0, (int)wc - 1);
            const int y = clampi((int)floorf(((float)i + 0.5f) * (float)hc / (float)h8), 0, (int)hc - 1);
            const size_t idx = (size_t)y * wc + (size_t)x;
            const float cm = maps[idx], ca = maps[n + idx], dv = maps[2 * n + idx];
            const float lm = maps[3 * n + idx], l2 = maps[4 * n + idx];
            const float sd = sqrtf(fmaxf(l2 - lm * lm, 0.0f));
            if (ca + eps < cm && dv > dmin && sd > tex) {
                const float xn = -1.0f + 2.0f * (float)j / (float)(w8 - 1 > 1 ? w8 - 1 : 1);
                const float yn = -1.0f + 2.0f * (float)i / (float)(h8 - 1 > 1 ? h8 - 1 : 1);
                for (uint32_t c = 0; c < 4; c++) wr(flow, h8, w8, 0, i, j, c, coef[c * 4] + coef[c * 4 + 1] * xn + coef[c * 4 + 2] * yn);
            }
        }
}

/* gm_steps (gmhs.rs:149-206): fit, cost maps, the two box windows (5 maps, then the costs and the displacement
 * difference), select */
void fho_gmhs(const fho_view* a, const fho_view* b, uint32_t h, uint32_t w, const fho_view* flow, uint32_t h8,
              uint32_t w8, uint32_t full_w, uint32_t level, float* coef, float* maps, float* tmp) {
    fho_gm_par p;
    fho_gm_params(h, w, full_w, level, &p);
    fho_gm_fit(flow, h8, w8, p.delta, 4, coef);
    fho_gm_cost(a, b, h, w, flow, h8, w8, coef, p.hc, p.wc, maps);
    fho_gm_box(maps, tmp, 5, p.hc, p.wc, p.r_blk, 0);
    fho_gm_box(tmp, maps, 5, p.hc, p.wc, p.r_blk, 1);
    fho_gm_box(maps, tmp, 3, p.hc, p.wc, p.r_dwin, 0);
    fho_gm_box(tmp, maps, 3, p.hc, p.wc, p.r_dwin, 1);
    fho_gm_select(maps, coef, flow, h8, w8, p.hc, p.wc, p.eps, p.dmin, p.tex);
}
