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

void fho_render(const fho_view* a, const fho_view* b, const fho_view* flow, const fho_view* vis, const fho_view* rt,
                const fho_view* out, uint32_t h, uint32_t w, uint32_t hq, uint32_t wq, float fsx, float fsy,
                int cubic, uint32_t flags) {
    const float sh = (float)hq / (float)h, sw = (float)wq / (float)w;
    for (uint32_t y = 0; y < h; y++)
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
