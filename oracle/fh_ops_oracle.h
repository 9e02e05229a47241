/* CPU oracle of the FlyHighFG network ops around the convs: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/ and bench.py's CPU-baseline leg call these functions, as the checker; the product (libfhconv.so)
 * never links or loads them. Each function restates one WGSL kernel of the reference, element by element, in f32
 * with the kernel's own order of operations, on NHWC f16 views: element (img, y, x, ch) of a view at
 * p[((img * H + y) * W + x) * cs + c0 + ch]. The reference's tensors are planar [C][H][W] with batch 1; a view's
 * channel offset there (Tensor::c0) is c0 here, and `scale` is its read scale (Tensor::scale,
 * crates/flyhigh-engine/src/ops/tensor.rs). Outputs are written through a view (cs, c0) so that a result can land
 * in a concat slice; their scale is not used.
 */
#ifndef FH_OPS_ORACLE_H
#define FH_OPS_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fho_view {
    void* p;        /* f16 bit patterns */
    uint32_t cs;    /* halves between consecutive pixels */
    uint32_t c0;    /* first channel of the view */
    float scale;    /* read scale (ops that take it) */
} fho_view;

/* backward warp, bilinear with border clamp: shaders/warp.wgsl:12-29 (flow channels c0, c0 + 1 = x, y pixels) */
void fho_warp(const fho_view* img, const fho_view* flow, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
              uint32_t c);
/* BGR -> luma (grad 0) or |d/dx| + |d/dy| of luma (grad 1): shaders/luma.wgsl:9-28 */
void fho_luma(const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w, int grad);
/* luma SAD cost volume over displacements |dy|, |dx| <= r, channel (dy + r) * (2r + 1) + dx + r:
 * shaders/sad.wgsl:10-29 */
void fho_sad(const fho_view* la, const fho_view* lb, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
             uint32_t r);
/* convex x2 upsample: softmax over 9 of wt (channel k * 4 + sy * 2 + sx) weighting x's 3x3 neighbourhood:
 * shaders/convex.wgsl:10-35; out is 2h x 2w */
void fho_convex(const fho_view* wt, const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
                uint32_t c);
/* FiLM modulate out = h * (1 + g[c]) + g[c + C], g f16 [n][2C]: shaders/film.wgsl:9-15 */
void fho_film(const fho_view* hv, const uint16_t* g, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
              uint32_t c);
/* visibility blend weights (softmax of 3 logits; the third class split half/half) -> 2 channels:
 * shaders/blend.wgsl:9-21 */
void fho_blend(const fho_view* vis, const fho_view* out, uint32_t n, uint32_t h, uint32_t w);
/* fused blend of two 3-channel images by those weights: shaders/blendmix.wgsl:12-28 */
void fho_blendmix(const fho_view* wa, const fho_view* wb, const fho_view* vis, const fho_view* out, uint32_t n,
                  uint32_t h, uint32_t w);
/* k x k average pool, stride k, out (h / k) x (w / k): shaders/avgpool.wgsl:8-19, ops/interp.rs:12-18 */
void fho_avgpool(const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c, uint32_t k);
/* bilinear resize (aa 0, align_corners false) or antialiased triangle-filter resize (aa 1):
 * shaders/interp.wgsl:11-45 */
void fho_interp(const fho_view* x, const fho_view* out, uint32_t n, uint32_t c, uint32_t ih, uint32_t iw,
                uint32_t oh, uint32_t ow, int aa);

/* elementwise binary: op 0 f16(a * sa + b * sb), op 1 f16((a * sa) * (b * sb)); cb == 1 broadcasts b's single
 * channel: shaders/binary.wgsl:9-17 */
void fho_binary(const fho_view* a, const fho_view* b, const fho_view* out, uint32_t n, uint32_t h, uint32_t w,
                uint32_t c, uint32_t cb, int op);
/* elementwise unary of v = x * scale: op 0 v * a, 1 clamp(v, a, b), 2 2 / (1 + exp(-v)) - 1 (affine_out), 3 -v:
 * shaders/unary.wgsl:9-20 */
void fho_unary(const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int op,
               float a, float b);
/* channel copy of a view into an output view, f16(x * scale) unless the scale is 1 (then the bits are copied):
 * one input of shaders/chcopy.wgsl:19-36 */
void fho_chcopy(const fho_view* x, const fho_view* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c);
/* render_pix: flow_tq (4 channels at the view's c0, x scaled by fsx, y by fsy), vis_tq (3 logits, read scale) and
 * R_t (3 channels) upsampled bilinearly from hq x wq to h x w; A warped by the forward flow, B by the backward one
 * (bilinear, or bicubic with cubic != 0); blended by the visibility weights; + R_t; clamped to [0, 1]. flags bit 0
 * the decisive blend, bit 1 the still test: shaders/render.wgsl:83-160. */
void fho_render(const fho_view* a, const fho_view* b, const fho_view* flow, const fho_view* vis, const fho_view* rt,
                const fho_view* out, uint32_t h, uint32_t w, uint32_t hq, uint32_t wq, float fsx, float fsy,
                int cubic, uint32_t flags);
/* rows y0 .. y1 - 1 of fho_render's output (the rows are independent: bands on threads give fho_render's result) */
void fho_render_rows(const fho_view* a, const fho_view* b, const fho_view* flow, const fho_view* vis,
                     const fho_view* rt, const fho_view* out, uint32_t h, uint32_t w, uint32_t hq, uint32_t wq,
                     float fsx, float fsy, int cubic, uint32_t flags, uint32_t y0, uint32_t y1);

/* rgba_in: n RGBA8 frames (R | G << 8 | B << 16 | A << 24 per 32-bit word, rows `pitch` words apart, frame i at
 * rgba + i * fstride words) -> BGR f16(byte / 255), replicate-padded to hp x wp, channels 0-2 of out:
 * shaders/rgba_in.wgsl:11-19 */
void fho_rgba_in(const uint32_t* rgba, uint32_t n, uint32_t w, uint32_t h, uint32_t pitch, uint64_t fstride,
                 const fho_view* out, uint32_t hp, uint32_t wp);
/* rgba_out: channels 0-2 (BGR) of an hp x wp view -> RGBA8 words, cropped to w x h, alpha 255:
 * shaders/rgba_out.wgsl:9-18 */
void fho_rgba_out(const fho_view* in, uint32_t n, uint32_t hp, uint32_t wp, uint32_t* rgba, uint32_t w, uint32_t h,
                  uint32_t pitch, uint64_t fstride);


/* GMHS, the periodic-structure repair of the pair's E8 flow (crates/flyhigh-engine/src/gmhs.rs:149-206): a robust
 * affine fit of the 4 flow channels, photometric cost maps of the model flow and the affine hypothesis on a grid of
 * 2 x 2 network pixels, two box windows, and a select that rewrites the flow where the hypothesis wins. Maps are
 * planar f32 [5][hc][wc]; coef is [4][4] (a0, a1, a2, 0 per flow channel). */
typedef struct fho_gm_par {
    uint32_t hc, wc, r_blk, r_dwin;
    float s, dmin, delta, eps, tex;
} fho_gm_par;
/* gmhs.rs:149-160: the grid and windows for an h x w network of a frame padded to full_w columns, repair level */
void fho_gm_params(uint32_t h, uint32_t w, uint32_t full_w, uint32_t level, fho_gm_par* p);
/* `iters` rounds of gm_fit_reduce.wgsl (32 workgroups) + gm_fit_solve.wgsl on the E8 flow (channels c0 .. c0 + 3) */
void fho_gm_fit(const fho_view* flow, uint32_t h8, uint32_t w8, float delta, uint32_t iters, float* coef);
/* gm_cost.wgsl:55-75, maps 0-4 (a, b: the network pictures, BGR) */
void fho_gm_cost(const fho_view* a, const fho_view* b, uint32_t h, uint32_t w, const fho_view* flow, uint32_t h8,
                 uint32_t w8, const float* coef, uint32_t hc, uint32_t wc, float* maps);
/* gm_box.wgsl: box_h (vert 0) or box_v of radius r over c planes */
void fho_gm_box(const float* src, float* dst, uint32_t c, uint32_t h, uint32_t w, uint32_t r, int vert);
/* gm_select.wgsl:14-27, the flow rewritten in place */
void fho_gm_select(const float* maps, const float* coef, const fho_view* flow, uint32_t h8, uint32_t w8, uint32_t hc,
                   uint32_t wc, float eps, float dmin, float tex);
/* the whole stage (gmhs.rs:149-206); maps and tmp hold 5 * hc * wc floats, maps ends as the decision maps */
void fho_gmhs(const fho_view* a, const fho_view* b, uint32_t h, uint32_t w, const fho_view* flow, uint32_t h8,
              uint32_t w8, uint32_t full_w, uint32_t level, float* coef, float* maps, float* tmp);

#ifdef __cplusplus
}
#endif
#endif
