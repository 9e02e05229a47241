/* fhc_ops: the FlyHighFG network ops between the convs, on MI355X (gfx950), as a C ABI.
 *
 * The reference runs each of these as one WGSL dispatch recorded by the planner (crates/flyhigh-engine/src/net/
 * build.rs) through a Gpu method (ops/network.rs, ops/interp.rs, ops/render.rs); there is no FFI at op level, so
 * each entry point below replaces that Gpu method plus the dispatch it records, and a maintainer would call it from
 * the planner arm named in its comment (a Step::Foreign replayed in order with the conv steps of fhc_conv.h).
 *
 * Conventions are those of fhc_conv.h: 0 on success, a negative value on error with the message in
 * fhc_last_error() (thread-local); nothing aborts or throws; the library allocates nothing and never synchronises,
 * so calls can be captured in a HIP graph. An empty tensor (a zero size) is a no-op.
 *
 * Tensors are NHWC f16 views (fhc_tensor): element (img, y, x, ch) at p[((img * H + y) * W + x) * cstride + c0 +
 * ch]. The reference's Tensor is planar [C][H][W] with batch 1 and carries a channel offset and a read scale
 * (ops/tensor.rs); both are kept: `c0` is the channel offset, `scale` multiplies every value read where the
 * reference's kernel applies its view's scale (noted per op; the other inputs must have scale 1). Outputs are
 * written through a view, so an op can write straight into its slice of a concat (the graph's concat ops become
 * free); an output's scale is not used. Arithmetic is f32 from f16 inputs, rounded once to f16 (RTNE) on store, in
 * the reference kernel's order of operations.
 */
#ifndef FHC_OPS_H
#define FHC_OPS_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct fhc_tensor {
    void* p;          /* device memory, f16 bit patterns                                                */
    uint32_t cstride; /* halves from one pixel to the next (>= c0 + the channels the op reads/writes)   */
    uint32_t c0;      /* first channel of the view                                                       */
    float scale;      /* read scale (Tensor::scale, ops/tensor.rs); 1 where the op takes none              */
} fhc_tensor;

/* Backward warp out[p] = img[p + flow[p]] in pixels, bilinear, coordinates clamped to the border; the flow view's
 * channels c0 and c0 + 1 are x and y. Both scales apply. Replaces Gpu::warp (ops/network.rs:6-19,
 * shaders/warp.wgsl:12-29), the planner's "warp" arm (net/build.rs:283). */
int fhc_warp(const fhc_tensor* img, const fhc_tensor* flow, const fhc_tensor* out, uint32_t n, uint32_t h,
             uint32_t w, uint32_t c, void* stream);

/* Luma of a BGR view (channel 0 B, 1 G, 2 R) into one channel; grad != 0: |luma(x+1) - luma| + |luma(y+1) -
 * luma| (0 past the last column / row). The scale applies. Replaces Gpu::luma (ops/network.rs:22-33,
 * shaders/luma.wgsl:9-28), the "luma" and "luma_grad" arms (net/build.rs:321-325). */
int fhc_luma(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, int grad,
             void* stream);

/* Luma SAD cost volume: for each displacement (dy, dx) in [-radius, radius]^2, channel (dy + r) * (2r + 1) + dx
 * + r, the 3x3 zero-padded mean of |la(y, x) - lb(y + dy, x + dx)| with lb's coordinates clamped. One-channel
 * inputs; radius <= 7. Replaces Gpu::sad (ops/network.rs:34-47, shaders/sad.wgsl:10-29), the "sad_volume" arm
 * (net/build.rs:326-329). */
int fhc_sad_volume(const fhc_tensor* la, const fhc_tensor* lb, const fhc_tensor* out, uint32_t n, uint32_t h,
                   uint32_t w, uint32_t radius, void* stream);

/* Convex x2 upsample: out (2h x 2w x c) = the softmax over 9 of wt's channels k * 4 + sy * 2 + sx (36 channels,
 * at the input pixel) weighting x's zero-padded 3x3 neighbourhood; c <= 256. wt is the up.w conv's output. Replaces
 * Gpu::convex (ops/network.rs:48-55, shaders/convex.wgsl:10-35), the "convex_upsample" arm after its conv
 * (net/build.rs:379-416). */
int fhc_convex_upsample(const fhc_tensor* wt, const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h,
                        uint32_t w, uint32_t c, void* stream);

/* FiLM modulate out = hv * (1 + g[c]) + g[C + c], g dense f16 [n][2C] in device memory (one vector per image: the
 * reference's batch 1 has one). Replaces Gpu::film (ops/network.rs:56-62, shaders/film.wgsl:9-15), the
 * "film_modulate" arm (net/build.rs:360-363). */
int fhc_film_modulate(const fhc_tensor* hv, const void* g, const fhc_tensor* out, uint32_t n, uint32_t h,
                      uint32_t w, uint32_t c, void* stream);

/* Visibility blend weights: the softmax (p0, p1, p2) of 3 logits -> 2 channels (p0 + p2 / 2, p1 + p2 / 2). The
 * scale applies. Replaces Gpu::blend (ops/network.rs:63-68, shaders/blend.wgsl:9-21), "blend_weights" unfused. */
int fhc_blend_weights(const fhc_tensor* vis, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w,
                      void* stream);

/* The fused blend of two 3-channel images by those weights, each product and the weights rounded to f16 as the
 * unfused path rounds them. vis's scale applies. Replaces Gpu::blendmix (ops/render.rs:102-115,
 * shaders/blendmix.wgsl:12-28), the blend_weights + mul + mul + add peephole (net/build.rs:417-450). */
int fhc_blendmix(const fhc_tensor* wa, const fhc_tensor* wb, const fhc_tensor* vis, const fhc_tensor* out,
                 uint32_t n, uint32_t h, uint32_t w, void* stream);

/* k x k average pool, stride k: out (h / k) x (w / k) x c (the remainder rows and columns are dropped). Replaces
 * Gpu::avgpool (ops/interp.rs:12-18, shaders/avgpool.wgsl:8-19), the "avgpool" arm (net/build.rs:279-282). */
int fhc_avgpool(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                uint32_t k, void* stream);

/* Resize ih x iw -> oh x ow: bilinear with align_corners false (antialias 0) or the separable triangle filter of
 * support max(scale, 1) (antialias 1, torch's antialiased bilinear). The scale applies to the result. Replaces
 * Gpu::interp (ops/interp.rs:6-11, shaders/interp.wgsl:11-45), the "interpolate" arm (net/build.rs:199-208). */
int fhc_interpolate(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t c, uint32_t ih, uint32_t iw,
                    uint32_t oh, uint32_t ow, int antialias, void* stream);

/* Elementwise binary: op 0 out = a * sa + b * sb, op 1 out = (a * sa) * (b * sb), sa and sb the views' scales;
 * cb (b's channels) is c, or 1 to broadcast b's one channel. Replaces Gpu::binary (ops/elementwise.rs:8-27,
 * shaders/binary.wgsl:9-17), the "add" and "mul" arms (net/build.rs:310-311). */
int fhc_binary(const fhc_tensor* a, const fhc_tensor* b, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w,
               uint32_t c, uint32_t cb, int op, void* stream);

/* Elementwise unary of v = x * scale: op 0 v * a, 1 clamp(v, a, b), 2 2 / (1 + exp(-v)) - 1, 3 -v. Replaces
 * Gpu::unary (shaders/unary.wgsl:9-20): the "mul_t" arm (op 0 with a = 2t or 2(1 - t), net/build.rs:290-308),
 * "affine_out" (op 2) and "clamp" (op 1). */
int fhc_unary(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c, int op,
              float a, float b, void* stream);

/* Channel copy of a view into an output view (a concat slice): the bits at scale 1, else f16(x * scale). One input
 * of the reference's concat (Gpu::concat, ops/elementwise.rs:65-77, shaders/chcopy.wgsl:19-36); the graph's other
 * concat inputs need no copy here, since their producers write into the slice. */
int fhc_chcopy(const fhc_tensor* x, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
               void* stream);

/* render_pix: flow (4 channels: A's x, y then B's, times fsx for x and fsy for y), vis (3 logits, read scale) and rt
 * (3 channels) upsampled bilinearly from hq x wq to h x w; a warped by the forward flow and b by the backward one
 * (bilinear, or bicubic with cubic != 0: Keys a = -0.75, every tap clamped to the border), blended by the visibility
 * weights, + rt, clamped to [0, 1], 3 channels into out. flags: bit 0 the decisive blend, bit 1 the still test.
 * Replaces Gpu::render_ex_to (ops/render.rs:43-101, shaders/render.wgsl:83-160), the "render_pix" arm
 * (net/build.rs:364-378); the static-age variant is not built. Views of a and b with 8-byte pixels (4-channel
 * strides and offsets) read each tap with one load. */
int fhc_render(const fhc_tensor* a, const fhc_tensor* b, const fhc_tensor* flow, const fhc_tensor* vis,
               const fhc_tensor* rt, const fhc_tensor* out, uint32_t h, uint32_t w, uint32_t hq, uint32_t wq, float fsx,
               float fsy, int cubic, uint32_t flags, void* stream);

/* ---- The host's 8-bit frames. A frame is RGBA8, one 32-bit word per pixel (R | G << 8 | B << 16 | A << 24), rows
 * `pitch` words apart, n frames `fstride` words apart; hp x wp is the padded working size (the frame rounded up to
 * 32). The network reads BGR f16 in [0, 1], replicate-padded: padded pixel (x, y) is frame pixel (min(x, w - 1),
 * min(y, h - 1)). Frames must be 4-byte aligned. */

/* rgba_in: n frames -> BGR f16(byte / 255), padded to hp x wp, channels c0..c0 + 2 of out (n, hp, wp); a view of
 * 4-channel pixels (cstride 4, c0 0, 8-byte aligned) gets channel 3 written 0. Replaces the Session's rgba_in steps
 * (crates/flyhigh-engine/src/net/session.rs:56-60, shaders/rgba_in.wgsl:11-19). */
int fhc_rgba_in(const void* rgba, uint32_t n, uint32_t w, uint32_t h, uint32_t pitch, uint64_t fstride,
                const fhc_tensor* out, uint32_t hp, uint32_t wp, void* stream);

/* rgba_out: channels c0..c0 + 2 (B, G, R) of in (n, hp, wp) -> n frames of w x h, each byte
 * u32(clamp(v, 0, 1) * 255 + 0.5), alpha 255 (the crop of the padding). Replaces the Session's rgba_out step
 * (net/session.rs:63, shaders/rgba_out.wgsl:9-18). */
int fhc_rgba_out(const fhc_tensor* in, uint32_t n, uint32_t hp, uint32_t wp, void* rgba, uint32_t w, uint32_t h,
                 uint32_t pitch, uint64_t fstride, void* stream);

/* rgba_in of n frames at hp x wp, then the antialiased resize to oh x ow (fhc_interpolate with antialias 1), in one
 * launch that reads the 8-bit frames directly: the internal-size mode's inputs A, B (net/session.rs:56-60, then
 * net/build.rs:615-620). out has 4-channel pixels (cstride 4, c0 0, 8-byte aligned), channel 3 written 0.
 * Bit-identical to the two steps. Downscales up to about 5x (at most 10 taps per axis and an 84-pixel window for
 * 16 outputs: 2160p frames to the 864 x 480 network take 10 taps and 78). */
int fhc_rgba_resize(const void* rgba, uint32_t n, uint32_t w, uint32_t h, uint32_t pitch, uint64_t fstride,
                    uint32_t hp, uint32_t wp, const fhc_tensor* out, uint32_t oh, uint32_t ow, void* stream);

/* The frame-size render of the internal-size mode and rgba_out in one launch: render_pix (fhc_render) of the padded
 * frames a and b (each w x h RGBA8, rows `pitch` words apart, read as rgba_in converts them) at hp x wp from the maps
 * flow / vis / rt at hq x wq, the flow's x times fsx and y times fsy (ftq.scale * wp / iwp and * hp / ihp,
 * net/build.rs:717-736), each result rounded to f16 and written as the RGBA8 frame out (w x h, rows opitch words
 * apart, alpha 255). flags: bits 0-1 fhc_render's modes; bit 2 set: the reference's f32 operations in its order,
 * bit-identical to rgba_in, fhc_render and rgba_out in turn; bit 2 clear (the frame path): the same expressions with
 * each product fused into the sum it feeds (one rounding where the reference rounds twice: about a fifth fewer
 * instructions), bytes within 1 of the exact order. Flow and vis as channels 0-3 and 4-6 of one 16-byte aligned
 * 8-channel view, with rt of 4-channel pixels, take two loads a map tap. w >= 4. */
int fhc_render_rgba(const void* a, const void* b, uint32_t w, uint32_t h, uint32_t pitch, uint32_t hp, uint32_t wp,
                    const fhc_tensor* flow, const fhc_tensor* vis, const fhc_tensor* rt, uint32_t hq, uint32_t wq,
                    float fsx, float fsy, int cubic, uint32_t flags, void* out, uint32_t opitch, void* stream);
/* fhc_render_rgba of pairs x phases generated frames in one launch, pair-major: pair p's frames A, B are frames
 * 2p, 2p + 1 (fstride words apart), phase j's maps image j * pairs + p of flow, vis and rt (each view's tensor holds
 * phases * pairs images of hq x wq), its output frame j * pairs + p (ostride words apart). Bit-identical to one call
 * per generated frame. pairs * phases <= 65535. The batched program's form; the reference renders one frame a mid(t). */
int fhc_render_rgba_n(const void* frames, uint32_t pairs, uint32_t phases, uint32_t w, uint32_t h, uint32_t pitch,
                      uint64_t fstride, uint32_t hp, uint32_t wp, const fhc_tensor* flow, const fhc_tensor* vis,
                      const fhc_tensor* rt, uint32_t hq, uint32_t wq, float fsx, float fsy, int cubic, uint32_t flags,
                      void* out, uint32_t opitch, uint64_t ostride, void* stream);

/* ---- The graph's op chains, fused. Each computes what its ops compute one after another (the same f32 operations
 * and f16 roundings at the tensors the ops store); no reference counterpart as one call: each replaces the listed
 * planner arms run in sequence. A and B arrive as a batch of 2. */

/* models/graph.json ops 14-18, 21-24: avgpool k 2 of q (2, h, w, 3) into i8 (2, h/2, w/2, 3), again into i16's
 * channels 3 * image (1, h/4, w/4: the img16 slice of the coarse input), and their luma into l16's channel image
 * (avgpool.wgsl:8-19, luma.wgsl:14-19; arms net/build.rs:279-282, :321). h, w >= 4. */
int fhc_pair_pyramid(const fhc_tensor* q, const fhc_tensor* i8, const fhc_tensor* i16, const fhc_tensor* l16,
                     uint32_t h, uint32_t w, void* stream);

/* graph.json ops 0-1, 14-18, 21-24: the antialiased resize of the pictures ab (2, ih, iw, 3) to q (2, oh, ow, 3), and
 * from it the pyramid of fhc_pair_pyramid (i8, i16, l16), in one launch where the resize's tiles hold whole pool
 * blocks (else the two calls). */
int fhc_pair_input(const fhc_tensor* ab, const fhc_tensor* q, const fhc_tensor* i8, const fhc_tensor* i16,
                   const fhc_tensor* l16, uint32_t ih, uint32_t iw, uint32_t oh, uint32_t ow, void* stream);

/* fhc_pair_input for `pairs` pairs in one launch: pair k's pictures are images 2k, 2k + 1 of ab, q and i8, its
 * i16 and l16 image k. Bit-identical to one call per pair. */
int fhc_pair_input_n(const fhc_tensor* ab, const fhc_tensor* q, const fhc_tensor* i8, const fhc_tensor* i16,
                     const fhc_tensor* l16, uint32_t ih, uint32_t iw, uint32_t oh, uint32_t ow, uint32_t pairs,
                     void* stream);

/* graph.json ops 7, 13 (the encoders' outputs f16a, f16b), their places in the concat of op 26 and f16b's in the
 * streaming state of op 43: x (2, h, w, c) holds both pictures' features as a batch; image i is copied to channels
 * c0 + i * c of out (batch 1) and image 1 also to `also` when not NULL. Lets the encoders run as one batch. */
int fhc_fold_pair(const fhc_tensor* x, const fhc_tensor* out, const fhc_tensor* also, uint32_t h, uint32_t w,
                  uint32_t c, void* stream);

/* graph.json ops 33-40 and 43's flow16: o (1, hi, wi) holds the coarse head's flow (channels 0-3) and visibility
 * logits (4-6); out (1, oh, ow) gets both resized bilinearly (align_corners false), the flow times flow_scale (flow16
 * = o * 16), in channels 0-3 and 4-6; state (when not NULL, hi <= oh, wi <= ow) gets the scaled flow at the input
 * size, as the copy into the streaming state does. */
int fhc_coarse_up(const fhc_tensor* o, const fhc_tensor* out, const fhc_tensor* state, uint32_t hi, uint32_t wi,
                  uint32_t oh, uint32_t ow, float flow_scale, void* stream);

/* graph.json op 42's body up to the concat: f8 (2, h, w, c) and i8 (2, h, w, 3) warped by flow (1, h, w: channels
 * 0-1 for A, 2-3 for B, at its read scale), written into fx's slices c0: wa, +c: wb, +2c: ia, +2c+3: ib, +2c+6: the
 * scaled flow (4 channels); the warped pictures' luma into l8's channel image (warp.wgsl, luma.wgsl, chcopy.wgsl). */
int fhc_fine_input(const fhc_tensor* f8, const fhc_tensor* i8, const fhc_tensor* flow, const fhc_tensor* fx,
                   const fhc_tensor* l8, uint32_t h, uint32_t w, uint32_t c, void* stream);

/* graph.json ops 44-48, 54-60: fv holds flow (channels 0-3) and vis (4-6), dfilm the FiLM head's output (d_flow
 * 0-3, d_mask 4); out = flow_t (0-3) = f16(flow * 2t) (forward, channels 0-1; 2(1 - t) backward, 2-3) + d_flow,
 * and vis_t (4-6) = vis + (d_mask, -d_mask, 0) (unary.wgsl op 0, binary.wgsl op 0, chcopy.wgsl; arms
 * net/build.rs:290-311). */
int fhc_flow_vis_t(const fhc_tensor* fv, const fhc_tensor* dfilm, const fhc_tensor* out, uint32_t n, uint32_t h,
                   uint32_t w, float t, void* stream);

/* graph.json ops 65-76: q (2, h, w, 3) warped by flow (1, h, w: channels 0-1 A, 2-3 B, at its read scale), the
 * blend of the two by the visibility logits vis (blendmix.wgsl), and the blend's luma gradient, written as rx:
 * c0 rwa, +3 rwb, +6 vis (copied), +9 the raw flow times flow_out_scale, +13 the gradient. */
int fhc_refine_input(const fhc_tensor* q, const fhc_tensor* flow, const fhc_tensor* vis, const fhc_tensor* rx,
                     uint32_t h, uint32_t w, float flow_out_scale, void* stream);
/* fhc_refine_input over n images in one launch: image i of flow, vis and rx (each view's tensor holding n images of
 * h x w) takes its two pictures from pair i % qmod of q (images 2p and 2p + 1 of a tensor of 2 qmod images), as a
 * batch of frame pairs and their phases lays them out. Bit-identical to n calls. 1 <= qmod <= n. */
int fhc_refine_input_n(const fhc_tensor* q, const fhc_tensor* flow, const fhc_tensor* vis, const fhc_tensor* rx,
                       uint32_t h, uint32_t w, float flow_out_scale, uint32_t n, uint32_t qmod, void* stream);


/* coarse_up then the fine block's input in one launch (graph ops 33-40 with 43's flow16, then op 42's input): the
 * coarse head's output o (hi x wi, 7 channels) resized bilinearly to the fine grid h x w, the flow channels times
 * flow_scale, stored into fv (7 channels) and the flow16 copy into state (NULL: none), as fhc_coarse_up; then, read
 * at fine_scale, the flow that warps f8 and i8 into fx with the lumas into l8, as fhc_fine_input on the view (fv,
 * fine_scale). Bit-identical to the two calls. */
int fhc_coarse_fine_input(const fhc_tensor* o, const fhc_tensor* fv, const fhc_tensor* state, uint32_t hi, uint32_t wi,
                          float flow_scale, const fhc_tensor* f8, const fhc_tensor* i8, float fine_scale,
                          const fhc_tensor* fx, const fhc_tensor* l8, uint32_t h, uint32_t w, uint32_t c,
                          void* stream);

/* fhc_coarse_fine_input for `pairs` pairs in one launch: pair k's maps and pictures are images 2k, 2k + 1 of f8 and
 * i8, its image k of o, fv, state, fx and l8. Bit-identical to one call per pair. */
int fhc_coarse_fine_input_n(const fhc_tensor* o, const fhc_tensor* fv, const fhc_tensor* state, uint32_t hi,
                            uint32_t wi, float flow_scale, const fhc_tensor* f8, const fhc_tensor* i8,
                            float fine_scale, const fhc_tensor* fx, const fhc_tensor* l8, uint32_t h, uint32_t w,
                            uint32_t c, uint32_t pairs, void* stream);

/* fhc_coarse_fine_input_n, then fhc_sad_volume(l8 channel 0, l8 channel 1, sad_out, pairs, h, w, radius) on its
 * lumas, in one launch (pair(): ops 33-42 with the fine block's cost volume): the cost volume's workgroups compute
 * the lumas they read themselves (the tile's and a ring of 1 + radius), with fine_input's arithmetic, beside the
 * fine input's. radius <= 3; sad_out (image k: pair k's volume) must not overlap what the fine input writes (fx's
 * first 2c + 10 channels, l8, fv, state). Bit-identical to the two calls. */
int fhc_coarse_fine_input_sad_n(const fhc_tensor* o, const fhc_tensor* fv, const fhc_tensor* state, uint32_t hi,
                                uint32_t wi, float flow_scale, const fhc_tensor* f8, const fhc_tensor* i8,
                                float fine_scale, const fhc_tensor* fx, const fhc_tensor* l8, uint32_t h, uint32_t w,
                                uint32_t c, uint32_t pairs, const fhc_tensor* sad_out, uint32_t radius,
                                void* stream);

/* fhc_flow_vis_t then fhc_convex_upsample of its output in one launch (graph ops 44-48, 54-62): the convex
 * upsample's 7-channel input (flow_t | vis_t) computed from fv and dfilm at phase t while it is staged, never
 * stored. Bit-identical to the two calls. */
int fhc_flow_vis_t_convex(const fhc_tensor* wt, const fhc_tensor* fv, const fhc_tensor* dfilm, float t,
                          const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, void* stream);

/* fhc_flow_vis_t_convex for `phases` phases ts[0 .. phases - 1] (at most 8) of n pairs in one launch: image j * n + p
 * of dfilm and out is phase j of pair p, whose wt and fv are image p. Bit-identical to one call per phase. The
 * reference runs one phase a mid(t) (model/graph.rs:182); this is the batched program's form. */
int fhc_flow_vis_t_convex_n(const fhc_tensor* wt, const fhc_tensor* fv, const fhc_tensor* dfilm, const float* ts,
                            uint32_t phases, const fhc_tensor* out, uint32_t n, uint32_t h, uint32_t w, void* stream);

/* fhc_flow_vis_t_convex_n into up (2h x 2w, 7 channels), then fhc_refine_input_n on it, in one launch (graph ops
 * 44-48, 54-76): image i = j * n + p of up and rx is phase j of pair p, its pictures pair p of q (images 2p, 2p + 1
 * of 2n), and the refine input reads up's flow (channels 0-3) at flow_scale and its visibility (4-6) unscaled, as
 * fhc_refine_input_n(q, (up, flow_scale), (up + 4, 1), rx, 2h, 2w, flow_out_scale, phases * n, n) would. Each
 * refine tile computes the upsampled values it reads itself (those at its right and lower edge twice, as the
 * neighbouring tile does), so no launch boundary sits between the two. Bit-identical to the two calls. */
int fhc_mid_input_n(const fhc_tensor* wt, const fhc_tensor* fv, const fhc_tensor* dfilm, const float* ts,
                    uint32_t phases, const fhc_tensor* up, const fhc_tensor* q, const fhc_tensor* rx, uint32_t n,
                    uint32_t h, uint32_t w, float flow_scale, float flow_out_scale, void* stream);

/* fhc_fold_pair and fhc_sad_volume in one launch, for a sad_volume that reads nothing the fold writes and writes
 * nothing it reads (pair(): the second encoder pair's fold, op 26 and 43's f16b, beside the 1/16 lumas' cost volume,
 * ops 25-26, ready since the pyramid). The fold's arguments as fhc_fold_pair's (h x w, c channels); the cost
 * volume's as fhc_sad_volume's (sn x sh x sw, radius). Bit-identical to the two calls. */
int fhc_fold_pair_sad(const fhc_tensor* x, const fhc_tensor* out, const fhc_tensor* also, uint32_t h, uint32_t w,
                      uint32_t c, const fhc_tensor* la, const fhc_tensor* lb, const fhc_tensor* sad_out, uint32_t sn,
                      uint32_t sh, uint32_t sw, uint32_t radius, void* stream);

/* fhc_fold_pair_sad with the fold over `pairs` pairs: pair k's two maps are images 2k, 2k + 1 of x, its fold
 * image k of out (and of also). Bit-identical to one call per pair. */
int fhc_fold_pair_sad_n(const fhc_tensor* x, const fhc_tensor* out, const fhc_tensor* also, uint32_t h, uint32_t w,
                        uint32_t c, uint32_t pairs, const fhc_tensor* la, const fhc_tensor* lb,
                        const fhc_tensor* sad_out, uint32_t sn, uint32_t sh, uint32_t sw, uint32_t radius,
                        void* stream);

/* GMHS, the periodic-structure repair of the pair's E8 flow (crates/flyhigh-engine/src/gmhs.rs:149-206, run at the
 * end of the pair stage when the repair level is above 0, net/build.rs:640-660; the reference's default level is 1,
 * options.rs:305). A robust affine motion is fitted to the flow (4 rounds of reweighted least squares,
 * gm_fit_reduce.wgsl and gm_fit_solve.wgsl); on a grid of 2 x 2 network pixels the luma mismatch under the flow and
 * under the affine motion, their displacement difference and the texture are mapped (gm_cost.wgsl) and box-filtered
 * (gm_box.wgsl); the flow is rewritten in place with the affine motion where that explains the frames better, differs
 * by a real jump and the texture is not flat (gm_select.wgsl). */
typedef struct fhc_gmhs_par {
    uint32_t hc, wc;        /* the cost grid, ceil(h / 2) x ceil(w / 2) */
    uint32_t r_blk, r_dwin; /* box radii: the texture window (all 5 maps), then the decision window (maps 0-2) */
    float s;                /* network pixels per half-frame pixel, w / (full_w / 2) */
    float dmin;             /* the jump a cell must show (0 at level 2) */
    float delta;            /* the fit's Huber scale */
    float eps, tex;         /* cost margin 0, texture floor 0.015 */
    uint64_t ws_bytes;      /* the workspace fhc_gmhs needs */
    uint64_t maps_offset;   /* byte offset of the cost maps after the texture window: f32 [5][hc][wc] (mismatch
                               under the flow, under the affine motion, displacement difference, luma, luma^2)
                               after a call; the affine coefficients, f32 [4][4] (a0, a1, a2, 0 per flow channel, a1
                               and a2 per unit of the coordinates normalised to [-1, 1]), are at byte 0 */
    uint64_t dec_offset;    /* byte offset of the values each E8 cell decides on: f32 [5][h8][w8], maps 0-2 after
                               the decision window and maps 3-4, at the cost cell the select reads for it */
} fhc_gmhs_par;

/* The stage's parameters for an h x w network of frames padded to full_w columns (gm_steps, gmhs.rs:149-160).
 * level 1 (safe) or 2 (aggressive, no jump gate). */
int fhc_gmhs_params(uint32_t h, uint32_t w, uint32_t full_w, uint32_t level, fhc_gmhs_par* out);

/* The repair, in place on channels 0-3 of `flow` (h8 x w8, the pair's plain E8 flow: x, y towards frame a, x, y
 * towards frame b, in network pixels). a, b: the network pictures (h x w, BGR in channels 0-2, scale 1). ws: a
 * 256-byte aligned workspace of fhc_gmhs_params' ws_bytes; nothing in it need be initialised. level 0 is a no-op.
 * The flow is the E8 grid of the network (h8 = h / 8, w8 = w / 8; a flow near the cost grid's size is an error).
 * Eight launches on `stream`. Replaces gmhs::gm_steps and its 14 dispatches. */
int fhc_gmhs(const fhc_tensor* a, const fhc_tensor* b, uint32_t h, uint32_t w, const fhc_tensor* flow, uint32_t h8,
             uint32_t w8, uint32_t full_w, uint32_t level, void* ws, size_t ws_bytes, void* stream);

/* fhc_gmhs for `pairs` independent pairs in the same eight launches: pair k's pictures are the images 2k past a and
 * b (a and b: images 0 and 1 of a buffer holding the pairs' pictures A0 B0 A1 B1 ...), its flow image k of flow,
 * its workspace at k * S bytes past ws, S = ws_bytes of fhc_gmhs_params rounded up to 256 (ws_bytes given >=
 * (pairs - 1) * S + that ws_bytes). Bit-identical to fhc_gmhs on each pair. The reference repairs one pair a
 * session (gmhs::gm_steps, gmhs.rs:149-206); this is the batched sessions' form. */
int fhc_gmhs_n(const fhc_tensor* a, const fhc_tensor* b, uint32_t h, uint32_t w, const fhc_tensor* flow, uint32_t h8,
               uint32_t w8, uint32_t full_w, uint32_t level, uint32_t pairs, void* ws, size_t ws_bytes, void* stream);

/* fhc_gmhs and the FiLM head: a FiLM pair plan (fhc_conv_pair_plan_create with FHC_PAIR_FILM_IN, fhc_conv.h) run
 * as fhc_conv_pair_run_film(pair, pair_x, pair_film, pair_y) runs it, with its workgroups inside the repair's first
 * launch, and, when conv is not NULL, a conv plan (the FiLM head's output conv on pair_y) run as
 * fhc_conv_run(conv, conv_x, conv_y, NULL, NULL) runs it, with its workgroups inside the second: the fit's 128
 * workgroups are latency-bound and leave the GPU to them. They touch none of the repair's data (the frame: the
 * repair of pair()'s flow, and mid()'s FiLM head, which reads h and the FiLM vectors of t). The pair's
 * configuration must be a one-tile configuration of 3 + 3 channel blocks on one wave row (the 48 -> 48 -> 48 FiLM
 * head at 2 or 4 rows per tile); the conv a one-launch direct plan without residual (its workgroups join the fit's
 * where its configuration is the one-row 64-channel kernel-row split, else it runs in its own launch after the
 * repair). level 0 runs the pair, then the conv. Eight launches (nine when the conv runs on its own) where the
 * three calls take ten. No counterpart in the reference. */
struct fhc_conv_plan;
int fhc_gmhs_film(const fhc_tensor* a, const fhc_tensor* b, uint32_t h, uint32_t w, const fhc_tensor* flow,
                  uint32_t h8, uint32_t w8, uint32_t full_w, uint32_t level, void* ws, size_t ws_bytes,
                  const struct fhc_conv_plan* pair, const void* pair_x, const void* pair_film, void* pair_y,
                  const struct fhc_conv_plan* conv, const void* conv_x, void* conv_y, void* stream);

#ifdef __cplusplus
}
#endif
#endif
