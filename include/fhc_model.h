/* fhc_model: the FlyHighFG model files and the static plan of a frame, as a C ABI (host logic, no GPU).
 *
 * The reference loads a model directory of three files (crates/flyhigh-engine/src/model/mod.rs:38-96): graph.json
 * (the op graph), flyhighfg.json (the manifest: tensor shapes and offsets in f16 elements, the meta block) and
 * flyhighfg.bin (little-endian f16 weights, model/blob.rs:29-41), and turns the graph into a static plan of steps
 * at session build (net/build.rs:149-484, :532-736; net/session.rs:26-66). This ABI does the same on the host: it
 * loads and validates the files, hands out weights as f16 bits, and walks the graph into a plan whose steps map one
 * to one onto the entry points of fhc_conv.h / fhc_ops.h (a host replays them, in order, on one HIP stream).
 *
 * Conventions are those of fhc_conv.h: 0 (or a size / count) on success, a negative value on error with the
 * message in fhc_last_error() (thread-local); nothing aborts or throws across the boundary; a model is immutable
 * after load and may be read from any thread.
 */
#ifndef FHC_MODEL_H
#define FHC_MODEL_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct fhc_model fhc_model;

/* Load dir/graph.json, dir/flyhighfg.json and dir/flyhighfg.bin (Model::from_dir, model/mod.rs:38-44) and validate
 * them as Model::from_shared does (:57-96): the format version, every manifest tensor an unsigned offset and integer
 * dimensions >= 1 lying inside the blob (check_tensor, :101-119), every op named with string operands, every
 * weight an op reads present (graph::validate, model/graph.rs:17-47). */
int fhc_model_load(const char* dir, fhc_model** out);

/* The same from the three files' bytes (Model::from_bytes, model/mod.rs:46-53). The blob is copied. */
int fhc_model_load_bytes(const char* graph_json, size_t graph_len, const char* manifest_json, size_t manifest_len,
                         const void* blob, size_t blob_len, fhc_model** out);

void fhc_model_destroy(fhc_model* model);

/* JSON {"model", "train_step", "graph_ops", "tensors", "params", "render_sampling", "format_version",
 * "default_k"} (ModelInfo, model/mod.rs:14-27). Bytes written or -1. */
int fhc_model_info(const fhc_model* model, char* json, size_t cap);

/* A manifest tensor: its dimensions (up to 8) and element count. Returns the number of dimensions, or -1 when the
 * manifest has no such tensor (Blob::shape, model/blob.rs:29-31). */
int fhc_model_tensor(const fhc_model* model, const char* name, uint32_t* dims, size_t cap, uint64_t* count);

/* A tensor's weights as f16 bit patterns, in the blob's order (OIHW for a conv): the little-endian halves
 * Blob::weight decodes (model/blob.rs:32-41), without the f32 widening. Returns the element count or -1. */
int64_t fhc_model_weight(const fhc_model* model, const char* name, uint16_t* out, size_t cap);

/* The static plan of one pair() + mid() as JSON: the reference Session's walk (net/session.rs:26-66,
 * net/build.rs:532-736, and the op walk of build(), :149-484) at tensor-shape level.
 *   k: the fine loop's repeat count (the session's K); frame_w x frame_h: the host's frames (padded to 32);
 *   net_w x net_h: the internal network size (padded to 32 here); equal to the padded frame, the graph's own
 *   render_pix renders; smaller, the frames are downscaled (antialiased) into the network and the render runs at
 *   the padded frame size with the flow scaled per axis (build.rs:615-620, :717-736);
 *   repair: the periodic-structure repair's level (0 off, 1 safe, the reference's default, 2 aggressive): above 0
 *   a "gmhs" step {level, full_w} rewrites the pair's plain 4-channel flow in place after the pair stage
 *   (build.rs:640-660; fhc_gmhs of fhc_ops.h).
 * The walk keeps the reference's rules: slices, scales, neg and copy are views; an op whose outputs nobody reads is
 * skipped; a view a kernel needs plain is materialised first ("mat"); a conv followed by an add of its output
 * (read once) and a plain same-shape tensor takes the add as its residual (:222-237); blend_weights + mul + mul +
 * add is one blendmix (:417-450); the repeat body runs k times; the pair / mid boundary is mid_start
 * (model/graph.rs:182). Static protection and the fast render path are not part of this plan. Output:
 *   {"frame":[w,h], "padded":[wp,hp], "network":[iwp,ihp], "internal":b, "k":k, "mid_start":i,
 *    "buffers":[{"c","h","w","zeros","name"}...],
 *    "steps":[{"stage":"pair"|"mid", "op":..., "in":[view...], "out":view, ...}...]}
 * with view = {"buf":id, "c0":..., "c":..., "scale":...} (its height and width are the buffer's). Step ops and
 * their extra fields: rgba_in {frame}; rgba_out; interp {antialias}; conv {weight, bias, slope|null, cin, cout,
 * stride, act, residual: view|null, name}; mat; concat; avgpool {k}; warp; binary {fn: 0 add, 1 mul}; unary {fn: 0
 * scale (mul_t, t-dependent: mode fwd|bwd), 1 clamp {lo, hi}, 2 affine_out}; luma; luma_grad; sad {radius};
 * film_mlp (host, t-dependent); film {g: view}; convex {weights: view}; blend; blendmix; render {fsx, fsy} (the
 * graph's render_pix, or the frame-size render of the internal mode); gmhs {level, full_w} (ins: A, B, the flow).
 * Bytes written or -1. */
int fhc_model_plan(const fhc_model* model, uint32_t k, uint32_t frame_w, uint32_t frame_h, uint32_t net_w,
                   uint32_t net_h, uint32_t repair, char* json, size_t cap);


/* The distinct conv shapes of the static plan (the walk of fhc_model_plan, repair aside) at batch n, in plan order:
 * 7 words each (cin, cout, h, w, stride, n, kernel size 3), h and w the input size: the key of the choice table
 * (fhc_tune_get_ex). The reference's discovery build (autotune(), ops/conv/autotune.rs:186-213: every ConvShape
 * of the plan, deduplicated by its key). Returns the count (the first cap / 7 written) or -1. */
int fhc_model_conv_shapes(const fhc_model* model, uint32_t k, uint32_t frame_w, uint32_t frame_h, uint32_t net_w,
                          uint32_t net_h, uint32_t n, uint32_t* out, size_t cap);

/* Time every variant for each of those shapes (fhc_conv_autotune, `reps` launches per candidate) on device buffers
 * this call allocates and frees (the layout of fhc_conv.h with channel strides rounded up to 8; seeded inputs; the
 * model's weights; the residual of the shape's first use), recording the fastest in the process-wide choice table:
 * the reference's autotune of a plan (ops/conv/autotune.rs:180-245, a TuneRequest's table) as one blocking call at
 * plan time. Fused pairs are not tuned here. Returns the number of shapes tuned or a negative status. */
int fhc_model_autotune(const fhc_model* model, uint32_t k, uint32_t frame_w, uint32_t frame_h, uint32_t net_w,
                       uint32_t net_h, uint32_t n, int reps);

#ifdef __cplusplus
}
#endif
#endif
