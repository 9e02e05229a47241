/* fhc_conv: the FlyHigh convolution hot path on MI355X (gfx950), as a C ABI.
 *
 * A drop-in for the reference engine's conv op. The reference has no FFI at conv level: its conv boundary is the
 * Rust-internal record/replay pair
 *   plan time  BuildCtx::conv_pick(&ConvOp, Option<&Tensor>)  crates/flyhigh-engine/src/ops/conv/autotune.rs:159
 *              -> Gpu::conv_tc / conv_tiled_with / conv_direct crates/flyhigh-engine/src/ops/conv/kernels.rs:100-279
 *   run time   replay of the recorded Steps                   crates/flyhigh-engine/src/gpu/exec.rs:62-87
 * This ABI keeps that split: fhc_conv_plan_create is conv_pick + the weight packing (buildb/buildb_tap), and
 * fhc_conv_run is the replay of the plan's dispatches onto a HIP stream.
 *
 * Conventions (those of the reference's C ABI, crates/flyhigh-capi/src/lib.rs:27-48 and include/flyhigh.h:12):
 *  - every call returns 0 (or a size / count) on success and a negative value on error; the message is then in
 *    fhc_last_error(), which is thread-local; nothing aborts and nothing throws across this boundary;
 *  - handles are opaque; a plan is immutable after create; single-threaded use per handle for create/destroy,
 *    fhc_conv_run may be called from any thread on a stream of the device the plan was created on;
 *  - tensors are caller-owned device buffers (the reference's arena, gpu/alloc.rs:85); the library never
 *    allocates during fhc_conv_run and never assumes zeroed memory.
 *
 * Tensors are NHWC f16 (IEEE binary16 bit patterns in uint16_t), batch-major: element (img, y, x, c) of a view
 * lives at ((img * H + y) * W + x) * cstride + c0 + c. The reference stores planar [C][H][W] f16 with batch 1
 * (crates/flyhigh-engine/src/ops/tensor.rs:6-17); a channel view there (c0) is a channel offset here, and a
 * concat slice is written in place by giving the producer the slice's cstride/c0. Each buffer spans its view's full
 * strided extent: N * H * W * cstride halves (the input of a 16-byte aligned view may be read in whole 8-channel
 * groups up to that extent; channels outside the view never reach the result).
 */
#ifndef FHC_CONV_H
#define FHC_CONV_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define FHC_ACT_NONE 0u  /* identity: the reference's conv2d op with the `ones` slope (net/build.rs:210-220) */
#define FHC_ACT_PRELU 1u /* v > 0 ? v : slope[co] * v (shaders/conv.wgsl:33, conv_tiled.wgsl:64-66) */
#define FHC_ACT_LEAKY 2u /* v > 0 ? v : alpha * v, alpha an f32 constant */

/* The conv descriptor. Mirrors ImplicitGemmParams (crates/flyhigh-engine/src/ops/params.rs:188-210) and ConvArgs
 * (ops/conv/kernels.rs:7-22) with NHWC views added. Zero in a cstride means "dense" (cin for x, cout for y/r). */
typedef struct fhc_conv_desc {
    uint32_t n, h, w;            /* batch (1 in the reference), input height and width                       */
    uint32_t cin, cout;          /* true channel counts (no padding)                                           */
    uint32_t kh, kw;             /* 3,3 (the reference) or 1,1 (the 1x1 extension)                            */
    uint32_t stride, pad;        /* 3x3: stride 1 or 2, pad 1 (kernels.rs:40-42); 1x1: stride 1, pad 0         */
    uint32_t x_cstride, x_c0;    /* input view                                                                  */
    uint32_t y_cstride, y_c0;    /* output view (a concat slice)                                                */
    uint32_t r_cstride, r_c0;    /* residual view                                                               */
    uint32_t act;                /* FHC_ACT_*                                                                   */
    float alpha;                 /* FHC_ACT_LEAKY slope                                                         */
    uint32_t residual;           /* 1: y = f16(f32(f16(act(acc + bias))) + f32(r)) (conv_tiled.wgsl:57-61)      */
    uint32_t variant;            /* 0: planner (tune table, else heuristic); else a forced MI355X variant code  */
    uint32_t ksplit;             /* 0: planner; else a forced split-K count (1, 2, 4, 8)                        */
    uint32_t ref_cand;           /* 0xFF: none; else the reference's candidate code (candidates.rs:3-16), taken
                                    as a hint: its forced split-K nibble applies when ksplit is 0              */
} fhc_conv_desc;

typedef struct fhc_conv_plan fhc_conv_plan;

/* Message of the last failed call on this thread ("" if none). Replaces fh_last_error
 * (crates/flyhigh-capi/include/flyhigh.h:32) at conv granularity. */
const char* fhc_last_error(void);

/* Build a plan: validate the descriptor, choose the kernel variant and split-K (replaces BuildCtx::conv_pick,
 * ops/conv/autotune.rs:159-235, fixed-routing and tune-table branches), pack the OIHW f16 weights
 * [cout][cin][kh][kw] into MFMA fragment order (replaces Gpu::buildb / buildb_tap, ops/conv/kernels.rs:66-78,
 * :194-207) and upload them, with bias and slope, to the current HIP device. w, bias and slope are host
 * pointers; slope may be NULL unless act == FHC_ACT_PRELU. */
int fhc_conv_plan_create(const fhc_conv_desc* desc, const uint16_t* w_oihw, const uint16_t* bias,
                         const uint16_t* slope, fhc_conv_plan** out);

/* Device scratch the plan needs per run, in bytes (split-K partials; 0 for most plans). The reference keeps this
 * in arena scratch released after the op (gpu/alloc.rs:101-111, kernels.rs:178-179). */
size_t fhc_conv_workspace_bytes(const fhc_conv_plan* plan);

/* Output shape of the plan (hout, wout); any pointer may be NULL. Replaces out_size (kernels.rs:40-42). */
int fhc_conv_out_shape(const fhc_conv_plan* plan, uint32_t* hout, uint32_t* wout);

/* Enqueue the conv on `stream` (a hipStream_t; NULL = the null stream). x, y, res, workspace are device
 * pointers; res is read only when desc.residual is 1; workspace must hold fhc_conv_workspace_bytes. Asynchronous:
 * no allocation, no synchronisation, capturable in a hipGraph. Replaces the replay of the conv's Steps
 * (gpu/exec.rs:15-87). 16-byte aligned pointers and cstride/c0 multiples of 8 select the vector load path; with
 * c0 + cin rounded up to 8 <= cstride a partial channel group loads as one 16-byte group too. */
int fhc_conv_run(const fhc_conv_plan* plan, const void* x, void* y, const void* res, void* workspace,
                 void* stream);

/* fhc_conv_run without a workspace argument, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, hosts that forbid hipMalloc). No counterpart in the reference. The plan's scratch
 * (the split-K partials, fhc_conv_workspace_bytes) comes from a device array the library holds, one per GPU for the
 * life of the process, of FHC_STATIC_SCRATCH_BYTES; a plan that needs more is refused with an error status. The array
 * is a file-scope device variable of the library: its memory is reserved on every GPU the library's code is loaded
 * onto, whether or not the process ever calls this function. 32 MiB holds the largest split-K plan of the 1080p
 * frame's layers (the 1080p/16 128 -> 128 conv split 8 ways: 33,423,360 bytes of f32 partials). The call
 * allocates nothing. Every call on one GPU shares that GPU's array: calls whose plans need scratch and that may
 * overlap on one GPU (other streams, other threads) race on it, so run them in one stream order. The array keeps
 * the last call's partials; every partial a call reads it has written itself first. Plans without scratch run
 * exactly as fhc_conv_run runs them. */
#define FHC_STATIC_SCRATCH_BYTES (32u << 20)
int fhc_conv_run_noalloc(const fhc_conv_plan* plan, const void* x, void* y, const void* res, void* stream);

/* JSON description of the plan: variant, tile, split-K, grid, packed sizes, algorithmic FLOPs and bytes. Returns
 * bytes written (without the NUL) or -1 when cap is too small. Replaces plan_dump for one conv
 * (ops/step.rs:51-88). */
int fhc_conv_describe(const fhc_conv_plan* plan, char* json, size_t cap);

void fhc_conv_plan_destroy(fhc_conv_plan* plan);

/* A fused pair: conv A (3x3, stride 1 or 2, no residual) and conv B (3x3 stride 1) that reads A's output, run as one
 * launch with A's output kept on chip. It serves two consecutive conv ops of the graph whose intermediate tensor has
 * no other reader (graph.json's enc.e1 -> enc.e2, enc.e3 -> enc.e4, film.h1 -> film.h2, refine.q1 -> q2, q3 -> q4,
 * fine.r2 -> r3). The result is the one the two plans give run in turn: A's output is rounded to f16 and B reads it
 * with zero padding. No counterpart in the reference, which records one dispatch per conv op (net/build.rs:209-278).
 * desc_b: B's n, h, w and cin equal A's n, output height and width and cout; B's input view is ignored. flags:
 * FHC_PAIR_RES_MID makes B's residual A's output (B.residual set, B.cout == B.cin; graph.json's "add" of e2 and e1,
 * e4 and e3), else B's residual, if any, is the `res` tensor of fhc_conv_run; bits 8-15: output rows per tile (1, 2,
 * 4 or 8 as instantiated; 0: the tallest that still gives 256 workgroups, else the shortest); bits 16-19: wave rows
 * splitting them (1 or 2; 0: 1 where instantiated, else 2); bits 20-21: the loop (1: one workgroup per tile, both
 * layers' weights loaded per tile; 2: a resident grid that loads them once and loops over the tiles, for 64 -> 64 ->
 * 64 at 4 rows x 2 wave rows and for the frame's pairs at 4 or 8 rows, 64-channel pairs with 2 wave rows; 3: a
 * resident grid whose A and B stages run on separate waves, pipelined across tiles, at 4 rows, and 8 rows for
 * 32-channel pairs; 0: the resident grid where it is instantiated and there are at least 2048 tiles, loop 3 first).
 * The plan runs with fhc_conv_run (x: A's input, y and res: B's output and residual), is described by
 * fhc_conv_describe (family "pair") and freed by fhc_conv_plan_destroy. The instantiated pairs cover, in channels
 * A.cin -> A.cout -> B.cout: stride 1 33..64 -> 49..64 -> 49..64 (resident grid only), stride 2 <= 32 -> 33..48 ->
 * 33..48 (2 or 4 rows) and 33..64 -> 65..80 -> 65..80 (1 or 2 rows, one wave row), and stride 1 33..64 -> 33..48 ->
 * 33..48, <= 32 -> 17..32 -> 17..32 and <= 32 -> 17..32 -> <= 16 (2 or 4 rows); other shapes are an error status. */
#define FHC_PAIR_RES_MID 1u
/* FHC_PAIR_AFFINE_OUT: B's f16 output then goes through the graph's affine_out op (unary.wgsl's op 2:
 * 2 / (1 + exp(-v)) - 1 in f32, rounded to f16 again; graph.json op 81 after refine.q4), so the pair writes that op's
 * output; it runs the one-workgroup-per-tile loop (bits 20-21 0 or 1) and needs B.cout <= 4 and no residual. No
 * counterpart in the reference, which dispatches the op on its own. */
#define FHC_PAIR_AFFINE_OUT 2u
/* FHC_PAIR_FILM_IN: A's input is modulated per channel as it is staged, the graph's film_modulate op
 * (film.wgsl: f16(x * (1 + gamma[c]) + beta[c]) in f32; graph.json op 50 before film.h1), so the pair reads the op's
 * input and the op's dispatch goes; the zero padding stays zero. The FiLM vectors (per image: cin gammas, then cin
 * betas, f16) are an argument of each run: the plan runs with fhc_conv_pair_run_film only (fhc_conv_run refuses it),
 * in the one-workgroup-per-tile loop (bits 20-21 0 or 1), without an external residual for B. No counterpart in the
 * reference, which dispatches the op on its own. */
#define FHC_PAIR_FILM_IN 4u
/* A's K order. By default, where A has at most 8 (or 16) input channels (graph.json's enc.e1: 3, refine.q1: 14) and
 * a configuration packs them, 4 (2) taps share each 32-wide K-step, each tap's channels padded to 8 (16): 3 (5) MFMA
 * K-steps per output where one tap a step takes 9, the reference's dense K (buildb, ops/conv/kernels.rs:64-78,
 * ⌈9 cin / 16⌉ 16) taken to whole taps. FHC_PAIR_TAP32 keeps one tap a step, channels padded to 32. */
#define FHC_PAIR_TAP32 0x400000u
int fhc_conv_pair_plan_create(const fhc_conv_desc* desc_a, const uint16_t* w_a, const uint16_t* bias_a,
                              const uint16_t* slope_a, const fhc_conv_desc* desc_b, const uint16_t* w_b,
                              const uint16_t* bias_b, const uint16_t* slope_b, uint32_t flags, fhc_conv_plan** out);

/* Sibling convs: two convs A and B that read the same input view with the same geometry, as one launch (the
 * one-tile direct kernel computing A's output channels, zero channels up to a multiple of 4, then B's, each with
 * the K loop the same configuration runs for it alone). A may take a residual; B takes none; identity or PReLU
 * activations. Instantiated: 3x3 stride 1, 33-64 input channels, A.cout rounded up to 4 plus B.cout at most 48
 * (graph.json's fine.out and up.w, which both read the fine block's h: 48 -> 7 + 36). The plan runs with
 * fhc_conv_sibling_run only (fhc_conv_run refuses it) and is freed by fhc_conv_plan_destroy. No counterpart in the
 * reference, which records a dispatch per conv (net/build.rs:209-278). */
int fhc_conv_sibling_plan_create(const fhc_conv_desc* desc_a, const uint16_t* w_a, const uint16_t* bias_a,
                                 const uint16_t* slope_a, const fhc_conv_desc* desc_b, const uint16_t* w_b,
                                 const uint16_t* bias_b, const uint16_t* slope_b, fhc_conv_plan** out);
/* x: the shared input; y_a, res_a: A's output and residual (res_a NULL without one); y_b: B's output. Async on
 * `stream`, no allocation, capturable in a HIP graph, as fhc_conv_run. Stands in for fhc_conv_run of A then of B. */
int fhc_conv_sibling_run(const fhc_conv_plan* plan, const void* x, void* y_a, const void* res_a, void* y_b,
                         void* stream);

/* Runs a pair plan created with FHC_PAIR_FILM_IN: x is A's input before the modulation, film the FiLM vectors
 * (n x 2 x A.cin f16, device memory), y B's output. Async on `stream`, no allocation, capturable in a HIP graph, as
 * fhc_conv_run. Stands in for fhc_conv_run(film_modulate's output, ...) after the reference's film dispatch
 * (`Gpu::film`, ops/network.rs:56-61, shaders/film.wgsl:11-14). */
int fhc_conv_pair_run_film(const fhc_conv_plan* pair, const void* x, const void* film, void* y, void* stream);

/* The planner's choice for a descriptor without creating a plan (no device call): the same JSON as
 * fhc_conv_describe, sizes included. For host-side tests and for tools that print the plan of a graph
 * (the reference's FH_TUNE_VERBOSE listing, ops/conv/autotune.rs:217-228). Bytes written or -1. */
int fhc_conv_plan_dry(const fhc_conv_desc* desc, char* json, size_t cap);

/* Time every variant fhc_variant_list gives for `desc` on the caller's device buffers (x, y, res: as for
 * fhc_conv_run; y is overwritten) with `reps` back-to-back launches captured in a HIP graph on a private stream,
 * record the fastest in the choice table under the descriptor's key, and return its code (or -1). *best_us
 * receives its time per launch when not NULL. The per-shape autotune of the reference's conv_pick
 * (ops/conv/autotune.rs:199-230): a blocking round trip per candidate, for plan time only. The host weights are
 * those of fhc_conv_plan_create. */
int fhc_conv_autotune(const fhc_conv_desc* desc, const uint16_t* w_oihw, const uint16_t* bias,
                      const uint16_t* slope, const void* x, void* y, const void* res, int reps, float* best_us);

/* ---- The planner's choice table ------------------------------------------------------------------------
 * The reference's TuneTable (ops/conv/tune_cache.rs:6-9, :39-64) keys a choice by (cin, cout, h, w, stride), h and
 * w the INPUT size, one "cin,cout,h,w,stride=code" per line. This table adds the batch n and the kernel size k (1 or
 * 3) to the key, since a batched conv and a 1x1 conv need choices of their own: the key of a batch-1 3x3 conv is
 * written in the reference's 5 fields, any other as "cin,cout,h,w,stride,n,k=code"; both forms parse, malformed
 * lines are skipped. The codes are MI355X variant codes (fhc_variant_name); fhc_tune_parse also takes a variant
 * name in place of the code, which stays valid across builds. The table is process-wide and consulted by
 * fhc_conv_plan_create (under the descriptor's n and kh) when desc.variant is 0. */
int fhc_tune_parse(const char* text);           /* merges; returns the number of entries read, or -1   */
int fhc_tune_format(char* text, size_t cap);    /* sorted lines; bytes written, or -1 if cap too small */
int fhc_tune_clear(void);
/* code or -1: the entry of a batch-1 3x3 conv (the reference's key) */
int fhc_tune_get(uint32_t cin, uint32_t cout, uint32_t h, uint32_t w, uint32_t stride);
/* code or -1: the entry of batch n, kernel size k */
int fhc_tune_get_ex(uint32_t cin, uint32_t cout, uint32_t h, uint32_t w, uint32_t stride, uint32_t n, uint32_t k);
/* Name of an MI355X variant code into buf; bytes written or -1. Codes 1..127 are the K-chunked kernels: bits 0-4
 * the configuration (1..10 the chunked implicit GEMM, "igemm.t8x16.n64"; 16..28 the deep-layer kernel with LDS
 * DMA, "gemm.t8x16.n48.f2x3.w4x1.c32.p2"), bits 5-6 the global split (1, 2, 4, 8: "/k2"); 128 + i the direct
 * kernel's configuration i ("direct.c64.t4x1.n64/p"). */
int fhc_variant_name(uint32_t code, char* buf, size_t cap);
/* The MI355X variant codes worth timing for a descriptor (the counterpart of cand_list); count written, or -1. */
int fhc_variant_list(const fhc_conv_desc* desc, uint32_t* codes, size_t cap);

/* ---- The reference planner, restated (host logic, no GPU) ---------------------------------------------
 * For parity of the planner itself: these reproduce the reference's kernel choice and dispatch words so that
 * tests can compare them with the reference's golden plans (crates/flyhigh-engine/tests/golden/<config>.<class>.txt). */

/* cand_list (ops/conv/candidates.rs:28-85); try_all stands for FH_TRY_ALL. Returns the count written, or -1. */
int fhc_ref_cand_list(int coop, uint32_t cout, uint32_t hout, uint32_t wout, int direct_ok, int try_all,
                      uint8_t* out, size_t cap);
/* cand_name (ops/conv/candidates.rs:17-24) into buf; bytes written or -1. */
int fhc_ref_cand_name(uint8_t code, char* buf, size_t cap);

/* One conv of the reference graph at plan time (ConvOp, ops/conv/autotune.rs:100-109, plus the planner's
 * residual peephole of net/build.rs:222-237). */
typedef struct fhc_ref_conv {
    uint32_t cin, cout, h, w, stride;
    uint32_t residual;  /* a fused `add` follows                                                   */
    uint32_t coop;      /* the device class has cooperative-matrix (tensor-core) kernels            */
    uint32_t cand;      /* 0xFF: fixed routing (autotune off, autotune.rs:191-198); else a CAND code */
    uint32_t ksplit_env;/* FH_KSPLIT (0 = unset)                                                    */
    uint32_t f32_mode;  /* the portable-f32 class: weights stored as f32 (4-byte elements)             */
} fhc_ref_conv;

/* The dispatches the reference records for that conv (conv_cand, autotune.rs:115-154, and the Gpu::conv_* launch
 * math, kernels.rs:99-279), one per line: "pipeline (gx,gy,gz) w<packed weight bytes> p<param words as 8-digit
 * hex, space separated>". Returns bytes written or -1. */
int fhc_ref_conv_steps(const fhc_ref_conv* c, char* text, size_t cap);

/* ---- Diagnostics -----------------------------------------------------------------------------------------
 * One v_mfma_f32_16x16x32_f16 with the operand layouts the conv kernels assume: d (16x16 f32, row-major) =
 * a (16x32 f16, row-major) x b (32x16 f16, row-major). Device pointers; asynchronous on `stream`. It has no
 * counterpart in the reference (the reference's own probes of its cooperative-matrix layout are
 * crates/flyhigh-cli/src/cli/coop_tests.rs:7-113). */
int fhc_probe_mfma_layout(const void* a, const void* b, void* d, void* stream);

/* The dense f16 MFMA rate the device sustains, for rooflines against an achievable peak next to the vendor one:
 * `blocks` workgroups of 256 threads, each wave issuing 16 * iters v_mfma_f32_16x16x32_f16 (16384 FLOPs each) on
 * register operands in 16 independent chains, so one launch does blocks * 4 * 16 * iters * 16384 FLOPs; the caller
 * times it on `stream` (4 workgroups per CU keep every SIMD busy).
 * out: device memory of blocks * 1024 floats. No counterpart in the reference. */
int fhc_probe_mfma_rate(uint32_t blocks, uint32_t iters, void* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
