/* CPU oracle of the FlyHigh convolution hot path: TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's conv arithmetic, used by tests/, by the smoke check and by the
 * CPU-baseline leg of bench.py, and only there, as the checker. The product (libfhconv.so) never links,
 * loads or calls anything in this directory.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference repository).
 * Pinning (what independently checks each function) is listed per function below; none is "parity unpinned"
 * except where said.
 */
#ifndef FH_ORACLE_H
#define FH_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* f32 -> f16 round-to-nearest-even, f16 -> f32 exact (the rounding of half 2.7.1 `f16::from_f32`, used by
 * crates/flyhigh-engine/src/gpu/alloc.rs:59-70, and of WGSL `f16(x)` as the build assumes it).
 * Pinned by tests against numpy's float16 conversion over all 65536 f16 patterns and 10^6 f32 values. */
uint16_t fho_f32_to_f16(float f);
float fho_f16_to_f32(uint16_t h);
/* the same over arrays */
void fho_f32_to_f16_n(const float* in, uint16_t* out, size_t n);
void fho_f16_to_f32_n(const uint16_t* in, float* out, size_t n);

/* The conv as the oracle sees it: NHWC f16 views with a pixel stride (cstride) and a channel offset (c0). */
typedef struct fho_conv {
    uint32_t n, h, w, cin, cout;
    uint32_t kh, kw, stride, pad;    /* 3,3,{1,2},1 (the reference); 1,1,1,0 (the 1x1 extension) */
    uint32_t x_cstride, x_c0, y_cstride, y_c0, r_cstride, r_c0;
    uint32_t act;                    /* 0 identity, 1 PReLU(slope[co]), 2 LeakyReLU(alpha) */
    float alpha;
    uint32_t residual;               /* y = f16(f32(f16(act(acc + b))) + f32(r)) */
} fho_conv;

/* summation orders of the reference kernels */
enum {
    FHO_ORDER_TILED = 0, /* shaders/conv_tiled.wgsl:89-127: acc = 0, k = ci*9 + tap ascending, then + bias */
    FHO_ORDER_NAIVE = 1, /* shaders/conv.wgsl:18-31: acc starts at the bias, ci, ky, kx ascending           */
    FHO_ORDER_SPLITK = 2 /* conv_tiled.wgsl:94-97 + splitk_reduce.wgsl:17-18: per-split partials summed z=0..  */
};

/* Output size (crates/flyhigh-engine/src/ops/conv/kernels.rs:40-42 for 3x3 pad 1; the same formula with the
 * descriptor's kh/pad for the 1x1 extension). */
uint32_t fho_out_size(uint32_t in, uint32_t k, uint32_t stride, uint32_t pad);

/* The reference conv, one output element at a time (shaders/conv.wgsl:14-35 for indexing and zero padding;
 * shaders/conv_tiled.wgsl:57-75 for the epilogue: bias, PReLU select, f16 round, then the residual add rounded
 * again, the same as the binary add of shaders/binary.wgsl:15-16 after the tensor-core kernels).
 * order: FHO_ORDER_*; ksplit: number of K splits for FHO_ORDER_SPLITK (the reference's z count), split over
 * kp/16 K-steps exactly as conv_tiled.wgsl:94-97 does. Returns 0, or -1 on a bad descriptor.
 * Pinned by: golden vectors computed with torch.nn.functional.conv2d in float64 (tests/golden), delta and
 * all-ones closed forms, and a constructed split-K case whose result depends on the z order. */
int fho_conv_run(const fho_conv* d, const uint16_t* x, const uint16_t* w_oihw, const uint16_t* bias,
                 const uint16_t* slope, const uint16_t* res, uint16_t* y, int order, uint32_t ksplit);

/* The same arithmetic (FHO_ORDER_TILED) split over output rows on `threads` POSIX threads: the CPU baseline. */
int fho_conv_run_mt(const fho_conv* d, const uint16_t* x, const uint16_t* w_oihw, const uint16_t* bias,
                    const uint16_t* slope, const uint16_t* res, uint16_t* y, int threads);

#ifdef __cplusplus
}
#endif
#endif
