/* CPU oracle of the FlyHigh convolution hot path: TEST INFRASTRUCTURE ONLY (see fh_oracle.h).
 * Only tests/, the smoke check and bench.py's CPU-baseline leg use this file, as the checker. */
#include "fh_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- f16 <-> f32 -------------------------------------------------------------------------------------- */

uint16_t fho_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t man = u & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan (quiet the nan, keep the top payload bits) */
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow to inf */
    if (e <= 0) {
        /* subnormal f16 (or zero): value = man24 * 2^(exp-150); f16 subnormal unit is 2^-24 */
        if (e < -10) return (uint16_t)sign; /* below half of the smallest subnormal: rounds to zero */
        uint32_t m = man | 0x800000u;     /* 24-bit significand */
        uint32_t shift = (uint32_t)(14 - e); /* bits to drop so that the unit becomes 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfw = 1u << (shift - 1u);
        if (rem > halfw || (rem == halfw && (q & 1u))) q++;
        return (uint16_t)(sign | q); /* q may carry into the exponent field: that is the correct result */
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry up to inf: correct */
    return (uint16_t)(sign | q);
}

float fho_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: normalise */
            int32_t e = -14;
            while (!(man & 0x400u)) {
                man <<= 1;
                e--;
            }
            man &= 0x3ffu;
            u = sign | ((uint32_t)(e + 127) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void fho_f32_to_f16_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = fho_f32_to_f16(in[i]);
}

void fho_f16_to_f32_n(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = fho_f16_to_f32(in[i]);
}

/* ---- the conv ------------------------------------------------------------------------------------------ */

uint32_t fho_out_size(uint32_t in, uint32_t k, uint32_t stride, uint32_t pad) {
    /* kernels.rs:40-42: (h + 2 - 3) / s + 1 for k = 3, pad = 1 */
    return (in + 2u * pad - k) / stride + 1u;
}

static int check_desc(const fho_conv* d) {
    if (!d || d->n == 0 || d->h == 0 || d->w == 0 || d->cin == 0 || d->cout == 0) return -1;
    if (d->stride == 0 || d->kh == 0 || d->kw == 0) return -1;
    if (d->h + 2u * d->pad < d->kh || d->w + 2u * d->pad < d->kw) return -1;
    if (d->x_cstride < d->x_c0 + d->cin || d->y_cstride < d->y_c0 + d->cout) return -1;
    if (d->residual && d->r_cstride < d->r_c0 + d->cout) return -1;
    return 0;
}

/* the epilogue of conv_tiled.wgsl:62-67 (store4) and :57-61 (fin): bias, activation, f16, residual */
static uint16_t epilogue(const fho_conv* d, float acc_plus_bias, const uint16_t* slope, uint32_t co,
                         const uint16_t* rpix) {
    float v = acc_plus_bias;
    float r = v;
    if (d->act == 1u) {
        float s = fho_f16_to_f32(slope[co]);
        r = v > 0.0f ? v : s * v;
    } else if (d->act == 2u) {
        r = v > 0.0f ? v : d->alpha * v;
    }
    uint16_t hq = fho_f32_to_f16(r);
    if (d->residual) {
        float sum = fho_f16_to_f32(hq) + fho_f16_to_f32(rpix[co]);
        hq = fho_f32_to_f16(sum);
    }
    return hq;
}

/* one input element of the implicit GEMM column k = ci * taps + tap (conv_tiled.wgsl:45-55); 0 outside */
static inline float gather(const fho_conv* d, const uint16_t* x, uint32_t img, uint32_t oy, uint32_t ox, uint32_t k,
                           int* inside) {
    uint32_t taps = d->kh * d->kw;
    uint32_t ci = k / taps, tap = k - ci * taps;
    uint32_t ky = tap / d->kw, kx = tap - ky * d->kw;
    int32_t yi = (int32_t)(oy * d->stride + ky) - (int32_t)d->pad;
    int32_t xi = (int32_t)(ox * d->stride + kx) - (int32_t)d->pad;
    if (yi < 0 || yi >= (int32_t)d->h || xi < 0 || xi >= (int32_t)d->w) {
        *inside = 0;
        return 0.0f;
    }
    *inside = 1;
    size_t p = ((size_t)img * d->h + (size_t)yi) * d->w + (size_t)xi;
    return fho_f16_to_f32(x[p * d->x_cstride + d->x_c0 + ci]);
}

static void conv_rows(const fho_conv* d, const uint16_t* x, const uint16_t* wt, const uint16_t* bias,
                      const uint16_t* slope, const uint16_t* res, uint16_t* y, int order, uint32_t ksplit,
                      uint32_t row0, uint32_t row1) {
    uint32_t hout = fho_out_size(d->h, d->kh, d->stride, d->pad);
    uint32_t wout = fho_out_size(d->w, d->kw, d->stride, d->pad);
    uint32_t taps = d->kh * d->kw;
    uint32_t K = d->cin * taps;
    uint32_t kp = (K + 15u) / 16u * 16u; /* kernels.rs:68 */
    uint32_t kt_count = kp / 16u;
    if (ksplit < 1u) ksplit = 1u;
    uint32_t per = (kt_count + ksplit - 1u) / ksplit; /* conv_tiled.wgsl:96 */
    for (uint32_t row = row0; row < row1; row++) {
        uint32_t img = row / hout, oy = row - img * hout;
        for (uint32_t ox = 0; ox < wout; ox++) {
            size_t op = ((size_t)img * hout + oy) * wout + ox;
            const uint16_t* rpix = d->residual ? res + op * d->r_cstride + d->r_c0 : NULL;
            for (uint32_t co = 0; co < d->cout; co++) {
                const uint16_t* wrow = wt + (size_t)co * K; /* OIHW: [co][ci][ky][kx] = [co][k] */
                float b = fho_f16_to_f32(bias[co]);
                float out;
                if (order == FHO_ORDER_NAIVE) {
                    /* conv.wgsl:18-31: acc = bias, then ci, ky, kx; out-of-image taps skipped */
                    float acc = b;
                    for (uint32_t k = 0; k < K; k++) {
                        int in;
                        float a = gather(d, x, img, oy, ox, k, &in);
                        if (in) acc = acc + a * fho_f16_to_f32(wrow[k]);
                    }
                    out = acc;
                } else if (order == FHO_ORDER_SPLITK) {
                    /* conv_tiled.wgsl:94-97 (z-th K range, acc from 0) + splitk_reduce.wgsl:17-18 (z order) */
                    float s = 0.0f;
                    for (uint32_t z = 0; z < ksplit; z++) {
                        uint32_t kt0 = z * per, kt1 = kt0 + per < kt_count ? kt0 + per : kt_count;
                        float part = 0.0f;
                        for (uint32_t k = kt0 * 16u; k < kt1 * 16u && k < K; k++) {
                            int in;
                            float a = gather(d, x, img, oy, ox, k, &in);
                            part = part + a * fho_f16_to_f32(wrow[k]);
                        }
                        s = z == 0 ? part : s + part;
                    }
                    out = s + b;
                } else {
                    /* conv_tiled.wgsl:99-118 then store4 :64-65: acc from 0 over k ascending, then + bias */
                    float acc = 0.0f;
                    for (uint32_t k = 0; k < K; k++) {
                        int in;
                        float a = gather(d, x, img, oy, ox, k, &in);
                        acc = acc + a * fho_f16_to_f32(wrow[k]);
                    }
                    out = acc + b;
                }
                y[op * d->y_cstride + d->y_c0 + co] = epilogue(d, out, slope, co, rpix);
            }
        }
    }
}

int fho_conv_run(const fho_conv* d, const uint16_t* x, const uint16_t* w_oihw, const uint16_t* bias,
                 const uint16_t* slope, const uint16_t* res, uint16_t* y, int order, uint32_t ksplit) {
    if (check_desc(d) || !x || !w_oihw || !bias || !y) return -1;
    if (d->act == 1u && !slope) return -1;
    if (d->residual && !res) return -1;
    uint32_t hout = fho_out_size(d->h, d->kh, d->stride, d->pad);
    conv_rows(d, x, w_oihw, bias, slope, res, y, order, ksplit, 0, d->n * hout);
    return 0;
}

typedef struct {
    const fho_conv* d;
    const uint16_t *x, *w, *b, *s, *r;
    uint16_t* y;
    uint32_t r0, r1;
} job_t;

static void* job_main(void* p) {
    job_t* j = (job_t*)p;
    conv_rows(j->d, j->x, j->w, j->b, j->s, j->r, j->y, FHO_ORDER_TILED, 1, j->r0, j->r1);
    return NULL;
}

int fho_conv_run_mt(const fho_conv* d, const uint16_t* x, const uint16_t* w_oihw, const uint16_t* bias,
                    const uint16_t* slope, const uint16_t* res, uint16_t* y, int threads) {
    if (check_desc(d) || !x || !w_oihw || !bias || !y || threads < 1 || threads > 1024) return -1;
    if (d->act == 1u && !slope) return -1;
    if (d->residual && !res) return -1;
    uint32_t rows = d->n * fho_out_size(d->h, d->kh, d->stride, d->pad);
    if ((uint32_t)threads > rows) threads = (int)rows;
    pthread_t* th = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    job_t* jobs = (job_t*)calloc((size_t)threads, sizeof(job_t));
    if (!th || !jobs) {
        free(th);
        free(jobs);
        return -1;
    }
    int started = 0, rc = 0;
    for (int t = 0; t < threads; t++) {
        jobs[t] = (job_t){d, x, w_oihw, bias, slope, res, y, (uint32_t)((uint64_t)rows * t / threads),
                          (uint32_t)((uint64_t)rows * (t + 1) / threads)};
        if (pthread_create(&th[t], NULL, job_main, &jobs[t]) != 0) {
            rc = -1;
            break;
        }
        started++;
    }
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
    return rc;
}
