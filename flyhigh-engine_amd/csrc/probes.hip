// Hardware probes: the MFMA operand layout the conv kernels assume, and the dense f16 MFMA rate the chip sustains.
// Built with -amdgpu-mfma-vgpr-form (Makefile): a loop-carried accumulator array otherwise lands in AGPRs with
// copies between iterations, and the probe then measures the copies.
#include "conv_kernels.h"
#include "direct_impl.h"

namespace fhc {

__global__ __launch_bounds__(64) void mfma_probe(const uint16_t* A, const uint16_t* B, float* D) {
    // A row-major 16x32, B row-major 32x16, D row-major 16x16
    const int l = threadIdx.x;
    h8 av, bv;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int k = 8 * (l >> 4) + i;
        av[i] = __builtin_bit_cast(_Float16, A[(l & 15) * 32 + k]);
        bv[i] = __builtin_bit_cast(_Float16, B[k * 16 + (l & 15)]);
    }
    f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; r++) D[(4 * (l >> 4) + r) * 16 + (l & 15)] = d[r];
}

// Each wave keeps kRateAcc independent 16x16x32 accumulators busy for `iters` rounds (operands in registers, no
// memory traffic besides one store per lane). A dependent MFMA waits about 50 cycles for its predecessor against
// 16 cycles of issue, so a wave needs several chains in flight; 16 per wave at 4 waves per SIMD measure the rate.
__global__ __launch_bounds__(256) void mfma_rate_probe(f4* out, int iters) {
    h8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (_Float16)((threadIdx.x & 7) * 0.001f + i * 0.01f);
        b[i] = (_Float16)(i * 0.02f);
    }
    f4 acc[kRateAcc];
#pragma unroll
    for (int j = 0; j < kRateAcc; j++) acc[j] = f4{(float)j, 0.0f, 0.0f, 0.0f};  // distinct: no chain is merged
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < kRateAcc; j++) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
    }
    f4 s = acc[0];
#pragma unroll
    for (int j = 1; j < kRateAcc; j++) s += acc[j];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

hipError_t mfma_probe_launch(const uint16_t* a, const uint16_t* b, float* d, hipStream_t s) {
    hipLaunchKernelGGL(mfma_probe, dim3(1), dim3(64), 0, s, a, b, d);
    return hipGetLastError();
}

hipError_t mfma_rate_probe_launch(unsigned blocks, int iters, float* out, hipStream_t s) {
    hipLaunchKernelGGL(mfma_rate_probe, dim3(blocks), dim3(256), 0, s, reinterpret_cast<f4*>(out), iters);
    return hipGetLastError();
}

}  // namespace fhc
