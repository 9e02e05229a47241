// Instantiations of the deep-layer conv (gemm_impl.h), one per kGemmCfgs entry.
#include "conv_kernels.h"
#include "gemm_impl.h"

namespace fhc {

namespace {

template <int I>
LaunchFn gemm_entry(const void** kernel) {
    constexpr GemmCfg c = kGemmCfgs[I];
    if (kernel) *kernel = gemm_kernel<c.s, c.ck, c.fm, c.na, c.wm, c.wn, c.st>();
    return launch_gemm<c.s, c.ck, c.fm, c.na, c.wm, c.wn, c.st>;
}

template <int... I>
LaunchFn gemm_pick(int index, const void** kernel, std::integer_sequence<int, I...>) {
    LaunchFn fn = nullptr;
    ((index == I ? (void)(fn = gemm_entry<I>(kernel)) : (void)0), ...);
    return fn;
}

}  // namespace

LaunchFn gemm_launcher(int index, const void** kernel) {
    if (index < 0 || index >= kNumGemm) return nullptr;
    return gemm_pick(index, kernel, std::make_integer_sequence<int, kNumGemm>{});
}

}  // namespace fhc
