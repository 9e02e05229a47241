// The instantiations of the fused conv pair (pair_impl.h), indexed like kPairCfgs.
#include <utility>

#include "gm_fit.h"
#include "pair_impl.h"

namespace fhc {

namespace {

template <int I>
PairLaunchFn pair_entry(const void** kernel) {
    constexpr PairCfg c = kPairCfgs[I];
    constexpr int cp = c.cpa ? c.cpa : 32;
    if constexpr (c.persist == 2) {
        if (kernel)
            *kernel = reinterpret_cast<const void*>(&conv_pair_ws<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, cp>);
        return launch_pair_ws<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, cp>;
    } else if constexpr (c.persist) {
        if (kernel)
            *kernel = reinterpret_cast<const void*>(&conv_pair_p<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm, cp>);
        return launch_pair_p<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm, cp>;
    } else {
        if (kernel)
            *kernel = reinterpret_cast<const void*>(
                &conv_pair<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm, true, false, cp>);
        return launch_pair<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm, cp>;
    }
}

template <int... I>
PairLaunchFn pair_pick(int index, const void** kernel, std::integer_sequence<int, I...>) {
    PairLaunchFn fn = nullptr;
    ((index == I ? (void)(fn = pair_entry<I>(kernel)) : (void)0), ...);
    return fn;
}

}  // namespace

PairLaunchFn pair_launcher(int index, const void** kernel) {
    if (index < 0 || index >= kNumPair) return nullptr;
    return pair_pick(index, kernel, std::make_integer_sequence<int, kNumPair>{});
}

namespace {

template <int SA, int CA32, int CB32, int TH>
union FitPairLds {
    gmfit::RoundLds fit;
    PairLds<SA, CA32, CB32, TH> pair;
};

template <int SA, int CA32, int CB32, int NBA, int NBB, int TH, bool VEC>
__global__ __launch_bounds__(192) void fit_film_pair_kernel(FitRoundArgs f, PairKArgs pk) {
    static_assert((NBA > NBB ? NBA : NBB) == 3, "the pair's workgroup is 192 threads");
    constexpr uint32_t NFIT = gmfit::kNwg * 4;
    __shared__ __align__(16) FitPairLds<SA, CA32, CB32, TH> lds;
    if (blockIdx.x < NFIT)  // uniform over the workgroup
        gmfit::round_body<192>(f.flow, f.cs, f.c0, f.h8, f.w8, f.delta, f.round, f.part_in, f.part_out,
                               blockIdx.x % gmfit::kNwg, blockIdx.x / gmfit::kNwg, lds.fit);
    else
        conv_pair_tile<SA, CA32, CB32, NBA, NBB, TH, 1, VEC, true>(pk, (int)(blockIdx.x - NFIT), lds.pair);
}

template <int I>
hipError_t fit_pair_launch(const FitRoundArgs& f, const PairKArgs& pk, uint32_t tiles, hipStream_t s) {
    constexpr PairCfg c = kPairCfgs[I];
    const dim3 grid(gmfit::kNwg * 4 + tiles);
    if (pk.a.xvec)
        hipLaunchKernelGGL((fit_film_pair_kernel<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, true>), grid, dim3(192), 0, s,
                           f, pk);
    else
        hipLaunchKernelGGL((fit_film_pair_kernel<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, false>), grid, dim3(192),
                           0, s, f, pk);
    return hipGetLastError();
}

constexpr int find_pair(int sa, int ca32, int cb32, int nba, int nbb, int th, int wm, int persist) {
    for (int i = 0; i < kNumPair; i++) {
        const PairCfg& c = kPairCfgs[i];
        if (c.sa == sa && c.ca32 == ca32 && c.cb32 == cb32 && c.nba == nba && c.nbb == nbb && c.th == th &&
            c.wm == wm && c.persist == persist && c.cpa == 0)
            return i;
    }
    return -1;
}

}  // namespace

FitPairLaunchFn fit_pair_launcher(int index) {
    // the FiLM head's pair (48 -> 48 -> 48) at 2 or 4 rows per tile, one wave row
    constexpr int p2 = find_pair(1, 64, 64, 3, 3, 2, 1, 0), p4 = find_pair(1, 64, 64, 3, 3, 4, 1, 0);
    static_assert(p2 >= 0 && p4 >= 0, "the FiLM pair's configurations");
    if (index == p2) return fit_pair_launch<p2>;
    if (index == p4) return fit_pair_launch<p4>;
    return nullptr;
}

}  // namespace fhc
