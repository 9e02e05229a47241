// The instantiations of the fused conv pair (pair_impl.h), indexed like kPairCfgs.
#include <utility>

#include "pair_impl.h"

namespace fhc {

namespace {

template <int I>
PairLaunchFn pair_entry(const void** kernel) {
    constexpr PairCfg c = kPairCfgs[I];
    if constexpr (c.persist == 2) {
        if (kernel) *kernel = reinterpret_cast<const void*>(&conv_pair_ws<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th>);
        return launch_pair_ws<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th>;
    } else if constexpr (c.persist) {
        if (kernel) *kernel = reinterpret_cast<const void*>(&conv_pair_p<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm>);
        return launch_pair_p<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm>;
    } else {
        if (kernel) *kernel = reinterpret_cast<const void*>(&conv_pair<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm, true>);
        return launch_pair<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm>;
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

}  // namespace fhc
