// The instantiations of the fused conv pair (pair_impl.h), indexed like kPairCfgs.
#include "pair_impl.h"

namespace fhc {

template <int I>
constexpr PairLaunchFn pair_entry() {
    constexpr PairCfg c = kPairCfgs[I];
    return launch_pair<c.sa, c.ca32, c.cb32, c.nba, c.nbb, c.th, c.wm>;
}

PairLaunchFn pair_launcher(int index) {
    static constexpr PairLaunchFn table[kNumPair] = {
        pair_entry<0>(),  pair_entry<1>(),  pair_entry<2>(),  pair_entry<3>(),  pair_entry<4>(),  pair_entry<5>(),
        pair_entry<6>(),  pair_entry<7>(),  pair_entry<8>(),  pair_entry<9>(),  pair_entry<10>(), pair_entry<11>(),
        pair_entry<12>(), pair_entry<13>(), pair_entry<14>(), pair_entry<15>(), pair_entry<16>(), pair_entry<17>()};
    return index >= 0 && index < kNumPair ? table[index] : nullptr;
}

}  // namespace fhc
