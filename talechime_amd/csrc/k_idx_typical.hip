// k_idx_typical.hip -- indextts with the typical warper (crates/indextts/src/generation.rs:196-248,
// applied at 649-651).

#include "tc_idx_general.h"

namespace tc {

// indextts with the typical warper (generation.rs:649-651, off by default):
// the general path with idx_typical between the penalty and the temperature.
template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_idx_typical(RowArgs a) {
  __shared__ IdxGenLds G;
  idx_general<InT, ITEMS, true>(a, G);
}


TC_DEFINE_LAUNCH(k_idx_typical)

}  // namespace tc
