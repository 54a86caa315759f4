// fp32 instantiations of the fused similarity + top-k kernel: euclidean.
#include "select_impl.h"

int launch_select_f32_euc(int sampled, const SelArgs& a, hipStream_t s) {
  return launch_select_t<float, true>(sampled, a, s);
}
