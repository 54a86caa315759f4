// bf16 instantiations of the fused similarity + top-k kernel: euclidean.
#include "select_impl.h"

int launch_select_bf16_euc(int sampled, const SelArgs& a, hipStream_t s) {
  return launch_select_t<uint16_t, true>(sampled, a, s);
}
