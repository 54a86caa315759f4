// fp16 instantiations of the fused similarity + top-k kernel: euclidean.
#include "select_impl.h"

int launch_select_f16_euc(int sampled, const SelArgs& a, hipStream_t s) {
  return launch_select_t<_Float16, true>(sampled, a, s);
}
