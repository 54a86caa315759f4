// bf16 instantiations of the fused similarity + top-k kernel.
#include "select_impl.h"

int launch_select_bf16(int euclid, int sampled, const SelArgs& a, hipStream_t s) {
  return launch_select_t<uint16_t>(euclid, sampled, a, s);
}
