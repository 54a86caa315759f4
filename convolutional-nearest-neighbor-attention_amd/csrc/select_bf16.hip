// bf16 instantiations of the fused similarity + top-k kernel: dot-product
// metrics (matmul, cosine).
#include "select_impl.h"

int launch_select_bf16_dot(int sampled, const SelArgs& a, hipStream_t s) {
  return launch_select_t<uint16_t, false>(sampled, a, s);
}
