// fp16 instantiations of the fused similarity + top-k kernel: dot-product
// metrics (matmul, cosine).
#include "select_impl.h"

int launch_select_f16_dot(int sampled, const SelArgs& a, hipStream_t s) {
  return launch_select_t<_Float16, false>(sampled, a, s);
}
