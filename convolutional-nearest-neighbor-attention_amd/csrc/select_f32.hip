// fp32 instantiations of the fused similarity + top-k kernel, and the
// dtype dispatch.
#include "select_impl.h"

int launch_select_bf16(int euclid, int sampled, const SelArgs& a, hipStream_t s);

int launch_select(int dtype, int euclid, int sampled, const SelArgs& a, hipStream_t s) {
  if (a.BH <= 0 || a.N <= 0) return 0;
  if (dtype == CNNA_BF16) return launch_select_bf16(euclid, sampled, a, s);
  if (dtype == CNNA_F32) return launch_select_t<float>(euclid, sampled, a, s);
  return CNNA_ERR_DTYPE;
}
