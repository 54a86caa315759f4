// fp32 instantiations of the fused similarity + top-k kernel (dot-product
// metrics), and the dtype / metric dispatch.
#include "select_impl.h"

int launch_select_bf16_dot(int sampled, const SelArgs& a, hipStream_t s);
int launch_select_bf16_euc(int sampled, const SelArgs& a, hipStream_t s);
int launch_select_f32_euc(int sampled, const SelArgs& a, hipStream_t s);
int launch_select_f16_dot(int sampled, const SelArgs& a, hipStream_t s);
int launch_select_f16_euc(int sampled, const SelArgs& a, hipStream_t s);

int launch_select(int dtype, int euclid, int sampled, const SelArgs& a, hipStream_t s) {
  if (a.BH <= 0 || a.N <= 0) return 0;
  if (dtype == CNNA_BF16)
    return euclid ? launch_select_bf16_euc(sampled, a, s) : launch_select_bf16_dot(sampled, a, s);
  if (dtype == CNNA_F16)
    return euclid ? launch_select_f16_euc(sampled, a, s) : launch_select_f16_dot(sampled, a, s);
  if (dtype == CNNA_F32)
    return euclid ? launch_select_f32_euc(sampled, a, s) : launch_select_t<float, false>(sampled, a, s);
  return CNNA_ERR_DTYPE;
}
