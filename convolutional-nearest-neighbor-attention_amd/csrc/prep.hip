// Row preparation of head-split tensors, one wave per row:
//  * coordinate channel linspace(-1, 1, rows) at channel d_k (layers.py:439-450),
//  * zero padding of channels [d_in, dkp),
//  * cosine: F.normalize(p=2, eps=1e-12) over the channels (layers.py:337-338),
//  * euclidean: fp32 squared norm per row (layers.py:328-329).
#include "common.h"
#include "kernels.h"

namespace {

template <typename T>
__global__ __launch_bounds__(256) void prep_kernel(PrepArgs p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows_total) return;
  T* t = static_cast<T*>(p.t) + (int64_t)row * p.dkp;
  const int din = p.dk + (p.coord ? 1 : 0);
  // the coordinate channel is written once: raw here, or normalised below
  if (p.coord && !p.normalize && lane == 0)
    stf(t + p.dk, linspace_f32(-1.0f, 1.0f, p.rows, row % p.rows));
  for (int c = din + lane; c < p.dkp; c += 64) stf(t + c, 0.0f);
  if (!p.normalize && p.norms == nullptr) return;
  float ss = 0.0f;
  for (int c = lane; c < din; c += 64) {
    float x = (c == p.dk && p.coord) ? linspace_f32(-1.0f, 1.0f, p.rows, row % p.rows) : ldf(t + c);
    ss += x * x;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if (p.norms != nullptr && lane == 0) p.norms[row] = ss;
  if (p.normalize) {
    const float nrm = fmaxf(sqrtf(ss), 1e-12f);
    for (int c = lane; c < din; c += 64) {
      float x = (c == p.dk && p.coord) ? linspace_f32(-1.0f, 1.0f, p.rows, row % p.rows) : ldf(t + c);
      stf(t + c, x / nrm);
    }
  }
}

}  // namespace

int launch_prep(int dtype, const PrepArgs& p, hipStream_t s) {
  if (p.rows_total <= 0) return 0;
  dim3 grid((p.rows_total + 3) / 4);
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(prep_kernel<uint16_t>, grid, dim3(256), 0, s, p);
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(prep_kernel<_Float16>, grid, dim3(256), 0, s, p);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(prep_kernel<float>, grid, dim3(256), 0, s, p);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}
