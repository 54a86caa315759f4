// Conv1d branch of MultiHeadBranchingConv (layers.py:452-499, 502-600):
// Conv1d(d_k, d_k, kernel_size, stride 1, padding 'same') along the tokens of
// every head of the W_x output, weights shared by the heads.
//
// A block owns TT consecutive tokens of one (b, h).  It stages the TT + ks - 1
// input rows it needs (zeros outside [0, N), torch's 'same' padding puts
// (ks - 1) / 2 zeros in front and the rest behind) and, when they fit, the
// weights as [c*ks + r][o] in LDS; each thread produces outputs (t, o) with
// adjacent lanes on adjacent output channels, so the weight reads are
// conflict-free and the input reads are broadcasts.  fp32 accumulation.
#include "common.h"
#include "kernels.h"

namespace {

template <typename T, bool WLDS>
__global__ __launch_bounds__(256) void conv1d_tok_kernel(Conv1dArgs a) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int nblk = (a.N + a.tt - 1) / a.tt;
  const int blk = xcd_swizzle(blockIdx.x, (int)gridDim.x);
  const int bh = blk / nblk;
  const int t0 = (blk - bh * nblk) * a.tt;
  const int b = bh / a.H, h = bh - b * a.H;
  const int dk = a.dk, ks = a.ks;
  const int rows = a.tt + ks - 1;
  float* su = sm;                  // (rows, dk)
  float* sw = su + rows * dk;      // (dk * ks, dk): [c*ks + r][o]
  const T* U = static_cast<const T*>(a.u) + (int64_t)b * a.N * a.ldu + h * dk;
  for (int e = threadIdx.x; e < rows * dk; e += 256) {
    const int rr = e / dk, c = e - rr * dk;
    const int t = t0 - a.padl + rr;
    su[e] = (t >= 0 && t < a.N) ? ldf(U + (int64_t)t * a.ldu + c) : 0.0f;
  }
  const T* W = static_cast<const T*>(a.w);
  if (WLDS) {
    for (int e = threadIdx.x; e < dk * dk * ks; e += 256) {
      const int o = e / (dk * ks), cr = e - o * dk * ks;
      sw[cr * dk + o] = ldf(W + e);
    }
  }
  __syncthreads();
  const int ntok = min(a.tt, a.N - t0);
  T* Y = static_cast<T*>(a.y) + ((int64_t)bh * a.N + t0) * dk;
  const T* Bs = static_cast<const T*>(a.bias);
  for (int e = threadIdx.x; e < ntok * dk; e += 256) {
    const int tl = e / dk, o = e - tl * dk;
    float acc = Bs != nullptr ? ldf(Bs + o) : 0.0f;
    const float* ur = su + tl * dk;
    for (int r = 0; r < ks; ++r) {
      for (int c = 0; c < dk; ++c) {
        const float wv = WLDS ? sw[(c * ks + r) * dk + o] : ldf(W + ((int64_t)o * dk + c) * ks + r);
        acc += wv * ur[r * dk + c];
      }
    }
    stf(Y + e, acc);
  }
}

template <typename T>
int launch_t(const Conv1dArgs& a0, hipStream_t s) {
  Conv1dArgs a = a0;
  a.tt = 64;
  const size_t wbytes = (size_t)a.dk * a.dk * a.ks * 4;
  auto ubytes = [&](int tt) { return (size_t)(tt + a.ks - 1) * a.dk * 4; };
  const bool wlds = wbytes + ubytes(a.tt) <= 64 * 1024;
  while (!wlds && a.tt > 8 && ubytes(a.tt) > 64 * 1024) a.tt >>= 1;
  if (ubytes(a.tt) > 64 * 1024) return CNNA_ERR_SHAPE;
  const size_t lds = ubytes(a.tt) + (wlds ? wbytes : 0);
  const int nblk = (a.N + a.tt - 1) / a.tt;
  const dim3 grid((unsigned)(a.B * a.H * nblk));
  if (wlds)
    hipLaunchKernelGGL((conv1d_tok_kernel<T, true>), grid, dim3(256), lds, s, a);
  else
    hipLaunchKernelGGL((conv1d_tok_kernel<T, false>), grid, dim3(256), lds, s, a);
  return (int)hipGetLastError();
}

}  // namespace

int launch_conv1d_tokens(int dtype, const Conv1dArgs& a, hipStream_t s) {
  if (a.B <= 0 || a.N <= 0) return 0;
  if (a.dk <= 0 || a.ks <= 0 || a.H <= 0 || a.padl < 0 || a.padl >= a.ks) return CNNA_ERR_SHAPE;
  if (dtype == CNNA_BF16) return launch_t<uint16_t>(a, s);
  if (dtype == CNNA_F32) return launch_t<float>(a, s);
  return CNNA_ERR_DTYPE;
}
