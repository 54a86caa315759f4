// Conv1d branch of MultiHeadBranchingConv (layers.py:452-499, 502-600):
// Conv1d(d_k, d_k, kernel_size, stride 1, padding 'same') along the tokens of
// every head of the W_x output, weights shared by the heads.
//
// A block owns TT consecutive tokens of one (b, h).  It stages the input rows
// it needs (zeros outside [0, N); torch's 'same' padding puts (ks - 1) / 2
// zeros in front and the rest behind) and, when they fit, the weights in LDS.
// A thread owns one output channel o of TG = 8 consecutive tokens: per input
// channel c it reads the TG + ks - 1 input values and the ks weights once and
// does TG * ks FMAs from registers (input reads are broadcasts across the
// lanes of one token group).  fp32 accumulation.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int TG = 8;

template <typename T, int KSM, bool WLDS>
__global__ __launch_bounds__(256) void conv1d_tok_kernel(Conv1dArgs a) {
  // KSM >= ks taps are evaluated; taps r >= ks have zero weight, so the tap
  // loops carry no runtime guards.  LDS: inputs channel-major [c][row] (a
  // thread's TG + KSM - 1 consecutive rows are 16-byte vector reads), weights
  // [c][o][r] (a thread's taps sit at immediate offsets; the lane stride KSM
  // is odd or 1, so adjacent output channels fall in distinct banks).
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int nblk = (a.N + a.tt - 1) / a.tt;
  const int blk = xcd_swizzle(blockIdx.x, (int)gridDim.x);
  const int bh = blk / nblk;
  const int t0 = (blk - bh * nblk) * a.tt;
  const int b = bh / a.H, h = bh - b * a.H;
  const int dk = a.dk, ks = a.ks;
  const int rows = a.tt + KSM - 1;
  const int rp = (rows + 3) & ~3;          // row pitch of a channel, whole 16-byte vectors
  float* su = sm;                          // (dk, rp)
  float* sw = su + dk * rp;                // (dk, dk, KSM): [c][o][r]
  const T* U = static_cast<const T*>(a.u) + (int64_t)b * a.N * a.ldu + h * dk;
  for (int e = threadIdx.x; e < rows * dk; e += 256) {
    const int rr = e / dk, c = e - rr * dk;
    const int t = t0 - a.padl + rr;
    su[c * rp + rr] = (t >= 0 && t < a.N) ? ldf(U + (int64_t)t * a.ldu + c) : 0.0f;
  }
  const T* W = static_cast<const T*>(a.w);
  if (WLDS) {
    // the launcher's prep kernel laid the weights out as [c][o][KSM] fp32
    const float4* src = reinterpret_cast<const float4*>(a.wprep);
    float4* dst = reinterpret_cast<float4*>(sw);
    for (int e = threadIdx.x; e < dk * dk * KSM / 4; e += 256) dst[e] = src[e];
  }
  __syncthreads();
  const int ntok = min(a.tt, a.N - t0);
  const int ngrp = (ntok + TG - 1) / TG;
  T* Y = static_cast<T*>(a.y) + ((int64_t)bh * a.N + t0) * dk;
  const T* Bs = static_cast<const T*>(a.bias);
  for (int e = threadIdx.x; e < ngrp * dk; e += 256) {
    const int g = e / dk, o = e - g * dk;
    const float* ur = su + g * TG;
    const float* wr = sw + o * KSM;
    float acc[TG];
    const float bias = Bs != nullptr ? ldf(Bs + o) : 0.0f;
#pragma unroll
    for (int t = 0; t < TG; ++t) acc[t] = bias;
    for (int c = 0; c < dk; ++c) {
      float u[TG + KSM - 1];
#pragma unroll
      for (int j = 0; j < TG + KSM - 1; ++j) u[j] = ur[c * rp + j];
#pragma unroll
      for (int r = 0; r < KSM; ++r) {
        float wv;
        if (WLDS) {
          wv = wr[c * dk * KSM + r];
        } else {
          wv = ldf(W + ((int64_t)o * dk + c) * ks + min(r, ks - 1));
          wv = r < ks ? wv : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < TG; ++t) acc[t] += wv * u[t + r];
      }
    }
#pragma unroll
    for (int t = 0; t < TG; ++t)
      if (g * TG + t < ntok) stf(Y + (g * TG + t) * dk + o, acc[t]);
  }
}

// weights (dk, dk, ks) -> fp32 [c][o][KSM], taps r >= ks zero
template <typename T, int KSM>
__global__ __launch_bounds__(256) void conv1d_wprep_kernel(const T* W, float* out, int dk, int ks) {
  const int n = dk * dk * KSM;
  for (int e = blockIdx.x * 256 + threadIdx.x; e < n; e += gridDim.x * 256) {
    const int co = e / KSM, r = e - co * KSM;
    const int c = co / dk, o = co - c * dk;
    out[e] = r < ks ? ldf(W + ((int64_t)o * dk + c) * ks + r) : 0.0f;
  }
}

template <typename T, int KSM>
int launch_ks(Conv1dArgs a, hipStream_t s) {
  a.tt = 64;
  const size_t wbytes = (size_t)a.dk * a.dk * KSM * 4;
  auto ubytes = [&](int tt) { return (size_t)((tt + KSM - 1 + 3) & ~3) * a.dk * 4; };
  const bool wlds = a.wprep != nullptr && wbytes <= a.wprep_bytes && (a.dk * a.dk * KSM) % 4 == 0 &&
                    wbytes + ubytes(a.tt) <= 64 * 1024;
  if (wlds) {
    const int n = a.dk * a.dk * KSM;
    hipLaunchKernelGGL((conv1d_wprep_kernel<T, KSM>), dim3((unsigned)((n + 255) / 256 < 256 ? (n + 255) / 256 : 256)),
                       dim3(256), 0, s, static_cast<const T*>(a.w), a.wprep, a.dk, a.ks);
  }
  while (!wlds && a.tt > TG && ubytes(a.tt) > 64 * 1024) a.tt >>= 1;
  if (ubytes(a.tt) > 64 * 1024) return CNNA_ERR_SHAPE;
  const size_t lds = ubytes(a.tt) + (wlds ? wbytes : 0);
  const int nblk = (a.N + a.tt - 1) / a.tt;
  const dim3 grid((unsigned)(a.B * a.H * nblk));
  if (wlds)
    hipLaunchKernelGGL((conv1d_tok_kernel<T, KSM, true>), grid, dim3(256), lds, s, a);
  else
    hipLaunchKernelGGL((conv1d_tok_kernel<T, KSM, false>), grid, dim3(256), lds, s, a);
  return (int)hipGetLastError();
}

template <typename T>
int launch_t(const Conv1dArgs& a, hipStream_t s) {
  if (a.ks == 1) return launch_ks<T, 1>(a, s);
  if (a.ks <= 3) return launch_ks<T, 3>(a, s);
  if (a.ks <= 5) return launch_ks<T, 5>(a, s);
  if (a.ks <= 9) return launch_ks<T, 9>(a, s);
  if (a.ks <= 17) return launch_ks<T, 17>(a, s);
  return launch_ks<T, 33>(a, s);
}

}  // namespace

int launch_conv1d_tokens(int dtype, const Conv1dArgs& a, hipStream_t s) {
  if (a.B <= 0 || a.N <= 0) return 0;
  if (a.dk <= 0 || a.ks <= 0 || a.ks > 33 || a.H <= 0 || a.padl < 0 || a.padl >= a.ks)
    return CNNA_ERR_SHAPE;
  if (dtype == CNNA_BF16) return launch_t<uint16_t>(a, s);
  else if (dtype == CNNA_F16) return launch_t<_Float16>(a, s);
  if (dtype == CNNA_F32) return launch_t<float>(a, s);
  return CNNA_ERR_DTYPE;
}
