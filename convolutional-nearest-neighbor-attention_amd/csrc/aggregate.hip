// Neighbour weights + V gather + Conv1d(kernel=K, stride=K) over the K
// gathered neighbours (layers.py:342-437 and self.conv at layers.py:313).
//
// Weights per token i (layers.py:352-355, 382-385, 394-397, 426-429):
//   softmax_topk_val: softmax(vals) (cosine/matmul) or softmax(-vals) (euclidean)
//   otherwise:        vals (cosine/matmul) or 1 / (vals + 1e-8) (euclidean)
// and prime[c, i, r] = w[i, r] * v[c, idx[i, r]] is never materialised.
//
// Output y is token-major (B*H, N, d_k); the head merge is applied by the
// output projection's A-operand loader.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int KCAP = 32;

CNNA_DEV void weights(const AggArgs& a, int64_t g, float (&w)[KCAP], int (&ix)[KCAP]) {
  const float* vals = a.vals + g * a.K;
  const int32_t* idx = a.idx + g * a.K;
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < KCAP; ++r) {
    if (r < a.K) {
      const float v = vals[r];
      ix[r] = idx[r];
      w[r] = (a.softmax && !a.maximum) ? -v : v;
      mx = fmaxf(mx, w[r]);
    } else {
      w[r] = 0.0f;
      ix[r] = 0;
    }
  }
  if (a.softmax) {
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < KCAP; ++r)
      if (r < a.K) {
        w[r] = expf(w[r] - mx);
        s += w[r];
      }
#pragma unroll
    for (int r = 0; r < KCAP; ++r)
      if (r < a.K) w[r] = w[r] / s;
  } else if (!a.maximum) {
#pragma unroll
    for (int r = 0; r < KCAP; ++r)
      if (r < a.K) w[r] = 1.0f / (w[r] + 1e-8f);
  }
}

// depthwise: one wave per token, lanes over channels
template <typename T>
__global__ __launch_bounds__(256) void agg_dw_kernel(AggArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= (int64_t)a.BH * a.N) return;
  const int64_t bh = g / a.N;
  float w[KCAP];
  int ix[KCAP];
  weights(a, g, w, ix);
  const T* V = static_cast<const T*>(a.v) + bh * a.N * a.dkp;
  const T* W0 = static_cast<const T*>(a.w0);
  T* y = static_cast<T*>(a.y) + g * a.dout;
  for (int c = lane; c < a.dout; c += 64) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < KCAP; ++r)
      if (r < a.K) acc += ldf(W0 + c * a.K + r) * (w[r] * ldf(V + (int64_t)ix[r] * a.dkp + c));
    stf(y + c, acc);
  }
}

// standard / depthwise-separable: one block per token
template <typename T>
__global__ __launch_bounds__(256) void agg_gen_kernel(AggArgs a) {
  extern __shared__ float sm[];
  const int64_t g = blockIdx.x;
  const int64_t bh = g / a.N;
  float w[KCAP];
  int ix[KCAP];
  weights(a, g, w, ix);
  const T* V = static_cast<const T*>(a.v) + bh * a.N * a.dkp;
  const T* W0 = static_cast<const T*>(a.w0);
  float* P = sm;                         // (K, din)
  float* t1 = sm + a.K * a.din;          // (din) depthwise stage of dw-separable
  for (int e = threadIdx.x; e < a.K * a.din; e += 256) {
    const int r = e / a.din, c = e - r * a.din;
    float wr = 0.0f;
    int jr = 0;
#pragma unroll
    for (int q = 0; q < KCAP; ++q)
      if (q == r) { wr = w[q]; jr = ix[q]; }
    P[e] = wr * ldf(V + (int64_t)jr * a.dkp + c);
  }
  __syncthreads();
  T* y = static_cast<T*>(a.y) + g * a.dout;
  if (a.conv == CNNA_CONV_STANDARD) {
    for (int o = threadIdx.x; o < a.dout; o += 256) {
      float acc = 0.0f;
      const T* wo = W0 + (int64_t)o * a.din * a.K;
      for (int c = 0; c < a.din; ++c)
        for (int r = 0; r < a.K; ++r) acc += ldf(wo + c * a.K + r) * P[r * a.din + c];
      stf(y + o, acc);
    }
  } else {
    const T* W1 = static_cast<const T*>(a.w1);
    for (int c = threadIdx.x; c < a.din; c += 256) {
      float acc = 0.0f;
      for (int r = 0; r < a.K; ++r) acc += ldf(W0 + c * a.K + r) * P[r * a.din + c];
      t1[c] = acc;
    }
    __syncthreads();
    for (int o = threadIdx.x; o < a.dout; o += 256) {
      float acc = 0.0f;
      for (int c = 0; c < a.din; ++c) acc += ldf(W1 + (int64_t)o * a.din + c) * t1[c];
      stf(y + o, acc);
    }
  }
}

template <typename T>
int launch_t(const AggArgs& a, hipStream_t s) {
  const int64_t tokens = (int64_t)a.BH * a.N;
  if (a.conv == CNNA_CONV_DEPTHWISE) {
    hipLaunchKernelGGL(agg_dw_kernel<T>, dim3((unsigned)((tokens + 3) / 4)), dim3(256), 0, s, a);
  } else {
    const size_t smem = ((size_t)a.K * a.din + a.din) * sizeof(float);
    hipLaunchKernelGGL(agg_gen_kernel<T>, dim3((unsigned)tokens), dim3(256), smem, s, a);
  }
  return (int)hipGetLastError();
}

}  // namespace

int launch_aggregate(int dtype, const AggArgs& a, hipStream_t s) {
  if (a.BH <= 0 || a.N <= 0) return 0;
  if (a.K > KCAP) return CNNA_ERR_K_RANGE;
  if (dtype == CNNA_BF16) return launch_t<uint16_t>(a, s);
  if (dtype == CNNA_F32) return launch_t<float>(a, s);
  return CNNA_ERR_DTYPE;
}
