// Backward kernels of the operator (autograd of layers.py:261-450).
//
// The reference differentiates a dense (BH, N, Nq) similarity matrix; here the
// similarity gradient is nonzero only at the K selected entries of each row,
// so every stage works on the (BH, N, K) neighbour lists:
//
//   tok_bwd     per token i: dw[i, r] = sum_c dP[c, i, r] * v[c, idx[i, r]],
//               softmax / weight backward -> dS[i, r], stored as a coefficient
//               coef = dS * (1/sqrt(d_k) | 1 | 1/s) per metric, and the key
//               gradient dk_i = sum_r coef * q_col(r) (+ normalisation /
//               distance terms); depthwise weight partial sums.
//   csr_*       reverse adjacency of the lists (count, scan, fill, sort by
//               entry id), so that
//   pull        dv_j = sum over entries reading v_j of w * dP and
//               dq_j = sum over entries selecting column j of coef * k_i
//               are summed in a fixed order (no floating-point atomics).
//
// dP (gradient of the gathered input prime) is W0[c, r] * g[c, i] for the
// depthwise conv and the depthwise stage of the separable conv, and a
// materialised GEMM result for the standard conv.
#include "common.h"
#include "kernels.h"

namespace {

CNNA_DEV float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// CPL consecutive channels starting at c0 of a row; zero beyond lim.
template <typename T, int CPL> struct Row;
// 16-bit rows (bf16 or fp16)
template <typename T> struct Row16_1 {
  static CNNA_DEV void load(const T* p, float (&o)[1]) { o[0] = ldf(p); }
};
template <typename T> struct Row16_2 {
  static CNNA_DEV void load(const T* p, float (&o)[2]) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
    o[0] = Pair16<T>::lo(u);
    o[1] = Pair16<T>::hi(u);
  }
};
template <typename T> struct Row16_4 {
  static CNNA_DEV void load(const T* p, float (&o)[4]) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    o[0] = Pair16<T>::lo(u.x);
    o[1] = Pair16<T>::hi(u.x);
    o[2] = Pair16<T>::lo(u.y);
    o[3] = Pair16<T>::hi(u.y);
  }
};
template <typename T> struct Row16_8 {
  static CNNA_DEV void load(const T* p, float (&o)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = Pair16<T>::lo(w[i]);
      o[2 * i + 1] = Pair16<T>::hi(w[i]);
    }
  }
};
template <> struct Row<uint16_t, 1> : Row16_1<uint16_t> {};
template <> struct Row<uint16_t, 2> : Row16_2<uint16_t> {};
template <> struct Row<uint16_t, 4> : Row16_4<uint16_t> {};
template <> struct Row<uint16_t, 8> : Row16_8<uint16_t> {};
template <> struct Row<_Float16, 1> : Row16_1<_Float16> {};
template <> struct Row<_Float16, 2> : Row16_2<_Float16> {};
template <> struct Row<_Float16, 4> : Row16_4<_Float16> {};
template <> struct Row<_Float16, 8> : Row16_8<_Float16> {};
template <> struct Row<float, 1> {
  static CNNA_DEV void load(const float* p, float (&o)[1]) { o[0] = *p; }
};
template <> struct Row<float, 2> {
  static CNNA_DEV void load(const float* p, float (&o)[2]) {
    const float2 u = *reinterpret_cast<const float2*>(p);
    o[0] = u.x;
    o[1] = u.y;
  }
};
template <> struct Row<float, 4> {
  static CNNA_DEV void load(const float* p, float (&o)[4]) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    o[0] = u.x; o[1] = u.y; o[2] = u.z; o[3] = u.w;
  }
};

template <typename T, int CPL>
CNNA_DEV void load_row(const T* row, int c0, int lim, bool vec, float (&o)[CPL]) {
  if (vec && c0 + CPL <= lim) {
    Row<T, CPL>::load(row + c0, o);
  } else {
#pragma unroll
    for (int u = 0; u < CPL; ++u) o[u] = (c0 + u < lim) ? ldf(row + c0 + u) : 0.0f;
  }
}

// channels [c0, c0 + CPL) below dk into an unsplit (rows, C) destination
template <typename T, int CPL>
CNNA_DEV void store_row(T* row, int c0, int dk, const float (&o)[CPL]) {
#pragma unroll
  for (int u = 0; u < CPL; ++u)
    if (c0 + u < dk) stf(row + c0 + u, o[u]);
}

// ------------------------------------------------------------------ unmerge
// Inverse of the head merge Z[b, t, h*dk + a] = y_bh[a*N + t] (H > 1) and of
// the transpose Z[b, i, c] = y_b[i*dk + c] (H == 1), y_bh flat token-major;
// concat: Z[b, t, h*dk + c] = y_bh[t*dk + c] for every H.
template <typename T>
__global__ __launch_bounds__(256) void unmerge_kernel(const T* dz, T* dy, int BH, int N, int dk,
                                                      int H, int C, int concat) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per = (int64_t)N * dk;
  if (e >= (int64_t)BH * per) return;
  const int bh = (int)(e / per);
  const int64_t f = e - (int64_t)bh * per;
  const int b = bh / H, h = bh - b * H;
  int64_t src;
  if (H == 1 || concat) {
    const int t = (int)(f / dk), c = (int)(f - (int64_t)t * dk);
    src = ((int64_t)b * N + t) * C + h * dk + c;
  } else {
    const int a = (int)(f / N), t = (int)(f - (int64_t)a * N);
    src = ((int64_t)b * N + t) * C + h * dk + a;
  }
  dy[e] = dz[src];
}

// Mixing case (H > 1, reference merge) as a tiled transpose: for one (b, h),
// y_bh viewed as (dk, N) [a][t] is the transpose of the (N, dk) slice
// Z[b, :, h*dk : (h+1)*dk].  64 x 64 tiles through LDS: reads run along the
// channels, writes along the tokens, both coalesced.
template <typename T>
__global__ __launch_bounds__(256) void unmerge_tile_kernel(const T* dz, T* dy, int N, int dk, int H,
                                                           int C) {
  __shared__ T tile[64][65];
  const int bh = blockIdx.z, b = bh / H, h = bh - b * H;
  const int t0 = blockIdx.x * 64, a0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const T* src = dz + (int64_t)b * N * C + h * dk;
  for (int r = ty; r < 64; r += 4) {
    const int t = t0 + r, a = a0 + tx;
    if (t < N && a < dk) tile[r][tx] = src[(int64_t)t * C + a];
  }
  __syncthreads();
  T* dst = dy + (int64_t)bh * N * dk;
  for (int r = ty; r < 64; r += 4) {
    const int a = a0 + r, t = t0 + tx;
    if (t < N && a < dk) dst[(int64_t)a * N + t] = tile[tx][r];
  }
}

// ------------------------------------------------------------------ tok_bwd

// sum over groups of N lanes (N = 8 or 16) inside a DPP row
template <int N>
CNNA_DEV float rowN_sum(float v) {
  v += dpp_f<0xB1>(v);                    // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);                    // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);                   // row_half_mirror: the two quads of 8 lanes
  if (N == 16) v += dpp_f<0x140>(v);      // row_mirror: the two halves of 16 lanes
  return v;
}

// DV (depthwise, din a multiple of the 16-byte vector): the neighbour-weight
// gradients use LPR = 64*CPL/V16 lanes per neighbour row with 16-byte loads of
// v and g, 64/LPR neighbours per pass and DPP sums over the LPR lanes; the
// depthwise-weight partials accumulate in that layout.
template <typename T, int CPL, int KMAX, bool DW, bool DV = false>
__global__ __launch_bounds__(256) void tok_bwd_kernel(TokBwdArgs a) {
  constexpr int CW = 64 * CPL;
  constexpr int V16 = 16 / sizeof(T);
  constexpr int LPR = CW / V16 > 0 ? CW / V16 : 1;   // lanes per neighbour row (DV)
  constexpr int RPP = 64 / LPR;                        // neighbours per pass (DV)
  constexpr int NPS = (KMAX + RPP - 1) / RPP;          // passes (DV)
  static_assert(!DV || (DW && (LPR == 8 || LPR == 16)), "DV needs 8 or 16 lanes per row");
  __shared__ float sW[DW ? KMAX * CW : 1];   // W0 as [r][c]; reused for the block reduction
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c0 = lane * CPL;
  const int K = a.K;
  if (DW) {
    const T* W0 = static_cast<const T*>(a.w0);
    for (int e = tid; e < KMAX * CW; e += 256) {
      const int r = e / CW, c = e - r * CW;
      sW[e] = (r < K && c < a.din) ? ldf(W0 + c * K + r) : 0.0f;
    }
    __syncthreads();
  }
  float acc[(DW && !DV) ? KMAX : 1][CPL];
#pragma unroll
  for (int r = 0; r < ((DW && !DV) ? KMAX : 1); ++r)
#pragma unroll
    for (int u = 0; u < CPL; ++u) acc[r][u] = 0.0f;
  float accd[DV ? NPS : 1][DV ? V16 : 1];
#pragma unroll
  for (int p = 0; p < (DV ? NPS : 1); ++p)
#pragma unroll
    for (int u = 0; u < (DV ? V16 : 1); ++u) accd[p][u] = 0.0f;
  const int dgrp = lane / LPR, dgl = lane % LPR, dc = dgl * V16;   // DV lane layout

  const bool euc = a.metric == CNNA_EUCLIDEAN, cos_ = a.metric == CNNA_COSINE;
  const bool gvec = (a.din % CPL) == 0;
  const bool svec = (a.din % (16 / (int)sizeof(T))) == 0;   // 16-byte rows of dP and v
  const int ntok = a.BH * a.N;
  const int nw = gridDim.x * 4;
  for (int tok = blockIdx.x * 4 + wv; tok < ntok; tok += nw) {
    const int bh = tok / a.N, i = tok - bh * a.N;
    const int b = bh / a.H, h = bh - b * a.H;
    const int64_t ebase = (int64_t)tok * K;
    const bool valid = lane < K;
    int my_j = 0;
    float my_w = 0.0f, my_val = 0.0f, my_mul = 1.0f;
    if (valid) {
      my_j = a.idx[ebase + lane];
      my_w = a.w[ebase + lane];
      my_val = a.vals[ebase + lane];
      if (a.wmul != nullptr) my_mul = a.wmul[ebase + lane];
    }
    const float my_wa = my_w * my_mul;   // the weight the aggregation used
    const T* V = static_cast<const T*>(a.v) + (int64_t)bh * a.N * a.dkp;
    float gv[CPL];
    if (DW && !DV) load_row<T, CPL>(static_cast<const T*>(a.g) + (int64_t)tok * a.din, c0, a.din, gvec, gv);

    // dw[r] = sum_c dP[c, r] * v[c, idx[r]]
    float my_dw = 0.0f;
    if constexpr (DV) {
      const bool cok = dc < a.din;
      float gq[V16];
      if (cok) {
        Row<T, V16>::load(static_cast<const T*>(a.g) + (int64_t)tok * a.din + dc, gq);
      } else {
#pragma unroll
        for (int u = 0; u < V16; ++u) gq[u] = 0.0f;
      }
#pragma unroll
      for (int ps = 0; ps < NPS; ++ps) {
        const int r0 = ps * RPP;
        if (r0 < K) {
          const int r = r0 + dgrp;
          const int rr = min(r, K - 1);
          const int t = __shfl(my_j, rr);
          const float wr = __shfl(my_wa, rr);
          float p = 0.0f;
          if (cok) {
            float vv[V16];
            Row<T, V16>::load(V + (int64_t)t * a.dkp + dc, vv);
            const bool rok = r < K;
#pragma unroll
            for (int u = 0; u < V16; ++u) {
              const float pr = gq[u] * vv[u];
              if (rok) accd[ps][u] += wr * pr;
              p += sW[rr * CW + dc + u] * pr;
            }
          }
          p = rowN_sum<LPR>(p);
#pragma unroll
          for (int q = 0; q < RPP; ++q) {
            const float sq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), q * LPR));
            if (lane == r0 + q) my_dw = sq;
          }
        }
      }
    }
    if (!DW && svec) {
      // standard conv: four neighbours per pass, 16 lanes per neighbour row
      // with 16-byte loads of dP and v, row sums by DPP inside the 16 lanes
      constexpr int V16 = 16 / sizeof(T);
      constexpr int NP = (64 * CPL + 16 * V16 - 1) / (16 * V16);
      const int grp = lane >> 4, gl = lane & 15;
#pragma unroll
      for (int r0 = 0; r0 < KMAX; r0 += 4) {
        if (r0 < K) {
          const int rr = min(r0 + grp, K - 1);
          const int t = __shfl(my_j, rr);
          const T* vrow = V + (int64_t)t * a.dkp;
          const T* prow = static_cast<const T*>(a.dP) + (ebase + rr) * a.din;
          float acc = 0.0f;
#pragma unroll
          for (int ps = 0; ps < NP; ++ps) {
            const int c = (ps * 16 + gl) * V16;
            if (c < a.din) {
              float vv[V16], pp[V16];
              Row<T, V16>::load(vrow + c, vv);
              Row<T, V16>::load(prow + c, pp);
#pragma unroll
              for (int u = 0; u < V16; ++u) acc += pp[u] * vv[u];
            }
          }
          acc = row16_sum(acc);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float sq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 16 * q));
            if (lane == r0 + q) my_dw = sq;
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      if (r < K && ((DW && !DV) || (!DW && !svec))) {
        const int t = __builtin_amdgcn_readlane(my_j, r);
        float vv[CPL];
        load_row<T, CPL>(V + (int64_t)t * a.dkp, c0, a.dkp, true, vv);
        float p = 0.0f;
        if (DW) {
          const float wr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_wa), r));
#pragma unroll
          for (int u = 0; u < CPL; ++u) {
            const float pr = gv[u] * vv[u];
            acc[DW ? r : 0][u] += wr * pr;
            p += sW[(DW ? r : 0) * CW + c0 + u] * pr;
          }
        } else {
          float dp[CPL];
          load_row<T, CPL>(static_cast<const T*>(a.dP) + (ebase + r) * a.din, c0, a.din, gvec, dp);
#pragma unroll
          for (int u = 0; u < CPL; ++u) p += dp[u] * vv[u];
        }
        p = wave_sum(p);
        if (lane == r) my_dw = p;
      }
    }

    // through the dropout multiplier back to the weight itself
    my_dw *= my_mul;
    // weight backward -> dS (layers.py:342-437)
    float ds;
    if (a.softmax) {
      const float dot = wave_sum(valid ? my_w * my_dw : 0.0f);
      ds = my_w * (my_dw - dot);
      if (euc) ds = -ds;                       // softmax(-vals)
    } else if (euc) {
      const float den = my_val + 1e-8f;        // prime / (vals + 1e-8)
      ds = -my_dw / (den * den);
    } else {
      ds = my_dw;                              // vals * prime
    }
    // sampled: slot 0 is the constant self logit, a masked column is constant
    if (a.sampled && (lane == 0 || my_j == i)) ds = 0.0f;
    if (!valid) ds = 0.0f;
    float coef = ds;
    if (a.metric == CNNA_MATMUL) coef = ds * a.scale;
    else if (euc) coef = (ds == 0.0f) ? 0.0f : ds / my_val;   // d sqrt(d2) = 1/(2s) * d d2
    if (valid) a.coef[ebase + lane] = coef;
    int my_col = my_j;
    // sampled: the candidate column the forward selected (duplicate columns of
    // one token carry different q rows with coordinate encoding)
    if (a.sampled) my_col = (valid && coef != 0.0f) ? min(max(a.cols[ebase + lane], 0), a.Nq - 1) : 0;

    // dk_i = sum_r coef[r] * q[col(r)]  (+ metric terms)
    float dk[CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u) dk[u] = 0.0f;
    const T* Q = static_cast<const T*>(a.q) + (int64_t)bh * a.Nq * a.dkp;
#pragma unroll
    for (int r = 0; r < KMAX; ++r) {
      if (r < K) {
        const float cr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(coef), r));
        if (cr != 0.0f) {
          const int col = __builtin_amdgcn_readlane(my_col, r);
          float qv[CPL];
          load_row<T, CPL>(Q + (int64_t)col * a.dkp, c0, a.dkp, true, qv);
#pragma unroll
          for (int u = 0; u < CPL; ++u) dk[u] += cr * qv[u];
        }
      }
    }
    if (cos_ || euc) {
      float kv[CPL];
      load_row<T, CPL>(static_cast<const T*>(a.k) + (int64_t)tok * a.dkp, c0, a.dkp, true, kv);
      if (cos_) {
        // F.normalize backward: (dkh - kh (kh . dkh)) / max(|k|, eps)
        float d = 0.0f;
#pragma unroll
        for (int u = 0; u < CPL; ++u) d += kv[u] * dk[u];
        d = wave_sum(d);
        const float nrm = sqrtf(a.kn[tok]);
#pragma unroll
        for (int u = 0; u < CPL; ++u)
          dk[u] = nrm > 1e-12f ? (dk[u] - kv[u] * d) / nrm : dk[u] / 1e-12f;
      } else {
        // d/dk sqrt(|k|^2 + |q|^2 - 2 k.q) summed: k * sum(coef) - sum(coef * q)
        const float cs = wave_sum(coef);
#pragma unroll
        for (int u = 0; u < CPL; ++u) dk[u] = kv[u] * cs - dk[u];
      }
    }
    T* dst = static_cast<T*>(a.dst) + ((int64_t)b * a.N + i) * a.ldd + a.offd + h * a.dk;
    store_row<T, CPL>(dst, c0, a.dk, dk);
  }

  if (DW) {
    // block partial of dW0[c, r] = sum_tokens w[r] g[c] v[c, idx[r]], waves added in order
    __syncthreads();
    for (int w = 0; w < 4; ++w) {
      if (wv == w) {
        if constexpr (DV) {
          // every wave covers the same (r < K, c < din) entries
#pragma unroll
          for (int ps = 0; ps < NPS; ++ps) {
            const int r = ps * RPP + dgrp;
            if (r < K && dc < a.din) {
#pragma unroll
              for (int u = 0; u < V16; ++u) {
                float* p = &sW[r * CW + dc + u];
                *p = (w == 0 ? 0.0f : *p) + accd[ps][u];
              }
            }
          }
        } else {
#pragma unroll
          for (int r = 0; r < KMAX; ++r)
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
              float* p = &sW[(DW ? r : 0) * CW + c0 + u];
              *p = (w == 0 ? 0.0f : *p) + acc[(DW && !DV) ? r : 0][u];
            }
        }
      }
      __syncthreads();
    }
    float* out = a.w0part + (int64_t)blockIdx.x * a.din * K;
    for (int e = tid; e < a.din * K; e += 256) {
      const int c = e / K, r = e - c * K;
      out[e] = sW[r * CW + c];
    }
  }
}

template <typename T, int CPL, int KMAX>
int launch_tok_t(const TokBwdArgs& a, hipStream_t s) {
  dim3 grid(a.nblk);
  constexpr int LPR = 64 * CPL / (16 / (int)sizeof(T));
  if (a.std_conv)
    hipLaunchKernelGGL((tok_bwd_kernel<T, CPL, KMAX, false>), grid, dim3(256), 0, s, a);
  else if constexpr (LPR == 8 || LPR == 16) {
    if (a.din % (16 / (int)sizeof(T)) == 0)
      hipLaunchKernelGGL((tok_bwd_kernel<T, CPL, KMAX, true, true>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((tok_bwd_kernel<T, CPL, KMAX, true>), grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((tok_bwd_kernel<T, CPL, KMAX, true>), grid, dim3(256), 0, s, a);
  }
  return (int)hipGetLastError();
}

template <typename T, int CPL>
int launch_tok_k(const TokBwdArgs& a, hipStream_t s) {
  if (a.K <= 9) return launch_tok_t<T, CPL, 9>(a, s);
  if (a.K <= 16) return launch_tok_t<T, CPL, 16>(a, s);
  if (a.K <= 32) return launch_tok_t<T, CPL, 32>(a, s);
  if (a.K <= 64) return launch_tok_t<T, CPL, 64>(a, s);
  return CNNA_ERR_UNSUPPORTED;
}

template <typename T>
int launch_tok_c(const TokBwdArgs& a, hipStream_t s) {
  if (a.dkp <= 64) return launch_tok_k<T, 1>(a, s);
  if (a.dkp <= 128) return launch_tok_k<T, 2>(a, s);
  if (a.dkp <= 256) return launch_tok_k<T, 4>(a, s);
  return CNNA_ERR_SHAPE;
}

// Sum of the per-block depthwise-weight partials: a block owns 32 outputs; 32
// thread groups each add every 32nd partial (four loads in flight), then the
// group sums are added in group order.  Fixed order: deterministic.
template <typename T>
__global__ __launch_bounds__(1024) void w0_reduce_kernel(const float* part, int nblk, int n, T* out) {
  __shared__ float red[32][33];
  const int el = threadIdx.x & 31, gb = threadIdx.x >> 5;
  const int e = blockIdx.x * 32 + el;
  float acc = 0.0f;
  if (e < n) {
    int b = gb;
    for (; b + 96 < nblk; b += 128) {
      const float v0 = part[(int64_t)b * n + e];
      const float v1 = part[(int64_t)(b + 32) * n + e];
      const float v2 = part[(int64_t)(b + 64) * n + e];
      const float v3 = part[(int64_t)(b + 96) * n + e];
      acc += v0;
      acc += v1;
      acc += v2;
      acc += v3;
    }
    for (; b < nblk; b += 32) acc += part[(int64_t)b * n + e];
  }
  red[gb][el] = acc;
  __syncthreads();
  if (gb == 0 && e < n) {
    float sum = 0.0f;
    for (int g = 0; g < 32; ++g) sum += red[g][el];
    stf(out + e, sum);
  }
}

// ------------------------------------------------------------------ CSR
CNNA_DEV int entry_key(const CsrArgs& c, int64_t ge, int i, int r) {
  const int j = c.idx[ge];
  if (c.mode == CSR_TOKEN) return j;
  if (r == 0 || j == i) return -1;             // self slot / masked column
  const int col = c.cols[ge];
  return col < c.nkeys ? col : -1;
}

__global__ __launch_bounds__(256) void csr_count_kernel(CsrArgs c) {
  const int64_t ge = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t NK = (int64_t)c.N * c.K;
  if (ge >= (int64_t)c.BH * NK) return;
  const int bh = (int)(ge / NK);
  const int e = (int)(ge - (int64_t)bh * NK);
  const int i = e / c.K, r = e - i * c.K;
  const int key = entry_key(c, ge, i, r);
  if (key >= 0) atomicAdd(&c.cnt[(int64_t)bh * c.nkeys + key], 1);
}

// one block per (b, h): exclusive scan of the counts; counts reset to 0 (fill cursors)
__global__ __launch_bounds__(1024) void csr_scan_kernel(CsrArgs c) {
  __shared__ int part[1024];
  const int bh = blockIdx.x, tid = threadIdx.x;
  int32_t* cnt = c.cnt + (int64_t)bh * c.nkeys;
  int32_t* off = c.off + (int64_t)bh * (c.nkeys + 1);
  const int per = (c.nkeys + 1023) / 1024;
  const int k0 = tid * per, k1 = min(c.nkeys, k0 + per);
  int s = 0;
  for (int k = k0; k < k1; ++k) s += cnt[k];
  part[tid] = s;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {
    const int x = tid >= d ? part[tid - d] : 0;
    __syncthreads();
    part[tid] += x;
    __syncthreads();
  }
  int run = part[tid] - s;
  for (int k = k0; k < k1; ++k) {
    off[k] = run;
    run += cnt[k];
    cnt[k] = 0;
  }
  if (tid == 1023) off[c.nkeys] = part[1023];
}

__global__ __launch_bounds__(256) void csr_fill_kernel(CsrArgs c) {
  const int64_t ge = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t NK = (int64_t)c.N * c.K;
  if (ge >= (int64_t)c.BH * NK) return;
  const int bh = (int)(ge / NK);
  const int e = (int)(ge - (int64_t)bh * NK);
  const int i = e / c.K, r = e - i * c.K;
  const int key = entry_key(c, ge, i, r);
  if (key < 0) return;
  const int pos = atomicAdd(&c.cnt[(int64_t)bh * c.nkeys + key], 1);
  c.tmp[(int64_t)bh * NK + c.off[(int64_t)bh * (c.nkeys + 1) + key] + pos] = e;
}

// One block per (b, h) with the key counters in LDS: count, exclusive scan,
// then the bucket fill with LDS cursors (bucket order arbitrary; the rank sort
// below restores entry order).  Four entries per thread and step, their
// loads issued before the LDS atomics.
constexpr int CSR_LDS_MAX_KEYS = 16384;
__global__ __launch_bounds__(1024) void csr_lds_kernel(CsrArgs c) {
  extern __shared__ int sc[];                      // nkeys counters, then 1024 scan partials
  int* part = sc + c.nkeys;
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int64_t NK = (int64_t)c.N * c.K;
  const int nk = (int)NK;
  for (int k = tid; k < c.nkeys; k += 1024) sc[k] = 0;
  __syncthreads();
  auto walk = [&](auto visit) __attribute__((always_inline)) {
    for (int e0 = 0; e0 < nk; e0 += 4 * 1024) {
      int key[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = e0 + j * 1024 + tid;
        key[j] = -1;
        if (e < nk) {
          const int i = e / c.K, r = e - i * c.K;
          key[j] = entry_key(c, (int64_t)bh * NK + e, i, r);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (key[j] >= 0) visit(key[j], e0 + j * 1024 + tid);
    }
  };
  walk([&](int key, int) { atomicAdd(&sc[key], 1); });
  __syncthreads();
  // exclusive scan: per-thread chunk sums, Hillis-Steele over the partials
  const int per = (c.nkeys + 1023) / 1024;
  const int k0 = tid * per, k1 = min(c.nkeys, k0 + per);
  int sum = 0;
  for (int k = k0; k < k1; ++k) sum += sc[k];
  part[tid] = sum;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {
    const int x = tid >= d ? part[tid - d] : 0;
    __syncthreads();
    part[tid] += x;
    __syncthreads();
  }
  int32_t* off = c.off + (int64_t)bh * (c.nkeys + 1);
  int run = part[tid] - sum;
  for (int k = k0; k < k1; ++k) {
    const int n = sc[k];
    off[k] = run;
    sc[k] = run;                                   // fill cursor
    run += n;
  }
  if (tid == 1023) off[c.nkeys] = part[1023];
  __syncthreads();
  int32_t* tmp = c.tmp + (int64_t)bh * NK;
  walk([&](int key, int e) { tmp[atomicAdd(&sc[key], 1)] = e; });
}

// one wave per key: rank sort of the bucket (entry ids are distinct)
constexpr int SORT_LDS = 1024;
__global__ __launch_bounds__(256) void csr_sort_kernel(CsrArgs c) {
  __shared__ int buf[4][SORT_LDS];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t gw = (int64_t)blockIdx.x * 4 + wv;
  if (gw >= (int64_t)c.BH * c.nkeys) return;
  const int bh = (int)(gw / c.nkeys), key = (int)(gw - (int64_t)bh * c.nkeys);
  const int64_t NK = (int64_t)c.N * c.K;
  const int32_t* off = c.off + (int64_t)bh * (c.nkeys + 1);
  const int beg = off[key], n = off[key + 1] - beg;
  const int32_t* src = c.tmp + bh * NK + beg;
  int32_t* dst = c.list + bh * NK + beg;
  if (n <= SORT_LDS) {
    for (int x = lane; x < n; x += 64) buf[wv][x] = src[x];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    for (int x = lane; x < n; x += 64) {
      const int me = buf[wv][x];
      int rank = 0;
      for (int y = 0; y < n; ++y) rank += buf[wv][y] < me;
      dst[rank] = me;
    }
  } else {
    for (int x = lane; x < n; x += 64) {
      const int me = src[x];
      int rank = 0;
      for (int y = 0; y < n; ++y) rank += src[y] < me;
      dst[rank] = me;
    }
  }
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e < n) p[e] = v;
}

// ------------------------------------------------------------------ pull
template <typename T, int CPL>
__global__ __launch_bounds__(256) void pull_kernel(PullArgs a) {
  constexpr int CW = 64 * CPL;
  extern __shared__ float sW[];                   // depthwise: W0 as [r][c]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c0 = lane * CPL;
  const bool dwv = a.do_v && !a.std_conv;
  if (dwv) {
    const T* W0 = static_cast<const T*>(a.w0);
    for (int e = tid; e < a.K * CW; e += 256) {
      const int r = e / CW, c = e - r * CW;
      sW[e] = c < a.din ? ldf(W0 + c * a.K + r) : 0.0f;
    }
    __syncthreads();
  }
  const int64_t gw = (int64_t)blockIdx.x * 4 + wv;
  if (gw >= (int64_t)a.BH * a.nkeys) return;
  const int bh = (int)(gw / a.nkeys), key = (int)(gw - (int64_t)bh * a.nkeys);
  const int b = bh / a.H, h = bh - b * a.H;
  const int64_t NK = (int64_t)a.N * a.K;
  const int32_t* off = a.off + (int64_t)bh * (a.nkeys + 1);
  const int beg = off[key], end = off[key + 1];
  const int32_t* list = a.list + bh * NK;
  const bool gvec = (a.din % CPL) == 0;
  const T* G = static_cast<const T*>(a.g);
  const T* DP = static_cast<const T*>(a.dP);
  const T* Kt = static_cast<const T*>(a.k) + (int64_t)bh * a.N * a.dkp;

  float dv[CPL], dq[CPL], cs = 0.0f;
#pragma unroll
  for (int u = 0; u < CPL; ++u) dv[u] = dq[u] = 0.0f;
  for (int x = beg; x < end; ++x) {
    const int e = list[x];
    const int i = e / a.K, r = e - i * a.K;
    if (a.do_v) {
      const float we = a.w[bh * NK + e] * (a.wmul != nullptr ? a.wmul[bh * NK + e] : 1.0f);
      float gg[CPL];
      if (a.std_conv) {
        load_row<T, CPL>(DP + (bh * NK + e) * a.din, c0, a.din, gvec, gg);
#pragma unroll
        for (int u = 0; u < CPL; ++u) dv[u] += we * gg[u];
      } else {
        load_row<T, CPL>(G + ((int64_t)bh * a.N + i) * a.din, c0, a.din, gvec, gg);
#pragma unroll
        for (int u = 0; u < CPL; ++u) dv[u] += we * (sW[r * CW + c0 + u] * gg[u]);
      }
    }
    if (a.do_q) {
      const float ce = a.coef[bh * NK + e];
      if (ce != 0.0f) {
        float kk[CPL];
        load_row<T, CPL>(Kt + (int64_t)i * a.dkp, c0, a.dkp, true, kk);
#pragma unroll
        for (int u = 0; u < CPL; ++u) dq[u] += ce * kk[u];
        cs += ce;
      }
    }
  }
  if (a.do_v) {
    T* dst = static_cast<T*>(a.dst_v) + ((int64_t)b * a.N + key) * a.ld_v + a.off_v + h * a.dk;
    store_row<T, CPL>(dst, c0, a.dk, dv);
  }
  if (a.do_q) {
    if (a.metric != CNNA_MATMUL) {
      float qv[CPL];
      load_row<T, CPL>(static_cast<const T*>(a.q) + ((int64_t)bh * a.nkeys + key) * a.dkp, c0,
                       a.dkp, true, qv);
      if (a.metric == CNNA_COSINE) {
        float d = 0.0f;
#pragma unroll
        for (int u = 0; u < CPL; ++u) d += qv[u] * dq[u];
        d = wave_sum(d);
        const float nrm = sqrtf(a.qn[(int64_t)bh * a.nkeys + key]);
#pragma unroll
        for (int u = 0; u < CPL; ++u)
          dq[u] = nrm > 1e-12f ? (dq[u] - qv[u] * d) / nrm : dq[u] / 1e-12f;
      } else {
        // q * sum(coef) - sum(coef * k)
#pragma unroll
        for (int u = 0; u < CPL; ++u) dq[u] = qv[u] * cs - dq[u];
      }
    }
    T* dst = static_cast<T*>(a.dst_q) + ((int64_t)b * a.nkeys + key) * a.ld_q + a.off_q + h * a.dk;
    store_row<T, CPL>(dst, c0, a.dk, dq);
  }
}

template <typename T, int CPL>
constexpr int pull_lanes_per_key() {
  return (64 * CPL) / (16 / (int)sizeof(T)) <= 8 ? 8 : 16;
}

// Same sums with four (or eight) keys per wave: a group of 16 (or 8, when a
// row is 8 vectors) lanes owns one key and walks its entries in list order
// with 16-byte row loads (NP passes of LPK * V16 channels); the cosine row dot
// product is a DPP sum over the group.  Rows of dP / g and
// k must be whole 16-byte vectors (din % V16 == 0).
template <typename T, int CPL>
__global__ __launch_bounds__(256) void pull16_kernel(PullArgs a) {
  constexpr int V16 = 16 / sizeof(T);
  constexpr int CW = 64 * CPL;
  constexpr int LPK = pull_lanes_per_key<T, CPL>();   // 8 when a row is 8 vectors, else 16
  constexpr int KPW = 64 / LPK;                       // keys per wave
  constexpr int NP = (CW + LPK * V16 - 1) / (LPK * V16);
  extern __shared__ float sW[];                   // depthwise: W0 as [r][c]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int grp = lane / LPK, gl = lane % LPK;
  const bool dwv = a.do_v && !a.std_conv;
  if (dwv) {
    const T* W0 = static_cast<const T*>(a.w0);
    for (int e = tid; e < a.K * CW; e += 256) {
      const int r = e / CW, c = e - r * CW;
      sW[e] = c < a.din ? ldf(W0 + c * a.K + r) : 0.0f;
    }
    __syncthreads();
  }
  const int64_t nk = (int64_t)a.BH * a.nkeys;
  const int64_t gk = ((int64_t)blockIdx.x * 4 + wv) * KPW + grp;
  const bool kvalid = gk < nk;
  const int64_t gkc = kvalid ? gk : nk - 1;      // idle groups walk a real key, store nothing
  const int bh = (int)(gkc / a.nkeys), key = (int)(gkc - (int64_t)bh * a.nkeys);
  const int b = bh / a.H, h = bh - b * a.H;
  const int64_t NK = (int64_t)a.N * a.K;
  const int32_t* off = a.off + (int64_t)bh * (a.nkeys + 1);
  const int beg = off[key], end = off[key + 1];
  const int32_t* list = a.list + bh * NK;
  const T* G = static_cast<const T*>(a.g);
  const T* DP = static_cast<const T*>(a.dP);
  const T* Kt = static_cast<const T*>(a.k) + (int64_t)bh * a.N * a.dkp;

  float dv[NP][V16], dq[NP][V16], cs = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int u = 0; u < V16; ++u) dv[p][u] = dq[p][u] = 0.0f;
  for (int x = beg; x < end; ++x) {
    const int e = list[x];
    const int i = e / a.K, r = e - i * a.K;
    if (a.do_v) {
      const float we = a.w[bh * NK + e] * (a.wmul != nullptr ? a.wmul[bh * NK + e] : 1.0f);
      const T* row = a.std_conv ? DP + (bh * NK + e) * a.din : G + ((int64_t)bh * a.N + i) * a.din;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int c = (p * LPK + gl) * V16;
        if (c < a.din) {
          float gg[V16];
          Row<T, V16>::load(row + c, gg);
          if (a.std_conv) {
#pragma unroll
            for (int u = 0; u < V16; ++u) dv[p][u] += we * gg[u];
          } else {
#pragma unroll
            for (int u = 0; u < V16; ++u) dv[p][u] += we * (sW[r * CW + c + u] * gg[u]);
          }
        }
      }
    }
    if (a.do_q) {
      const float ce = a.coef[bh * NK + e];
      if (ce != 0.0f) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const int c = (p * LPK + gl) * V16;
          if (c < a.dkp) {
            float kk[V16];
            Row<T, V16>::load(Kt + (int64_t)i * a.dkp + c, kk);
#pragma unroll
            for (int u = 0; u < V16; ++u) dq[p][u] += ce * kk[u];
          }
        }
        cs += ce;
      }
    }
  }
  if (a.do_v && kvalid) {
    T* dst = static_cast<T*>(a.dst_v) + ((int64_t)b * a.N + key) * a.ld_v + a.off_v + h * a.dk;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int u = 0; u < V16; ++u) {
        const int c = (p * LPK + gl) * V16 + u;
        if (c < a.dk) stf(dst + c, dv[p][u]);
      }
  }
  if (a.do_q) {
    if (a.metric != CNNA_MATMUL) {
      const T* qrow = static_cast<const T*>(a.q) + ((int64_t)bh * a.nkeys + key) * a.dkp;
      float qv[NP][V16];
      float d = 0.0f;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int c = (p * LPK + gl) * V16;
        if (c < a.dkp) {
          Row<T, V16>::load(qrow + c, qv[p]);
        } else {
#pragma unroll
          for (int u = 0; u < V16; ++u) qv[p][u] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < V16; ++u) d += qv[p][u] * dq[p][u];
      }
      if (a.metric == CNNA_COSINE) {
        d = rowN_sum<LPK>(d);
        const float nrm = sqrtf(a.qn[(int64_t)bh * a.nkeys + key]);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int u = 0; u < V16; ++u)
            dq[p][u] = nrm > 1e-12f ? (dq[p][u] - qv[p][u] * d) / nrm : dq[p][u] / 1e-12f;
      } else {
        // q * sum(coef) - sum(coef * k)
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int u = 0; u < V16; ++u) dq[p][u] = qv[p][u] * cs - dq[p][u];
      }
    }
    if (kvalid) {
      T* dst = static_cast<T*>(a.dst_q) + ((int64_t)b * a.nkeys + key) * a.ld_q + a.off_q + h * a.dk;
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int u = 0; u < V16; ++u) {
          const int c = (p * LPK + gl) * V16 + u;
          if (c < a.dk) stf(dst + c, dq[p][u]);
        }
    }
  }
}

template <typename T>
int launch_pull_t(const PullArgs& a, hipStream_t s) {
  const int64_t waves = (int64_t)a.BH * a.nkeys;
  if (waves <= 0) return 0;
  dim3 grid((unsigned)((waves + 3) / 4));
  auto lds = [&](int cpl) { return (size_t)((a.do_v && !a.std_conv) ? a.K * 64 * cpl * 4 : 0); };
  constexpr int V16 = 16 / sizeof(T);
  if (a.din % V16 == 0 && a.dkp <= 256) {
    auto g16 = [&](int cpl) {
      const int kpw = 64 / (cpl == 1 ? pull_lanes_per_key<T, 1>()
                                     : (cpl == 2 ? pull_lanes_per_key<T, 2>() : pull_lanes_per_key<T, 4>()));
      return dim3((unsigned)((waves + 4 * kpw - 1) / (4 * kpw)));
    };
    if (a.dkp <= 64)
      hipLaunchKernelGGL((pull16_kernel<T, 1>), g16(1), dim3(256), lds(1), s, a);
    else if (a.dkp <= 128)
      hipLaunchKernelGGL((pull16_kernel<T, 2>), g16(2), dim3(256), lds(2), s, a);
    else
      hipLaunchKernelGGL((pull16_kernel<T, 4>), g16(4), dim3(256), lds(4), s, a);
    return (int)hipGetLastError();
  }
  if (a.dkp <= 64)
    hipLaunchKernelGGL((pull_kernel<T, 1>), grid, dim3(256), lds(1), s, a);
  else if (a.dkp <= 128)
    hipLaunchKernelGGL((pull_kernel<T, 2>), grid, dim3(256), lds(2), s, a);
  else if (a.dkp <= 256)
    hipLaunchKernelGGL((pull_kernel<T, 4>), grid, dim3(256), lds(4), s, a);
  else
    return CNNA_ERR_SHAPE;
  return (int)hipGetLastError();
}

// ------------------------------------------------------------------ sampled rows
template <typename T>
__global__ __launch_bounds__(256) void gather_rows_kernel(const T* x, int64_t ldx,
                                                          const int32_t* cand, T* xs, int B, int N,
                                                          int Nq, int C) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)B * Nq * C) return;
  const int64_t row = e / C;
  const int c = (int)(e - row * C);
  const int b = (int)(row / Nq), j = (int)(row - (int64_t)b * Nq);
  xs[e] = x[((int64_t)b * N + cand[j]) * ldx + c];
}

// one thread per (b, c): rows added in column order j = 0 .. Nq-1
template <typename T>
__global__ __launch_bounds__(256) void scatter_rows_kernel(const T* dxs, const int32_t* cand, T* dx,
                                                           int B, int N, int Nq, int C) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)B * C) return;
  const int b = (int)(e / C), c = (int)(e - (int64_t)b * C);
  for (int j = 0; j < Nq; ++j) {
    T* p = dx + ((int64_t)b * N + cand[j]) * C + c;
    stf(p, ldf(p) + ldf(dxs + ((int64_t)b * Nq + j) * C + c));
  }
}

// Column sums (the bias gradient of the projections): 32 columns per block,
// 32 row groups strided over the rows, the group partials added in order.
template <typename T>
__global__ __launch_bounds__(1024) void colsum_kernel(const T* a, int64_t rows, int cols, int64_t lda, T* out) {
  __shared__ float part[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int c = blockIdx.x * 32 + tx;
  float s = 0.0f;
  if (c < cols)
    for (int64_t r = ty; r < rows; r += 32) s += ldf(a + r * lda + c);
  part[ty][tx] = s;
  __syncthreads();
  if (ty == 0 && c < cols) {
    float t = 0.0f;
    for (int i = 0; i < 32; ++i) t += part[i][tx];
    stf(out + c, t);
  }
}

inline dim3 grid_for(int64_t n) { return dim3((unsigned)((n + 255) / 256)); }

}  // namespace

int launch_unmerge(int dtype, const void* dz, void* dy, int BH, int N, int dk, int H, int C,
                   int concat, hipStream_t s) {
  const int64_t n = (int64_t)BH * N * dk;
  if (n <= 0) return 0;
  if (H > 1 && !concat && BH <= 65535) {
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((dk + 63) / 64), (unsigned)BH);
    if (dtype == CNNA_BF16)
      hipLaunchKernelGGL(unmerge_tile_kernel<uint16_t>, grid, dim3(256), 0, s,
                         static_cast<const uint16_t*>(dz), static_cast<uint16_t*>(dy), N, dk, H, C);
    else if (dtype == CNNA_F16)
      hipLaunchKernelGGL(unmerge_tile_kernel<_Float16>, grid, dim3(256), 0, s,
                         static_cast<const _Float16*>(dz), static_cast<_Float16*>(dy), N, dk, H, C);
    else if (dtype == CNNA_F32)
      hipLaunchKernelGGL(unmerge_tile_kernel<float>, grid, dim3(256), 0, s,
                         static_cast<const float*>(dz), static_cast<float*>(dy), N, dk, H, C);
    else
      return CNNA_ERR_DTYPE;
    return (int)hipGetLastError();
  }
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(unmerge_kernel<uint16_t>, grid_for(n), dim3(256), 0, s,
                       static_cast<const uint16_t*>(dz), static_cast<uint16_t*>(dy), BH, N, dk, H, C, concat);
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(unmerge_kernel<_Float16>, grid_for(n), dim3(256), 0, s,
                       static_cast<const _Float16*>(dz), static_cast<_Float16*>(dy), BH, N, dk, H, C, concat);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(unmerge_kernel<float>, grid_for(n), dim3(256), 0, s,
                       static_cast<const float*>(dz), static_cast<float*>(dy), BH, N, dk, H, C, concat);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}

int launch_tok_bwd(int dtype, const TokBwdArgs& a0, hipStream_t s) {
  if (a0.BH <= 0 || a0.N <= 0) return 0;
  TokBwdArgs a = a0;
  a.nblk = tok_bwd_blocks(a.BH, a.N);
  if (dtype == CNNA_BF16) return launch_tok_c<uint16_t>(a, s);
  else if (dtype == CNNA_F16) return launch_tok_c<_Float16>(a, s);
  if (dtype == CNNA_F32) return launch_tok_c<float>(a, s);
  return CNNA_ERR_DTYPE;
}

int launch_w0_reduce(int dtype, const float* part, int nblk, int n, void* out, hipStream_t s) {
  if (n <= 0) return 0;
  const dim3 grid((unsigned)((n + 31) / 32));
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(w0_reduce_kernel<uint16_t>, grid, dim3(1024), 0, s, part, nblk, n,
                       static_cast<uint16_t*>(out));
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(w0_reduce_kernel<_Float16>, grid, dim3(1024), 0, s, part, nblk, n,
                       static_cast<_Float16*>(out));
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(w0_reduce_kernel<float>, grid, dim3(1024), 0, s, part, nblk, n,
                       static_cast<float*>(out));
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}

int launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_i32_kernel, grid_for(n), dim3(256), 0, s, p, n, v);
  return (int)hipGetLastError();
}

int launch_csr(const CsrArgs& c, hipStream_t s) {
  const int64_t ne = (int64_t)c.BH * c.N * c.K;
  if (ne <= 0 || c.nkeys <= 0) return 0;
  if (c.nkeys <= CSR_LDS_MAX_KEYS && (int64_t)c.N * c.K <= INT32_MAX) {
    hipLaunchKernelGGL(csr_lds_kernel, dim3(c.BH), dim3(1024), (size_t)(c.nkeys + 1024) * sizeof(int), s,
                       c);
    hipLaunchKernelGGL(csr_sort_kernel, dim3((unsigned)(((int64_t)c.BH * c.nkeys + 3) / 4)), dim3(256),
                       0, s, c);
    return (int)hipGetLastError();
  }
  int st = launch_fill_i32(c.cnt, (int64_t)c.BH * c.nkeys, 0, s);
  if (st) return st;
  hipLaunchKernelGGL(csr_count_kernel, grid_for(ne), dim3(256), 0, s, c);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(c.BH), dim3(1024), 0, s, c);
  hipLaunchKernelGGL(csr_fill_kernel, grid_for(ne), dim3(256), 0, s, c);
  hipLaunchKernelGGL(csr_sort_kernel, dim3((unsigned)(((int64_t)c.BH * c.nkeys + 3) / 4)), dim3(256),
                     0, s, c);
  return (int)hipGetLastError();
}

int launch_pull(int dtype, const PullArgs& p, hipStream_t s) {
  if (dtype == CNNA_BF16) return launch_pull_t<uint16_t>(p, s);
  else if (dtype == CNNA_F16) return launch_pull_t<_Float16>(p, s);
  if (dtype == CNNA_F32) return launch_pull_t<float>(p, s);
  return CNNA_ERR_DTYPE;
}

int launch_gather_rows(int dtype, const void* x, int64_t ldx, const int32_t* cand, void* xs, int B,
                       int N, int Nq, int C, hipStream_t s) {
  const int64_t n = (int64_t)B * Nq * C;
  if (n <= 0) return 0;
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(gather_rows_kernel<uint16_t>, grid_for(n), dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), ldx, cand, static_cast<uint16_t*>(xs), B, N,
                       Nq, C);
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(gather_rows_kernel<_Float16>, grid_for(n), dim3(256), 0, s,
                       static_cast<const _Float16*>(x), ldx, cand, static_cast<_Float16*>(xs), B, N,
                       Nq, C);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(gather_rows_kernel<float>, grid_for(n), dim3(256), 0, s,
                       static_cast<const float*>(x), ldx, cand, static_cast<float*>(xs), B, N, Nq, C);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}

int launch_scatter_rows(int dtype, const void* dxs, const int32_t* cand, void* dx, int B, int N,
                        int Nq, int C, hipStream_t s) {
  const int64_t n = (int64_t)B * C;
  if (n <= 0 || Nq <= 0) return 0;
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(scatter_rows_kernel<uint16_t>, grid_for(n), dim3(256), 0, s,
                       static_cast<const uint16_t*>(dxs), cand, static_cast<uint16_t*>(dx), B, N, Nq,
                       C);
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(scatter_rows_kernel<_Float16>, grid_for(n), dim3(256), 0, s,
                       static_cast<const _Float16*>(dxs), cand, static_cast<_Float16*>(dx), B, N, Nq,
                       C);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(scatter_rows_kernel<float>, grid_for(n), dim3(256), 0, s,
                       static_cast<const float*>(dxs), cand, static_cast<float*>(dx), B, N, Nq, C);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}

int launch_colsum(int dtype, const void* a, int64_t rows, int cols, int64_t lda, void* out, hipStream_t s) {
  if (cols <= 0) return 0;
  const dim3 grid((unsigned)((cols + 31) / 32));
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(colsum_kernel<uint16_t>, grid, dim3(1024), 0, s, static_cast<const uint16_t*>(a), rows,
                       cols, lda, static_cast<uint16_t*>(out));
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(colsum_kernel<_Float16>, grid, dim3(1024), 0, s, static_cast<const _Float16*>(a), rows,
                       cols, lda, static_cast<_Float16*>(out));
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(colsum_kernel<float>, grid, dim3(1024), 0, s, static_cast<const float*>(a), rows, cols,
                       lda, static_cast<float*>(out));
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}
