// Neighbour aggregation (layers.py:342-437 and self.conv at layers.py:313)
// and the reference head merge (layers.py:316-317, 247-259).
//
//  * agg_kernel<T, VW, COPY=false>: depthwise Conv1d(kernel=K, stride=K) over
//    the K gathered neighbours,  y[i, c] = sum_r W0[c, r] * w[i, r] * v[idx[i, r], c],
//    where w are the neighbour weights written by the select kernel.  prime
//    (layers.py:348-358, 402-405) is never materialised.
//  * agg_kernel<T, VW, COPY=true>: the head merge of an already computed
//    token-major y (standard / depthwise-separable conv paths).
//
// Both write the plain token-major tensor (B*H, N, dout) or a merged tensor
// Z (B, N, C) (AggArgs::merged, MERGE_*).  The reference merge (H > 1, and the
// Conv1d branch's batch_split for every H, layers.py:490-493) mixes tokens:
//   Z[b, t, h*dk + a] = y_bh[f] with f = a*N + t, y_bh flat token-major;
// MERGE_CONCAT places head h at columns [h*dk, (h+1)*dk) of token t.
// A block owns TI consecutive tokens of one (b, h), i.e. the flat range
// f in [i0*dk, (i0+TI)*dk); it stages that range in LDS as rows a of length N
// and writes each Z row's run of consecutive columns a with adjacent lanes.
//
// Lanes: a token is handled by LPT lanes, VW channels each (16-byte vectors).
#include "common.h"
#include "kernels.h"

namespace {

__host__ __device__ inline bool merge_mixes(const AggArgs& a) {
  return (a.merged == MERGE_REFERENCE && a.H > 1) || a.merged == MERGE_MIX;
}

template <typename T, int VW> struct Vec;
// eight 16-bit values (bf16 or fp16) as one 16-byte vector
template <typename T> struct Vec16 {
  typedef uint4 Raw;
  static CNNA_DEV Raw raw(const T* p) { return *reinterpret_cast<const uint4*>(p); }
  static CNNA_DEV void load(const T* p, float (&o)[8]) { unpack(raw(p), o); }
  static CNNA_DEV void unpack(const uint4 u, float (&o)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = Pair16<T>::lo(w[i]);
      o[2 * i + 1] = Pair16<T>::hi(w[i]);
    }
  }
  static CNNA_DEV void store(T* p, const float (&o)[8]) {
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = Pair16<T>::pack(o[2 * i], o[2 * i + 1]);
    *reinterpret_cast<u32x4_t*>(p) = w;
  }
  static CNNA_DEV Raw pack(const float (&o)[8]) {
    Raw u;
    u.x = Pair16<T>::pack(o[0], o[1]);
    u.y = Pair16<T>::pack(o[2], o[3]);
    u.z = Pair16<T>::pack(o[4], o[5]);
    u.w = Pair16<T>::pack(o[6], o[7]);
    return u;
  }
};
template <> struct Vec<uint16_t, 8> : Vec16<uint16_t> {};
template <> struct Vec<_Float16, 8> : Vec16<_Float16> {};
template <> struct Vec<float, 4> {
  typedef float4 Raw;
  static CNNA_DEV Raw raw(const float* p) { return *reinterpret_cast<const float4*>(p); }
  static CNNA_DEV void load(const float* p, float (&o)[4]) { unpack(raw(p), o); }
  static CNNA_DEV void unpack(const float4 u, float (&o)[4]) {
    o[0] = u.x; o[1] = u.y; o[2] = u.z; o[3] = u.w;
  }
  static CNNA_DEV void store(float* p, const float (&o)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(o[0], o[1], o[2], o[3]);
  }
  static CNNA_DEV Raw pack(const float (&o)[4]) { return make_float4(o[0], o[1], o[2], o[3]); }
};
template <typename T> struct Vec<T, 1> {
  static CNNA_DEV void load(const T* p, float (&o)[1]) { o[0] = ldf(p); }
  static CNNA_DEV void store(T* p, const float (&o)[1]) { stf(p, o[0]); }
};

// KM > 0: K <= KM; the K neighbour rows of the next token group are loaded
// while the current group is convolved
// blocks per CU the register budget is held to: three for K <= 9 (one round
// of blocks at the config-3 shape), two for the K <= 16 instance
template <int KM> constexpr int agg_min_blocks() { return KM == 0 ? 1 : (KM <= 9 ? 3 : 1); }

template <typename T, int VW, bool COPY, int KM>
__global__ __launch_bounds__(256, agg_min_blocks<KM>()) void agg_kernel(AggArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  const int total = a.BH * a.nblk;
  const int wblk = xcd_swizzle(blockIdx.x, total);
  const int bh = wblk / a.nblk;
  const int i0 = (wblk - bh * a.nblk) * a.ti;
  const int ntok = min(a.ti, a.N - i0);
  const int dout = a.dout;
  const bool stage_z = merge_mixes(a);

  // LDS carve-up
  float* sW = reinterpret_cast<float*>(smem);                       // (K, dout) conv weights
  float* sw = sW + (COPY ? 0 : a.K * dout);                         // (ti, K) neighbour weights
  int* sj = reinterpret_cast<int*>(sw + (COPY ? 0 : a.ti * a.K));   // (ti, K) neighbour indices
  T* stage = reinterpret_cast<T*>(sj + (COPY ? 0 : a.ti * a.K));    // (na, NP)
  // staged row pitch: a multiple of the vector width, so whole vectors land aligned
  const int NP = (int)cnna_round_up((size_t)a.N, 8) + 8;
  const int64_t F0 = (int64_t)i0 * dout;
  const int a_lo = (int)(F0 / a.N);

  if (!COPY) {
    const T* W0 = static_cast<const T*>(a.w0);
    // (K, dout) fp32 conv weights: a lane reads its VW channels of a tap as
    // 16-byte vectors
    for (int e = tid; e < a.K * dout; e += 256) {
      const int c = e / a.K, r = e - c * a.K;
      sW[r * dout + c] = W0 != nullptr ? ldf(W0 + e) : 1.0f;
    }
    const int64_t base = ((int64_t)bh * a.N + i0) * a.K;
    for (int e = tid; e < ntok * a.K; e += 256) {
      sw[e] = a.w[base + e];
      sj[e] = a.idx[base + e];
    }
    __syncthreads();
  }

  const int LPT = a.lpt;                 // lanes per token (power of two)
  const int g = tid & (LPT - 1);
  const int c0 = g * VW;
  const T* V = static_cast<const T*>(a.v) + (int64_t)bh * a.N * a.dkp;
  const int b = bh / a.H, h = bh - b * a.H;

  // one token's conv output (VW channels from c0) to Z / the staged range / y
  auto emit = [&](int i, const float (&acc)[VW]) __attribute__((always_inline)) {
    if (stage_z) {
      const int64_t f0 = (int64_t)i * dout + c0;
      int aa = (int)(f0 / a.N);
      int t = (int)(f0 - (int64_t)aa * a.N);
      if (VW > 1 && t % VW == 0 && t + VW <= a.N) {
        Vec<T, VW>::store(stage + (aa - a_lo) * NP + t, acc);   // one 16-byte LDS write
      } else {
#pragma unroll
        for (int u = 0; u < VW; ++u) {
          stf(stage + (aa - a_lo) * NP + t, acc[u]);
          if (++t == a.N) { t = 0; ++aa; }
        }
      }
    } else if (a.merged) {
      // reference merge with H == 1: Z[b, i, c] = y[b, c, i] (layers.py:248-249, 255-256);
      // MERGE_CONCAT: Z[b, i, h*dk + c]
      Vec<T, VW>::store(static_cast<T*>(a.out) + ((int64_t)b * a.N + i) * a.C + h * dout + c0, acc);
    } else {
      Vec<T, VW>::store(static_cast<T*>(a.out) + ((int64_t)bh * a.N + i) * dout + c0, acc);
    }
  };

  if constexpr (!COPY && KM > 0) {
    // Software-pipelined gather: the K neighbour rows of the next token group
    // are in flight while the current group is convolved.  Per element: one
    // unpack, one multiply by the neighbour weight, one FMA with the conv
    // weight (fp32 LDS vectors); gather offsets in 32 bits; the staged
    // position (row a, column t of the merge) stepped, not divided.
    typedef typename Vec<T, VW>::Raw Raw;
    const int step = 256 / LPT;
    if (c0 < dout) {
      // Unconditional loads (token and neighbour slot clamped into range): the
      // compiler then knows how many loads follow each group's and waits for
      // that group alone (a conditional prefetch made every use wait for all
      // loads, the next group's included, so the gathers did not overlap).
      auto load = [&](int tt, Raw (&raw)[KM]) __attribute__((always_inline)) {
        const int tc = min(tt, ntok - 1);
        // the gathers are issued at a raised wave priority, ahead of the other
        // waves' FMA work, so more rows are in flight sooner (c3 about 1 %)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int r = 0; r < KM; ++r)
          raw[r] = Vec<T, VW>::raw(V + (uint32_t)(sj[tc * a.K + min(r, a.K - 1)] * a.dkp + c0));
        __builtin_amdgcn_s_setprio(0);
      };
      // merge position of (token i0 + tt, channel c0) and its step per pass
      int tt0 = tid / LPT;
      int f0 = (i0 + tt0) * dout + c0;
      int za = f0 / a.N, zt = f0 - za * a.N;
      const int dstep = step * dout;
      const int qa = dstep / a.N, qt = dstep - qa * a.N;
      const bool fastv = (a.N % VW) == 0;
      auto conv_emit = [&](int tt, const Raw (&raw)[KM]) __attribute__((always_inline)) {
        float acc[VW];
#pragma unroll
        for (int u = 0; u < VW; ++u) acc[u] = 0.0f;
#pragma unroll
        for (int r = 0; r < KM; ++r) {
          if (r < a.K) {
            const float wr = sw[tt * a.K + r];
            float vv[VW];
            Vec<T, VW>::unpack(raw[r], vv);
            const float4* wp = reinterpret_cast<const float4*>(sW + r * dout + c0);
#pragma unroll
            for (int q4 = 0; q4 < VW / 4; ++q4) {
              const float4 w4 = wp[q4];
              acc[4 * q4 + 0] += w4.x * (wr * vv[4 * q4 + 0]);
              acc[4 * q4 + 1] += w4.y * (wr * vv[4 * q4 + 1]);
              acc[4 * q4 + 2] += w4.z * (wr * vv[4 * q4 + 2]);
              acc[4 * q4 + 3] += w4.w * (wr * vv[4 * q4 + 3]);
            }
          }
        }
        if (stage_z) {
          T* dst = stage + (za - a_lo) * NP + zt;
          if (fastv) {
            Vec<T, VW>::store(dst, acc);                  // one 16-byte LDS write
          } else {
            int aa = za, t = zt;
#pragma unroll
            for (int u = 0; u < VW; ++u) {
              stf(stage + (aa - a_lo) * NP + t, acc[u]);
              if (++t == a.N) { t = 0; ++aa; }
            }
          }
          zt += qt;
          za += qa;
          if (zt >= a.N) { zt -= a.N; ++za; }
        } else {
          emit(i0 + tt, acc);
        }
      };
      Raw ra[KM], rb[KM];
      int tt = tt0;
      load(tt, ra);
      // two steps per iteration so the buffers alternate without copies
      for (; tt < ntok; tt += 2 * step) {
        load(tt + step, rb);
        conv_emit(tt, ra);
        if (tt + step >= ntok) break;
        load(tt + 2 * step, ra);
        conv_emit(tt + step, rb);
      }
    }
  } else {
    for (int tt = tid / LPT; tt < ntok; tt += 256 / LPT) {
      if (c0 >= dout) continue;
      const int i = i0 + tt;
      float acc[VW];
      if (COPY) {
        Vec<T, VW>::load(static_cast<const T*>(a.v) + ((int64_t)bh * a.N + i) * dout + c0, acc);
      } else {
#pragma unroll
        for (int u = 0; u < VW; ++u) acc[u] = 0.0f;
        for (int r = 0; r < a.K; ++r) {
          const int j = sj[tt * a.K + r];
          const float wr = sw[tt * a.K + r];
          float vv[VW];
          Vec<T, VW>::load(V + (int64_t)j * a.dkp + c0, vv);
#pragma unroll
          for (int u = 0; u < VW; ++u) acc[u] += sW[r * dout + c0 + u] * (wr * vv[u]);
        }
      }
      emit(i, acc);
    }
  }
  if (!stage_z) return;
  __syncthreads();

  // write the staged flat range into Z
  const int64_t F1 = (int64_t)(i0 + ntok) * dout;
  const int na = (int)((F1 - 1) / a.N) - a_lo + 1;
  constexpr int ZV = 16 / sizeof(T);
  if (F0 % a.N == 0 && F1 % a.N == 0 && na % ZV == 0 && (h * dout + a_lo) % ZV == 0 && a.C % ZV == 0) {
    // the block covers na whole columns of Z, a multiple of ZV (16 aligned
    // bytes per row and group): a thread per (row t, column group) gathers the
    // group from ZV staged rows, one 16-byte store; the groups of a row are on
    // adjacent lanes, so a row's segment is one contiguous write (c3: 30 -> 27 us)
    T* Zb = static_cast<T*>(a.out) + (int64_t)b * a.N * a.C + h * dout + a_lo;
    const int ng = na / ZV;
    for (int e = tid; e < a.N * ng; e += 256) {
      const int t = e / ng, gq = e - t * ng;
      union {
        u32x4_t u;
        T e[ZV];
      } pk;
#pragma unroll
      for (int u = 0; u < ZV; ++u) pk.e[u] = stage[(gq * ZV + u) * NP + t];
      *reinterpret_cast<u32x4_t*>(Zb + (int64_t)t * a.C + gq * ZV) = pk.u;
    }
    return;
  }
  // general case: lanes run along the columns a of a row t
  const int rows_per_it = 256 / na;
  const int ar = tid % na, trow = tid / na;
  if (trow >= rows_per_it) return;
  T* Z = static_cast<T*>(a.out) + (int64_t)b * a.N * a.C + h * dout + a_lo + ar;
  const int64_t fa = (int64_t)(a_lo + ar) * a.N;
  for (int t = trow; t < a.N; t += rows_per_it) {
    const int64_t f = fa + t;
    if (f < F0 || f >= F1) continue;
    Z[(int64_t)t * a.C] = stage[ar * NP + t];
  }
}

template <typename T, bool COPY>
int launch_vw(const AggArgs& a0, hipStream_t s) {
  AggArgs a = a0;
  constexpr int V = 16 / sizeof(T);
  const bool vec = (a.dout % V == 0) && (COPY || a.dkp % V == 0);
  const int vw = vec ? V : 1;
  int lpt = 1;
  while (lpt < (a.dout + vw - 1) / vw) lpt <<= 1;
  if (lpt > 256) return CNNA_ERR_SHAPE;
  a.lpt = lpt;
  // tokens per block: about sixteen Z columns per row when merging (two
  // 16-byte vectors per row of the write-back), within LDS
  const bool stage_z = merge_mixes(a);
  int ti = 128;
  if (stage_z) {
    ti = (int)cnna_round_up((size_t)((16LL * a.N + a.dout - 1) / a.dout), 16);
    ti = ti < 16 ? 16 : (ti > 256 ? 256 : ti);
  }
  auto lds = [&](int t) {
    size_t n = COPY ? 0 : ((size_t)a.K * a.dout * 4 + (size_t)t * a.K * 8);
    if (stage_z) {
      const int na = (int)(((int64_t)t * a.dout - 1) / a.N) + 2;
      if (na > 256) return (size_t)1 << 40;
      n += (size_t)na * (cnna_round_up((size_t)a.N, 8) + 8) * sizeof(T);
    }
    return n;
  };
  while (ti > 1 && lds(ti) > 96 * 1024) ti >>= 1;
  if (lds(ti) > 96 * 1024) return CNNA_ERR_SHAPE;
  a.ti = ti;
  a.nblk = (a.N + ti - 1) / ti;
  dim3 grid(a.BH * a.nblk);
  if constexpr (!COPY) {
    if (vec && a.K <= 9) {
      hipLaunchKernelGGL((agg_kernel<T, V, COPY, 9>), grid, dim3(256), lds(ti), s, a);
      return (int)hipGetLastError();
    }
    if (vec && a.K <= 16) {
      hipLaunchKernelGGL((agg_kernel<T, V, COPY, 16>), grid, dim3(256), lds(ti), s, a);
      return (int)hipGetLastError();
    }
  }
  if (vec)
    hipLaunchKernelGGL((agg_kernel<T, V, COPY, 0>), grid, dim3(256), lds(ti), s, a);
  else
    hipLaunchKernelGGL((agg_kernel<T, 1, COPY, 0>), grid, dim3(256), lds(ti), s, a);
  return (int)hipGetLastError();
}

}  // namespace

int launch_aggregate(int dtype, const AggArgs& a, hipStream_t s) {
  if (a.BH <= 0 || a.N <= 0) return 0;
  if (dtype == CNNA_BF16) return launch_vw<uint16_t, false>(a, s);
  if (dtype == CNNA_F16) return launch_vw<_Float16, false>(a, s);
  if (dtype == CNNA_F32) return launch_vw<float, false>(a, s);
  return CNNA_ERR_DTYPE;
}

int launch_merge(int dtype, const AggArgs& a, hipStream_t s) {
  if (a.BH <= 0 || a.N <= 0) return 0;
  if (dtype == CNNA_BF16) return launch_vw<uint16_t, true>(a, s);
  if (dtype == CNNA_F16) return launch_vw<_Float16, true>(a, s);
  if (dtype == CNNA_F32) return launch_vw<float, true>(a, s);
  return CNNA_ERR_DTYPE;
}
