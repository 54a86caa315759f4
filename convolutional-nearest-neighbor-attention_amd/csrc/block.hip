// ViT block around the operator (vit.py:247-269): LayerNorm over the hidden
// dimension, optionally with the residual add in front of it (x + attention
// output before norm2, vit.py:264, 267).
//
// The row is read once into registers; mean and variance are two fp32
// reductions over the row (mean first, then the mean of squared deviations),
// rstd = 1/sqrt(var + eps) as nn.LayerNorm.  Rows of 16-byte vectors: 16 lanes
// per row with DPP reductions; otherwise one wave per row, element by element.
// With a residual the sum is rounded to the storage type first (the unfused
// x + y produces that tensor) and optionally written out.  A statistics-only
// kernel writes the per-tile partials a folded LayerNorm (gemm.hip) reads.
#include "common.h"
#include "kernels.h"

namespace {


CNNA_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <typename T, int E>
__global__ __launch_bounds__(256) void layernorm_kernel(LnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const T* x = static_cast<const T*>(a.x) + row * a.ldx;
  const T* r = a.res ? static_cast<const T*>(a.res) + row * a.ldr : nullptr;
  float v[E];
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = lane + 64 * e;
    v[e] = 0.0f;
    if (c < a.C) {
      float t = ldf(x + c);
      if (r != nullptr) t = rnd_to(t + ldf(r + c), T(0));
      v[e] = t;
      s += t;
    }
  }
  const float mean = wave_sum(s) / (float)a.C;
  float q = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = lane + 64 * e;
    if (c < a.C) {
      const float d = v[e] - mean;
      q += d * d;
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)a.C + a.eps);
  T* so = a.sum_out ? static_cast<T*>(a.sum_out) + row * a.lds : nullptr;
  T* y = static_cast<T*>(a.y) + row * a.ldy;
  const T* gm = static_cast<const T*>(a.gamma);
  const T* bt = static_cast<const T*>(a.beta);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = lane + 64 * e;
    if (c < a.C) {
      if (so != nullptr) stf(so + c, v[e]);
      float o = (v[e] - mean) * rstd;
      if (gm != nullptr) o *= ldf(gm + c);
      if (bt != nullptr) o += ldf(bt + c);
      stf(y + c, o);
    }
  }
}

// Vector form: 16 lanes per row (4 rows per wave), 16-byte vectors; lane g of
// a row holds vectors g, g + 16, ... (EV per lane).  The row sums are DPP
// reductions inside the 16-lane row (no LDS traffic).

template <typename T, int EV>
__global__ __launch_bounds__(256) void layernorm_vec_kernel(LnArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  const int g = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  // rows past the end still run the reductions (DPP reads neighbouring lanes) but touch no memory
  const bool ok = row < a.rows;
  const int nv = a.C / VEC;
  const T* x = static_cast<const T*>(a.x) + row * a.ldx;
  const T* r = a.res ? static_cast<const T*>(a.res) + row * a.ldr : nullptr;
  float v[EV][VEC];
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < EV; ++e) {
    const int cv = g + 16 * e;
#pragma unroll
    for (int u = 0; u < VEC; ++u) v[e][u] = 0.0f;
    if (ok && cv < nv) {
      union {
        u32x4_t q;
        T t[VEC];
      } lx, lr;
      lx.q = *reinterpret_cast<const u32x4_t*>(x + cv * VEC);
      if (r != nullptr) lr.q = *reinterpret_cast<const u32x4_t*>(r + cv * VEC);
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
        float t = ldf(&lx.t[u]);
        if (r != nullptr) t = rnd_to(t + ldf(&lr.t[u]), T(0));
        v[e][u] = t;
        s += t;
      }
    }
  }
  const float mean = row16_sum(s) / (float)a.C;
  float q = 0.0f;
#pragma unroll
  for (int e = 0; e < EV; ++e) {
    if (g + 16 * e < nv) {
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
        const float d = v[e][u] - mean;
        q += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(row16_sum(q) / (float)a.C + a.eps);
  if (!ok) return;
  T* so = a.sum_out ? static_cast<T*>(a.sum_out) + row * a.lds : nullptr;
  T* y = static_cast<T*>(a.y) + row * a.ldy;
  const T* gm = static_cast<const T*>(a.gamma);
  const T* bt = static_cast<const T*>(a.beta);
#pragma unroll
  for (int e = 0; e < EV; ++e) {
    const int cv = g + 16 * e;
    if (cv < nv) {
      union {
        u32x4_t q;
        T t[VEC];
      } o, sv, lg, lb;
      if (gm != nullptr) lg.q = *reinterpret_cast<const u32x4_t*>(gm + cv * VEC);
      if (bt != nullptr) lb.q = *reinterpret_cast<const u32x4_t*>(bt + cv * VEC);
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
        float t = (v[e][u] - mean) * rstd;
        if (gm != nullptr) t *= ldf(&lg.t[u]);
        if (bt != nullptr) t += ldf(&lb.t[u]);
        stf(&o.t[u], t);
        stf(&sv.t[u], v[e][u]);
      }
      *reinterpret_cast<u32x4_t*>(y + cv * VEC) = o.q;
      if (so != nullptr) *reinterpret_cast<u32x4_t*>(so + cv * VEC) = sv.q;
    }
  }
}

// Statistics only, for a LayerNorm folded into the GEMM that consumes its
// output: per ROW_STAT_TILE-column tile of each row, the tile's mean and M2
// (the sum of squared deviations from that mean), two passes.  One wave per
// row, two columns per lane per tile.
template <typename T>
__global__ __launch_bounds__(256) void row_stats_kernel(LnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const T* x = static_cast<const T*>(a.x) + row * a.ldx;
  const int parts = (a.C + ROW_STAT_TILE - 1) / ROW_STAT_TILE;
  for (int t = 0; t < parts; ++t) {
    const int c0 = t * ROW_STAT_TILE, nt = min(ROW_STAT_TILE, a.C - c0);
    const bool k0 = lane < nt, k1 = lane + 64 < nt;
    const float v0 = k0 ? ldf(x + c0 + lane) : 0.0f;
    const float v1 = k1 ? ldf(x + c0 + 64 + lane) : 0.0f;
    const float mean = wave_sum(v0 + v1) / (float)nt;
    const float d0 = k0 ? v0 - mean : 0.0f, d1 = k1 ? v1 - mean : 0.0f;
    const float q = wave_sum(d0 * d0 + d1 * d1);
    if (lane == 0) *reinterpret_cast<float2*>(a.stats + (row * parts + t) * 2) = make_float2(mean, q);
  }
}

inline bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename T>
int launch_ln_t(const LnArgs& a, hipStream_t s) {
  constexpr int VEC = 16 / sizeof(T);
  const bool vec = a.C % VEC == 0 && a16(a.x) && a16(a.y) && (a.ldx % VEC == 0) && (a.ldy % VEC == 0) &&
                   (!a.res || (a16(a.res) && a.ldr % VEC == 0)) &&
                   (!a.sum_out || (a16(a.sum_out) && a.lds % VEC == 0)) &&
                   (!a.gamma || a16(a.gamma)) && (!a.beta || a16(a.beta));
  if (vec && a.C <= 1024) {
    const dim3 grid16((unsigned)((a.rows + 15) / 16));
    const int ev = (a.C / VEC + 15) / 16;
    if (ev <= 2)
      hipLaunchKernelGGL((layernorm_vec_kernel<T, 2>), grid16, dim3(256), 0, s, a);
    else if (ev <= 4)
      hipLaunchKernelGGL((layernorm_vec_kernel<T, 4>), grid16, dim3(256), 0, s, a);
    else if (ev <= 8)
      hipLaunchKernelGGL((layernorm_vec_kernel<T, 8>), grid16, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((layernorm_vec_kernel<T, 16>), grid16, dim3(256), 0, s, a);
    return (int)hipGetLastError();
  }
  const dim3 grid((unsigned)((a.rows + 3) / 4));
  if (a.C <= 256)
    hipLaunchKernelGGL((layernorm_kernel<T, 4>), grid, dim3(256), 0, s, a);
  else if (a.C <= 512)
    hipLaunchKernelGGL((layernorm_kernel<T, 8>), grid, dim3(256), 0, s, a);
  else if (a.C <= 1024)
    hipLaunchKernelGGL((layernorm_kernel<T, 16>), grid, dim3(256), 0, s, a);
  else
    return CNNA_ERR_SHAPE;
  return (int)hipGetLastError();
}

}  // namespace

int launch_layernorm(int dtype, const LnArgs& a, hipStream_t s) {
  if (a.rows <= 0) return 0;
  if (a.C <= 0) return CNNA_ERR_SHAPE;
  if (a.stats != nullptr) {
    const dim3 grid((unsigned)((a.rows + 3) / 4));
    if (dtype == CNNA_BF16)
      hipLaunchKernelGGL(row_stats_kernel<uint16_t>, grid, dim3(256), 0, s, a);
    else if (dtype == CNNA_F16)
      hipLaunchKernelGGL(row_stats_kernel<_Float16>, grid, dim3(256), 0, s, a);
    else if (dtype == CNNA_F32)
      hipLaunchKernelGGL(row_stats_kernel<float>, grid, dim3(256), 0, s, a);
    else
      return CNNA_ERR_DTYPE;
    return (int)hipGetLastError();
  }
  if (dtype == CNNA_BF16) return launch_ln_t<uint16_t>(a, s);
  else if (dtype == CNNA_F16) return launch_ln_t<_Float16>(a, s);
  if (dtype == CNNA_F32) return launch_ln_t<float>(a, s);
  return CNNA_ERR_DTYPE;
}
