// Implementation of the fused similarity + top-k kernel; included by
// select_bf16.hip and select_f32.hip so the two dtypes compile in parallel.
#pragma once
// Fused similarity + streaming top-k (replaces layers.py:323-340 followed by
// torch.topk in layers.py:344, 363, 391, 410 and the sampled self mask
// layers.py:291-292, 304-305).  The N x Nq similarity never reaches HBM.
//
// Block = 4 waves; a wave owns 32 tokens of one (batch, head).  Candidate
// (query) tiles of 64 rows are staged through LDS, double buffered, and each
// wave computes S^T for its tokens with v_mfma_f32_32x32x{16 bf16|2 f32}:
// the A operand is the candidate tile and the B operand the wave's 32 key
// rows (kept in registers), so lane l holds 16 candidates of token l % 32 per
// 32-candidate block; lanes l and l + 32 split a token's candidates.
//
// Ranking key (larger is better): dot metrics use acc * kscale (matmul scale
// 1/sqrt(d_k), cosine inputs are pre-normalised); euclidean uses -d^2 with
// d^2 = (|k|^2 + |q|^2) - 2 acc, and a negative d^2 (NaN distance in the
// reference) ranks last.  Ties break by the lowest candidate index.
//
// Two passes over the candidates:
//  1. per lane, the maximum of each 16-candidate group goes into a sorted
//     register list (med3 insertion); the K-th largest of the union of both
//     half-lanes' lists is a lower bound tau of the token's K-th key, because
//     it is attained by K distinct candidates.
//  2. the tiles are recomputed and every key >= tau is appended to a per-lane
//     LDS queue (about K + few entries per token).  Queues are merged into a
//     sorted (key, index) register list when they fill and at the end; after a
//     merge tau rises to just above the list's K-th key.  The two half-lane
//     lists are finally merged and written out.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int TJ = 64;      // candidates per tile (two MFMA blocks)
constexpr int QC = 32;      // queue capacity per lane
constexpr int NT = 256;     // threads per block

template <typename T> struct SelCfg;
template <> struct SelCfg<uint16_t> { static constexpr int MAXCH = 16, VEC = 8; };  // d <= 256
template <> struct SelCfg<float> { static constexpr int MAXCH = 64, VEC = 4; };     // d <= 128

CNNA_DEV bool better(float v, int j, float ov, int oj) { return v > ov || (v == ov && j < oj); }

template <int KMAX>
CNNA_DEV void list_insert(float (&SV)[KMAX], int (&SI)[KMAX], float v, int j) {
  bool b[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) b[r] = better(v, j, SV[r], SI[r]);
#pragma unroll
  for (int r = KMAX - 1; r >= 1; --r) {
    SV[r] = b[r - 1] ? SV[r - 1] : (b[r] ? v : SV[r]);
    SI[r] = b[r - 1] ? SI[r - 1] : (b[r] ? j : SI[r]);
  }
  SV[0] = b[0] ? v : SV[0];
  SI[0] = b[0] ? j : SI[0];
}

template <int KMAX>
CNNA_DEV void bound_insert(float (&L)[KMAX], float x) {
#pragma unroll
  for (int r = KMAX - 1; r >= 1; --r) L[r] = __builtin_amdgcn_fmed3f(L[r - 1], x, L[r]);
  L[0] = fmaxf(L[0], x);
}

// L[r] for a runtime (wave-uniform) r, written as masked ORs so the
// compiler keeps the list in registers instead of indexing scratch memory.
template <int KMAX>
CNNA_DEV int pick(const int (&L)[KMAX], int r) {
  int t = 0;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) t |= L[i] & -(int)(i == r);
  return t;
}
template <int KMAX>
CNNA_DEV float pick(const float (&L)[KMAX], int r) {
  int t = 0;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) t |= __float_as_int(L[i]) & -(int)(i == r);
  return __int_as_float(t);
}

// NCH: compile-time upper bound of the MFMA reduction chunks (d / KC)
template <typename T, int NCH, int KMAX, bool EUC, bool SMP>
__global__ __launch_bounds__(NT) void select_kernel(SelArgs a) {
  using M_ = Mfma<T>;
  constexpr int VEC = SelCfg<T>::VEC;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int total = a.BH * a.rb_per_bh;
  const int w = xcd_swizzle(blockIdx.x, total);
  const int bh = w / a.rb_per_bh, rb = w - bh * a.rb_per_bh;
  const int ti = rb * 128 + wave * 32 + col;
  const bool tvalid = ti < a.N;
  const int tic = tvalid ? ti : a.N - 1;

  const int dkp = a.dkp, nch = dkp / M_::KC;
  const int QS = dkp + VEC;  // LDS row stride of a candidate tile (elements)
  T* qt = reinterpret_cast<T*>(smem);
  float* qnt = reinterpret_cast<float*>(smem + 2 * TJ * QS * sizeof(T));
  int* cdt = reinterpret_cast<int*>(qnt + 2 * TJ);
  float* qkey = reinterpret_cast<float*>(cdt + 2 * TJ);
  int* qidx = reinterpret_cast<int*>(qkey + QC * NT);

  const T* Kb = static_cast<const T*>(a.k) + ((int64_t)bh * a.N + tic) * dkp;
  const T* Qb = static_cast<const T*>(a.q) + (int64_t)bh * a.Nq * dkp;
  const float kni = EUC ? a.kn[(int64_t)bh * a.N + tic] : 0.0f;

  typename M_::frag kf[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    kf[c] = (c < nch) ? M_::load(Kb + c * M_::KC + half * M_::KL) : M_::zero();

  const int ntiles = (a.Nq + TJ - 1) / TJ;
  const int vpr = dkp / VEC;  // 16-byte vectors per candidate row
  constexpr int NPF = (TJ * (NCH * Mfma<T>::KC / VEC) + NT - 1) / NT;

  uint4 pf[NPF];
  float pfn = 0.0f;
  int pfc = 0;
  auto fetch = [&](int tile) __attribute__((always_inline)) {
    const int j0 = tile * TJ;
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const int e = tid + i * NT;
      const int r = e / vpr, cv = e - r * vpr;
      pf[i] = make_uint4(0, 0, 0, 0);
      if (r < TJ && j0 + r < a.Nq)
        pf[i] = *reinterpret_cast<const uint4*>(Qb + (int64_t)(j0 + r) * dkp + cv * VEC);
    }
    if (tid < TJ) {
      const int j = j0 + tid;
      if (EUC) pfn = (j < a.Nq) ? a.qn[(int64_t)bh * a.Nq + j] : 0.0f;
      if (SMP) pfc = (j < a.Nq) ? a.cand[j] : -1;
    }
  };
  auto stash = [&](int buf) __attribute__((always_inline)) {
    T* dst = qt + buf * TJ * QS;
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const int e = tid + i * NT;
      const int r = e / vpr, cv = e - r * vpr;
      if (r < TJ) *reinterpret_cast<uint4*>(dst + r * QS + cv * VEC) = pf[i];
    }
    if (tid < TJ) {
      if (EUC) qnt[buf * TJ + tid] = pfn;
      if (SMP) cdt[buf * TJ + tid] = pfc;
    }
  };

  // S^T tile for this wave: acc[blk][v] = k_ti . q_{j0 + blk*32 + mfma_row(v)}
  auto compute = [&](int buf, f32x16_t (&acc)[2]) __attribute__((always_inline)) {
    const T* base = qt + buf * TJ * QS;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c < nch) {
        const typename M_::frag a0 = M_::load(base + col * QS + c * M_::KC + half * M_::KL);
        const typename M_::frag a1 = M_::load(base + (32 + col) * QS + c * M_::KC + half * M_::KL);
        acc[0] = M_::mma(a0, kf[c], acc[0]);
        acc[1] = M_::mma(a1, kf[c], acc[1]);
      }
    }
  };
  // ranking key of one accumulator entry (NaN = not a candidate)
  auto keyof = [&](float accv, int buf, int jl, int j) __attribute__((always_inline)) -> float {
    float key;
    if (EUC) {
      const float d2 = __builtin_fmaf(-2.0f, accv, kni + qnt[buf * TJ + jl]);
      key = (d2 >= 0.0f) ? -d2 : -INFINITY;
    } else {
      key = accv * a.kscale;
    }
    if (SMP && cdt[buf * TJ + jl] == ti) key = a.mask_key;
    return (j < a.Nq) ? key : __builtin_nanf("");
  };

  // drive the double-buffered tile loop; body(buf, j0) per tile
  auto sweep = [&](auto&& body) __attribute__((always_inline)) {
    fetch(0);
    stash(0);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
      const int buf = t & 1;
      if (t + 1 < ntiles) fetch(t + 1);
      body(buf, t * TJ);
      if (t + 1 < ntiles) stash(buf ^ 1);
      __syncthreads();
    }
  };

  float SV[KMAX];
  int SI[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) { SV[r] = -INFINITY; SI[r] = 0x7fffffff; }

  if (a.Ksel > 0) {
    // ---------------- pass 1: group-max bound
    float L[KMAX];
#pragma unroll
    for (int r = 0; r < KMAX; ++r) L[r] = -INFINITY;
    sweep([&](int buf, int j0) __attribute__((always_inline)) {
      f32x16_t acc[2];
      compute(buf, acc);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float gm = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int jl = b * 32 + mfma_row(v, lane);
          gm = fmaxf(gm, keyof(acc[b][v], buf, jl, j0 + jl));
        }
        bound_insert<KMAX>(L, gm);
      }
    });
    {
      float P[KMAX];
#pragma unroll
      for (int r = 0; r < KMAX; ++r) P[r] = __shfl_xor(L[r], 32);
#pragma unroll
      for (int r = 0; r < KMAX; ++r) bound_insert<KMAX>(L, P[r]);
    }
    float tau = pick<KMAX>(L, a.Ksel - 1);

    // ---------------- pass 2: filter + queue
    int cnt = 0;
    float* myk = qkey + tid;
    int* myi = qidx + tid;
    auto drain = [&]() __attribute__((always_inline)) {
      for (int e = 0; __any(e < cnt); ++e) {
        if (e < cnt) list_insert<KMAX>(SV, SI, myk[e * NT], myi[e * NT]);
      }
      cnt = 0;
      const int kth = pick<KMAX>(SI, a.Ksel - 1);
      if (kth != 0x7fffffff) tau = fmaxf(tau, next_up(pick<KMAX>(SV, a.Ksel - 1)));
    };
    sweep([&](int buf, int j0) __attribute__((always_inline)) {
      f32x16_t acc[2];
      compute(buf, acc);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        if (__any(cnt > QC - 16)) drain();
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int jl = b * 32 + mfma_row(v, lane);
          const float key = keyof(acc[b][v], buf, jl, j0 + jl);
          if (key >= tau) {
            myk[cnt * NT] = key;
            myi[cnt * NT] = j0 + jl;
            ++cnt;
          }
        }
      }
    });
    drain();
  }

  // ---------------- merge the two half-lane lists and write out
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    qkey[r * NT + tid] = SV[r];
    qidx[r * NT + tid] = SI[r];
  }
  __syncthreads();
  if (half == 0 && tvalid) {
    const int64_t o = ((int64_t)bh * a.N + ti) * a.K;
    int off = 0;
    if (SMP) {
      a.idx[o] = ti;
      a.vals[o] = 1.0f;
      off = 1;
    }
    int ia = 0, ib = 0;
    for (int r = 0; r < a.Ksel; ++r) {
      const int ra = ia < KMAX ? ia : KMAX - 1, rb2 = ib < KMAX ? ib : KMAX - 1;
      const float va = qkey[ra * NT + tid], vb = qkey[rb2 * NT + tid + 32];
      const int ja = qidx[ra * NT + tid], jb = qidx[rb2 * NT + tid + 32];
      const bool ta = (ia < KMAX) && (ib >= KMAX || better(va, ja, vb, jb));
      const float key = ta ? va : vb;
      const int j = ta ? ja : jb;
      ia += ta ? 1 : 0;
      ib += ta ? 0 : 1;
      float val = key;
      int tok = j;
      if (SMP) tok = a.cand[j];
      if (EUC) val = (key == -INFINITY) ? __builtin_nanf("") : sqrtf(-key);
      if (SMP && EUC && tok == ti) val = a.mask_val;
      a.idx[o + off + r] = tok;
      a.vals[o + off + r] = val;
    }
  }
}

template <typename T, int NCH, int KMAX>
int launch_k(int euclid, int sampled, const SelArgs& a, size_t smem, dim3 grid, hipStream_t s) {
  if (!euclid && !sampled)
    hipLaunchKernelGGL((select_kernel<T, NCH, KMAX, false, false>), grid, dim3(NT), smem, s, a);
  else if (!euclid && sampled)
    hipLaunchKernelGGL((select_kernel<T, NCH, KMAX, false, true>), grid, dim3(NT), smem, s, a);
  else if (euclid && !sampled)
    hipLaunchKernelGGL((select_kernel<T, NCH, KMAX, true, false>), grid, dim3(NT), smem, s, a);
  else
    hipLaunchKernelGGL((select_kernel<T, NCH, KMAX, true, true>), grid, dim3(NT), smem, s, a);
  return (int)hipGetLastError();
}

template <typename T, int NCH>
int launch_n(int euclid, int sampled, const SelArgs& a, size_t smem, dim3 grid, hipStream_t s) {
  if (a.Ksel <= 9) return launch_k<T, NCH, 9>(euclid, sampled, a, smem, grid, s);
  if (a.Ksel <= 16) return launch_k<T, NCH, 16>(euclid, sampled, a, smem, grid, s);
  if (a.Ksel <= 32) return launch_k<T, NCH, 32>(euclid, sampled, a, smem, grid, s);
  return CNNA_ERR_K_RANGE;
}

template <typename T>
int launch_select_t(int euclid, int sampled, const SelArgs& a, hipStream_t s) {
  if (a.dkp % Mfma<T>::KC != 0 || a.dkp > SelCfg<T>::MAXCH * Mfma<T>::KC || a.dkp % SelCfg<T>::VEC != 0)
    return CNNA_ERR_SHAPE;
  const size_t smem = 2 * TJ * (a.dkp + SelCfg<T>::VEC) * sizeof(T) + 2 * TJ * (sizeof(float) + sizeof(int)) +
                      (size_t)QC * NT * (sizeof(float) + sizeof(int));
  dim3 grid(a.BH * a.rb_per_bh);
  const int nch = a.dkp / Mfma<T>::KC;
  const int q = SelCfg<T>::MAXCH / 4;   // chunk classes: d <= 64, 128, 256 (bf16) / 32, 64, 128 (f32)
  if (nch <= q) return launch_n<T, SelCfg<T>::MAXCH / 4>(euclid, sampled, a, smem, grid, s);
  if (nch <= 2 * q) return launch_n<T, SelCfg<T>::MAXCH / 2>(euclid, sampled, a, smem, grid, s);
  return launch_n<T, SelCfg<T>::MAXCH>(euclid, sampled, a, smem, grid, s);
}
}  // namespace

