// MFMA GEMM  out[m][n] = sum_k A[m][k] * W[n][k]  (nn.Linear: x @ W^T).
//
// Used for the Q/K/V projections with the head split in the epilogue
// (layers.py:264-265, 274, 237-245), the output projection W_o (layers.py:320),
// the standard conv as a gather-GEMM over the K neighbours (layers.py:313 with
// the prime tensor of layers.py:402-405 built on the fly in the A loader) and
// the pointwise half of the depthwise-separable conv.
//
// Tile 128 x 128 x BK, 256 threads = 4 waves in a 2 x 2 grid, each wave owns a
// 64 x 64 block = 2 x 2 v_mfma_f32_32x32x{16 bf16 | 2 f32} accumulators.  The
// MFMA computes the transposed tile (W as the A operand), so each lane ends
// with 4 consecutive output columns of one row and stores them as one vector.
// The next k-tile is fetched into registers while the current one is
// multiplied from LDS (rows padded by 16 bytes).  Blocks are ordered so that
// all column tiles of a row tile run on the same XCD (shared L2).
//
// LayerNorm folding (the pre-norm ViT block, vit.py:260-267): with a LN
// prologue the A rows are normalised in registers between the global load and
// the LDS store, from per-row statistics combined out of per-128-column
// (mean, M2) partials; with a statistics epilogue the bf16 GEMM that writes a
// residual-stream row (W_o + residual, fc2 + residual) also writes those
// partials for the rows it stores, so the LayerNorm that follows costs no
// pass of its own.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace {

constexpr int BM = 128, BN = 128;
static_assert(BN == ROW_STAT_TILE, "one statistics partial per column tile");
// widest row a LayerNorm prologue normalises (gamma / beta staged in LDS)
constexpr int LN_MAX_K = 1024;

template <typename T> struct GemmCfg;
template <> struct GemmCfg<uint16_t> { static constexpr int BK = 64, VEC = 8; };
template <> struct GemmCfg<_Float16> { static constexpr int BK = 64, VEC = 8; };
template <> struct GemmCfg<float> { static constexpr int BK = 32, VEC = 4; };

template <typename T, int VEC>
union Pack {
  u32x4_t u;
  T e[VEC];
};

// w * (16-byte vector of T), rounded back to T
template <typename T>
CNNA_DEV u32x4_t scale_vec16(u32x4_t s, float w) {
  u32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = Pair16<T>::pack(w * Pair16<T>::lo(s[i]), w * Pair16<T>::hi(s[i]));
  return o;
}
CNNA_DEV u32x4_t scale_vec(u32x4_t s, float w, uint16_t) { return scale_vec16<uint16_t>(s, w); }
CNNA_DEV u32x4_t scale_vec(u32x4_t s, float w, _Float16) { return scale_vec16<_Float16>(s, w); }
CNNA_DEV u32x4_t scale_vec(u32x4_t s, float w, float) {
  u32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = __float_as_uint(w * __uint_as_float(s[i]));
  return o;
}

// Linear epilogue before the store: v + bias[n], then the activation.  For
// bf16 the biased value is rounded to bf16 first, as the unfused nn.Linear ->
// nn.GELU sequence rounds it.
template <typename T, int EPI>
CNNA_DEV float lin_epi(const GemmArgs& g, float v, int n) {
  if (g.bias != nullptr) v += ldf(static_cast<const T*>(g.bias) + n);
  if (EPI == 2) {
    v = rnd_to(v, T(0));
    v = gelu_erf(v);
  }
  return v;
}

// four consecutive outputs -> one 8-byte (bf16) or 16-byte (fp32) store
template <typename T>
CNNA_DEV void store4_16(T* p, float a, float b, float c, float d) {
  uint2 u;
  u.x = Pair16<T>::pack(a, b);
  u.y = Pair16<T>::pack(c, d);
  *reinterpret_cast<uint2*>(p) = u;
}
CNNA_DEV void store4(uint16_t* p, float a, float b, float c, float d) { store4_16(p, a, b, c, d); }
CNNA_DEV void store4(_Float16* p, float a, float b, float c, float d) { store4_16(p, a, b, c, d); }
CNNA_DEV void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}

// FAST: 16-byte loads everywhere and Kd % BK == 0 (decided by the launcher);
// EPI: the nn.Linear extras of a plain output are compiled in (0: none, 1: bias
// and residual, 2: bias, GELU and residual), as separate instances so the
// operator's own GEMMs keep their epilogues lean
// XF: bit 0 the LayerNorm prologue on A, bit 1 the row-statistics epilogue
// (three blocks per CU: accumulators in AGPRs + VGPRs within 168 registers)
template <typename T, int AMODE, int OMODE, bool FAST, int EPI = 0, int XF = 0>
__global__ __launch_bounds__(256, 3) void gemm_kernel(GemmArgs g) {
  using M_ = Mfma<T>;
  constexpr int BK = GemmCfg<T>::BK, VEC = GemmCfg<T>::VEC;
  constexpr int LDS_STRIDE = BK + VEC;      // elements; rows stay 16-byte aligned
  constexpr int VPR = BK / VEC;             // 16-byte vectors per tile row
  constexpr int NV = BM * VPR / 256;        // vectors per thread per operand tile
  __shared__ __attribute__((aligned(16))) T smem_ab[(BM + BN) * LDS_STRIDE];
  T* As = smem_ab;
  T* Bs = smem_ab + BM * LDS_STRIDE;
  // LayerNorm prologue: gamma, beta (fp32, zero past Kd) and each tile row's
  // (rstd, -mean * rstd), read back as the A tiles are stashed
  __shared__ __attribute__((aligned(16))) float ln_smem[(XF & 1) ? 2 * LN_MAX_K + 2 * BM : 4];
  float* ln_g = ln_smem;
  float* ln_b = ln_smem + LN_MAX_K;
  float* ln_row = ln_smem + 2 * LN_MAX_K;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int ncol = (g.Nc + BN - 1) / BN;
  const int nrow = (g.M + BM - 1) / BM;
  const int wid = xcd_swizzle(blockIdx.x, ncol * nrow);
  const int n0 = (wid % ncol) * BN, m0 = (wid / ncol) * BM;
  const T* A = static_cast<const T*>(g.a);

  // per-thread rows of the A and W tiles
  int rowv[NV], kvv[NV];
  const T* arow_ptr[NV];
  const T* wrow_ptr[NV];
  bool arow_ok[NV], wrow_ok[NV];
  int64_t gather_base[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = tid + i * 256;
    rowv[i] = e / VPR;
    kvv[i] = (e % VPR) * VEC;
    const int m = m0 + rowv[i];
    arow_ok[i] = m < g.M;
    int64_t sr = arow_ok[i] ? m : 0;
    if (AMODE == GEMM_A_ROWS && g.arow != nullptr && arow_ok[i]) {
      const int b = m / g.a_rows, rr = m - b * g.a_rows;
      sr = (int64_t)b * g.a_src_rows + g.arow[rr];
    }
    arow_ptr[i] = A + sr * g.lda;
    const int mc = arow_ok[i] ? m : g.M - 1;
    gather_base[i] = (AMODE == GEMM_A_GATHER) ? (int64_t)mc - (mc % g.g_N) : 0;
    const int n = n0 + rowv[i];
    wrow_ok[i] = n < g.Nc;
    const int mat = wrow_ok[i] ? n / g.ncol_each : 0;
    const int rn = wrow_ok[i] ? n - mat * g.ncol_each : 0;
    wrow_ptr[i] = static_cast<const T*>(g.w[mat]) + (int64_t)rn * g.Kd;
  }

  Pack<T, VEC> ra[NV], rw[NV];
  auto fetch = [&](int k0) __attribute__((always_inline)) {
    if (FAST) {
      // every vector in range (rows clamped; Kd % BK == 0): no branches, so
      // the loads stay in flight while the previous tile is multiplied
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int k = k0 + kvv[i];
        if (AMODE == GEMM_A_ROWS) {
          ra[i].u = *reinterpret_cast<const u32x4_t*>(arow_ptr[i] + k);
        } else {
          const int m = min(m0 + rowv[i], g.M - 1);
          const int r = k / g.g_din, c = k - r * g.g_din;
          const int j = g.g_idx[(int64_t)m * g.g_K + r];
          const float wr = g.g_w[(int64_t)m * g.g_K + r];
          ra[i].u = scale_vec(*reinterpret_cast<const u32x4_t*>(A + (gather_base[i] + j) * g.g_dkp + c), wr, T(0));
        }
        rw[i].u = *reinterpret_cast<const u32x4_t*>(wrow_ptr[i] + k);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int k = k0 + kvv[i];
      // ---- A
      if (AMODE == GEMM_A_ROWS) {
        if (arow_ok[i] && g.avec && k + VEC <= g.Kd) {
          ra[i].u = *reinterpret_cast<const u32x4_t*>(arow_ptr[i] + k);
        } else {
#pragma unroll
          for (int t = 0; t < VEC; ++t)
            ra[i].e[t] = (arow_ok[i] && k + t < g.Kd) ? arow_ptr[i][k + t] : T(0);
        }
      } else {
        const int m = m0 + rowv[i];
#pragma unroll
        for (int t = 0; t < VEC; ++t) {
          float val = 0.0f;
          if (arow_ok[i] && k + t < g.Kd) {
            const int r = (k + t) / g.g_din, c = (k + t) - r * g.g_din;
            const int j = g.g_idx[(int64_t)m * g.g_K + r];
            val = g.g_w[(int64_t)m * g.g_K + r] * ldf(A + (gather_base[i] + j) * g.g_dkp + c);
          }
          stf(&ra[i].e[t], val);
        }
      }
      // ---- W
      if (wrow_ok[i] && g.bvec && k + VEC <= g.Kd) {
        rw[i].u = *reinterpret_cast<const u32x4_t*>(wrow_ptr[i] + k);
      } else {
#pragma unroll
        for (int t = 0; t < VEC; ++t)
          rw[i].e[t] = (wrow_ok[i] && k + t < g.Kd) ? wrow_ptr[i][k + t] : T(0);
      }
    }
  };
  auto stash = [&](int k0) __attribute__((always_inline)) {
    float gv[(XF & 1) ? VEC : 1], bv[(XF & 1) ? VEC : 1];
    if (XF & 1) {
      // every vector of a thread covers the same columns (256 % VPR == 0)
#pragma unroll
      for (int t = 0; t < VEC; t += 4) {
        const float4 g4 = *reinterpret_cast<const float4*>(&ln_g[k0 + kvv[0] + t]);
        const float4 b4 = *reinterpret_cast<const float4*>(&ln_b[k0 + kvv[0] + t]);
        gv[t] = g4.x; gv[t + 1] = g4.y; gv[t + 2] = g4.z; gv[t + 3] = g4.w;
        bv[t] = b4.x; bv[t + 1] = b4.y; bv[t + 2] = b4.z; bv[t + 3] = b4.w;
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (XF & 1) {
        // (x - mean) * rstd * gamma + beta as two FMAs (x * rstd + (-mean * rstd)),
        // rounded to T as nn.LayerNorm's output; columns past Kd stay zero
        const float2 st = *reinterpret_cast<const float2*>(&ln_row[2 * rowv[i]]);
#pragma unroll
        for (int t = 0; t < VEC; ++t) {
          float y = __builtin_fmaf(ldf(&ra[i].e[t]), st.x, st.y);
          y = __builtin_fmaf(y, gv[t], bv[t]);
          if (!FAST && k0 + kvv[i] + t >= g.Kd) y = 0.0f;
          stf(&ra[i].e[t], y);
        }
      }
      *reinterpret_cast<u32x4_t*>(&As[rowv[i] * LDS_STRIDE + kvv[i]]) = ra[i].u;
      *reinterpret_cast<u32x4_t*>(&Bs[rowv[i] * LDS_STRIDE + kvv[i]]) = rw[i].u;
    }
  };

  // acc[i][j] holds the transposed 32 x 32 block: rows = output columns
  // n0 + wn*64 + j*32 + .., columns = output rows m0 + wm*64 + i*32 + lane%32
  f32x16_t acc[2][2];

  fetch(0);
  if (XF & 1) {
    // (after the first tile's loads are issued, so both latencies overlap)
    // gamma / beta over the k-tiles (Kd <= LN_MAX_K, a multiple of BK)
    const T* gp = static_cast<const T*>(g.ln_gamma);
    const T* bp = static_cast<const T*>(g.ln_beta);
    const int kpad = (g.Kd + BK - 1) / BK * BK;
    for (int c = tid; c < kpad; c += 256) {
      const bool in = c < g.Kd;
      ln_g[c] = in ? (gp ? ldf(gp + c) : 1.0f) : 0.0f;
      ln_b[c] = (in && bp) ? ldf(bp + c) : 0.0f;
    }
    // mean and 1/sqrt(var + eps) of tile row tid from the row's per-tile
    // (mean, M2) partials (tile t holds min(ROW_STAT_TILE, Kd - t * ROW_STAT_TILE) columns)
    if (tid < BM) {
      const int m = min(m0 + tid, g.M - 1);
      int64_t sr = m;
      if (g.arow != nullptr) {
        const int b = m / g.a_rows, rr = m - b * g.a_rows;
        sr = (int64_t)b * g.a_src_rows + g.arow[rr];
      }
      const float* sp = g.ln_stats + sr * (2 * g.ln_parts);
      float sm = 0.0f;
      for (int t = 0; t < g.ln_parts; ++t) sm += (float)min(ROW_STAT_TILE, g.Kd - t * ROW_STAT_TILE) * sp[2 * t];
      const float mean = sm / (float)g.Kd;
      float q = 0.0f;
      for (int t = 0; t < g.ln_parts; ++t) {
        const float d = sp[2 * t] - mean;
        q += sp[2 * t + 1] + (float)min(ROW_STAT_TILE, g.Kd - t * ROW_STAT_TILE) * d * d;
      }
      const float rstd = 1.0f / sqrtf(q / (float)g.Kd + g.ln_eps);
      ln_row[2 * tid] = rstd;
      ln_row[2 * tid + 1] = -mean * rstd;
    }
    __syncthreads();
  }

  // one k-tile; FIRST: the first one starts the accumulators from zero (a zero
  // C operand in the MFMA instead of 64 register clears per tile)
  auto kstep = [&](int k0, auto FIRST) __attribute__((always_inline)) {
    stash(k0);
    __syncthreads();
    // the next tile's loads and the MFMA loop at a raised wave priority, ahead
    // of the other blocks' prologue / epilogue VALU work on the SIMD (ViT
    // forward about 1.5 % faster; the direct-to-LDS kernel measured no gain)
    __builtin_amdgcn_s_setprio(1);
    if (k0 + BK < g.Kd) fetch(k0 + BK);
#pragma unroll
    for (int ks = 0; ks < BK / M_::KC; ++ks) {
      const int kk = ks * M_::KC + (lane >> 5) * M_::KL;
      typename M_::frag af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[i] = M_::load(&As[(wm * 64 + i * 32 + (lane & 31)) * LDS_STRIDE + kk]);
        bfr[i] = M_::load(&Bs[(wn * 64 + i * 32 + (lane & 31)) * LDS_STRIDE + kk]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if (decltype(FIRST)::value && ks == 0) {
            f32x16_t z;
#pragma unroll
            for (int v = 0; v < 16; ++v) z[v] = 0.0f;
            acc[i][j] = M_::mma(bfr[j], af[i], z);
          } else {
            acc[i][j] = M_::mma(bfr[j], af[i], acc[i][j]);
          }
        }
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();
  };
  if (g.Kd > 0) {
    kstep(0, std::true_type{});
    for (int k0 = BK; k0 < g.Kd; k0 += BK) kstep(k0, std::false_type{});
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  }

  if constexpr (sizeof(T) == 2) if (g.ostage) {
    // ---- bf16 epilogue through LDS: the 128 x 128 tile is staged (reusing the
    // operand buffers) and written back as whole 16-byte row segments
    constexpr int CP = BN + 8;                              // staged row pitch
    T* Cs = As;                                             // 128 * 136 <= As + Bs
    // linear extras: per column block j, this lane's 16 bias values (the same
    // for both row blocks), 4 consecutive columns at a time
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float bq[EPI ? 4 : 1][4];
      if (EPI) {
        const T* bp = static_cast<const T*>(g.bias);
#pragma unroll
        for (int vq = 0; vq < (EPI ? 4 : 1); ++vq) {
          const int n = n0 + wn * 64 + j * 32 + vq * 8 + (lane >> 5) * 4;
#pragma unroll
          for (int u = 0; u < 4; ++u) bq[vq][u] = 0.0f;
          if (bp != nullptr) {
            if (n + 4 <= g.Nc && ((uintptr_t)(bp + n) % 8) == 0) {
              const uint2 b2 = *reinterpret_cast<const uint2*>(bp + n);
              bq[vq][0] = Pair16<T>::lo(b2.x);
              bq[vq][1] = Pair16<T>::hi(b2.x);
              bq[vq][2] = Pair16<T>::lo(b2.y);
              bq[vq][3] = Pair16<T>::hi(b2.y);
            } else {
#pragma unroll
              for (int u = 0; u < 4; ++u) bq[vq][u] = ldf(bp + min(n + u, g.Nc - 1));
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const int ml = wm * 64 + i * 32 + (lane & 31);
          const int nl = wn * 64 + j * 32 + vq * 8 + (lane >> 5) * 4;
          const f32x16_t& a = acc[i][j];
          float e[4] = {a[vq * 4], a[vq * 4 + 1], a[vq * 4 + 2], a[vq * 4 + 3]};
          if (EPI) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              float v = e[u] + bq[EPI ? vq : 0][u];
              if (EPI == 2) v = gelu_erf(rnd_to(v, T(0)));   // rounded as nn.Linear's output
              e[u] = v;
            }
          }
          uint2 u;
          u.x = Pair16<T>::pack(e[0], e[1]);
          u.y = Pair16<T>::pack(e[2], e[3]);
          *reinterpret_cast<uint2*>(&Cs[ml * CP + nl]) = u;
        }
    }
    __syncthreads();
    // thread -> fixed 8-column group nl, rows ml = (tid >> 4) + 16 * it: the
    // head-split coordinates are derived once and stepped, not divided per row
    const int nl = (tid & 15) * 8;
    const int n = n0 + nl;
    int mat = 0, hh = 0, cc = n, b = 0, r = 0;
    bool whole = n + 8 <= g.Nc;
    if (OMODE == GEMM_O_HEADSPLIT) {
      mat = n / g.ncol_each;
      const int nn = n - mat * g.ncol_each;
      hh = nn / g.o_dk;
      cc = nn - hh * g.o_dk;
      whole = whole && (cc + 8 <= g.o_dk);
      const int m = m0 + (tid >> 4);
      b = m / g.o_rows;
      r = m - b * g.o_rows;
    }
    T* obase = static_cast<T*>(g.o[OMODE == GEMM_O_HEADSPLIT ? (mat > 2 ? 2 : mat) : 0]);
    // statistics epilogue: the 16 threads of a row segment are one DPP row
    const int st_parts = (g.Nc + ROW_STAT_TILE - 1) / ROW_STAT_TILE;
    const float st_inv = 1.0f / (float)min(BN, g.Nc - n0);
#pragma unroll
    for (int it = 0; it < (BM * BN / 8) / 256; ++it) {
      const int ml = (tid >> 4) + it * 16;
      const int m = m0 + ml;
      if (it > 0 && OMODE == GEMM_O_HEADSPLIT) {
        r += 16;
        while (r >= g.o_rows) {
          r -= g.o_rows;
          ++b;
        }
      }
      if (XF & 2) {
        // plain output, Nc % 8 == 0 (so every segment in range is whole): store
        // the row segment, then (mean, M2) of the row's stored values in this
        // column tile, two passes over registers
        const bool ok = m < g.M && n < g.Nc;
        u32x4_t val = {0u, 0u, 0u, 0u};
        if (ok) {
          val = *reinterpret_cast<const u32x4_t*>(&Cs[ml * CP + nl]);
          if (EPI && g.res != nullptr) {
            const u32x4_t rv = *reinterpret_cast<const u32x4_t*>(static_cast<const T*>(g.res) + (int64_t)m * g.ldr + n);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              val[q] = Pair16<T>::pack(Pair16<T>::lo(val[q]) + Pair16<T>::lo(rv[q]),
                                       Pair16<T>::hi(val[q]) + Pair16<T>::hi(rv[q]));
          }
          *reinterpret_cast<u32x4_t*>(obase + (int64_t)m * g.ldo + n) = val;
        }
        float xv[8], sm = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          xv[2 * q] = Pair16<T>::lo(val[q]);
          xv[2 * q + 1] = Pair16<T>::hi(val[q]);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) sm += xv[u];
        const float mean = row16_sum(sm) * st_inv;
        float sq = 0.0f;
        if (ok) {
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const float d = xv[u] - mean;
            sq += d * d;
          }
        }
        sq = row16_sum(sq);
        if ((tid & 15) == 0 && m < g.M)
          *reinterpret_cast<float2*>(g.st_out + ((int64_t)m * st_parts + n0 / ROW_STAT_TILE) * 2) = make_float2(mean, sq);
        continue;
      }
      if (m >= g.M || n >= g.Nc) continue;
      u32x4_t val = *reinterpret_cast<const u32x4_t*>(&Cs[ml * CP + nl]);
      if (EPI && g.res != nullptr && whole) {
        // residual: bf16 linear output + bf16 residual, added in fp32 and rounded once
        const u32x4_t r = *reinterpret_cast<const u32x4_t*>(static_cast<const T*>(g.res) + (int64_t)m * g.ldr + n);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          val[q] = Pair16<T>::pack(Pair16<T>::lo(val[q]) + Pair16<T>::lo(r[q]),
                                   Pair16<T>::hi(val[q]) + Pair16<T>::hi(r[q]));
      }
      T* dst;
      if (OMODE == GEMM_O_HEADSPLIT)
        dst = obase + (((int64_t)b * g.o_H + hh) * g.o_rows + r) * g.o_dkp + cc;
      else
        dst = obase + (int64_t)m * g.ldo + n;
      if (whole) {
        *reinterpret_cast<u32x4_t*>(dst) = val;
      } else {
        // tile or head edge: element by element (rare)
        for (int u = 0; u < 8 && n + u < g.Nc; ++u) {
          const T v = Cs[ml * CP + nl + u];
          if (OMODE == GEMM_O_HEADSPLIT) {
            const int nu = n + u;
            const int mt = nu / g.ncol_each, nn = nu - mt * g.ncol_each;
            const int h = nn / g.o_dk, c = nn - h * g.o_dk;
            static_cast<T*>(g.o[mt])[(((int64_t)b * g.o_H + h) * g.o_rows + r) * g.o_dkp + c] = v;
          } else {
            if (EPI && g.res != nullptr)
              stf(&dst[u], ldf(&v) + ldf(static_cast<const T*>(g.res) + (int64_t)m * g.ldr + n + u));
            else
              dst[u] = v;
          }
        }
      }
    }
    return;
  }

  // ---- epilogue: lane owns row m (per i) and columns nq..nq+3 (per j, vq)
  int64_t roff[2];
  bool mok[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + wm * 64 + i * 32 + (lane & 31);
    mok[i] = m < g.M;
    const int mc = mok[i] ? m : 0;
    if (OMODE == GEMM_O_HEADSPLIT) {
      const int b = mc / g.o_rows, r = mc - b * g.o_rows;
      roff[i] = ((int64_t)b * g.o_H * g.o_rows + r) * g.o_dkp;
    } else {
      roff[i] = (int64_t)mc * g.ldo;
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int vq = 0; vq < 4; ++vq) {
      const int nq = n0 + wn * 64 + j * 32 + vq * 8 + (lane >> 5) * 4;
      if (nq >= g.Nc) continue;
      T* ob;
      int64_t oc;
      bool vec = g.ovec && nq + 3 < g.Nc;
      if (OMODE == GEMM_O_HEADSPLIT) {
        const int mat = nq / g.ncol_each, nn = nq - mat * g.ncol_each;
        const int h = nn / g.o_dk, c = nn - h * g.o_dk;
        ob = static_cast<T*>(g.o[mat]);
        oc = (int64_t)h * g.o_rows * g.o_dkp + c;
        vec = vec && (c + 3 < g.o_dk);
      } else {
        ob = static_cast<T*>(g.o[0]);
        oc = nq;
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (!mok[i]) continue;
        f32x16_t a = acc[i][j];
        if (EPI) {
          const int64_t rrow = (int64_t)(m0 + wm * 64 + i * 32 + (lane & 31)) * g.ldr;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int n = min(nq + u, g.Nc - 1);
            float v = lin_epi<T, EPI>(g, a[vq * 4 + u], n);
            if (g.res != nullptr) {
              v = rnd_to(v, T(0));
              v += ldf(static_cast<const T*>(g.res) + rrow + n);
            }
            a[vq * 4 + u] = v;
          }
        }
        if (vec) {
          store4(ob + roff[i] + oc, a[vq * 4], a[vq * 4 + 1], a[vq * 4 + 2], a[vq * 4 + 3]);
        } else {
          // tile edge: element by element (the head split re-derived per column)
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int n = nq + u;
            if (n >= g.Nc) break;
            if (OMODE == GEMM_O_HEADSPLIT) {
              const int mat = n / g.ncol_each, nn = n - mat * g.ncol_each;
              const int h = nn / g.o_dk, c = nn - h * g.o_dk;
              stf(static_cast<T*>(g.o[mat]) + roff[i] + (int64_t)h * g.o_rows * g.o_dkp + c, a[vq * 4 + u]);
            } else {
              stf(ob + roff[i] + n, a[vq * 4 + u]);
            }
          }
        }
      }
    }
}

// ---- Direct-to-LDS variant for 16-bit types with row-major A, Kd % 64 == 0,
// 16-byte aligned rows and the staged epilogue (no LayerNorm prologue, no
// statistics epilogue).  Tile 128 x 192 x 64, 4 waves of 64 x 96 (2 x 3 MFMA
// blocks), two blocks per CU.  The operand tiles go from global memory straight
// into LDS (global_load_lds_dwordx4: lane l of an instruction writes bytes
// [16 l, 16 l + 16) after the wave-uniform base in M0), so one instruction
// fills 8 rows of 128 bytes; a lane fetches the 16-byte chunk
// (l % 8) ^ ((row / 2) % 8) of its row, so the MFMA operand reads (16 lanes =
// 16 rows at one chunk) hit 16 distinct 16-byte slots of each 256-byte bank
// window.  Two LDS stages: the loads of k-tile t + 1 are in flight while tile t
// is multiplied.  Measured against the register-staged kernel at the workload
// shapes: Q/K/V projection (M = 32768, N = 1152, K = 384) 41 vs 52 us, W_o
// (N = K = 384) 15.6 vs 17.3 us.
constexpr int DL_BM = 128, DL_BN = 192, DL_BK = 64;

CNNA_DEV void load_to_lds16(const void* gp, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gp), "{m0}"(lds_base) : "memory");
}

template <typename T, int OMODE, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_dl_kernel(GemmArgs g) {
  using M_ = Mfma<T>;
  constexpr int MI = 2, NJ = 3, BM = DL_BM, BN = DL_BN, BK = DL_BK;
  constexpr int ROWB = BK * (int)sizeof(T);   // 128-byte LDS rows, unpadded
  constexpr int RPI = 1024 / ROWB;            // rows filled by one wave instruction
  constexpr int STAGE = (BM + BN) * ROWB;
  constexpr int CP = BN + 8;                  // staged output row pitch (elements)
  constexpr int SMB = 2 * STAGE > BM * CP * (int)sizeof(T) ? 2 * STAGE : BM * CP * (int)sizeof(T);
  constexpr int AI = BM / RPI / 4, WI = BN / RPI / 4;
  static_assert(ROWB == 128 && BM % (RPI * 4) == 0 && BN % (RPI * 4) == 0, "tile shape");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[SMB];
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int ncol = (g.Nc + BN - 1) / BN;
  const int nrow = (g.M + BM - 1) / BM;
  const int wid = xcd_swizzle(blockIdx.x, ncol * nrow);
  const int n0 = (wid % ncol) * BN, m0 = (wid / ncol) * BM;
  auto chunk = [](int row, int c) { return c ^ ((row >> 1) & 7); };

  // sources of this lane's load instructions (rows clamped into range)
  const T* A = static_cast<const T*>(g.a);
  const T* asrc[AI];
  const T* wsrc[WI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int r = (i * 4 + wave) * RPI + (lane >> 3);
    const int m = min(m0 + r, g.M - 1);
    int64_t sr = m;
    if (g.arow != nullptr) {
      const int b = m / g.a_rows, rr = m - b * g.a_rows;
      sr = (int64_t)b * g.a_src_rows + g.arow[rr];
    }
    asrc[i] = A + sr * g.lda + chunk(r, lane & 7) * 8;
  }
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int r = (i * 4 + wave) * RPI + (lane >> 3);
    const int n = min(n0 + r, g.Nc - 1);
    // at most three stacked matrices: the index by two compares, not a division
    const int mat = (n >= g.ncol_each ? 1 : 0) + (n >= 2 * g.ncol_each ? 1 : 0);
    wsrc[i] = static_cast<const T*>(g.w[mat]) + (int64_t)(n - mat * g.ncol_each) * g.Kd + chunk(r, lane & 7) * 8;
  }
  auto issue = [&](int buf, int k0) __attribute__((always_inline)) {
    const uint32_t st = sbase + buf * STAGE;
#pragma unroll
    for (int i = 0; i < AI; ++i) load_to_lds16(asrc[i] + k0, st + (i * 4 + wave) * RPI * ROWB);
#pragma unroll
    for (int i = 0; i < WI; ++i) load_to_lds16(wsrc[i] + k0, st + (BM + (i * 4 + wave) * RPI) * ROWB);
  };

  f32x16_t acc[MI][NJ];
  const int arow = wm * MI * 32 + (lane & 31), brow = wn * NJ * 32 + (lane & 31);
  // FIRST: the first k-tile starts the accumulators from zero (a zero C
  // operand in the MFMA instead of 96 register clears per tile)
  auto compute = [&](int buf, auto FIRST) __attribute__((always_inline)) {
    const unsigned char* sp = smem + buf * STAGE;
#pragma unroll
    for (int ks = 0; ks < BK / M_::KC; ++ks) {
      const int cb = chunk(lane & 31, ks * 2 + (lane >> 5)) * 16;
      typename M_::frag af[MI], bfr[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i)
        af[i] = __builtin_bit_cast(typename M_::frag, *reinterpret_cast<const u32x4_t*>(sp + (arow + i * 32) * ROWB + cb));
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        bfr[j] = __builtin_bit_cast(typename M_::frag, *reinterpret_cast<const u32x4_t*>(sp + (BM + brow + j * 32) * ROWB + cb));
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          if (decltype(FIRST)::value && ks == 0) {
            f32x16_t z;
#pragma unroll
            for (int v = 0; v < 16; ++v) z[v] = 0.0f;
            acc[i][j] = M_::mma(bfr[j], af[i], z);
          } else {
            acc[i][j] = M_::mma(bfr[j], af[i], acc[i][j]);
          }
        }
    }
  };
  const int nk = g.Kd / BK;
  issue(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's loads of tile kt are in LDS
    __syncthreads();                      // ... everyone's; and tile kt - 1 is consumed
    if (kt + 1 < nk) issue((kt + 1) & 1, (kt + 1) * BK);
    if (kt == 0)
      compute(0, std::true_type{});
    else
      compute(kt & 1, std::false_type{});
  }
  __syncthreads();

  // ---- epilogue: the tile is staged through LDS (bias / GELU applied on the
  // way) and written back as 16-byte row segments
  T* Cs = reinterpret_cast<T*>(smem);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    float bq[EPI ? 4 : 1][4];
    if (EPI) {
      const T* bp = static_cast<const T*>(g.bias);
#pragma unroll
      for (int vq = 0; vq < (EPI ? 4 : 1); ++vq) {
        const int n = n0 + wn * NJ * 32 + j * 32 + vq * 8 + (lane >> 5) * 4;
#pragma unroll
        for (int u = 0; u < 4; ++u) bq[vq][u] = bp != nullptr ? ldf(bp + min(n + u, g.Nc - 1)) : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int vq = 0; vq < 4; ++vq) {
        const int ml = wm * MI * 32 + i * 32 + (lane & 31);
        const int nl = wn * NJ * 32 + j * 32 + vq * 8 + (lane >> 5) * 4;
        const f32x16_t& a = acc[i][j];
        float e[4] = {a[vq * 4], a[vq * 4 + 1], a[vq * 4 + 2], a[vq * 4 + 3]};
        if (EPI) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            float v = e[u] + bq[EPI ? vq : 0][u];
            if (EPI == 2) v = gelu_erf(rnd_to(v, T(0)));   // rounded as nn.Linear's output
            e[u] = v;
          }
        }
        uint2 u;
        u.x = Pair16<T>::pack(e[0], e[1]);
        u.y = Pair16<T>::pack(e[2], e[3]);
        *reinterpret_cast<uint2*>(&Cs[ml * CP + nl]) = u;
      }
  }
  __syncthreads();
  // 192 threads: thread -> fixed 8-column group, rows (tid / 24) + 8 * it, so
  // the head-split coordinates are derived once and stepped
  constexpr int SEGS = BN / 8;
  if (tid >= SEGS * 8) return;
  const int nl = (tid % SEGS) * 8;
  const int n = n0 + nl;
  if (n >= g.Nc) return;
  int mat = 0, hh = 0, cc = n, b = 0, r = 0;
  bool whole = n + 8 <= g.Nc;
  const int mfirst = m0 + tid / SEGS;
  if (OMODE == GEMM_O_HEADSPLIT) {
    mat = (n >= g.ncol_each ? 1 : 0) + (n >= 2 * g.ncol_each ? 1 : 0);
    const int nn = n - mat * g.ncol_each;
    hh = nn / g.o_dk;
    cc = nn - hh * g.o_dk;
    whole = whole && (cc + 8 <= g.o_dk);
    b = mfirst / g.o_rows;
    r = mfirst - b * g.o_rows;
  }
  T* obase = static_cast<T*>(g.o[OMODE == GEMM_O_HEADSPLIT ? (mat > 2 ? 2 : mat) : 0]);
  // output offset of this thread's segment, stepped by 8 rows (recomputed when
  // the head-split row wraps into the next sequence)
  auto seg_off = [&](int m) -> int64_t {
    return OMODE == GEMM_O_HEADSPLIT ? (((int64_t)b * g.o_H + hh) * g.o_rows + r) * g.o_dkp + cc
                                     : (int64_t)m * g.ldo + n;
  };
  int64_t off = seg_off(mfirst);
  const int64_t ostep = OMODE == GEMM_O_HEADSPLIT ? 8 * (int64_t)g.o_dkp : 8 * g.ldo;
#pragma unroll
  for (int it = 0; it < BM / 8; ++it) {
    const int ml = tid / SEGS + it * 8;
    const int m = m0 + ml;
    if (it > 0) {
      if (OMODE == GEMM_O_HEADSPLIT) {
        r += 8;
        if (r >= g.o_rows) {
          b = m / g.o_rows;
          r = m - b * g.o_rows;
          off = seg_off(m);
        } else {
          off += ostep;
        }
      } else {
        off += ostep;
      }
    }
    if (m >= g.M) break;
    u32x4_t val = *reinterpret_cast<const u32x4_t*>(&Cs[ml * CP + nl]);
    if (EPI && g.res != nullptr && whole) {
      // residual: 16-bit linear output + 16-bit residual, added in fp32 and rounded once
      const u32x4_t rv = *reinterpret_cast<const u32x4_t*>(static_cast<const T*>(g.res) + (int64_t)m * g.ldr + n);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        val[q] = Pair16<T>::pack(Pair16<T>::lo(val[q]) + Pair16<T>::lo(rv[q]),
                                 Pair16<T>::hi(val[q]) + Pair16<T>::hi(rv[q]));
    }
    T* dst = obase + off;
    if (whole) {
      *reinterpret_cast<u32x4_t*>(dst) = val;
    } else {
      // tile or head edge: element by element
      for (int u = 0; u < 8 && n + u < g.Nc; ++u) {
        const T v = Cs[ml * CP + nl + u];
        if (OMODE == GEMM_O_HEADSPLIT) {
          const int nu = n + u;
          const int mt = nu / g.ncol_each, nn = nu - mt * g.ncol_each;
          const int h = nn / g.o_dk, c = nn - h * g.o_dk;
          static_cast<T*>(g.o[mt])[(((int64_t)b * g.o_H + h) * g.o_rows + r) * g.o_dkp + c] = v;
        } else {
          if (EPI && g.res != nullptr)
            stf(&dst[u], ldf(&v) + ldf(static_cast<const T*>(g.res) + (int64_t)m * g.ldr + n + u));
          else
            dst[u] = v;
        }
      }
    }
  }
}

// the direct-to-LDS kernel for the linear GEMMs it covers; DL_SKIP when the
// call is not one of them
constexpr int DL_SKIP = 0x7fffffff;
template <typename T>
int launch_dl(int amode, int omode, const GemmArgs& g, hipStream_t s) {
  if constexpr (sizeof(T) != 2) {
    return DL_SKIP;
  } else {
    if (amode != GEMM_A_ROWS || !g.ostage || g.ln_stats || g.st_out) return DL_SKIP;
    if (!g.avec || !g.bvec || g.Kd <= 0 || g.Kd % DL_BK != 0) return DL_SKIP;
    // 16-byte aligned sources for every row (the loads bypass the registers)
    if ((uintptr_t)g.a % 16 != 0 || (g.lda * (int64_t)sizeof(T)) % 16 != 0) return DL_SKIP;
    for (int i = 0; i < 3; ++i)
      if (g.w[i] && (uintptr_t)g.w[i] % 16 != 0) return DL_SKIP;
    const dim3 grid(((g.Nc + DL_BN - 1) / DL_BN) * ((g.M + DL_BM - 1) / DL_BM));
    const bool gelu = g.act == GEMM_ACT_GELU;
    if (omode == GEMM_O_HEADSPLIT) {
      if (g.res || gelu) return CNNA_ERR_OPTION;
      if (g.bias)
        hipLaunchKernelGGL((gemm_dl_kernel<T, GEMM_O_HEADSPLIT, 1>), grid, dim3(256), 0, s, g);
      else
        hipLaunchKernelGGL((gemm_dl_kernel<T, GEMM_O_HEADSPLIT, 0>), grid, dim3(256), 0, s, g);
    } else if (gelu) {
      hipLaunchKernelGGL((gemm_dl_kernel<T, GEMM_O_PLAIN, 2>), grid, dim3(256), 0, s, g);
    } else if (g.bias || g.res) {
      hipLaunchKernelGGL((gemm_dl_kernel<T, GEMM_O_PLAIN, 1>), grid, dim3(256), 0, s, g);
    } else {
      hipLaunchKernelGGL((gemm_dl_kernel<T, GEMM_O_PLAIN, 0>), grid, dim3(256), 0, s, g);
    }
    return (int)hipGetLastError();
  }
}

template <typename T, bool FAST>
int launch_x(int omode, const GemmArgs& g, hipStream_t s, dim3 grid) {
  // LayerNorm prologue and / or statistics epilogue (row-major A)
  const int xf = (g.ln_stats ? 1 : 0) | (g.st_out ? 2 : 0);
  if (omode == GEMM_O_HEADSPLIT) {
    if (xf != 1 || g.res || g.act != GEMM_ACT_NONE) return CNNA_ERR_OPTION;
    if (g.bias)
      hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_HEADSPLIT, FAST, 1, 1>), grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_HEADSPLIT, FAST, 0, 1>), grid, dim3(256), 0, s, g);
    return (int)hipGetLastError();
  }
  const bool gelu = g.act == GEMM_ACT_GELU;
  if (xf == 1) {
    if (gelu)
      hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST, 2, 1>), grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST, 1, 1>), grid, dim3(256), 0, s, g);
    return (int)hipGetLastError();
  }
  if constexpr (sizeof(T) == 2) {
    // the statistics come from the staged bf16 epilogue
    if (!g.ostage || g.Nc % 8 != 0) return CNNA_ERR_UNSUPPORTED;
    if (gelu && xf == 2)
      hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST, 2, 2>), grid, dim3(256), 0, s, g);
    else if (gelu)
      hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST, 2, 3>), grid, dim3(256), 0, s, g);
    else if (xf == 2)
      hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST, 1, 2>), grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST, 1, 3>), grid, dim3(256), 0, s, g);
    return (int)hipGetLastError();
  } else {
    return CNNA_ERR_UNSUPPORTED;
  }
}

template <typename T, bool FAST>
int launch_f(int amode, int omode, const GemmArgs& g, hipStream_t s) {
  dim3 grid(((g.Nc + BN - 1) / BN) * ((g.M + BM - 1) / BM));
  if (g.ln_stats || g.st_out) {
    if (amode != GEMM_A_ROWS) return CNNA_ERR_OPTION;
    if (g.ln_stats && g.Kd > LN_MAX_K) return CNNA_ERR_UNSUPPORTED;
    return launch_x<T, FAST>(omode, g, s, grid);
  }
  if (amode == GEMM_A_ROWS && omode == GEMM_O_HEADSPLIT && (g.res || g.act != GEMM_ACT_NONE))
    return CNNA_ERR_OPTION;   // the head split takes a bias only
  else if (amode == GEMM_A_ROWS && omode == GEMM_O_HEADSPLIT && g.bias)
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_HEADSPLIT, FAST, 1>), grid, dim3(256), 0, s, g);
  else if (amode == GEMM_A_ROWS && omode == GEMM_O_HEADSPLIT)
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_HEADSPLIT, FAST>), grid, dim3(256), 0, s, g);
  else if (amode == GEMM_A_ROWS && omode == GEMM_O_PLAIN && g.act == GEMM_ACT_GELU)
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST, 2>), grid, dim3(256), 0, s, g);
  else if (amode == GEMM_A_ROWS && omode == GEMM_O_PLAIN && (g.bias || g.res))
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST, 1>), grid, dim3(256), 0, s, g);
  else if (amode == GEMM_A_ROWS && omode == GEMM_O_PLAIN)
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN, FAST>), grid, dim3(256), 0, s, g);
  else if (g.bias || g.act != GEMM_ACT_NONE || g.res)
    return CNNA_ERR_OPTION;   // linear extras only with row-major A and a plain output
  else if (amode == GEMM_A_GATHER && omode == GEMM_O_PLAIN)
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_GATHER, GEMM_O_PLAIN, FAST>), grid, dim3(256), 0, s, g);
  else
    return CNNA_ERR_OPTION;
  return (int)hipGetLastError();
}

template <typename T>
int launch_t(int amode, int omode, const GemmArgs& g0, hipStream_t s) {
  GemmArgs g = g0;
  // vector epilogue: 4 consecutive columns land contiguously and aligned
  const int es = sizeof(T);
  bool ovec = true;
  for (int i = 0; i < 3; ++i)
    if (g.o[i] && ((uintptr_t)g.o[i] % (4 * es)) != 0) ovec = false;
  if (omode == GEMM_O_PLAIN) ovec = ovec && (g.ldo % 4 == 0);
  else ovec = ovec && (g.o_dkp % 4 == 0) && (g.ncol_each % 4 == 0) && (g.o_dk % 4 == 0);
  g.ovec = ovec;
  // staged bf16 epilogue: 8-column (16-byte) segments stay aligned and inside a head
  bool ostage = sizeof(T) == 2;
  for (int i = 0; i < 3; ++i)
    if (g.o[i] && ((uintptr_t)g.o[i] % 16) != 0) ostage = false;
  if (omode == GEMM_O_PLAIN) ostage = ostage && (g.ldo % 8 == 0);
  if (g.res != nullptr) ostage = ostage && ((uintptr_t)g.res % 16 == 0) && (g.ldr % 8 == 0);
  else ostage = ostage && (g.o_dkp % 8 == 0) && (g.ncol_each % 8 == 0) && (g.o_dk % 8 == 0);
  g.ostage = ostage;
  const int dl = launch_dl<T>(amode, omode, g, s);
  if (dl != DL_SKIP) return dl;
  const bool fast = g.avec && g.bvec && (g.Kd % GemmCfg<T>::BK == 0);
  return fast ? launch_f<T, true>(amode, omode, g, s) : launch_f<T, false>(amode, omode, g, s);
}

template <typename T>
__global__ void permute_w0_kernel(const T* w0, T* w0p, int dout, int din, int K) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)dout * din * K;
  if (e >= total) return;
  const int o = (int)(e / ((int64_t)din * K));
  const int rem = (int)(e - (int64_t)o * din * K);
  const int c = rem / K, r = rem - c * K;
  w0p[(int64_t)o * din * K + (int64_t)r * din + c] = w0[e];
}

// W0 (dout, din, K) -> W0t (K*din, dout) with W0t[r*din + c][o] = W0[o][c][r]:
// the transpose of W0p, the weight operand of dP = dy @ W0p as a row GEMM
template <typename T>
__global__ void permute_w0t_kernel(const T* w0, T* w0t, int dout, int din, int K) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)dout * din * K;
  if (e >= total) return;
  const int o = (int)(e / ((int64_t)din * K));
  const int rem = (int)(e - (int64_t)o * din * K);
  const int c = rem / K, r = rem - c * K;
  w0t[((int64_t)r * din + c) * dout + o] = w0[e];
}

// dst[c * ldd + k] = src[k * cols + c] for a (rows, cols) source: 32 x 32
// tiles through LDS (many small blocks: the matrices are weights, a few MB),
// reads and writes coalesced
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* src, T* dst, int rows, int cols,
                                                        int64_t ldd) {
  __shared__ T tile[32][33];
  const int k0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int k = k0 + r, c = c0 + tx;
    if (k < rows && c < cols) tile[r][tx] = src[(int64_t)k * cols + c];
  }
  __syncthreads();
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int c = c0 + r, k = k0 + tx;
    if (k < rows && c < cols) dst[(int64_t)c * ldd + k] = tile[tx][r];
  }
}

}  // namespace

int launch_transpose(int dtype, const void* src, void* dst, int rows, int cols, int64_t ldd,
                     hipStream_t s) {
  if (rows <= 0 || cols <= 0) return 0;
  const dim3 grid((unsigned)((rows + 31) / 32), (unsigned)((cols + 31) / 32));
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), rows, cols, ldd);
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(transpose_kernel<_Float16>, grid, dim3(256), 0, s,
                       static_cast<const _Float16*>(src), static_cast<_Float16*>(dst), rows, cols, ldd);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(src),
                       static_cast<float*>(dst), rows, cols, ldd);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}

int launch_permute_w0t(int dtype, const void* w0, void* w0t, int dout, int din, int K, hipStream_t s) {
  const int64_t total = (int64_t)dout * din * K;
  dim3 grid((unsigned)((total + 255) / 256));
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(permute_w0t_kernel<uint16_t>, grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(w0), static_cast<uint16_t*>(w0t), dout, din, K);
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(permute_w0t_kernel<_Float16>, grid, dim3(256), 0, s,
                       static_cast<const _Float16*>(w0), static_cast<_Float16*>(w0t), dout, din, K);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(permute_w0t_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(w0),
                       static_cast<float*>(w0t), dout, din, K);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}

int launch_gemm(int dtype, int amode, int omode, const GemmArgs& g, hipStream_t s) {
  if (g.M <= 0 || g.Nc <= 0 || g.Kd <= 0) return 0;
  if (dtype == CNNA_BF16) return launch_t<uint16_t>(amode, omode, g, s);
  else if (dtype == CNNA_F16) return launch_t<_Float16>(amode, omode, g, s);
  if (dtype == CNNA_F32) return launch_t<float>(amode, omode, g, s);
  return CNNA_ERR_DTYPE;
}

int launch_permute_w0(int dtype, const void* w0, void* w0p, int dout, int din, int K, hipStream_t s) {
  const int64_t total = (int64_t)dout * din * K;
  dim3 grid((unsigned)((total + 255) / 256));
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(permute_w0_kernel<uint16_t>, grid, dim3(256), 0, s,
                       static_cast<const uint16_t*>(w0), static_cast<uint16_t*>(w0p), dout, din, K);
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(permute_w0_kernel<_Float16>, grid, dim3(256), 0, s,
                       static_cast<const _Float16*>(w0), static_cast<_Float16*>(w0p), dout, din, K);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(permute_w0_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(w0),
                       static_cast<float*>(w0p), dout, din, K);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}
