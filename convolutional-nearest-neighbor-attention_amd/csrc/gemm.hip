// MFMA GEMM for the projections: Q/K/V (x @ W^T with head split, layers.py:
// 264-265, 274, 237-245) and the output projection W_o whose A operand is
// the reference's head merge read in place (layers.py:247-259, 317, 320).
//
// Tile 128 x 128, 256 threads = 4 waves in a 2 x 2 grid, each wave owns a
// 64 x 64 block = 2 x 2 v_mfma_f32_32x32x{16 bf16 | 2 f32} accumulators.
// A and W tiles are staged through LDS (rows padded by 16 bytes).
#include "common.h"
#include "kernels.h"

namespace {

constexpr int BM = 128, BN = 128;

template <typename T> struct GemmCfg;
template <> struct GemmCfg<uint16_t> { static constexpr int BK = 32, VEC = 8; };
template <> struct GemmCfg<float> { static constexpr int BK = 16, VEC = 4; };

template <typename T, int AMODE, int OMODE>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  using M_ = Mfma<T>;
  constexpr int BK = GemmCfg<T>::BK, VEC = GemmCfg<T>::VEC;
  constexpr int LDS_STRIDE = BK + VEC;  // elements; rows stay 16-byte aligned
  __shared__ __attribute__((aligned(16))) T As[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) T Bs[BN * LDS_STRIDE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const T* A = static_cast<const T*>(g.a);

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // per-thread source rows for the A_ROWS / W loads (2 vectors each)
  constexpr int VPR = BK / VEC;  // vectors per tile row (4)
  const T* arow_ptr[2];
  bool arow_ok[2];
  const T* wrow_ptr[2];
  bool wrow_ok[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int e = tid + i * 256;
    const int r = e / VPR;
    const int m = m0 + r;
    arow_ok[i] = m < g.M;
    int64_t sr = m;
    if (AMODE == GEMM_A_ROWS && g.arow != nullptr && arow_ok[i]) {
      const int b = m / g.a_rows, rr = m - b * g.a_rows;
      sr = (int64_t)b * g.a_src_rows + g.arow[rr];
    }
    arow_ptr[i] = A + (arow_ok[i] ? sr : 0) * g.lda;
    const int n = n0 + r;
    wrow_ok[i] = n < g.Nc;
    const int mat = wrow_ok[i] ? n / g.ncol_each : 0;
    const int rn = wrow_ok[i] ? n - mat * g.ncol_each : 0;
    wrow_ptr[i] = static_cast<const T*>(g.w[mat]) + (int64_t)rn * g.Kd;
  }

  for (int k0 = 0; k0 < g.Kd; k0 += BK) {
    // ---- stage A
    if (AMODE == GEMM_A_ROWS) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid + i * 256;
        const int r = e / VPR, kv = (e % VPR) * VEC;
        const int k = k0 + kv;
        T* dst = &As[r * LDS_STRIDE + kv];
        if (arow_ok[i] && g.avec && k + VEC <= g.Kd) {
          *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(arow_ptr[i] + k);
        } else {
#pragma unroll
          for (int t = 0; t < VEC; ++t)
            dst[t] = (arow_ok[i] && k + t < g.Kd) ? arow_ptr[i][k + t] : T(0);
        }
      }
    } else {
      // head-merge gather: consecutive threads read consecutive tokens t
      const T* Y = A;
      const int64_t head_sz = (int64_t)g.mix_N * g.mix_dk;
#pragma unroll 4
      for (int e = tid; e < BM * BK; e += 256) {
        const int r = e % BM, kc = e / BM;
        const int m = m0 + r, k = k0 + kc;
        T val = T(0);
        if (m < g.M && k < g.Kd) {
          const int b = m / g.mix_N, t = m - b * g.mix_N;
          const int h = k / g.mix_dk, c = k - h * g.mix_dk;
          val = Y[((int64_t)b * g.mix_H + h) * head_sz + (int64_t)c * g.mix_N + t];
        }
        As[r * LDS_STRIDE + kc] = val;
      }
    }
    // ---- stage W
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + i * 256;
      const int r = e / VPR, kv = (e % VPR) * VEC;
      const int k = k0 + kv;
      T* dst = &Bs[r * LDS_STRIDE + kv];
      if (wrow_ok[i] && g.bvec && k + VEC <= g.Kd) {
        *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(wrow_ptr[i] + k);
      } else {
#pragma unroll
        for (int t = 0; t < VEC; ++t)
          dst[t] = (wrow_ok[i] && k + t < g.Kd) ? wrow_ptr[i][k + t] : T(0);
      }
    }
    __syncthreads();

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
        for (int j = 0; j < 2; ++j) acc[i][j] = M_::mma(af[i], bfr[j], acc[i][j]);
    }
    __syncthreads();
  }

  // ---- epilogue
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + (lane & 31);
    if (n >= g.Nc) continue;
    T* obase;
    int64_t ocol;
    if (OMODE == GEMM_O_HEADSPLIT) {
      const int mat = n / g.ncol_each, nn = n - mat * g.ncol_each;
      const int h = nn / g.o_dk, c = nn - h * g.o_dk;
      obase = static_cast<T*>(g.o[mat]);
      ocol = (int64_t)h * g.o_rows * g.o_dkp + c;
    } else {
      obase = static_cast<T*>(g.o[0]);
      ocol = n;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 64 + i * 32 + mfma_row(v, lane);
        if (m >= g.M) continue;
        int64_t off;
        if (OMODE == GEMM_O_HEADSPLIT) {
          const int b = m / g.o_rows, r = m - b * g.o_rows;
          off = ((int64_t)b * g.o_H * g.o_rows + r) * g.o_dkp + ocol;
        } else {
          off = (int64_t)m * g.ldo + ocol;
        }
        stf(obase + off, acc[i][j][v]);
      }
  }
}

template <typename T>
int launch_t(int amode, int omode, const GemmArgs& g, hipStream_t s) {
  dim3 grid((g.Nc + BN - 1) / BN, (g.M + BM - 1) / BM);
  if (amode == GEMM_A_ROWS && omode == GEMM_O_HEADSPLIT)
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_HEADSPLIT>), grid, dim3(256), 0, s, g);
  else if (amode == GEMM_A_ROWS && omode == GEMM_O_PLAIN)
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_ROWS, GEMM_O_PLAIN>), grid, dim3(256), 0, s, g);
  else if (amode == GEMM_A_MIXED && omode == GEMM_O_PLAIN)
    hipLaunchKernelGGL((gemm_kernel<T, GEMM_A_MIXED, GEMM_O_PLAIN>), grid, dim3(256), 0, s, g);
  else
    return CNNA_ERR_OPTION;
  return (int)hipGetLastError();
}

}  // namespace

int launch_gemm(int dtype, int amode, int omode, const GemmArgs& g, hipStream_t s) {
  if (g.M <= 0 || g.Nc <= 0 || g.Kd <= 0) return 0;
  if (dtype == CNNA_BF16) return launch_t<uint16_t>(amode, omode, g, s);
  if (dtype == CNNA_F32) return launch_t<float>(amode, omode, g, s);
  return CNNA_ERR_DTYPE;
}
