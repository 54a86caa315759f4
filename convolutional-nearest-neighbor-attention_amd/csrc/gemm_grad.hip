// MFMA GEMM for the backward pass: out[m][n] = sum_k A[m][k] * W[n][k] with
// either operand row-major or transposed.  Transposed operands are read along
// their contiguous index and transposed while being staged into LDS.  Covers
// the gradients of the projections (nn.Linear at layers.py:264-265, 274, 320)
// and of the standard / pointwise convolutions (layers.py:187-228).
//
// Tiling as in the forward GEMM: 128 x 128 x BK tiles, four waves of 64 x 64,
// fp32 accumulation, register prefetch of the next k-tile.  Weight gradients
// reduce over B*N rows: they split k into chunks written as fp32 partials and
// summed in a fixed order by splitk_reduce, so results are deterministic.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int BM = 128, BN = 128;

template <typename T> struct GCfg;
template <> struct GCfg<uint16_t> { static constexpr int BK = 64, VEC = 8; };
template <> struct GCfg<float> { static constexpr int BK = 32, VEC = 4; };

template <typename T, int VEC>
union GPack {
  u32x4_t u;
  T e[VEC];
};

// One operand tile (128 rows of the output dimension x BK of k) per k-step.
// ROWS: thread slot -> (row, k-vector), 16-byte loads along k.
// TRANS: thread slot -> (k, row-vector), 16-byte loads along the rows.
template <typename T, int MODE>
struct Operand {
  static constexpr int BK = GCfg<T>::BK, VEC = GCfg<T>::VEC;
  static constexpr int NV = BM * (BK / VEC) / 256;
  static constexpr int LDS_STRIDE = BK + VEC;

  static CNNA_DEV void slot(int tid, int i, int& x, int& y) {
    const int e = tid + i * 256;
    if (MODE == GG_ROWS) {
      x = e / (BK / VEC);              // row
      y = (e % (BK / VEC)) * VEC;      // k
    } else {
      x = e / (BM / VEC);              // k
      y = (e % (BM / VEC)) * VEC;      // row
    }
  }

  // rows [r0, r0 + 128) of a (nrows x Kd) operand, k in [k0, k0 + BK) below kend
  static CNNA_DEV void fetch(GPack<T, VEC> (&reg)[NV], const T* const (&base)[3], int krows,
                             int64_t ld, bool vec, int nrows, int r0, int k0, int kend, int tid) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      int x, y;
      slot(tid, i, x, y);
      if (MODE == GG_ROWS) {
        const int r = r0 + x, k = k0 + y;
        const T* p = base[0] + (int64_t)r * ld + k;
        if (r < nrows && vec && k + VEC <= kend) {
          reg[i].u = *reinterpret_cast<const u32x4_t*>(p);
        } else {
#pragma unroll
          for (int t = 0; t < VEC; ++t) reg[i].e[t] = (r < nrows && k + t < kend) ? p[t] : T(0);
        }
      } else {
        const int k = k0 + x, r = r0 + y;
        int kb = 0, kr = k;
        if (krows > 0) {
          kb = k / krows;
          kr = k - kb * krows;
          kb = kb > 2 ? 2 : kb;
        }
        const T* p = base[kb] + (int64_t)kr * ld + r;
        if (k < kend && vec && r + VEC <= nrows) {
          reg[i].u = *reinterpret_cast<const u32x4_t*>(p);
        } else {
#pragma unroll
          for (int t = 0; t < VEC; ++t) reg[i].e[t] = (k < kend && r + t < nrows) ? p[t] : T(0);
        }
      }
    }
  }

  static CNNA_DEV void stash(const GPack<T, VEC> (&reg)[NV], T* S, int tid) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      int x, y;
      slot(tid, i, x, y);
      if (MODE == GG_ROWS) {
        *reinterpret_cast<u32x4_t*>(&S[x * LDS_STRIDE + y]) = reg[i].u;
      } else {
#pragma unroll
        for (int t = 0; t < VEC; ++t) S[(y + t) * LDS_STRIDE + x] = reg[i].e[t];
      }
    }
  }
};

template <typename T, int AM, int WM>
__global__ __launch_bounds__(256) void gemm_grad_kernel(GradGemmArgs g) {
  using M_ = Mfma<T>;
  using OA = Operand<T, AM>;
  using OW = Operand<T, WM>;
  constexpr int BK = GCfg<T>::BK, VEC = GCfg<T>::VEC;
  constexpr int LDS_STRIDE = BK + VEC;
  __shared__ __attribute__((aligned(16))) T As[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) T Bs[BN * LDS_STRIDE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int ncol = (g.Nc + BN - 1) / BN;
  const int nrow = (g.M + BM - 1) / BM;
  const int ntile = ncol * nrow;
  const int wid = xcd_swizzle(blockIdx.x, ntile * g.splits);
  const int split = wid / ntile, tile = wid - split * ntile;
  const int n0 = (tile % ncol) * BN, m0 = (tile / ncol) * BM;
  const int kbeg = split * g.kchunk;
  const int kend = min(g.Kd, kbeg + g.kchunk);

  const T* const abase[3] = {static_cast<const T*>(g.a), nullptr, nullptr};
  const T* const wbase[3] = {static_cast<const T*>(g.w[0]), static_cast<const T*>(g.w[1]),
                             static_cast<const T*>(g.w[2])};

  GPack<T, VEC> ra[OA::NV], rw[OW::NV];
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  if (kbeg < kend) {
    OA::fetch(ra, abase, 0, g.lda, g.avec, g.M, m0, kbeg, kend, tid);
    OW::fetch(rw, wbase, g.w_krows, g.ldw, g.bvec, g.Nc, n0, kbeg, kend, tid);
  }
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    OA::stash(ra, As, tid);
    OW::stash(rw, Bs, tid);
    __syncthreads();
    if (k0 + BK < kend) {
      OA::fetch(ra, abase, 0, g.lda, g.avec, g.M, m0, k0 + BK, kend, tid);
      OW::fetch(rw, wbase, g.w_krows, g.ldw, g.bvec, g.Nc, n0, k0 + BK, kend, tid);
    }
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

  // acc[i][j][v] = out[m][n], m = m0 + wm*64 + i*32 + mfma_row(v, lane),
  //                n = n0 + wn*64 + j*32 + lane%32 (adjacent lanes, adjacent columns)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + (lane & 31);
    if (n >= g.Nc) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 64 + i * 32 + mfma_row(v, lane);
        if (m >= g.M) continue;
        if (g.part != nullptr)
          g.part[((int64_t)split * g.M + m) * g.Nc + n] = acc[i][j][v];
        else
          stf(static_cast<T*>(g.o) + (int64_t)m * g.ldo + n, acc[i][j][v]);
      }
  }
}

template <typename T>
int launch_grad_t(const GradGemmArgs& g, hipStream_t s) {
  dim3 grid(((g.Nc + BN - 1) / BN) * ((g.M + BM - 1) / BM) * g.splits);
  if (g.amode == GG_ROWS && g.wmode == GG_ROWS)
    hipLaunchKernelGGL((gemm_grad_kernel<T, GG_ROWS, GG_ROWS>), grid, dim3(256), 0, s, g);
  else if (g.amode == GG_ROWS && g.wmode == GG_TRANS)
    hipLaunchKernelGGL((gemm_grad_kernel<T, GG_ROWS, GG_TRANS>), grid, dim3(256), 0, s, g);
  else if (g.amode == GG_TRANS && g.wmode == GG_TRANS)
    hipLaunchKernelGGL((gemm_grad_kernel<T, GG_TRANS, GG_TRANS>), grid, dim3(256), 0, s, g);
  else if (g.amode == GG_TRANS && g.wmode == GG_ROWS)
    hipLaunchKernelGGL((gemm_grad_kernel<T, GG_TRANS, GG_ROWS>), grid, dim3(256), 0, s, g);
  else
    return CNNA_ERR_OPTION;
  return (int)hipGetLastError();
}

template <typename T>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceArgs r) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t MN = (int64_t)r.M * r.Nc;
  if (e >= MN) return;
  const int m = (int)(e / r.Nc), n = (int)(e - (int64_t)m * r.Nc);
  float acc = 0.0f;
  for (int s = 0; s < r.splits; ++s) acc += r.part[s * MN + e];
  const int blk = min(m / r.rows_each, 2), mm = m - blk * r.rows_each;
  int col = n;
  if (r.pdin > 0) {
    const int rr = n / r.pdin, c = n - rr * r.pdin;
    col = c * r.pK + rr;
  }
  stf(static_cast<T*>(r.o[blk]) + (int64_t)mm * r.ldo + col, acc);
}

}  // namespace

int launch_gemm_grad(int dtype, const GradGemmArgs& g0, hipStream_t s) {
  if (g0.M <= 0 || g0.Nc <= 0) return 0;
  GradGemmArgs g = g0;
  const int es = dtype == CNNA_BF16 ? 2 : 4;
  const int bk = grad_gemm_bk(dtype);
  if (g.splits < 1) g.splits = 1;
  // fp32 partials when part is given (any split count), else T into o (one split)
  if (g.part == nullptr && (g.splits > 1 || g.o == nullptr)) return CNNA_ERR_NULL;
  g.kchunk = (int)cnna_round_up((size_t)((g.Kd + g.splits - 1) / g.splits), (size_t)bk);
  if (g.kchunk < bk) g.kchunk = bk;
  // 16-byte loads need 16-byte aligned rows
  g.avec = ((uintptr_t)g.a % 16 == 0) && ((g.lda * es) % 16 == 0);
  bool bv = (g.ldw * es) % 16 == 0;
  for (int i = 0; i < 3; ++i) bv = bv && ((uintptr_t)g.w[i] % 16 == 0);
  g.bvec = bv;
  if (g.w_krows == 0) g.w[1] = g.w[2] = g.w[0];
  if (dtype == CNNA_BF16) return launch_grad_t<uint16_t>(g, s);
  if (dtype == CNNA_F32) return launch_grad_t<float>(g, s);
  return CNNA_ERR_DTYPE;
}

int launch_splitk_reduce(int dtype, const ReduceArgs& r, hipStream_t s) {
  const int64_t MN = (int64_t)r.M * r.Nc;
  if (MN <= 0) return 0;
  dim3 grid((unsigned)((MN + 255) / 256));
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(splitk_reduce_kernel<uint16_t>, grid, dim3(256), 0, s, r);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(splitk_reduce_kernel<float>, grid, dim3(256), 0, s, r);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}
