// MFMA GEMM for the backward pass: out[m][n] = sum_k A[m][k] * W[n][k] with
// either operand row-major (ROWS) or transposed (TRANS: k is the slow index),
// and a gathered transposed W (GATHER_T: the standard conv's input P, built
// from the neighbour lists on the fly).  Covers the gradients of the
// projections (nn.Linear at layers.py:264-265, 274, 320) and of the standard /
// pointwise convolutions (layers.py:187-228).
//
// Tiling: 128 x 128 output tiles, BK = 128 bytes of k per step, four waves of
// 64 x 64, fp32 accumulation, register prefetch of the next k-step.
//
// LDS holds each operand tile as 128 rows x 8 chunks of 16 bytes (k
// contiguous inside a chunk), chunk index XOR-swizzled by the row so that both
// the staging writes and the MFMA fragment reads spread over the banks.
//   ROWS   a thread loads 16-byte vectors along k and writes them as chunks;
//   TRANS  a thread loads 4 consecutive k of one 16-byte row-vector each,
//          transposes the 4 x RV block in registers and writes RV pieces of
//          4 consecutive k (8 or 16 bytes): no scalar LDS writes.
// Weight gradients reduce over B*N rows: they split k into chunks written as
// fp32 partials and summed in a fixed order by splitk_reduce (deterministic).
#include "common.h"
#include "kernels.h"

namespace {

constexpr int BM = 128, BN = 128;

template <typename T> struct GCfg {
  static constexpr int CE = 16 / sizeof(T);   // elements per 16-byte chunk
  static constexpr int BK = 8 * CE;           // k per step (one 128-byte row)
  static constexpr int RV = CE;               // rows per TRANS vector
  static constexpr int RB = 128 / RV;         // TRANS row-vectors per tile
};

CNNA_DEV int swz(int row) { return (row ^ (row >> 3)) & 7; }

// element offset of (row, k) in a swizzled tile
template <typename T>
CNNA_DEV int lds_off(int row, int k) {
  constexpr int CE = GCfg<T>::CE;
  return row * (8 * CE) + (((k / CE) ^ swz(row)) * CE) + (k % CE);
}

template <typename T>
union GPack {
  u32x4_t u;
  T e[GCfg<T>::CE];
};

struct GatherArgs {
  const int32_t* idx;
  const float* w;
  int K, N, din, dkp;
};

template <typename T, int MODE>
struct Operand {
  static constexpr int CE = GCfg<T>::CE, RV = GCfg<T>::RV, RB = GCfg<T>::RB;
  static constexpr int NV = 4;   // 16-byte vectors per thread per tile (both layouts)

  // GATHER_T: neighbour index and weight of each of this thread's NV tokens
  // for the k-step at k0, loaded one step ahead of the rows they select
  struct Index {
    int j[NV];
    float w[NV];
  };
  static CNNA_DEV void fetch_index(Index& ix, int nrows, int r0, int k0, int kend, int tid,
                                   const GatherArgs& ga) {
    const int n = r0 + (tid % RB) * RV, rr = min(n, nrows - 1) / ga.din;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int k = min(k0 + (tid / RB) * 4 + i, kend - 1);
      ix.j[i] = ga.idx[(int64_t)k * ga.K + rr];
      ix.w[i] = ga.w[(int64_t)k * ga.K + rr];
    }
  }

  // rows [r0, r0 + 128) of the operand, k in [k0, k0 + BK) below kend;
  // GATHER_T with ix: the fast path takes the prefetched index and weight
  static CNNA_DEV void fetch(GPack<T> (&reg)[NV], const T* const (&base)[3], int krows, int64_t ld,
                             bool vec, int nrows, int r0, int k0, int kend, int tid,
                             const GatherArgs& ga, const Index* ix = nullptr, float* wsave = nullptr) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (MODE == GG_ROWS) {
        const int e = tid + i * 256;
        const int r = r0 + (e >> 3), k = k0 + (e & 7) * CE;
        const T* p = base[0] + (int64_t)r * ld + k;
        if (r < nrows && vec && k + CE <= kend) {
          reg[i].u = *reinterpret_cast<const u32x4_t*>(p);
        } else {
#pragma unroll
          for (int t = 0; t < CE; ++t) reg[i].e[t] = (r < nrows && k + t < kend) ? p[t] : T(0);
        }
      } else if (MODE == GG_TRANS) {
        const int r = r0 + (tid % RB) * RV, k = k0 + (tid / RB) * 4 + i;
        int kb = 0, kr = k;
        if (krows > 0) {
          kb = k / krows;
          kr = k - kb * krows;
          kb = kb > 2 ? 2 : kb;
        }
        const T* p = base[kb] + (int64_t)kr * ld + r;
        if (k < kend && vec && r + RV <= nrows) {
          reg[i].u = *reinterpret_cast<const u32x4_t*>(p);
        } else {
#pragma unroll
          for (int t = 0; t < RV; ++t) reg[i].e[t] = (k < kend && r + t < nrows) ? p[t] : T(0);
        }
      } else {
        // GATHER_T: rows n = r*din + c .. + RV of token k
        const int n = r0 + (tid % RB) * RV, k = k0 + (tid / RB) * 4 + i;
        if (k < kend && vec && n + RV <= nrows) {
          const int rr = n / ga.din, c = n - rr * ga.din;
          const int j = ix ? ix->j[i] : ga.idx[(int64_t)k * ga.K + rr];
          const float wv = ix ? ix->w[i] : ga.w[(int64_t)k * ga.K + rr];
          const T* p = base[0] + ((int64_t)(k - k % ga.N) + j) * ga.dkp + c;
          // raw row; the weight is applied at stash time (no wait on the load here)
          reg[i].u = *reinterpret_cast<const u32x4_t*>(p);
          if (wsave) wsave[i] = wv;
          else {
            GPack<T> v = reg[i];
#pragma unroll
            for (int t = 0; t < RV; ++t) stf(&reg[i].e[t], wv * ldf(&v.e[t]));
          }
        } else {
#pragma unroll
          for (int t = 0; t < RV; ++t) {
            float x = 0.0f;
            if (k < kend && n + t < nrows) {
              const int rr = (n + t) / ga.din, c = (n + t) - rr * ga.din;
              const int j = ga.idx[(int64_t)k * ga.K + rr];
              x = ga.w[(int64_t)k * ga.K + rr] *
                  ldf(base[0] + ((int64_t)(k - k % ga.N) + j) * ga.dkp + c);
            }
            stf(&reg[i].e[t], x);
          }
          if (wsave) wsave[i] = 1.0f;
        }
      }
    }
  }

  // GATHER_T: scale each gathered row by its neighbour weight first
  static CNNA_DEV void scale(GPack<T> (&reg)[NV], const float (&wsave)[NV]) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const GPack<T> v = reg[i];
#pragma unroll
      for (int t = 0; t < RV; ++t) stf(&reg[i].e[t], wsave[i] * ldf(&v.e[t]));
    }
  }

  static CNNA_DEV void stash(const GPack<T> (&reg)[NV], T* S, int tid) {
    if (MODE == GG_ROWS) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = tid + i * 256;
        *reinterpret_cast<u32x4_t*>(&S[lds_off<T>(e >> 3, (e & 7) * CE)]) = reg[i].u;
      }
    } else {
      // reg[i] = RV consecutive rows at k = kb*4 + i; write row j's 4 k values
      const int rb = tid % RB, kb = tid / RB;
#pragma unroll
      for (int j = 0; j < RV; ++j) {
        T* dst = &S[lds_off<T>(rb * RV + j, kb * 4)];
        if constexpr (sizeof(T) == 2) {
          uint2 u;
          u.x = (uint32_t)__builtin_bit_cast(uint16_t, reg[0].e[j]) |
                ((uint32_t)__builtin_bit_cast(uint16_t, reg[1].e[j]) << 16);
          u.y = (uint32_t)__builtin_bit_cast(uint16_t, reg[2].e[j]) |
                ((uint32_t)__builtin_bit_cast(uint16_t, reg[3].e[j]) << 16);
          *reinterpret_cast<uint2*>(dst) = u;
        } else {
          u32x4_t u;
#pragma unroll
          for (int i = 0; i < 4; ++i) u[i] = __builtin_bit_cast(uint32_t, reg[i].e[j]);
          *reinterpret_cast<u32x4_t*>(dst) = u;
        }
      }
    }
  }
};

template <typename T, int AM, int WM>
__global__ __launch_bounds__(256) void gemm_grad_kernel(GradGemmArgs g) {
  using M_ = Mfma<T>;
  using OA = Operand<T, AM>;
  using OW = Operand<T, WM>;
  constexpr int BK = GCfg<T>::BK;
  __shared__ __attribute__((aligned(16))) T As[BM * BK];
  __shared__ __attribute__((aligned(16))) T Bs[BN * BK];

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
  GatherArgs ga;
  ga.idx = g.g_idx; ga.w = g.g_w; ga.K = g.g_K; ga.N = g.g_N; ga.din = g.g_din; ga.dkp = g.g_dkp;

  GPack<T> ra[OA::NV], rw[OW::NV];
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // GATHER_T: the neighbour indices of step k + BK are loaded during step k,
  // so the gathered rows of a step never wait on their own index loads
  constexpr bool GI = WM == GG_GATHER_T;
  typename OW::Index ix;
  float wsave[OW::NV];
  if (kbeg < kend) {
    OA::fetch(ra, abase, 0, g.lda, g.avec, g.M, m0, kbeg, kend, tid, ga);
    OW::fetch(rw, wbase, g.w_krows, g.ldw, g.bvec, g.Nc, n0, kbeg, kend, tid, ga, nullptr, GI ? wsave : nullptr);
    if (GI && kbeg + BK < kend) OW::fetch_index(ix, g.Nc, n0, kbeg + BK, kend, tid, ga);
  }
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    if (GI) OW::scale(rw, wsave);
    OA::stash(ra, As, tid);
    OW::stash(rw, Bs, tid);
    __syncthreads();
    // next tile's loads and the MFMA loop at a raised wave priority
    __builtin_amdgcn_s_setprio(1);
    if (k0 + BK < kend) {
      OA::fetch(ra, abase, 0, g.lda, g.avec, g.M, m0, k0 + BK, kend, tid, ga);
      OW::fetch(rw, wbase, g.w_krows, g.ldw, g.bvec, g.Nc, n0, k0 + BK, kend, tid, ga, GI ? &ix : nullptr,
                GI ? wsave : nullptr);
      if (GI && k0 + 2 * BK < kend) OW::fetch_index(ix, g.Nc, n0, k0 + 2 * BK, kend, tid, ga);
    }
#pragma unroll
    for (int ks = 0; ks < BK / M_::KC; ++ks) {
      const int kk = ks * M_::KC + (lane >> 5) * M_::KL;
      typename M_::frag af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[i] = M_::load(&As[lds_off<T>(wm * 64 + i * 32 + (lane & 31), kk)]);
        bfr[i] = M_::load(&Bs[lds_off<T>(wn * 64 + i * 32 + (lane & 31), kk)]);
      }
      // transposed blocks (W as the MFMA A operand): a lane ends with 4
      // consecutive output columns of one row, stored as one vector
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = M_::mma(bfr[j], af[i], acc[i][j]);
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();
  }

  // acc[i][j][v] = out[m][n], m = m0 + wm*64 + i*32 + lane%32,
  //                n = n0 + wn*64 + j*32 + mfma_row(v, lane) (4 consecutive per v / 4)
  const bool vec = (g.Nc % 4 == 0) && (g.part != nullptr || (g.ldo % 4 == 0 && ((uintptr_t)g.o % (4 * sizeof(T))) == 0));
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + wm * 64 + i * 32 + (lane & 31);
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int vq = 0; vq < 4; ++vq) {
        const int n = n0 + wn * 64 + j * 32 + vq * 8 + (lane >> 5) * 4;
        if (n >= g.Nc) continue;
        const float a4[4] = {acc[i][j][vq * 4], acc[i][j][vq * 4 + 1], acc[i][j][vq * 4 + 2], acc[i][j][vq * 4 + 3]};
        if (vec && n + 4 <= g.Nc) {
          if (g.part != nullptr) {
            *reinterpret_cast<float4*>(&g.part[((int64_t)split * g.M + m) * g.Nc + n]) =
                make_float4(a4[0], a4[1], a4[2], a4[3]);
          } else {
            T* dst = static_cast<T*>(g.o) + (int64_t)m * g.ldo + n;
            if constexpr (sizeof(T) == 2) {
              uint2 u;
              u.x = Pair16<T>::pack(a4[0], a4[1]);
              u.y = Pair16<T>::pack(a4[2], a4[3]);
              *reinterpret_cast<uint2*>(dst) = u;
            } else {
              *reinterpret_cast<float4*>(dst) = make_float4(a4[0], a4[1], a4[2], a4[3]);
            }
          }
        } else {
          for (int u = 0; u < 4 && n + u < g.Nc; ++u) {
            if (g.part != nullptr)
              g.part[((int64_t)split * g.M + m) * g.Nc + n + u] = a4[u];
            else
              stf(static_cast<T*>(g.o) + (int64_t)m * g.ldo + n + u, a4[u]);
          }
        }
      }
  }
}

template <typename T, int AM>
int launch_grad_w(const GradGemmArgs& g, dim3 grid, hipStream_t s) {
  if (g.wmode == GG_ROWS)
    hipLaunchKernelGGL((gemm_grad_kernel<T, AM, GG_ROWS>), grid, dim3(256), 0, s, g);
  else if (g.wmode == GG_TRANS)
    hipLaunchKernelGGL((gemm_grad_kernel<T, AM, GG_TRANS>), grid, dim3(256), 0, s, g);
  else if (g.wmode == GG_GATHER_T)
    hipLaunchKernelGGL((gemm_grad_kernel<T, AM, GG_GATHER_T>), grid, dim3(256), 0, s, g);
  else
    return CNNA_ERR_OPTION;
  return (int)hipGetLastError();
}

template <typename T>
int launch_grad_t(const GradGemmArgs& g, hipStream_t s) {
  dim3 grid(((g.Nc + BN - 1) / BN) * ((g.M + BM - 1) / BM) * g.splits);
  if (g.amode == GG_ROWS) return launch_grad_w<T, GG_ROWS>(g, grid, s);
  if (g.amode == GG_TRANS) return launch_grad_w<T, GG_TRANS>(g, grid, s);
  return CNNA_ERR_OPTION;
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
  const int es = dtype == CNNA_F32 ? 4 : 2;
  const int bk = grad_gemm_bk(dtype);
  if (g.splits < 1) g.splits = 1;
  // fp32 partials when part is given (any split count), else T into o (one split)
  if (g.part == nullptr && (g.splits > 1 || g.o == nullptr)) return CNNA_ERR_NULL;
  g.kchunk = (int)cnna_round_up((size_t)((g.Kd + g.splits - 1) / g.splits), (size_t)bk);
  if (g.kchunk < bk) g.kchunk = bk;
  // 16-byte loads need 16-byte aligned rows
  g.avec = ((uintptr_t)g.a % 16 == 0) && ((g.lda * es) % 16 == 0);
  if (g.wmode == GG_GATHER_T) {
    if (!g.g_idx || !g.g_w || g.g_K <= 0 || g.g_N <= 0 || g.g_din <= 0) return CNNA_ERR_NULL;
    const int ce = 16 / es;
    g.bvec = ((uintptr_t)g.w[0] % 16 == 0) && (g.g_din % ce == 0) && (g.g_dkp % ce == 0);
  } else {
    bool bv = (g.ldw * es) % 16 == 0;
    if (g.w_krows == 0) g.w[1] = g.w[2] = g.w[0];
    for (int i = 0; i < 3; ++i) bv = bv && ((uintptr_t)g.w[i] % 16 == 0);
    g.bvec = bv;
  }
  if (dtype == CNNA_BF16) return launch_grad_t<uint16_t>(g, s);
  else if (dtype == CNNA_F16) return launch_grad_t<_Float16>(g, s);
  if (dtype == CNNA_F32) return launch_grad_t<float>(g, s);
  return CNNA_ERR_DTYPE;
}

int launch_splitk_reduce(int dtype, const ReduceArgs& r, hipStream_t s) {
  const int64_t MN = (int64_t)r.M * r.Nc;
  if (MN <= 0) return 0;
  dim3 grid((unsigned)((MN + 255) / 256));
  if (dtype == CNNA_BF16)
    hipLaunchKernelGGL(splitk_reduce_kernel<uint16_t>, grid, dim3(256), 0, s, r);
  else if (dtype == CNNA_F16)
    hipLaunchKernelGGL(splitk_reduce_kernel<_Float16>, grid, dim3(256), 0, s, r);
  else if (dtype == CNNA_F32)
    hipLaunchKernelGGL(splitk_reduce_kernel<float>, grid, dim3(256), 0, s, r);
  else
    return CNNA_ERR_DTYPE;
  return (int)hipGetLastError();
}
