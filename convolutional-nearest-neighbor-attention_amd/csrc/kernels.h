// Kernel argument blocks and host launchers shared between the kernel
// translation units and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// ---------------------------------------------------------------- GEMM
// out[m][n] = sum_k A[m][k] * W[n][k]  (nn.Linear: x @ W^T), fp32 accumulate.
enum { GEMM_A_ROWS = 0, GEMM_A_GATHER = 1 };
enum { GEMM_O_PLAIN = 0, GEMM_O_HEADSPLIT = 1 };

struct GemmArgs {
  int M, Nc, Kd;
  // A_ROWS: A row m is source row (arow ? (m / a_rows) * a_src_rows + arow[m % a_rows] : m)
  const void* a;
  int64_t lda;
  const int32_t* arow;
  int a_rows, a_src_rows;
  // A_GATHER: weighted neighbour rows, r-major over the reduction index:
  //   A[m][r*g_din + c] = g_w[m*g_K + r] * a[(m - m % g_N + g_idx[m*g_K + r]) * g_dkp + c]
  const int32_t* g_idx;
  const float* g_w;
  int g_K, g_N, g_din, g_dkp;
  // B: up to three (ncol_each, Kd) weight matrices stacked along n
  const void* w[3];
  int ncol_each;
  // outputs
  void* o[3];
  int64_t ldo;
  int o_rows, o_H, o_dk, o_dkp;
  int avec, bvec;  // 16-byte vector loads allowed for A / W
  int ovec;        // set by the launcher: 4-column vector stores allowed
  int ostage;      // set by the launcher: 16-bit tile staged through LDS for 16-byte stores
  // nn.Linear extras: out = act(A W^T + bias) + res (act and res: plain output only)
  const void* bias;  // (Nc) or NULL, indexed by the stacked output column
  int act;           // GEMM_ACT_*
  const void* res;   // (M, Nc) residual with row stride ldr, or NULL
  int64_t ldr;
  // prologue (row-major A): A rows are LayerNorm-ed on load,
  //   a[m][k] = round((x[m][k] - mean_m) * rstd_m * gamma[k] + beta[k]),
  // mean_m / rstd_m combined from ln_parts per-tile (mean, M2) partials of
  // the row (ROW_STAT_TILE columns each, the last one partial), or NULL
  const float* ln_stats;
  int ln_parts;
  const void* ln_gamma;
  const void* ln_beta;
  float ln_eps;
  // epilogue (staged 16-bit, plain output): per ROW_STAT_TILE-column tile of
  // each output row, (mean, M2) of the stored values, at
  // st_out[(m * ceil(Nc / ROW_STAT_TILE) + tile) * 2], or NULL
  float* st_out;
};
enum { GEMM_ACT_NONE = 0, GEMM_ACT_GELU = 1 };
// columns per row-statistics partial (the GEMM's column tile)
constexpr int ROW_STAT_TILE = 128;

int launch_gemm(int dtype, int amode, int omode, const GemmArgs& g, hipStream_t s);

// ---------------------------------------------------------------- ViT block
// LayerNorm over rows of C (one wave per row), optional residual in front.
struct LnArgs {
  const void* x;
  int64_t ldx;
  const void* res;    // or NULL
  int64_t ldr;
  void* sum_out;      // x + res, or NULL
  int64_t lds;
  const void* gamma;  // or NULL
  const void* beta;   // or NULL
  float eps;
  void* y;
  int64_t ldy;
  int64_t rows;
  int C;
  // statistics only: y unused, (mean, M2) of each row over ROW_STAT_TILE
  // column tiles written to stats[(row * parts + t) * 2] (the GEMM
  // prologue's format), or NULL
  float* stats;
};
// deterministic column sums out[c] = sum_r a[r * lda + c] (fp32, fixed order), rounded to the dtype
int launch_colsum(int dtype, const void* a, int64_t rows, int cols, int64_t lda, void* out, hipStream_t s);
int launch_layernorm(int dtype, const LnArgs& a, hipStream_t s);

// ---------------------------------------------------------------- prep
// Per row of a head-split tensor: coordinate channel, zero padding, cosine
// normalisation or euclidean squared norm.
struct PrepArgs {
  void* t;          // (rows_total, dkp)
  float* norms;     // euclidean: squared norms per row, else NULL
  int rows_total;   // BH * rows
  int rows;         // rows per head (linspace length)
  int dk, dkp;
  int coord;        // write linspace(-1, 1, rows) into channel dk
  int normalize;    // cosine: divide channels [0, din) by max(||.||, 1e-12)
};
int launch_prep(int dtype, const PrepArgs& p, hipStream_t s);

// ---------------------------------------------------------------- select
struct SelArgs {
  const void* k;     // (BH, N, dkp)
  const void* q;     // (BH, Nq, dkp)
  const float* kn;   // euclidean squared norms (BH*N) or NULL
  const float* qn;   // (BH*Nq) or NULL
  const int32_t* cand;  // sampled candidate -> token map (Nq) or NULL
  int32_t* idx;      // (BH, N, K)
  float* vals;       // (BH, N, K) selected similarity values
  float* w;          // (BH, N, K) neighbour weights, or NULL
  int32_t* cols;     // sampled: (BH, N, K) candidate column of each entry (slot 0: Nq), or NULL
  int softmax;       // softmax_topk_val
  int BH, N, Nq, dkp, K, Ksel, rb_per_bh;
  int kbase;         // entries (after the sampled self slot) chosen by earlier rounds of a
                     // selection wider than one list; 0 for the first round
  float kscale;      // key = acc * kscale for dot metrics (raw keys: value = key * kscale, kscale > 0)
  int kneg;          // raw keys of a negative matmul scale: rank -k.q (the key rows are negated)
  float mask_key;    // key of the self-masked candidate (sampled)
  float mask_val;    // value reported for it
};
int launch_select(int dtype, int euclid, int sampled, const SelArgs& a, hipStream_t s);

// ---------------------------------------------------------------- aggregate
struct AggArgs {
  const void* v;       // (BH, N, dkp) values; for the merge: y (BH, N, dout)
  const int32_t* idx;  // (BH, N, K) neighbour token indices
  const float* w;      // (BH, N, K) neighbour weights
  const void* w0;      // depthwise conv weight (dout, 1, K)
  void* out;           // merged Z (B, N, C) or plain (BH, N, dout)
  int BH, N, K, dout, dkp;
  int H, C;
  int merged;          // MERGE_*
  int lpt, ti, nblk;   // set by the launcher
};
// Output layouts of the aggregate / merge kernels:
//   PLAIN      token-major (BH, N, dout)
//   REFERENCE  the ConvNN head merge (layers.py:247-259): token-mixing when H > 1, transpose when H == 1
//   CONCAT     heads side by side, Z[b, t, h*dout + c] (MultiHeadKvtAttention, layers.py:683)
//   MIX        the token-mixing merge for every H (MultiHeadConv1dAttention, layers.py:490-497)
enum { MERGE_PLAIN = 0, MERGE_REFERENCE = 1, MERGE_CONCAT = 2, MERGE_MIX = 3 };
// conv over the gathered neighbours; w0 == NULL: unit weights (plain weighted sum)
int launch_aggregate(int dtype, const AggArgs& a, hipStream_t s);
// head merge of a token-major y into Z
int launch_merge(int dtype, const AggArgs& a, hipStream_t s);
// W0 (dout, din, K) -> W0p (dout, K*din) with W0p[o][r*din + c] = W0[o][c][r]
int launch_permute_w0(int dtype, const void* w0, void* w0p, int dout, int din, int K, hipStream_t s);
// dst[c * ldd + k] = src[k * cols + c]: transpose of a (rows, cols) matrix into
// columns [0, rows) of a (cols, ldd) destination
int launch_transpose(int dtype, const void* src, void* dst, int rows, int cols, int64_t ldd,
                     hipStream_t s);
// W0 (dout, din, K) -> W0t (K*din, dout), W0t[r*din + c][o] = W0[o][c][r]
int launch_permute_w0t(int dtype, const void* w0, void* w0t, int dout, int din, int K, hipStream_t s);

// ================================================================ backward
// Gradient GEMM: out[m][n] = sum_k A[m][k] * W[n][k] with
//   A: ROWS a[m * lda + k]  |  TRANS a[k * lda + m]
//   W: ROWS w[n * ldw + k]  |  TRANS w[k * ldw + n], optionally three
//      matrices stacked along k (w_krows rows each)
//      | GATHER_T  W[n][k] = g_w[k*g_K + r] * w[0][(k - k % g_N + g_idx[k*g_K + r]) * g_dkp + c]
//        with n = r*g_din + c: the gathered conv input P of token k, read transposed.
// Without part: T into o (splits must be 1).  With part: fp32 partial sums
// part[s][m][n] over k-chunks of kchunk, summed by launch_splitk_reduce.
enum { GG_ROWS = 0, GG_TRANS = 1, GG_GATHER_T = 2 };
struct GradGemmArgs {
  int M, Nc, Kd;
  const void* a;
  int64_t lda;
  int amode;
  const void* w[3];
  int64_t ldw;
  int wmode;
  int w_krows;       // 0: single W; else rows of k per stacked pointer
  const int32_t* g_idx;
  const float* g_w;
  int g_K, g_N, g_din, g_dkp;
  void* o;
  int64_t ldo;
  float* part;
  int splits, kchunk;
  int avec, bvec;    // set by the launcher
};
// split count for a weight-gradient GEMM (shared by launcher and workspace sizing)
inline int grad_gemm_splits(int M, int Nc, int Kd, int bk) {
  const int tiles = ((M + 127) / 128) * ((Nc + 127) / 128);
  int s = (512 + tiles - 1) / tiles;
  const int maxs = (Kd + 8 * bk - 1) / (8 * bk);   // at least 8 k-tiles per split
  if (s > maxs) s = maxs;
  return s < 1 ? 1 : s;
}
inline int grad_gemm_bk(int dtype) { return dtype == 1 ? 64 : 32; }
int launch_gemm_grad(int dtype, const GradGemmArgs& g, hipStream_t s);

// Sum of split-K partials into up to three row blocks of T outputs, with an
// optional column permutation n = r*pdin + c -> c*pK + r (conv weight layout).
struct ReduceArgs {
  const float* part;
  int splits, M, Nc;
  void* o[3];
  int rows_each;
  int64_t ldo;
  int pdin, pK;      // pdin > 0: permute columns
};
int launch_splitk_reduce(int dtype, const ReduceArgs& r, hipStream_t s);

// Inverse head merge: dy (BH, N, dk) token-major from dZ (B, N, C), the
// reference merge or (concat) heads side by side.
int launch_unmerge(int dtype, const void* dz, void* dy, int BH, int N, int dk, int H, int C,
                   int concat, hipStream_t s);

// Per token: neighbour-weight gradient, softmax / weight backward, similarity
// gradient coefficients and the key gradient; depthwise-weight partial sums.
struct TokBwdArgs {
  const void* g;        // depthwise modes: (BH, N, din) gradient at the depthwise-conv output
  const void* dP;       // standard conv: (BH*N*K, din) gradient of the gathered input
  const void* v;        // (BH, N, dkp)
  const void* k;        // (BH, N, dkp), normalised for cosine
  const void* q;        // (BH, Nq, dkp), normalised for cosine
  const float* kn;      // squared key norms (cosine, euclidean)
  const int32_t* idx;   // (BH, N, K)
  const float* vals;    // (BH, N, K)
  const float* w;       // (BH, N, K)
  const float* wmul;    // (BH, N, K) multipliers applied to w before the aggregation, or NULL
  const int32_t* cols;  // sampled: (BH, N, K) candidate column of each entry
  const void* w0;       // depthwise weight (din, 1, K)
  float* coef;          // out: (BH, N, K) similarity-gradient coefficient
  float* w0part;        // out: (gridDim, din, K) depthwise-weight partials
  void* dst;            // dK rows (B*N) of stride ldd, columns offd + h*dk + c
  int64_t ldd;
  int offd;
  int BH, N, Nq, K, din, dk, dkp, H;
  int metric, softmax, sampled, std_conv;
  float scale;          // matmul: 1/sqrt(d_k)
  int nblk;             // set by the launcher
};
int launch_tok_bwd(int dtype, const TokBwdArgs& a, hipStream_t s);
// number of blocks of launch_tok_bwd (sizes the w0part buffer)
inline int tok_bwd_blocks(int BH, int N) {
  const long long w = ((long long)BH * N + 3) / 4;
  return (int)(w < 2048 ? (w < 1 ? 1 : w) : 2048);
}
int launch_w0_reduce(int dtype, const float* part, int nblk, int n, void* out, hipStream_t s);

// Deterministic reverse adjacency: entries e = i*K + r of each (b, h) bucketed
// by key (CSR_TOKEN: idx[e]; CSR_COLUMN: cols[e] for sampled r >= 1 that are
// not the masked self column), sorted by e inside each bucket.
enum { CSR_TOKEN = 0, CSR_COLUMN = 1 };
struct CsrArgs {
  const int32_t* idx;
  const int32_t* cols;
  int mode;
  int BH, N, K, nkeys;
  int32_t* cnt;    // (BH, nkeys)
  int32_t* off;    // (BH, nkeys + 1)
  int32_t* tmp;    // (BH, N*K)
  int32_t* list;   // (BH, N*K)
};
int launch_csr(const CsrArgs& c, hipStream_t s);

// Pull reductions over a CSR: dV (sum of w * dP over the entries that read a
// value row) and dQ (sum of coef * k over the entries that selected a column).
struct PullArgs {
  const int32_t* off;
  const int32_t* list;
  int nkeys;
  int do_v, do_q;
  // dV
  const void* g;       // depthwise modes: (BH, N, din)
  const void* dP;      // standard: (BH*N*K, din)
  const void* w0;      // depthwise weight (din, 1, K)
  const float* w;      // (BH, N, K)
  const float* wmul;   // (BH, N, K) or NULL, as in TokBwdArgs
  int std_conv;
  void* dst_v;
  int64_t ld_v;
  int off_v;
  // dQ
  const float* coef;
  const void* k;       // (BH, N, dkp)
  const void* q;       // (BH, nkeys, dkp)
  const float* qn;     // squared norms of q rows
  int metric;
  void* dst_q;
  int64_t ld_q;
  int off_q;
  int BH, N, K, din, dk, dkp, H;
};
int launch_pull(int dtype, const PullArgs& p, hipStream_t s);

// sampled rows: xs[b, j] = x[b, cand[j]];  dx[b, cand[j]] += dxs[b, j] in j order
int launch_gather_rows(int dtype, const void* x, int64_t ldx, const int32_t* cand, void* xs, int B,
                       int N, int Nq, int C, hipStream_t s);
int launch_scatter_rows(int dtype, const void* dxs, const int32_t* cand, void* dx, int B, int N,
                        int Nq, int C, hipStream_t s);
int launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t s);

// ================================================================ branches
// Conv1d(dk, dk, ks, stride 1, padding 'same') along the tokens of each head
// of u (B, N, H*dk) (MultiHeadConv1dAttention, layers.py:495-497):
//   y[b*H + h][t][o] = bias[o] + sum_{c, r} w[o][c][r] * u[b][t + r - padl][h*dk + c]
// (zero outside [0, N)), y token-major (B*H, N, dk).
struct Conv1dArgs {
  const void* u;
  int64_t ldu;
  const void* w;      // (dk, dk, ks)
  const void* bias;   // (dk) or NULL
  void* y;
  int B, N, H, dk, ks, padl;
  float* wprep;       // scratch for the weights as fp32 [c][o][taps], or NULL
  size_t wprep_bytes;
  int tt;             // set by the launcher: tokens per block
};
// bytes of Conv1dArgs::wprep that let the weights stage from LDS
inline size_t conv1d_wprep_bytes(int dk, int ks) {
  const int ksm = ks == 1 ? 1 : ks <= 3 ? 3 : ks <= 5 ? 5 : ks <= 9 ? 9 : ks <= 17 ? 17 : 33;
  return (size_t)dk * dk * ksm * 4;
}
int launch_conv1d_tokens(int dtype, const Conv1dArgs& a, hipStream_t s);
