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
  int ostage;      // set by the launcher: bf16 tile staged through LDS for 16-byte stores
};

int launch_gemm(int dtype, int amode, int omode, const GemmArgs& g, hipStream_t s);

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
  int softmax;       // softmax_topk_val
  int BH, N, Nq, dkp, K, Ksel, rb_per_bh;
  float kscale;      // key = acc * kscale for dot metrics
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
  int merged;          // 1: write Z (head merge), 0: plain token-major
  int lpt, ti, nblk;   // set by the launcher
};
// depthwise conv over the gathered neighbours
int launch_aggregate(int dtype, const AggArgs& a, hipStream_t s);
// head merge of a token-major y into Z
int launch_merge(int dtype, const AggArgs& a, hipStream_t s);
// W0 (dout, din, K) -> W0p (dout, K*din) with W0p[o][r*din + c] = W0[o][c][r]
int launch_permute_w0(int dtype, const void* w0, void* w0p, int dout, int din, int K, hipStream_t s);
