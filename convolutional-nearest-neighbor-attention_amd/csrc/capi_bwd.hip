// C-ABI backward entry points (declared in include/cnna.h): the autograd of
// MultiHeadConvNNAttention.forward (layers.py:261-321) expressed as GEMMs over
// the neighbour lists plus the per-token / reverse-adjacency kernels of
// backward.hip.  Workspaces are carved by one plan shared with the size query.
#include <math.h>
#include <string.h>

#include "common.h"
#include "kernels.h"

#include "desc_util.h"

using namespace cnna_desc_util;

namespace {

struct CorePlan {
  void *dy, *t1, *dt1, *w0p, *dP, *dqkv, *dqs, *xs, *dxs, *wt;
  float *coef, *w0part, *part;
  int32_t *cnt, *off, *tmp, *list, *cnt2, *off2, *tmp2, *list2;
  size_t bytes;
};

size_t part_floats(int dtype, int M, int Nc, int Kd) {
  return (size_t)grad_gemm_splits(M, Nc, Kd, grad_gemm_bk(dtype)) * M * Nc;
}

CorePlan plan_core(const cnna_desc* d, void* ws) {
  CorePlan p;
  memset(&p, 0, sizeof(p));
  Carve c(ws);
  const size_t es = elem_size(d->dtype), BH = (size_t)d->B * d->H;
  const size_t N = d->N, Nq = d->Nq, K = d->K, C = d->C, B = d->B;
  const size_t dk = C / d->H, din = din_of(d);
  const size_t tok = BH * N, ent = tok * K;
  p.dy = c.take(tok * dk * es);
  if (d->conv == CNNA_CONV_DWSEP) {
    p.t1 = c.take(tok * din * es);
    p.dt1 = c.take(tok * din * es);
  }
  if (d->conv == CNNA_CONV_STANDARD) {
    p.w0p = c.take(dk * K * din * es);
    p.dP = c.take(ent * din * es);
  }
  p.coef = static_cast<float*>(c.take(ent * 4));
  if (d->conv != CNNA_CONV_STANDARD)
    p.w0part = static_cast<float*>(c.take((size_t)tok_bwd_blocks((int)BH, (int)N) * din * K * 4));
  p.dqkv = c.take(B * N * (d->sampled ? 2 : 3) * C * es);
  p.wt = c.take(3 * C * C * es);                 // [W_q^T | W_k^T | W_v^T] for dx
  p.cnt = static_cast<int32_t*>(c.take(BH * N * 4));
  p.off = static_cast<int32_t*>(c.take(BH * (N + 1) * 4));
  p.tmp = static_cast<int32_t*>(c.take(ent * 4));
  p.list = static_cast<int32_t*>(c.take(ent * 4));
  size_t partf = 0;
  auto upd = [&](size_t f) { partf = f > partf ? f : partf; };
  if (d->sampled) {
    p.dqs = c.take(B * Nq * C * es);
    p.xs = c.take(B * Nq * C * es);
    p.dxs = c.take(B * Nq * C * es);
    p.cnt2 = static_cast<int32_t*>(c.take(BH * (Nq > 0 ? Nq : 1) * 4));
    p.off2 = static_cast<int32_t*>(c.take(BH * (Nq + 1) * 4));
    p.tmp2 = static_cast<int32_t*>(c.take(ent * 4));
    p.list2 = static_cast<int32_t*>(c.take(ent * 4));
    upd(part_floats(d->dtype, 2 * d->C, d->C, d->B * d->N));
    upd(part_floats(d->dtype, d->C, d->C, d->B * d->Nq));
  } else {
    upd(part_floats(d->dtype, 3 * d->C, d->C, d->B * d->N));
  }
  if (d->conv == CNNA_CONV_STANDARD) upd(part_floats(d->dtype, (int)dk, (int)(K * din), (int)tok));
  if (d->conv == CNNA_CONV_DWSEP) upd(part_floats(d->dtype, (int)dk, (int)din, (int)tok));
  p.part = static_cast<float*>(c.take(partf * 4));
  p.bytes = c.used;
  return p;
}

// weight gradient out = A^T-style GEMM through fp32 split-K partials
int weight_grad(int dtype, GradGemmArgs g, float* part, void* o0, void* o1, void* o2, int rows_each,
                int64_t ldo, int pdin, int pK, hipStream_t s) {
  g.splits = grad_gemm_splits(g.M, g.Nc, g.Kd, grad_gemm_bk(dtype));
  g.part = part;
  g.o = nullptr;
  int st = launch_gemm_grad(dtype, g, s);
  if (st) return st;
  ReduceArgs r;
  memset(&r, 0, sizeof(r));
  r.part = part;
  r.splits = g.splits;
  r.M = g.M;
  r.Nc = g.Nc;
  r.o[0] = o0; r.o[1] = o1; r.o[2] = o2;
  r.rows_each = rows_each;
  r.ldo = ldo;
  r.pdin = pdin;
  r.pK = pK;
  return launch_splitk_reduce(dtype, r, s);
}

GradGemmArgs gg(int M, int Nc, int Kd, const void* a, int64_t lda, int amode, const void* w,
                int64_t ldw, int wmode) {
  GradGemmArgs g;
  memset(&g, 0, sizeof(g));
  g.M = M; g.Nc = Nc; g.Kd = Kd;
  g.a = a; g.lda = lda; g.amode = amode;
  g.w[0] = w; g.ldw = ldw; g.wmode = wmode;
  g.splits = 1;
  return g;
}

}  // namespace

extern "C" {

size_t cnna_output_proj_backward_workspace(const cnna_desc* d) {
  if (cnna_check_desc(d)) return 0;
  return cnna_round_up(part_floats(d->dtype, d->C, d->C, d->B * d->N) * 4, 256) +
         cnna_round_up((size_t)d->C * d->C * elem_size(d->dtype), 256);   // W_o^T
}

int cnna_output_proj_backward(const cnna_desc* d, const void* z, const void* Wo, const void* dout,
                              int64_t ld_dout, void* dz, void* dWo, void* ws, size_t ws_bytes,
                              void* stream) {
  int st = cnna_check_desc(d);
  if (st) return st;
  if (!z || !Wo || !dout || !dz || !dWo || !ws) return CNNA_ERR_NULL;
  if (ld_dout < d->C) return CNNA_ERR_SHAPE;
  if (ws_bytes < cnna_output_proj_backward_workspace(d)) return CNNA_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  const int M = d->B * d->N, C = d->C;
  // dz[m][c] = sum_n dout[m][n] Wo[n][c]: a row GEMM against W_o^T (the forward kernel)
  char* wtp = static_cast<char*>(ws) + cnna_round_up(part_floats(d->dtype, C, C, M) * 4, 256);
  if ((st = launch_transpose(d->dtype, Wo, wtp, C, C, C, s))) return st;
  {
    const int es = elem_size(d->dtype);
    GemmArgs f;
    memset(&f, 0, sizeof(f));
    f.M = M; f.Nc = C; f.Kd = C;
    f.a = dout; f.lda = ld_dout;
    f.avec = ((C * es) % 16 == 0) && ((ld_dout * es) % 16 == 0) && aligned16(dout);
    f.w[0] = wtp; f.ncol_each = C;
    f.bvec = ((C * es) % 16 == 0) && aligned16(wtp);
    f.o[0] = dz; f.ldo = C;
    if ((st = launch_gemm(d->dtype, GEMM_A_ROWS, GEMM_O_PLAIN, f, s))) return st;
  }
  // dWo[n][c] = sum_m dout[m][n] z[m][c]
  GradGemmArgs g = gg(C, C, M, dout, ld_dout, GG_TRANS, z, C, GG_TRANS);
  return weight_grad(d->dtype, g, static_cast<float*>(ws), dWo, nullptr, nullptr, C, C, 0, 0, s);
}

size_t cnna_core_backward_workspace(const cnna_desc* d) {
  if (cnna_check_desc(d)) return 0;
  return plan_core(d, nullptr).bytes;
}

int cnna_core_backward(const cnna_desc* d, const void* x, int64_t ldx, const int32_t* cand,
                       const void* Wq, const void* Wk, const void* Wv, const void* conv_w0,
                       const void* conv_w1, const cnna_saved* sv, const void* dz,
                       const cnna_grads* gr, void* ws, size_t ws_bytes, void* stream) {
  int st = cnna_check_desc(d);
  if (st) return st;
  // the per-token backward holds a token's entries one per lane
  if (d->K > 64) return CNNA_ERR_UNSUPPORTED;
  if (!x || !Wq || !Wk || !Wv || !conv_w0 || !sv || !dz || !gr || !ws) return CNNA_ERR_NULL;
  if (!sv->q || !sv->k || !sv->v || !sv->idx || !sv->vals || !sv->w) return CNNA_ERR_NULL;
  if (d->metric != CNNA_MATMUL && (!sv->qn || !sv->kn)) return CNNA_ERR_NULL;
  if (!gr->dx || !gr->dWq || !gr->dWk || !gr->dWv || !gr->dconv_w0) return CNNA_ERR_NULL;
  if (d->conv == CNNA_CONV_DWSEP && (!conv_w1 || !gr->dconv_w1)) return CNNA_ERR_NULL;
  if (d->sampled && (!cand || !sv->cols)) return CNNA_ERR_NULL;
  if (sv->wmul && d->conv != CNNA_CONV_DEPTHWISE) return CNNA_ERR_OPTION;
  if (ldx < d->C) return CNNA_ERR_SHAPE;
  if (ws_bytes < cnna_core_backward_workspace(d)) return CNNA_ERR_WORKSPACE;
  if (!aligned16(ws)) return CNNA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const CorePlan p = plan_core(d, ws);
  const int dt = d->dtype;
  const int B = d->B, N = d->N, Nq = d->Nq, K = d->K, C = d->C, H = d->H, BH = B * H;
  const int dk = C / H, din = din_of(d), dkp = dkp_of(d);
  const int ntok = BH * N;

  // 1. inverse head merge: dy (BH, N, dk)
  if ((st = launch_unmerge(dt, dz, p.dy, BH, N, dk, H, C, d->merge == CNNA_MERGE_CONCAT, s)))
    return st;

  // 2. conv backward down to dP / g
  const void* g_dw = nullptr;   // gradient at the depthwise-conv output (depthwise modes)
  if (d->conv == CNNA_CONV_DEPTHWISE) {
    g_dw = p.dy;
  } else if (d->conv == CNNA_CONV_DWSEP) {
    // recompute the depthwise stage t1 (BH*N, din)
    AggArgs a;
    memset(&a, 0, sizeof(a));
    a.v = sv->v; a.idx = sv->idx; a.w = sv->w; a.w0 = conv_w0; a.out = p.t1;
    a.BH = BH; a.N = N; a.K = K; a.dout = din; a.dkp = dkp; a.H = H; a.C = C; a.merged = 0;
    if ((st = launch_aggregate(dt, a, s))) return st;
    // dt1 = dy @ W1 ; dW1 = dy^T t1
    GradGemmArgs g = gg(ntok, din, dk, p.dy, dk, GG_ROWS, conv_w1, din, GG_TRANS);
    g.o = p.dt1;
    g.ldo = din;
    if ((st = launch_gemm_grad(dt, g, s))) return st;
    g = gg(dk, din, ntok, p.dy, dk, GG_TRANS, p.t1, din, GG_TRANS);
    if ((st = weight_grad(dt, g, p.part, gr->dconv_w1, nullptr, nullptr, dk, din, 0, 0, s)))
      return st;
    g_dw = p.dt1;
  } else {
    // standard: dP = dy @ W0p ; dW0p = dy^T P with P[tok][r*din + c] = w * v[idx] gathered
    // inside the GEMM, permuted back to (dk, din, K)
    // dP as a row GEMM against W0p^T (the forward kernel: LDS-staged 16-byte stores
    // of the 805 MB-class output)
    if ((st = launch_permute_w0t(dt, conv_w0, p.w0p, dk, din, K, s))) return st;
    {
      const int es = elem_size(dt);
      GemmArgs f;
      memset(&f, 0, sizeof(f));
      f.M = ntok; f.Nc = K * din; f.Kd = dk;
      f.a = p.dy; f.lda = dk;
      f.avec = ((dk * es) % 16 == 0) && aligned16(p.dy);
      f.w[0] = p.w0p; f.ncol_each = K * din;
      f.bvec = ((dk * es) % 16 == 0) && aligned16(p.w0p);
      f.o[0] = p.dP; f.ldo = (int64_t)K * din;
      if ((st = launch_gemm(dt, GEMM_A_ROWS, GEMM_O_PLAIN, f, s))) return st;
    }
    GradGemmArgs g = gg(dk, K * din, ntok, p.dy, dk, GG_TRANS, sv->v, 0, GG_GATHER_T);
    g.g_idx = sv->idx; g.g_w = sv->w; g.g_K = K; g.g_N = N; g.g_din = din; g.g_dkp = dkp;
    if ((st = weight_grad(dt, g, p.part, gr->dconv_w0, nullptr, nullptr, dk, (int64_t)din * K, din,
                          K, s)))
      return st;
  }

  // 3. per token: weight / softmax / similarity backward, dK, depthwise-weight partials
  const int ld3 = (d->sampled ? 2 : 3) * C;
  const int offK = d->sampled ? 0 : C, offV = offK + C;
  TokBwdArgs t;
  memset(&t, 0, sizeof(t));
  t.g = g_dw; t.dP = p.dP; t.v = sv->v; t.k = sv->k; t.q = sv->q; t.kn = sv->kn;
  t.idx = sv->idx; t.vals = sv->vals; t.w = sv->w; t.cols = sv->cols; t.w0 = conv_w0;
  t.coef = p.coef; t.w0part = p.w0part;
  t.dst = p.dqkv; t.ldd = ld3; t.offd = offK;
  t.BH = BH; t.N = N; t.Nq = Nq; t.K = K; t.din = din; t.dk = dk; t.dkp = dkp; t.H = H;
  t.metric = d->metric; t.softmax = d->softmax; t.sampled = d->sampled;
  t.std_conv = d->conv == CNNA_CONV_STANDARD;
  t.scale = matmul_scale(d);
  t.wmul = sv->wmul;
  if ((st = launch_tok_bwd(dt, t, s))) return st;
  if (d->conv != CNNA_CONV_STANDARD &&
      (st = launch_w0_reduce(dt, p.w0part, tok_bwd_blocks(BH, N), din * K, gr->dconv_w0, s)))
    return st;

  // 4. reverse adjacency by value row; dV (and dQ for 'all') pulled in entry order
  CsrArgs c;
  memset(&c, 0, sizeof(c));
  c.idx = sv->idx; c.cols = sv->cols; c.mode = CSR_TOKEN;
  c.BH = BH; c.N = N; c.K = K; c.nkeys = N;
  c.cnt = p.cnt; c.off = p.off; c.tmp = p.tmp; c.list = p.list;
  if ((st = launch_csr(c, s))) return st;
  PullArgs pa;
  memset(&pa, 0, sizeof(pa));
  pa.off = p.off; pa.list = p.list; pa.nkeys = N;
  pa.do_v = 1;
  pa.g = g_dw; pa.dP = p.dP; pa.w0 = conv_w0; pa.w = sv->w; pa.wmul = sv->wmul;
  pa.std_conv = t.std_conv;
  pa.dst_v = p.dqkv; pa.ld_v = ld3; pa.off_v = offV;
  pa.coef = p.coef; pa.k = sv->k; pa.q = sv->q; pa.qn = sv->qn; pa.metric = d->metric;
  pa.BH = BH; pa.N = N; pa.K = K; pa.din = din; pa.dk = dk; pa.dkp = dkp; pa.H = H;
  if (!d->sampled) {
    pa.do_q = 1;
    pa.dst_q = p.dqkv; pa.ld_q = ld3; pa.off_q = 0;
  }
  if ((st = launch_pull(dt, pa, s))) return st;
  if (d->sampled) {
    // reverse adjacency by candidate column for dQ of the sampled rows
    c.mode = CSR_COLUMN; c.nkeys = Nq;
    c.cnt = p.cnt2; c.off = p.off2; c.tmp = p.tmp2; c.list = p.list2;
    if ((st = launch_csr(c, s))) return st;
    pa.off = p.off2; pa.list = p.list2; pa.nkeys = Nq;
    pa.do_v = 0; pa.do_q = 1;
    pa.dst_q = p.dqs; pa.ld_q = C; pa.off_q = 0;
    if ((st = launch_pull(dt, pa, s))) return st;
  }

  // bias gradients of the projections: column sums of dQ, dK, dV
  if (gr->dbqkv != nullptr) {
    char* db = static_cast<char*>(gr->dbqkv);
    const size_t es = elem_size(dt);
    if (!d->sampled) {
      if ((st = launch_colsum(dt, p.dqkv, (int64_t)B * N, 3 * C, ld3, db, s))) return st;
    } else {
      if ((st = launch_colsum(dt, p.dqkv, (int64_t)B * N, 2 * C, ld3, db + C * es, s))) return st;
      if ((st = launch_colsum(dt, p.dqs, (int64_t)B * Nq, C, C, db, s))) return st;
    }
  }

  // 5. projections: dx and the weight gradients.  dx = dqkv @ [W_q; W_k; W_v]
  // as a row GEMM against the transposed stack (the forward kernel)
  {
    const void* ws3[3] = {Wq, Wk, Wv};
    const void* ws2[2] = {Wk, Wv};
    const int nm = d->sampled ? 2 : 3;
    for (int j = 0; j < nm; ++j) {
      const void* src = d->sampled ? ws2[j] : ws3[j];
      if ((st = launch_transpose(dt, src, static_cast<char*>(p.wt) + (size_t)j * C * elem_size(dt), C, C,
                                 ld3, s)))
        return st;
    }
    const int es = elem_size(dt);
    GemmArgs f;
    memset(&f, 0, sizeof(f));
    f.M = B * N; f.Nc = C; f.Kd = ld3;
    f.a = p.dqkv; f.lda = ld3;
    f.avec = ((ld3 * es) % 16 == 0) && aligned16(p.dqkv);
    f.w[0] = p.wt; f.ncol_each = C;
    f.bvec = ((ld3 * es) % 16 == 0) && aligned16(p.wt);
    f.o[0] = gr->dx; f.ldo = C;
    if ((st = launch_gemm(dt, GEMM_A_ROWS, GEMM_O_PLAIN, f, s))) return st;
  }
  GradGemmArgs g = gg(ld3, C, B * N, p.dqkv, ld3, GG_TRANS, x, ldx, GG_TRANS);
  if (d->sampled) {
    if ((st = weight_grad(dt, g, p.part, gr->dWk, gr->dWv, nullptr, C, C, 0, 0, s))) return st;
    if (Nq > 0) {
      // x[:, cand] rows: dx += scatter(dQs @ Wq), dWq = dQs^T x[:, cand]
      g = gg(B * Nq, C, C, p.dqs, C, GG_ROWS, Wq, C, GG_TRANS);
      g.o = p.dxs;
      g.ldo = C;
      if ((st = launch_gemm_grad(dt, g, s))) return st;
      if ((st = launch_scatter_rows(dt, p.dxs, cand, gr->dx, B, N, Nq, C, s))) return st;
      if ((st = launch_gather_rows(dt, x, ldx, cand, p.xs, B, N, Nq, C, s))) return st;
      g = gg(C, C, B * Nq, p.dqs, C, GG_TRANS, p.xs, C, GG_TRANS);
      if ((st = weight_grad(dt, g, p.part, gr->dWq, nullptr, nullptr, C, C, 0, 0, s))) return st;
    }
  } else {
    if ((st = weight_grad(dt, g, p.part, gr->dWq, gr->dWk, gr->dWv, C, C, 0, 0, s))) return st;
  }
  return CNNA_OK;
}

}  // extern "C"
