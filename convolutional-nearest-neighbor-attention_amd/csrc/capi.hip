// C-ABI entry points of libcnna.so (declared in include/cnna.h).
// Validation mirrors the exceptions the reference raises (layers.py:149,
// 251, 310, 344/365 via torch.topk, Conv1d groups check) so callers can map
// status codes to the same Python exception types before any launch.
#include <math.h>
#include <string.h>

#include "common.h"
#include "kernels.h"

#include "desc_util.h"

using namespace cnna_desc_util;

static_assert(CNNA_STAT_TILE == ROW_STAT_TILE, "statistics tile of the ABI and the kernels");

extern "C" {

int cnna_abi_version(void) { return CNNA_ABI_VERSION; }

const char* cnna_error_string(int code) {
  switch (code) {
    case CNNA_OK: return "ok";
    case CNNA_ERR_NULL: return "cnna: required pointer is NULL";
    case CNNA_ERR_SHAPE: return "cnna: inconsistent or unsupported shape";
    case CNNA_ERR_DTYPE: return "cnna: unsupported dtype (float32, bfloat16 or float16)";
    case CNNA_ERR_OPTION: return "cnna: unknown magnitude_type / convolution_type / option combination";
    case CNNA_ERR_K_RANGE: return "cnna: selected index k out of range";
    case CNNA_ERR_SEQ_LENGTH: return "cnna: seq_length must equal the number of tokens when num_heads > 1";
    case CNNA_ERR_WORKSPACE: return "cnna: workspace too small";
    case CNNA_ERR_GROUPS: return "cnna: out_channels must be divisible by groups";
    case CNNA_ERR_SCRATCH:
      return "cnna: the call needs more intermediate memory than the 128 MiB static scratch of "
             "cnna_forward_noalloc; call cnna_forward with a workspace";
    case CNNA_ERR_UNSUPPORTED:
      return "cnna: configuration not supported by this build (limits: K <= 64 neighbours in the "
             "backward, head width d_k (+1 with coordinate encoding) <= 256, at most 65536 "
             "candidates; folded LayerNorm: C <= 1024; row statistics "
             "epilogue: 16-bit types, Nout % 8 == 0, 16-byte aligned out / res with row strides that "
             "are multiples of 8 elements)";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "cnna: unknown error";
}

int cnna_check_desc(const cnna_desc* d) {
  if (d == nullptr) return CNNA_ERR_NULL;
  if (d->dtype != CNNA_F32 && d->dtype != CNNA_BF16 && d->dtype != CNNA_F16) return CNNA_ERR_DTYPE;
  if (d->B <= 0 || d->N <= 0 || d->C <= 0 || d->H <= 0 || d->C % d->H != 0) return CNNA_ERR_SHAPE;
  if (d->metric < CNNA_MATMUL || d->metric > CNNA_EUCLIDEAN) return CNNA_ERR_OPTION;
  if (d->conv < CNNA_CONV_STANDARD || d->conv > CNNA_CONV_DWSEP) return CNNA_ERR_OPTION;
  if (d->conv == CNNA_CONV_DEPTHWISE && d->coord) return CNNA_ERR_GROUPS;
  if (d->K < 1) return CNNA_ERR_K_RANGE;
  if (d->Nq < 0 || (!d->sampled && d->Nq != d->N)) return CNNA_ERR_SHAPE;
  if (ksel_of(d) > d->Nq) return CNNA_ERR_K_RANGE;
  if (d->merge != CNNA_MERGE_REFERENCE && d->merge != CNNA_MERGE_CONCAT) return CNNA_ERR_OPTION;
  if (d->scale != 0.0f && (d->metric != CNNA_MATMUL || !isfinite(d->scale))) return CNNA_ERR_OPTION;
  if (d->merge == CNNA_MERGE_REFERENCE && d->H > 1 && d->seq_length != d->N) return CNNA_ERR_SEQ_LENGTH;
  // the reference accepts these; the kernels' tiles do not
  const int dkp = dkp_of(d);
  if (dkp > 256) return CNNA_ERR_UNSUPPORTED;
  if (d->Nq > 65536) return CNNA_ERR_UNSUPPORTED;
  return CNNA_OK;
}

int cnna_head_stride(const cnna_desc* d) { return d ? dkp_of(d) : 0; }

}  // extern "C"

namespace {

// LayerNorm prologue of a GEMM over Kd-channel rows (NULL: none)
int set_ln(GemmArgs& g, const cnna_ln* ln) {
  if (ln == nullptr) return CNNA_OK;
  if (!ln->stats) return CNNA_ERR_NULL;
  if (((uintptr_t)ln->stats & 3) != 0) return CNNA_ERR_SHAPE;
  g.ln_stats = ln->stats;
  g.ln_parts = (g.Kd + ROW_STAT_TILE - 1) / ROW_STAT_TILE;
  g.ln_gamma = ln->gamma;
  g.ln_beta = ln->beta;
  g.ln_eps = ln->eps;
  return CNNA_OK;
}

int project_qkv_impl(const cnna_desc* d, const void* x, int64_t ldx, const cnna_ln* ln, const int32_t* cand,
                     const void* Wq, const void* Wk, const void* Wv, const void* bqkv, void* q, void* k,
                     void* v, float* qn, float* kn, void* stream) {
  int st = cnna_check_desc(d);
  if (st) return st;
  if (!x || !Wq || !Wk || !Wv || !q || !k || !v) return CNNA_ERR_NULL;
  if (d->sampled && !cand) return CNNA_ERR_NULL;
  if (d->metric == CNNA_EUCLIDEAN && (!qn || !kn)) return CNNA_ERR_NULL;
  if (ldx < d->C) return CNNA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int es = elem_size(d->dtype), dk = d->C / d->H, dkp = dkp_of(d);
  const int BH = d->B * d->H;

  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.Kd = d->C;
  g.a = x;
  g.lda = ldx;
  g.ncol_each = d->C;
  g.o_H = d->H;
  g.o_dk = dk;
  g.o_dkp = dkp;
  g.avec = ((ldx * es) % 16 == 0) && aligned16(x);
  g.bvec = ((d->C * es) % 16 == 0) && aligned16(Wq) && aligned16(Wk) && aligned16(Wv);
  if ((st = set_ln(g, ln))) return st;
  if (!d->sampled) {
    // one launch: [Q | K | V] = x @ [Wq; Wk; Wv]^T
    g.M = d->B * d->N;
    g.Nc = 3 * d->C;
    g.w[0] = Wq; g.w[1] = Wk; g.w[2] = Wv;
    g.o[0] = q; g.o[1] = k; g.o[2] = v;
    g.o_rows = d->N;
    g.bias = bqkv;
    if ((st = launch_gemm(d->dtype, GEMM_A_ROWS, GEMM_O_HEADSPLIT, g, s))) return st;
  } else {
    g.M = d->B * d->N;
    g.Nc = 2 * d->C;
    g.w[0] = Wk; g.w[1] = Wv;
    g.o[0] = k; g.o[1] = v;
    g.o_rows = d->N;
    g.bias = bqkv ? static_cast<const char*>(bqkv) + (size_t)d->C * es : nullptr;
    if ((st = launch_gemm(d->dtype, GEMM_A_ROWS, GEMM_O_HEADSPLIT, g, s))) return st;
    // Q on the sampled tokens x[:, cand, :] (layers.py:285-286, 298-299)
    g.M = d->B * d->Nq;
    g.Nc = d->C;
    g.w[0] = Wq; g.o[0] = q;
    g.bias = bqkv;
    g.arow = cand;
    g.a_rows = d->Nq;
    g.a_src_rows = d->N;
    g.o_rows = d->Nq;
    if (d->Nq > 0 && (st = launch_gemm(d->dtype, GEMM_A_ROWS, GEMM_O_HEADSPLIT, g, s))) return st;
  }
  // coordinate channel / padding / cosine normalisation / euclidean norms
  const bool pad = dkp != dk;
  const bool cos = d->metric == CNNA_COSINE, euc = d->metric == CNNA_EUCLIDEAN;
  PrepArgs p;
  memset(&p, 0, sizeof(p));
  p.dk = dk;
  p.dkp = dkp;
  p.coord = d->coord;
  if (pad || cos || euc) {
    p.t = k; p.rows = d->N; p.rows_total = BH * d->N; p.normalize = cos; p.norms = (euc || cos) ? kn : nullptr;
    if ((st = launch_prep(d->dtype, p, s))) return st;
    p.t = q; p.rows = d->Nq; p.rows_total = BH * d->Nq; p.normalize = cos; p.norms = (euc || cos) ? qn : nullptr;
    if ((st = launch_prep(d->dtype, p, s))) return st;
  }
  if (pad) {
    p.t = v; p.rows = d->N; p.rows_total = BH * d->N; p.normalize = 0; p.norms = nullptr;
    if ((st = launch_prep(d->dtype, p, s))) return st;
  }
  return CNNA_OK;
}

}  // namespace

extern "C" {

int cnna_project_qkv(const cnna_desc* d, const void* x, int64_t ldx, const int32_t* cand,
                     const void* Wq, const void* Wk, const void* Wv, void* q, void* k, void* v,
                     float* qn, float* kn, void* stream) {
  return project_qkv_impl(d, x, ldx, nullptr, cand, Wq, Wk, Wv, nullptr, q, k, v, qn, kn, stream);
}

int cnna_project_qkv_ex(const cnna_desc* d, const void* x, int64_t ldx, const cnna_ln* ln,
                        const int32_t* cand, const void* Wq, const void* Wk, const void* Wv,
                        const void* bqkv, void* q, void* k, void* v, float* qn, float* kn, void* stream) {
  return project_qkv_impl(d, x, ldx, ln, cand, Wq, Wk, Wv, bqkv, q, k, v, qn, kn, stream);
}

int cnna_select(const cnna_desc* d, const void* k, const void* q, const float* kn, const float* qn,
                const int32_t* cand, int32_t* idx, float* vals, float* w, int32_t* cols,
                void* stream) {
  int st = cnna_check_desc(d);
  if (st) return st;
  if (!k || !q || !idx || !vals) return CNNA_ERR_NULL;
  if (d->sampled && !cand) return CNNA_ERR_NULL;
  if (d->metric == CNNA_EUCLIDEAN && (!kn || !qn)) return CNNA_ERR_NULL;
  if (!aligned16(k) || !aligned16(q)) return CNNA_ERR_SHAPE;
  SelArgs a;
  memset(&a, 0, sizeof(a));
  a.k = k; a.q = q; a.kn = kn; a.qn = qn; a.cand = d->sampled ? cand : nullptr;
  a.idx = idx; a.vals = vals; a.w = w; a.cols = d->sampled ? cols : nullptr; a.softmax = d->softmax;
  a.BH = d->B * d->H; a.N = d->N; a.Nq = d->Nq; a.dkp = dkp_of(d);
  a.K = d->K; a.Ksel = ksel_of(d);
  a.rb_per_bh = (d->N + 127) / 128;
  // matmul: S = k.q / d_k**0.5 (layers.py:324); cosine inputs are normalised.
  // Raw keys rank the accumulator itself: a negative scale (KVT qk_scale)
  // ranks -k.q with the magnitude as the value scale.
  a.kscale = (d->metric == CNNA_MATMUL) ? matmul_scale(d) : 1.0f;
  if (d->metric == CNNA_MATMUL && !d->sampled && a.kscale < 0.0f) {
    a.kscale = -a.kscale;
    a.kneg = 1;
  }
  if (d->metric == CNNA_EUCLIDEAN) {
    a.mask_val = 1.1f;                         // INF (layers.py:234)
    a.mask_key = -(a.mask_val * a.mask_val);
  } else {
    a.mask_val = -0.1f;                        // NEG_INF (layers.py:235)
    a.mask_key = a.mask_val;
  }
  return launch_select(d->dtype, d->metric == CNNA_EUCLIDEAN, d->sampled, a, (hipStream_t)stream);
}

size_t cnna_aggregate_workspace(const cnna_desc* d) {
  if (cnna_check_desc(d)) return 0;
  const size_t es = elem_size(d->dtype), BH = (size_t)d->B * d->H;
  const size_t dk = d->C / d->H, din = din_of(d);
  if (d->conv == CNNA_CONV_DEPTHWISE) return 0;
  size_t n = cnna_round_up(BH * d->N * dk * es, 256);                      // y
  if (d->conv == CNNA_CONV_STANDARD) n += cnna_round_up(dk * din * d->K * es, 256);   // W0 permuted
  else n += cnna_round_up(BH * d->N * din * es, 256);                      // depthwise stage
  return n;
}

int cnna_aggregate(const cnna_desc* d, const void* v, const int32_t* idx, const float* w,
                   const void* conv_w0, const void* conv_w1, void* z, void* ws, size_t ws_bytes,
                   void* stream) {
  int st = cnna_check_desc(d);
  if (st) return st;
  if (!v || !idx || !w || !conv_w0 || !z) return CNNA_ERR_NULL;
  if (d->conv == CNNA_CONV_DWSEP && !conv_w1) return CNNA_ERR_NULL;
  const size_t need = cnna_aggregate_workspace(d);
  if (need > 0 && (!ws || ws_bytes < need)) return CNNA_ERR_WORKSPACE;
  if (need > 0 && !aligned16(ws)) return CNNA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int es = elem_size(d->dtype), BH = d->B * d->H, dk = d->C / d->H, din = din_of(d);
  const int dkp = dkp_of(d);
  AggArgs a;
  memset(&a, 0, sizeof(a));
  a.idx = idx; a.w = w; a.BH = BH; a.N = d->N; a.K = d->K; a.dkp = dkp; a.H = d->H; a.C = d->C;
  if (d->conv == CNNA_CONV_DEPTHWISE) {
    // y = depthwise conv over the gathered neighbours, written merged
    a.v = v; a.w0 = conv_w0; a.out = z; a.dout = dk; a.merged = merge_mode(d);
    return launch_aggregate(d->dtype, a, s);
  }
  char* p = static_cast<char*>(ws);
  void* y = p;
  p += cnna_round_up((size_t)BH * d->N * dk * es, 256);
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.M = BH * d->N;
  g.Nc = dk;
  g.ncol_each = dk;
  g.o[0] = y;
  g.ldo = dk;
  if (d->conv == CNNA_CONV_STANDARD) {
    // y = P @ W0p^T with P[m][r*din + c] = w[m, r] * v[idx[m, r], c] gathered in the A loader
    void* w0p = p;
    if ((st = launch_permute_w0(d->dtype, conv_w0, w0p, dk, din, d->K, s))) return st;
    g.Kd = din * d->K;
    g.a = v;
    g.g_idx = idx; g.g_w = w; g.g_K = d->K; g.g_N = d->N; g.g_din = din; g.g_dkp = dkp;
    g.avec = (din % (16 / es) == 0) && (dkp % (16 / es) == 0) && aligned16(v);
    g.w[0] = w0p;
    g.bvec = ((g.Kd * es) % 16 == 0);
    if ((st = launch_gemm(d->dtype, GEMM_A_GATHER, GEMM_O_PLAIN, g, s))) return st;
  } else {
    // depthwise stage (din channels) then the pointwise conv as a GEMM
    void* t1 = p;
    a.v = v; a.w0 = conv_w0; a.out = t1; a.dout = din; a.merged = MERGE_PLAIN;
    if ((st = launch_aggregate(d->dtype, a, s))) return st;
    g.Kd = din;
    g.a = t1;
    g.lda = din;
    g.avec = ((din * es) % 16 == 0);
    g.w[0] = conv_w1;
    g.bvec = ((din * es) % 16 == 0) && aligned16(conv_w1);
    if ((st = launch_gemm(d->dtype, GEMM_A_ROWS, GEMM_O_PLAIN, g, s))) return st;
  }
  // head merge of y into z
  a.v = y; a.out = z; a.dout = dk; a.merged = merge_mode(d); a.w0 = nullptr;
  return launch_merge(d->dtype, a, s);
}

int cnna_output_proj(const cnna_desc* d, const void* z, const void* Wo, void* out, int64_t ldo,
                     void* stream) {
  int st = cnna_check_desc(d);
  if (st) return st;
  if (!z || !Wo || !out) return CNNA_ERR_NULL;
  if (ldo < d->C) return CNNA_ERR_SHAPE;
  const int es = elem_size(d->dtype);
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.M = d->B * d->N;
  g.Nc = d->C;
  g.Kd = d->C;
  g.a = z;
  g.lda = d->C;
  g.avec = ((d->C * es) % 16 == 0) && aligned16(z);
  g.w[0] = Wo;
  g.ncol_each = d->C;
  g.bvec = ((d->C * es) % 16 == 0) && aligned16(Wo);
  g.o[0] = out;
  g.ldo = ldo;
  return launch_gemm(d->dtype, GEMM_A_ROWS, GEMM_O_PLAIN, g, (hipStream_t)stream);
}

int cnna_layernorm(int32_t dtype, int64_t rows, int32_t C, const void* x, int64_t ldx, const void* res,
                   int64_t ldr, void* sum_out, int64_t ld_sum, const void* gamma, const void* beta,
                   float eps, void* y, int64_t ldy, void* stream) {
  if (dtype != CNNA_F32 && dtype != CNNA_BF16 && dtype != CNNA_F16) return CNNA_ERR_DTYPE;
  if (rows < 0 || C <= 0 || C > 1024 || ldx < C || ldy < C || (res && ldr < C) || (sum_out && ld_sum < C))
    return CNNA_ERR_SHAPE;
  if (rows > 0 && (!x || !y)) return CNNA_ERR_NULL;
  LnArgs a;
  memset(&a, 0, sizeof(a));
  a.x = x;
  a.ldx = ldx;
  a.res = res;
  a.ldr = ldr;
  a.sum_out = sum_out;
  a.lds = ld_sum;
  a.gamma = gamma;
  a.beta = beta;
  a.eps = eps;
  a.y = y;
  a.ldy = ldy;
  a.rows = rows;
  a.C = C;
  return launch_layernorm(dtype, a, (hipStream_t)stream);
}

int cnna_row_stats(int32_t dtype, int64_t rows, int32_t C, const void* x, int64_t ldx, float* stats,
                   void* stream) {
  if (dtype != CNNA_F32 && dtype != CNNA_BF16 && dtype != CNNA_F16) return CNNA_ERR_DTYPE;
  if (rows < 0 || C <= 0 || ldx < C) return CNNA_ERR_SHAPE;
  if (rows == 0) return 0;
  if (!x || !stats) return CNNA_ERR_NULL;
  if (((uintptr_t)stats & 7) != 0) return CNNA_ERR_SHAPE;
  LnArgs a;
  memset(&a, 0, sizeof(a));
  a.x = x;
  a.ldx = ldx;
  a.rows = rows;
  a.C = C;
  a.stats = stats;
  return launch_layernorm(dtype, a, (hipStream_t)stream);
}

int cnna_linear(int32_t dtype, int64_t M, int32_t Nout, int32_t Kd, const void* a, int64_t lda,
                const void* W, const void* bias, int32_t act, const void* res, int64_t ldr, void* out,
                int64_t ldo, void* stream) {
  return cnna_linear_ln(dtype, M, Nout, Kd, a, lda, nullptr, W, bias, act, res, ldr, out, ldo, nullptr,
                        stream);
}

int cnna_linear_ln(int32_t dtype, int64_t M, int32_t Nout, int32_t Kd, const void* a, int64_t lda,
                   const cnna_ln* ln, const void* W, const void* bias, int32_t act, const void* res,
                   int64_t ldr, void* out, int64_t ldo, float* stats_out, void* stream) {
  if (dtype != CNNA_F32 && dtype != CNNA_BF16 && dtype != CNNA_F16) return CNNA_ERR_DTYPE;
  if (act != CNNA_ACT_NONE && act != CNNA_ACT_GELU) return CNNA_ERR_OPTION;
  if (M < 0 || M > INT32_MAX || Nout <= 0 || Kd <= 0 || lda < Kd || ldo < Nout || (res && ldr < Nout))
    return CNNA_ERR_SHAPE;
  if (M == 0) return 0;
  if (!a || !W || !out) return CNNA_ERR_NULL;
  const int es = elem_size(dtype);
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.M = (int)M;
  g.Nc = Nout;
  g.Kd = Kd;
  g.a = a;
  g.lda = lda;
  g.avec = ((Kd * es) % 16 == 0) && ((lda * es) % 16 == 0) && aligned16(a);
  g.w[0] = W;
  g.ncol_each = Nout;
  g.bvec = ((Kd * es) % 16 == 0) && aligned16(W);
  g.o[0] = out;
  g.ldo = ldo;
  g.bias = bias;
  g.act = act == CNNA_ACT_GELU ? GEMM_ACT_GELU : GEMM_ACT_NONE;
  g.res = res;
  g.ldr = ldr;
  int st = set_ln(g, ln);
  if (st) return st;
  if (stats_out != nullptr && ((uintptr_t)stats_out & 7) != 0) return CNNA_ERR_SHAPE;
  g.st_out = stats_out;
  return launch_gemm(dtype, GEMM_A_ROWS, GEMM_O_PLAIN, g, (hipStream_t)stream);
}

size_t cnna_forward_workspace(const cnna_desc* d) {
  if (cnna_check_desc(d)) return 0;
  const size_t es = elem_size(d->dtype), dkp = dkp_of(d), BH = (size_t)d->B * d->H;
  size_t n = 0;
  n += cnna_round_up(BH * d->Nq * dkp * es, 256);         // q
  n += 2 * cnna_round_up(BH * d->N * dkp * es, 256);      // k, v
  n += cnna_round_up(BH * d->Nq * 4, 256);                // qn
  n += cnna_round_up(BH * d->N * 4, 256);                 // kn
  n += 3 * cnna_round_up(BH * d->N * d->K * 4, 256);      // idx, vals, w
  n += cnna_round_up((size_t)d->B * d->N * d->C * es, 256);   // z
  n += cnna_aggregate_workspace(d);
  return n;
}

int cnna_forward(const cnna_desc* d, const void* x, int64_t ldx, const int32_t* cand, const void* Wq,
                 const void* Wk, const void* Wv, const void* Wo, const void* conv_w0,
                 const void* conv_w1, void* out, int64_t ldo, void* ws, size_t ws_bytes,
                 void* stream) {
  int st = cnna_check_desc(d);
  if (st) return st;
  if (!ws) return CNNA_ERR_NULL;
  if (ws_bytes < cnna_forward_workspace(d)) return CNNA_ERR_WORKSPACE;
  if (!aligned16(ws)) return CNNA_ERR_SHAPE;
  const size_t es = elem_size(d->dtype), dkp = dkp_of(d), BH = (size_t)d->B * d->H;
  char* p = static_cast<char*>(ws);
  auto take = [&](size_t bytes) { void* r = p; p += cnna_round_up(bytes, 256); return r; };
  void* q = take(BH * d->Nq * dkp * es);
  void* k = take(BH * d->N * dkp * es);
  void* v = take(BH * d->N * dkp * es);
  float* qn = static_cast<float*>(take(BH * d->Nq * 4));
  float* kn = static_cast<float*>(take(BH * d->N * 4));
  int32_t* idx = static_cast<int32_t*>(take(BH * d->N * d->K * 4));
  float* vals = static_cast<float*>(take(BH * d->N * d->K * 4));
  float* w = static_cast<float*>(take(BH * d->N * d->K * 4));
  void* z = take((size_t)d->B * d->N * d->C * es);
  const size_t agg_ws = cnna_aggregate_workspace(d);
  void* aws = take(agg_ws);
  const bool euc = d->metric == CNNA_EUCLIDEAN;
  if ((st = cnna_project_qkv(d, x, ldx, cand, Wq, Wk, Wv, q, k, v, euc ? qn : nullptr,
                             euc ? kn : nullptr, stream)))
    return st;
  if ((st = cnna_select(d, k, q, euc ? kn : nullptr, euc ? qn : nullptr, cand, idx, vals, w, nullptr,
                        stream)))
    return st;
  if ((st = cnna_aggregate(d, v, idx, w, conv_w0, conv_w1, z, aws, agg_ws, stream))) return st;
  return cnna_output_proj(d, z, Wo, out, ldo, stream);
}

}  // extern "C"
