/* C-ABI of the MI355X (gfx950) ConvNN-Attention library, libcnna.so.
 *
 * The reference operator is the Python class MultiHeadConvNNAttention
 * (layers.py:132-450 of mingikang31/Convolutional-Nearest-Neighbor-Attention);
 * it has no FFI of its own.  Each entry point below replaces one stage of its
 * forward (layers.py:261-321) or the autograd backward of those stages.
 *
 * Conventions
 *  - Every pointer is device memory owned by the caller; the library never
 *    allocates or frees device memory and never synchronises the stream.
 *  - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *  - Return value: 0 ok; negative = invalid argument (cnna_error_string);
 *    positive = hipError_t of a failed launch.
 *  - Tensors are row-major.  "Head-split" tensors are (B*H, rows, dkp):
 *    token-major per head, dkp = cnna_head_stride(desc) channels of which the
 *    first d_k (+1 with coordinate encoding) are used and the rest are zero.
 *  - idx is int32 token indices (B*H, N, K); vals is fp32 (B*H, N, K) holding
 *    the selected similarity values (for sampled paths slot 0 is the token
 *    itself with value 1.0, layers.py:369-376).
 */
#ifndef CNNA_H
#define CNNA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CNNA_ABI_VERSION 4

/* Storage and product type; every kernel accumulates in fp32 (the MFMA
 * instructions' accumulators) and rounds to nearest-even when it stores.
 * CNNA_F16 serves torch.autocast(dtype=torch.float16), the reference's AMP
 * default (train_eval.py:137-146). */
enum cnna_dtype { CNNA_F32 = 0, CNNA_BF16 = 1, CNNA_F16 = 2 };
/* magnitude_type (layers.py:167-168, 323-340) */
enum cnna_metric { CNNA_MATMUL = 0, CNNA_COSINE = 1, CNNA_EUCLIDEAN = 2 };
/* convolution_type (layers.py:186-228) */
enum cnna_conv { CNNA_CONV_STANDARD = 0, CNNA_CONV_DEPTHWISE = 1, CNNA_CONV_DWSEP = 2 };
/* Head layout of the aggregated tensor z:
 *   REFERENCE  the operator's own merge (layers.py:247-259, 316-317)
 *   CONCAT     heads side by side, z[b, t, h*d_k + c] = y[b*H + h][t][c]: the
 *              (attn @ v).transpose(1, 2).reshape(B, N, C) of
 *              MultiHeadKvtAttention (layers.py:681) */
enum cnna_merge { CNNA_MERGE_REFERENCE = 0, CNNA_MERGE_CONCAT = 1 };

enum cnna_status {
  CNNA_OK = 0,
  CNNA_ERR_NULL = -1,         /* required pointer is NULL */
  CNNA_ERR_SHAPE = -2,        /* inconsistent or unsupported sizes */
  CNNA_ERR_DTYPE = -3,        /* unknown dtype */
  CNNA_ERR_OPTION = -4,       /* unknown metric / conv / option combination */
  CNNA_ERR_K_RANGE = -5,      /* K larger than the candidates (torch.topk RuntimeError) */
  CNNA_ERR_SEQ_LENGTH = -6,   /* seq_length != N with num_heads > 1 (layers.py:251) */
  CNNA_ERR_WORKSPACE = -7,    /* workspace too small */
  CNNA_ERR_GROUPS = -8,       /* depthwise with coordinate encoding (Conv1d ValueError) */
  CNNA_ERR_UNSUPPORTED = -9,  /* a valid reference configuration beyond this library's limits
                                 (cnna_error_string names the limit) */
  CNNA_ERR_SCRATCH = -10      /* the call needs more than the static scratch of
                                 cnna_forward_noalloc (CNNA_NOALLOC_SCRATCH_BYTES) */
};

/* Operator configuration: the constructor arguments of layers.py:133-146
 * plus the call's shapes. */
typedef struct cnna_desc {
  int32_t B;            /* batch */
  int32_t N;            /* tokens (x.shape[1]) */
  int32_t C;            /* d_hidden */
  int32_t H;            /* num_heads */
  int32_t Nq;           /* candidates: N for sampling 'all', num_samples otherwise */
  int32_t K;            /* neighbours per token (self included for sampled paths) */
  int32_t seq_length;   /* constructor seq_length; must equal N when H > 1 */
  int32_t dtype;        /* enum cnna_dtype */
  int32_t metric;       /* enum cnna_metric */
  int32_t conv;         /* enum cnna_conv */
  int32_t softmax;      /* softmax_topk_val */
  int32_t sampled;      /* 1 for 'random' / 'spatial' (layers.py:283-307) */
  int32_t coord;        /* coordinate_encoding (layers.py:269-270, 439-450) */
  int32_t merge;        /* enum cnna_merge, 0 = the operator's own */
  float scale;          /* matmul similarity scale; 0 = 1/sqrt(d_k) (layers.py:324) */
} cnna_desc;

/* MultiHeadKvtAttention (layers.py:654-686) is this operator with
 *   metric MATMUL, conv DEPTHWISE with unit weights (d_k, 1, K) of ones,
 *   softmax 1, sampled 0, K = topk, merge CONCAT, scale = its self.scale,
 *   Wq := qkv.weight[C:2C] (its keys are the candidates, layers.py:672),
 *   Wk := qkv.weight[0:C]  (its queries are the rows that choose),
 *   Wv := qkv.weight[2C:3C], Wo := proj.weight:
 * softmax over the topk largest q_i . k_j * scale of each row equals its
 * dense row with the rest masked to -inf (layers.py:674-679). */

int cnna_abi_version(void);
const char* cnna_error_string(int code);

/* Validate a descriptor (the checks the reference performs at construction
 * and call time, layers.py:149, 251, 310, 344/365, Conv1d groups). */
int cnna_check_desc(const cnna_desc* d);

/* Channel stride dkp of head-split tensors for this descriptor. */
int cnna_head_stride(const cnna_desc* d);

/* Q/K/V projections + head split (layers.py:264-265, 274, 286, 299 and
 * split_head/batch_combine layers.py:237-245), plus coordinate channel and
 * cosine normalisation / euclidean squared norms (layers.py:327-340, 439-450).
 *   x    (B, N, C) with row stride ldx elements (channels contiguous)
 *   cand (Nq) int32 sampled token indices, NULL for 'all'
 *   W*   (C, C) nn.Linear weights [out, in]
 *   q    (B*H, Nq, dkp); k, v (B*H, N, dkp)
 *   qn, kn  fp32 squared norms (B*H*Nq), (B*H*N) of the rows before
 *           normalisation: required for euclidean, optional for cosine (the
 *           backward needs them), else NULL */
int cnna_project_qkv(const cnna_desc* d, const void* x, int64_t ldx, const int32_t* cand,
                     const void* Wq, const void* Wk, const void* Wv,
                     void* q, void* k, void* v, float* qn, float* kn, void* stream);

/* Fused similarity + streaming top-k (layers.py:323-340 then torch.topk in
 * _prime/_prime_softmax/_prime_N/_prime_softmax_N, layers.py:344, 363, 391,
 * 410, with the sampled self mask layers.py:291-292, 304-305).  The N x Nq
 * similarity matrix is never written.  Ties break by lowest candidate index.
 * Also writes the neighbour weights w (softmax of the values, or the raw
 * values / 1/(value + 1e-8) without softmax) when w is not NULL, and for
 * sampled paths the candidate column of each entry, cols (B*H, N, K) int32
 * (slot 0, the token itself: Nq), when cols is not NULL: several columns can
 * hold one token (spatial linspace with more samples than tokens), and with
 * coordinate encoding their q rows differ; the backward needs the column. */
int cnna_select(const cnna_desc* d, const void* k, const void* q, const float* kn, const float* qn,
                const int32_t* cand, int32_t* idx, float* vals, float* w, int32_t* cols,
                void* stream);

/* V gather and the Conv1d(kernel=K, stride=K) over the neighbours
 * (layers.py:346-358, 378-386, 393-405, 425-436, 313), then the head merge
 * (layers.py:316-317, 247-259), producing the tensor that enters W_o.
 *   w       (B*H, N, K) neighbour weights from cnna_select
 *   conv_w0 standard (d_k, d_in, K) / depthwise (d_k, 1, K) / dw part (d_in, 1, K)
 *   conv_w1 pointwise (d_k, d_in, 1) for depthwise-separable, else NULL
 *   z       (B, N, C) merged:  z[b, t, h*d_k + a] = y[b*H + h][f] with f = a*N + t
 *           over the token-major flat conv output y (H == 1: a transpose)
 *   ws      cnna_aggregate_workspace(d) bytes (0 for depthwise) */
size_t cnna_aggregate_workspace(const cnna_desc* d);
int cnna_aggregate(const cnna_desc* d, const void* v, const int32_t* idx, const float* w,
                   const void* conv_w0, const void* conv_w1, void* z, void* ws, size_t ws_bytes,
                   void* stream);

/* Output projection W_o (layers.py:320):  out = z @ Wo^T.
 *   out (B, N, C) with row stride ldo elements */
int cnna_output_proj(const cnna_desc* d, const void* z, const void* Wo, void* out, int64_t ldo,
                     void* stream);

/* Bytes of workspace cnna_forward needs for this descriptor. */
size_t cnna_forward_workspace(const cnna_desc* d);

/* Whole forward of MultiHeadConvNNAttention in eval mode (dropout identity):
 * the four stages above on one stream, intermediates in `ws`. */
int cnna_forward(const cnna_desc* d, const void* x, int64_t ldx, const int32_t* cand,
                 const void* Wq, const void* Wk, const void* Wv, const void* Wo,
                 const void* conv_w0, const void* conv_w1, void* out, int64_t ldo,
                 void* ws, size_t ws_bytes, void* stream);

/* Size of the file-scope device array cnna_forward_noalloc works in. */
#define CNNA_NOALLOC_SCRATCH_BYTES (128u << 20)

/* cnna_forward without a workspace argument, for callers that cannot
 * allocate device memory (HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference (its forward is
 * eager PyTorch that allocates every intermediate, layers.py:261-321).
 * The intermediates live in a static device array of
 * CNNA_NOALLOC_SCRATCH_BYTES per GPU, held from the first call until the
 * process ends; it allocates and frees nothing.  Returns CNNA_ERR_SCRATCH
 * when cnna_forward_workspace(d) exceeds that size (c3, B=32 N=1024 C=384 in
 * bf16, needs 112 MB).  Calls on one GPU share the array: calls that overlap
 * on one GPU race; results are those of cnna_forward. */
int cnna_forward_noalloc(const cnna_desc* d, const void* x, int64_t ldx, const int32_t* cand,
                         const void* Wq, const void* Wk, const void* Wv, const void* Wo,
                         const void* conv_w0, const void* conv_w1, void* out, int64_t ldo,
                         void* stream);

/* ------------------------------------------------------------ backward
 * Autograd of the stages above (what loss.backward() computes through
 * layers.py:261-450).  The reference differentiates the dense (B*H, N, Nq)
 * similarity matrix; these entry points only touch the K selected entries
 * of each row.  All sums run in a fixed order: results are deterministic. */

/* Tensors saved by the forward stages (outputs of cnna_project_qkv and
 * cnna_select). qn/kn are required for cosine and euclidean. */
typedef struct cnna_saved {
  const void* q;
  const void* k;
  const void* v;
  const float* qn;
  const float* kn;
  const int32_t* idx;
  const float* vals;
  const float* w;
  /* per-entry multipliers (B*H, N, K) the forward applied to w before the
   * aggregation (dropout on the attention probabilities: 0 or 1/(1-p),
   * layers.py:680), or NULL; depthwise conv only */
  const float* wmul;
  /* sampled paths: the cols output of cnna_select (required), else NULL */
  const int32_t* cols;
} cnna_saved;

/* Gradients written by cnna_core_backward, dtype of the descriptor.
 *   dx (B, N, C) contiguous; dWq, dWk, dWv (C, C); dconv_w0 / dconv_w1 shaped
 *   like conv_w0 / conv_w1 (dconv_w1 only for depthwise-separable). */
typedef struct cnna_grads {
  void* dx;
  void* dWq;
  void* dWk;
  void* dWv;
  void* dconv_w0;
  void* dconv_w1;
  /* (3C) [dbq | dbk | dbv]: gradient of the projection biases of
   * cnna_project_qkv_ex (MultiHeadKvtAttention's qkv_bias, layers.py:662), or
   * NULL when the projections have no bias */
  void* dbqkv;
} cnna_grads;

/* Backward of cnna_output_proj (nn.Linear W_o, layers.py:320):
 *   dz = dout @ Wo,  dWo = dout^T @ z.   dout (B, N, C) row stride ld_dout;
 *   z, dz (B, N, C) contiguous; dWo (C, C). */
size_t cnna_output_proj_backward_workspace(const cnna_desc* d);
int cnna_output_proj_backward(const cnna_desc* d, const void* z, const void* Wo, const void* dout,
                              int64_t ld_dout, void* dz, void* dWo, void* ws, size_t ws_bytes,
                              void* stream);

/* Backward of cnna_project_qkv + cnna_select + cnna_aggregate: from dz, the
 * gradient at the input of W_o (B, N, C contiguous), to x, W_q, W_k, W_v and
 * the conv weights.  Covers the head merge (layers.py:247-259, 316-317), the
 * conv (layers.py:313), the weights of _prime/_prime_softmax/_prime_N/
 * _prime_softmax_N (layers.py:342-437, softmax backward and the self-slot /
 * self-mask constants), the similarity (layers.py:323-340) and the projections
 * (layers.py:264-265, 274, 286, 299). */
size_t cnna_core_backward_workspace(const cnna_desc* d);
int cnna_core_backward(const cnna_desc* d, const void* x, int64_t ldx, const int32_t* cand,
                       const void* Wq, const void* Wk, const void* Wv, const void* conv_w0,
                       const void* conv_w1, const cnna_saved* saved, const void* dz,
                       const cnna_grads* grads, void* ws, size_t ws_bytes, void* stream);

/* ---- ViT block around the operator (vit.py:247-269), inference path ----
 * Activation codes for cnna_linear. */
enum cnna_act { CNNA_ACT_NONE = 0, CNNA_ACT_GELU = 1 };

/* nn.LayerNorm(C) over the last dimension (vit.py:247-248, applied at
 * vit.py:262 and 267), optionally with the residual add in front of it
 * (x + attention output, vit.py:264):  s = x + res (rounded to dtype, written
 * to sum_out when not NULL), y = (s - mean) / sqrt(var + eps) * gamma + beta.
 * rows x C with row strides in elements; res, sum_out, gamma, beta may be NULL
 * (no residual / not written / 1 / 0).  C <= 1024. */
int cnna_layernorm(int32_t dtype, int64_t rows, int32_t C, const void* x, int64_t ldx, const void* res,
                   int64_t ldr, void* sum_out, int64_t ld_sum, const void* gamma, const void* beta,
                   float eps, void* y, int64_t ldy, void* stream);

/* nn.Linear with the epilogues of the ViT block fused:
 *   out = act(a @ W^T + bias) + res
 * the MLP (nn.Linear -> nn.GELU -> nn.Linear, vit.py:253-257) with its residual
 * (vit.py:269), and W_o followed by the attention residual (vit.py:263-264).
 * a (M, Kd) row stride lda; W (Nout, Kd) contiguous; bias (Nout) or NULL;
 * act CNNA_ACT_*; res (M, Nout) row stride ldr or NULL; out (M, Nout) row
 * stride ldo.  For bf16 the biased value is rounded before the activation and
 * before the residual add, as the unfused modules round their outputs. */
int cnna_linear(int32_t dtype, int64_t M, int32_t Nout, int32_t Kd, const void* a, int64_t lda,
                const void* W, const void* bias, int32_t act, const void* res, int64_t ldr, void* out,
                int64_t ldo, void* stream);

/* LayerNorm folded into the GEMM that consumes it (the pre-norm block,
 * vit.py:260-267: norm1 -> attention's W_q/W_k/W_v, norm2 -> fc1).
 * nn.LayerNorm's two steps are split between two kernels:
 *  - the statistics, written by the kernel that produces the rows: the
 *    statistics epilogue of cnna_linear_ln (W_o + residual, fc2 + residual)
 *    or, for the first block, cnna_row_stats;
 *  - the normalisation (x - mean) / sqrt(var + eps) * gamma + beta, rounded to
 *    the dtype as nn.LayerNorm's output is, applied by the consuming GEMM
 *    (cnna_linear_ln, cnna_project_qkv_ex) as it loads each row.
 * The statistics are fp32 partials, stats[(row * CNNA_STAT_PARTS(C) + t) * 2
 * + {0, 1}] = the mean and the sum of squared deviations from that mean of the
 * row's columns [128 t, min(128 (t + 1), C)); mean and var (biased, as
 * nn.LayerNorm) of the row are combined from them. */
#define CNNA_STAT_TILE 128
#define CNNA_STAT_PARTS(C) (((C) + CNNA_STAT_TILE - 1) / CNNA_STAT_TILE)

typedef struct cnna_ln {
  const float* stats;   /* partials of the GEMM's A rows (indexed by A row) */
  const void* gamma;    /* (C) LayerNorm weight, or NULL (1) */
  const void* beta;     /* (C) LayerNorm bias, or NULL (0) */
  float eps;
} cnna_ln;

/* Statistics partials of x (rows, C) row stride ldx into stats (8-byte
 * aligned, rows * CNNA_STAT_PARTS(C) * 2 floats). */
int cnna_row_stats(int32_t dtype, int64_t rows, int32_t C, const void* x, int64_t ldx, float* stats,
                   void* stream);

/* cnna_linear with the LayerNorm of a folded in (ln; C = Kd) and, when
 * stats_out is not NULL, the statistics partials of the stored out rows
 * ((M, CNNA_STAT_PARTS(Nout), 2), 8-byte aligned).  The statistics epilogue
 * needs bfloat16, Nout % 8 == 0 and 16-byte aligned out / res with row strides
 * that are multiples of 8 elements (else CNNA_ERR_UNSUPPORTED).  ln may be
 * NULL (no prologue). */
int cnna_linear_ln(int32_t dtype, int64_t M, int32_t Nout, int32_t Kd, const void* a, int64_t lda,
                   const cnna_ln* ln, const void* W, const void* bias, int32_t act, const void* res,
                   int64_t ldr, void* out, int64_t ldo, float* stats_out, void* stream);

/* cnna_project_qkv with two optional extras:
 *  ln    LayerNorm(x) instead of x (vit.py:262 feeding layers.py:264-265): the
 *        rows of x are normalised (C = d->C; stats indexed by the row b * N + t
 *        of x, also for the sampled Q rows) as the projection GEMM loads them;
 *        NULL: x itself;
 *  bqkv  (3C) [bq | bk | bv] biases added to the projections (nn.Linear with
 *        bias: MultiHeadKvtAttention's qkv_bias, layers.py:662, in this
 *        operator's role order); NULL: none. */
int cnna_project_qkv_ex(const cnna_desc* d, const void* x, int64_t ldx, const cnna_ln* ln,
                        const int32_t* cand, const void* Wq, const void* Wk, const void* Wv,
                        const void* bqkv, void* q, void* k, void* v, float* qn, float* kn, void* stream);

/* ---- branching callers (layers.py:502-652) ----
 * MultiHeadConv1dAttention (layers.py:452-499), the Conv1d branch of
 * MultiHeadBranchingConv, inference path:
 *   u = x @ Wx^T + bx;  per head, Conv1d(d_k, d_k, ks, stride 1, padding
 *   'same', weights conv_w (d_k, d_k, ks), bias conv_b) along the tokens;
 *   the token-mixing reshape of layers.py:483-497, z[b, t, h*d_k + a] =
 *   y[b*H + h][f] over the flat token-major conv output, f = a*N + t, for
 *   every H;  out = z @ Wo^T + bo.
 * x (B, N, C) row stride ldx; out row stride ldo (a channel slice of a wider
 * tensor: the concatenation of layers.py:596-597 without a copy).  bx,
 * conv_b, bo may be NULL; ks <= 33.  ws: cnna_conv1d_branch_workspace bytes. */
size_t cnna_conv1d_branch_workspace(int32_t dtype, int32_t B, int32_t N, int32_t C, int32_t H,
                                    int32_t ks);
int cnna_conv1d_branch(int32_t dtype, int32_t B, int32_t N, int32_t C, int32_t H, int32_t ks,
                       const void* x, int64_t ldx, const void* Wx, const void* bx,
                       const void* conv_w, const void* conv_b, const void* Wo, const void* bo,
                       void* out, int64_t ldo, void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CNNA_H */
