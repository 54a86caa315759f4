// C-ABI of the branching callers' Conv1d branch (declared in include/cnna.h).
//
// MultiHeadConv1dAttention (layers.py:452-499), the sibling of the ConvNN
// branch in MultiHeadBranchingConv (layers.py:502-600), inference path:
//   u = x @ Wx^T + bx                               W_x (layers.py:463, 495)
//   y = Conv1d(d_k, d_k, ks, 'same') per head         split_head / batch_combine / conv (:476-497)
//   z = the token-mixing merge of y                   permute / batch_split / combine_heads (:483-497)
//   out = z @ Wo^T + bo                               W_o (layers.py:464, 497)
#include <string.h>

#include "common.h"
#include "kernels.h"

#include "desc_util.h"

using namespace cnna_desc_util;

namespace {

bool conv1d_shape_ok(int32_t dtype, int32_t B, int32_t N, int32_t C, int32_t H, int32_t ks) {
  (void)dtype;
  return B > 0 && N > 0 && C > 0 && H > 0 && C % H == 0 && ks > 0 && ks <= 33 &&
         (int64_t)B * N * C <= INT32_MAX;
}

}  // namespace

extern "C" {

size_t cnna_conv1d_branch_workspace(int32_t dtype, int32_t B, int32_t N, int32_t C, int32_t H,
                                    int32_t ks) {
  const int es = elem_size(dtype);
  if (!es || !conv1d_shape_ok(dtype, B, N, C, H, ks)) return 0;
  return 3 * cnna_round_up((size_t)B * N * C * es, 256) +   // u, y, z
         cnna_round_up(conv1d_wprep_bytes(C / H, ks), 256);  // conv weights, fp32 [c][o][taps]
}

int cnna_conv1d_branch(int32_t dtype, int32_t B, int32_t N, int32_t C, int32_t H, int32_t ks,
                       const void* x, int64_t ldx, const void* Wx, const void* bx,
                       const void* conv_w, const void* conv_b, const void* Wo, const void* bo,
                       void* out, int64_t ldo, void* ws, size_t ws_bytes, void* stream) {
  const int es = elem_size(dtype);
  if (!es) return CNNA_ERR_DTYPE;
  if (!conv1d_shape_ok(dtype, B, N, C, H, ks) || ldx < C || ldo < C) return CNNA_ERR_SHAPE;
  if (!x || !Wx || !conv_w || !Wo || !out || !ws) return CNNA_ERR_NULL;
  if (ws_bytes < cnna_conv1d_branch_workspace(dtype, B, N, C, H, ks)) return CNNA_ERR_WORKSPACE;
  if (!aligned16(ws)) return CNNA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int dk = C / H;
  Carve cv(ws);
  void* u = cv.take((size_t)B * N * C * es);
  void* y = cv.take((size_t)B * N * C * es);
  void* z = cv.take((size_t)B * N * C * es);
  const size_t wpb = conv1d_wprep_bytes(dk, ks);
  float* wprep = static_cast<float*>(cv.take(wpb));
  int st;
  if ((st = cnna_linear(dtype, (int64_t)B * N, C, C, x, ldx, Wx, bx, CNNA_ACT_NONE, nullptr, 0, u, C,
                        stream)))
    return st;
  Conv1dArgs c;
  memset(&c, 0, sizeof(c));
  c.u = u; c.ldu = C; c.w = conv_w; c.bias = conv_b; c.y = y;
  c.B = B; c.N = N; c.H = H; c.dk = dk; c.ks = ks;
  c.padl = (ks - 1) / 2;                 // torch 'same': the odd extra zero goes behind
  c.wprep = wprep; c.wprep_bytes = wpb;
  if ((st = launch_conv1d_tokens(dtype, c, s))) return st;
  AggArgs a;
  memset(&a, 0, sizeof(a));
  a.v = y; a.out = z; a.BH = B * H; a.N = N; a.dout = dk; a.dkp = dk; a.H = H; a.C = C;
  a.merged = MERGE_MIX;
  if ((st = launch_merge(dtype, a, s))) return st;
  return cnna_linear(dtype, (int64_t)B * N, C, C, z, C, Wo, bo, CNNA_ACT_NONE, nullptr, 0, out, ldo,
                     stream);
}

}  // extern "C"
