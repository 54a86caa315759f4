"""ctypes binding of libcnna.so and the autograd functions of the operator.

The library is loaded from this directory; importing this module fails loudly
when it is missing (there is no CPU or eager-PyTorch fallback).  Launches go
on ``torch.cuda.current_stream()``; outputs and workspaces are allocated by
PyTorch's caching allocator and handed to the C-ABI as raw pointers.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import List, Optional, Tuple

import torch
from torch.utils._python_dispatch import _get_current_dispatch_mode

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcnna.so")

CNNA_F32, CNNA_BF16, CNNA_F16 = 0, 1, 2
METRICS = {"matmul": 0, "cosine": 1, "euclidean": 2}
CONVS = {"standard": 0, "depthwise": 1, "depthwise-separable": 2}
MERGE_REFERENCE, MERGE_CONCAT = 0, 1

ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_OPTION, ERR_K_RANGE, ERR_SEQ, ERR_WS, ERR_GROUPS, ERR_UNSUPPORTED = (
    -1, -2, -3, -4, -5, -6, -7, -8, -9)
ERR_SCRATCH = -10
NOALLOC_SCRATCH_BYTES = 128 << 20    # CNNA_NOALLOC_SCRATCH_BYTES
STAT_TILE = 128                      # CNNA_STAT_TILE: columns per row-statistics partial


class Desc(ctypes.Structure):
    """Mirror of ``cnna_desc`` in include/cnna.h."""

    _fields_ = [(n, ctypes.c_int32) for n in (
        "B", "N", "C", "H", "Nq", "K", "seq_length", "dtype", "metric", "conv",
        "softmax", "sampled", "coord", "merge")] + [("scale", ctypes.c_float)]


class Saved(ctypes.Structure):
    """Mirror of ``cnna_saved``."""

    _fields_ = [(n, ctypes.c_void_p) for n in ("q", "k", "v", "qn", "kn", "idx", "vals", "w", "wmul",
                                               "cols")]


class Grads(ctypes.Structure):
    """Mirror of ``cnna_grads``."""

    _fields_ = [(n, ctypes.c_void_p) for n in ("dx", "dWq", "dWk", "dWv", "dconv_w0", "dconv_w1", "dbqkv")]


class Ln(ctypes.Structure):
    """Mirror of ``cnna_ln``: a LayerNorm folded into the GEMM that loads its rows."""

    _fields_ = [("stats", ctypes.c_void_p), ("gamma", ctypes.c_void_p), ("beta", ctypes.c_void_p),
                ("eps", ctypes.c_float)]


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libcnna.so not found at {LIB_PATH}; build it with "
            "`python convolutional-nearest-neighbor-attention_amd/build.py` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    D = ctypes.POINTER(Desc)
    sigs = {
        "cnna_abi_version": ([], I32),
        "cnna_error_string": ([I32], ctypes.c_char_p),
        "cnna_check_desc": ([D], I32),
        "cnna_head_stride": ([D], I32),
        "cnna_project_qkv": ([D, P, I64, P, P, P, P, P, P, P, P, P, P], I32),
        "cnna_select": ([D, P, P, P, P, P, P, P, P, P, P], I32),
        "cnna_aggregate_workspace": ([D], ctypes.c_size_t),
        "cnna_aggregate": ([D, P, P, P, P, P, P, P, ctypes.c_size_t, P], I32),
        "cnna_output_proj": ([D, P, P, P, I64, P], I32),
        "cnna_forward_workspace": ([D], ctypes.c_size_t),
        "cnna_forward": ([D, P, I64, P, P, P, P, P, P, P, P, I64, P, ctypes.c_size_t, P], I32),
        "cnna_forward_noalloc": ([D, P, I64, P, P, P, P, P, P, P, P, I64, P], I32),
        "cnna_output_proj_backward_workspace": ([D], ctypes.c_size_t),
        "cnna_output_proj_backward": ([D, P, P, P, I64, P, P, P, ctypes.c_size_t, P], I32),
        "cnna_core_backward_workspace": ([D], ctypes.c_size_t),
        "cnna_core_backward": ([D, P, I64, P, P, P, P, P, P, ctypes.POINTER(Saved), P,
                                ctypes.POINTER(Grads), P, ctypes.c_size_t, P], I32),
        "cnna_layernorm": ([I32, I64, I32, P, I64, P, I64, P, I64, P, P, ctypes.c_float, P, I64, P], I32),
        "cnna_linear": ([I32, I64, I32, I32, P, I64, P, P, I32, P, I64, P, I64, P], I32),
        "cnna_row_stats": ([I32, I64, I32, P, I64, P, P], I32),
        "cnna_linear_ln": ([I32, I64, I32, I32, P, I64, ctypes.POINTER(Ln), P, P, I32, P, I64, P, I64, P, P],
                           I32),
        "cnna_project_qkv_ex": ([D, P, I64, ctypes.POINTER(Ln), P, P, P, P, P, P, P, P, P, P, P], I32),
        "cnna_conv1d_branch_workspace": ([I32] * 6, ctypes.c_size_t),
        "cnna_conv1d_branch": ([I32] * 6 + [P, I64, P, P, P, P, P, P, P, I64, P, ctypes.c_size_t, P], I32),
    }
    for name, (args, res) in sigs.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    return lib


ABI_VERSION = 4        # CNNA_ABI_VERSION of the include/cnna.h this binding mirrors
LIB = _load()
if LIB.cnna_abi_version() != ABI_VERSION:
    raise ImportError(f"libcnna.so ABI {LIB.cnna_abi_version()} != {ABI_VERSION}: rebuild it with "
                      "`python convolutional-nearest-neighbor-attention_amd/build.py`")
EXPORTED = ("cnna_abi_version", "cnna_error_string", "cnna_check_desc", "cnna_head_stride",
            "cnna_project_qkv", "cnna_select", "cnna_aggregate_workspace", "cnna_aggregate",
            "cnna_output_proj", "cnna_forward_workspace", "cnna_forward", "cnna_forward_noalloc",
            "cnna_output_proj_backward_workspace", "cnna_output_proj_backward",
            "cnna_core_backward_workspace", "cnna_core_backward", "cnna_layernorm", "cnna_linear",
            "cnna_row_stats", "cnna_linear_ln", "cnna_project_qkv_ex",
            "cnna_conv1d_branch_workspace", "cnna_conv1d_branch")
ACT_NONE, ACT_GELU = 0, 1


def check(status: int) -> None:
    """Map a C-ABI status to the exception type the reference raises."""
    if status == 0:
        return
    msg = LIB.cnna_error_string(status).decode()
    if status in (ERR_K_RANGE, ERR_SEQ):
        raise RuntimeError(msg)
    if status in (ERR_GROUPS, ERR_OPTION):
        raise ValueError(msg)
    if status in (ERR_DTYPE,):
        raise TypeError(msg)
    if status == ERR_UNSUPPORTED:
        # a configuration the reference runs but this build's kernels do not
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return CNNA_F32
    if dt == torch.bfloat16:
        return CNNA_BF16
    if dt == torch.float16:
        return CNNA_F16
    raise TypeError(f"cnna: unsupported dtype {dt} (float32, bfloat16 or float16)")


def make_desc(B, N, C, H, Nq, K, seq_length, dtype, metric, conv, softmax, sampled, coord,
              merge=MERGE_REFERENCE, scale=0.0) -> Desc:
    d = Desc(B, N, C, H, Nq, K, seq_length, dtype_code(dtype), METRICS[metric], CONVS[conv],
             int(bool(softmax)), int(bool(sampled)), int(bool(coord)), int(merge), float(scale))
    check(LIB.cnna_check_desc(ctypes.byref(d)))
    return d


def head_stride(d: Desc) -> int:
    return LIB.cnna_head_stride(ctypes.byref(d))


# --------------------------------------------------------------------------
# stage wrappers (each allocates its outputs with torch, launches, no sync)
# --------------------------------------------------------------------------

def _token_rows(x: torch.Tensor) -> torch.Tensor:
    """(B, N, C) whose tokens are rows of one stride (a channel slice of a wider
    tensor qualifies) as is, anything else as a contiguous copy."""
    if x.stride(2) != 1 or x.stride(0) != x.shape[1] * x.stride(1):
        return x.contiguous()
    return x


def _out_rows(out: torch.Tensor, B: int, N: int, C: int) -> int:
    """Row stride of a caller-provided (B, N, C) output view."""
    if (tuple(out.shape) != (B, N, C) or out.stride(2) != 1 or out.stride(0) != N * out.stride(1)):
        raise ValueError("cnna: out must be (B, N, C) with unit channel stride and one token stride")
    return out.stride(1)


def project_qkv(d: Desc, x: torch.Tensor, cand: Optional[torch.Tensor], Wq, Wk, Wv, ln=None, bqkv=None):
    """Returns q (BH,Nq,dkp), k, v (BH,N,dkp), qn, kn (euclidean norms or None).

    ``ln``: a :class:`FoldedNorm` of x's rows; the projections then run on
    LayerNorm(x), normalised as the GEMM loads x (inference only).
    ``bqkv``: (3C) [bq | bk | bv] projection biases, or None."""
    x = _token_rows(x)
    ldx = x.stride(1)
    BH, dkp = d.B * d.H, head_stride(d)
    q = torch.empty((BH, d.Nq, dkp), dtype=x.dtype, device=x.device)
    k = torch.empty((BH, d.N, dkp), dtype=x.dtype, device=x.device)
    v = torch.empty((BH, d.N, dkp), dtype=x.dtype, device=x.device)
    qn = kn = None
    if d.metric != METRICS["matmul"]:
        # euclidean distances need the norms; the cosine backward needs them too
        qn = torch.empty((BH * d.Nq,), dtype=torch.float32, device=x.device)
        kn = torch.empty((BH * d.N,), dtype=torch.float32, device=x.device)
    if ln is None and bqkv is None:
        check(LIB.cnna_project_qkv(ctypes.byref(d), _ptr(x), ldx, _ptr(cand), _ptr(Wq.contiguous()),
                                   _ptr(Wk.contiguous()), _ptr(Wv.contiguous()), _ptr(q), _ptr(k),
                                   _ptr(v), _ptr(qn), _ptr(kn), _stream()))
    else:
        if ln is not None:
            ln.check(x)
        if bqkv is not None:
            if tuple(bqkv.shape) != (3 * d.C,) or bqkv.dtype != x.dtype:
                raise ValueError(f"cnna: bqkv must be ({3 * d.C},) {x.dtype}, got {tuple(bqkv.shape)} {bqkv.dtype}")
            bqkv = bqkv.contiguous()
        check(LIB.cnna_project_qkv_ex(ctypes.byref(d), _ptr(x), ldx,
                                      None if ln is None else ctypes.byref(ln.struct()), _ptr(cand),
                                      _ptr(Wq.contiguous()), _ptr(Wk.contiguous()), _ptr(Wv.contiguous()),
                                      _ptr(bqkv), _ptr(q), _ptr(k), _ptr(v), _ptr(qn), _ptr(kn), _stream()))
    return q, k, v, qn, kn


def select(d: Desc, k, q, kn=None, qn=None, cand=None):
    """Fused similarity + top-k: idx int32, vals fp32, neighbour weights fp32, all (BH,N,K)."""
    return select_cols(d, k, q, kn, qn, cand)[:3]


def select_cols(d: Desc, k, q, kn=None, qn=None, cand=None):
    """``select`` plus, for sampled paths, the candidate column of each entry
    (int32 (BH,N,K), slot 0 = Nq); cols is None for sampling 'all'."""
    BH = d.B * d.H
    idx = torch.empty((BH, d.N, d.K), dtype=torch.int32, device=k.device)
    vals = torch.empty((BH, d.N, d.K), dtype=torch.float32, device=k.device)
    w = torch.empty((BH, d.N, d.K), dtype=torch.float32, device=k.device)
    cols = torch.empty((BH, d.N, d.K), dtype=torch.int32, device=k.device) if d.sampled else None
    check(LIB.cnna_select(ctypes.byref(d), _ptr(k), _ptr(q), _ptr(kn), _ptr(qn), _ptr(cand),
                          _ptr(idx), _ptr(vals), _ptr(w), _ptr(cols), _stream()))
    return idx, vals, w, cols


def aggregate(d: Desc, v, idx, w, w0, w1=None):
    """Gather + conv + head merge: z (B, N, C), the tensor that enters W_o."""
    z = torch.empty((d.B, d.N, d.C), dtype=v.dtype, device=v.device)
    w0 = w0.to(v.dtype).contiguous()
    w1 = None if w1 is None else w1.to(v.dtype).contiguous()
    nws = LIB.cnna_aggregate_workspace(ctypes.byref(d))
    ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=v.device) if nws else None
    check(LIB.cnna_aggregate(ctypes.byref(d), _ptr(v), _ptr(idx), _ptr(w), _ptr(w0), _ptr(w1),
                             _ptr(z), _ptr(ws), nws, _stream()))
    return z


def output_proj(d: Desc, z, Wo, out=None):
    """out = z @ Wo^T (z already carries the reference's head-merge mixing).
    ``out``: optional (B, N, C) view to write into (e.g. a channel slice)."""
    if out is None:
        out = torch.empty((d.B, d.N, d.C), dtype=z.dtype, device=z.device)
    ldo = _out_rows(out, d.B, d.N, d.C)
    check(LIB.cnna_output_proj(ctypes.byref(d), _ptr(z.contiguous()), _ptr(Wo.contiguous()),
                               _ptr(out), ldo, _stream()))
    return out


def forward_fused(d: Desc, x, cand, Wq, Wk, Wv, Wo, w0, w1=None):
    """Whole forward through the single ``cnna_forward`` entry point."""
    x = x.contiguous()
    ws_bytes = LIB.cnna_forward_workspace(ctypes.byref(d))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=x.device)
    out = torch.empty((d.B, d.N, d.C), dtype=x.dtype, device=x.device)
    w0 = w0.to(x.dtype).contiguous()
    w1 = None if w1 is None else w1.to(x.dtype).contiguous()
    check(LIB.cnna_forward(ctypes.byref(d), _ptr(x), x.stride(1), _ptr(cand), _ptr(Wq.contiguous()),
                           _ptr(Wk.contiguous()), _ptr(Wv.contiguous()), _ptr(Wo.contiguous()),
                           _ptr(w0), _ptr(w1), _ptr(out), d.C, _ptr(ws), ws_bytes, _stream()))
    return out


def forward_noalloc(d: Desc, x, cand, Wq, Wk, Wv, Wo, w0, w1=None, out=None):
    """Whole forward through ``cnna_forward_noalloc``: the library works in its
    static device scratch (no workspace); ``out`` may be passed in so that the
    call allocates nothing on this side either."""
    x = x.contiguous()
    if out is None:
        out = torch.empty((d.B, d.N, d.C), dtype=x.dtype, device=x.device)
    check(LIB.cnna_forward_noalloc(ctypes.byref(d), _ptr(x), x.stride(1), _ptr(cand), _ptr(Wq), _ptr(Wk),
                                   _ptr(Wv), _ptr(Wo), _ptr(w0), _ptr(w1), _ptr(out), d.C, _stream()))
    return out


def _rows(t: torch.Tensor) -> torch.Tensor:
    """(..., C) with unit stride in C -> (rows, C) view or contiguous copy."""
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def layernorm(x, weight, bias, eps, residual=None, want_sum=False):
    """nn.LayerNorm over the last dimension of ``x`` (+ ``residual`` first).

    Returns y, or (y, x + residual) with ``want_sum``.  Inference helper of
    the ViT block (vit.py:247-248, 262-267); no autograd."""
    xr = _rows(x)
    rows, C = xr.shape
    rr = None if residual is None else _rows(residual)
    y = torch.empty((rows, C), dtype=x.dtype, device=x.device)
    s = torch.empty_like(y) if (want_sum and residual is not None) else None
    check(LIB.cnna_layernorm(dtype_code(x.dtype), rows, C, _ptr(xr), xr.stride(0), _ptr(rr),
                             0 if rr is None else rr.stride(0), _ptr(s), 0 if s is None else s.stride(0),
                             _ptr(None if weight is None else weight.contiguous()),
                             _ptr(None if bias is None else bias.contiguous()), float(eps), _ptr(y),
                             y.stride(0), _stream()))
    y = y.view(x.shape)
    if want_sum:
        return y, (x if residual is None else s.view(x.shape))
    return y


def linear(a, W, bias=None, gelu=False, residual=None, ln=None, want_stats=False):
    """act(a @ W^T + bias) + residual through the MFMA GEMM (nn.Linear with the
    ViT block's epilogues fused: vit.py:253-257, 263-264, 269); no autograd.

    ``ln``: a :class:`FoldedNorm` of a's rows; the GEMM then runs on
    LayerNorm(a), normalised as it loads a.  ``want_stats``: also return the
    row-statistics partials of the output (a :class:`FoldedNorm` without its
    module), from the GEMM's epilogue where the library supports it (16-bit,
    aligned rows), else from a statistics pass over the output."""
    ar = _rows(a)
    M, Kd = ar.shape
    Nout = W.shape[0]
    rr = None if residual is None else _rows(residual)
    out = torch.empty((M, Nout), dtype=a.dtype, device=a.device)
    epi = want_stats and _stats_epilogue_ok(out, rr)
    st = torch.empty((M, stat_parts(Nout), 2), dtype=torch.float32, device=a.device) if epi else None
    lns = None
    if ln is not None:
        ln.check(ar)
        lns = ln.struct()
    check(LIB.cnna_linear_ln(dtype_code(a.dtype), M, Nout, Kd, _ptr(ar), ar.stride(0),
                             None if lns is None else ctypes.byref(lns), _ptr(W.contiguous()),
                             _ptr(None if bias is None else bias.contiguous()), ACT_GELU if gelu else ACT_NONE,
                             _ptr(rr), 0 if rr is None else rr.stride(0), _ptr(out), out.stride(0), _ptr(st),
                             _stream()))
    out = out.view(*a.shape[:-1], Nout)
    if not want_stats:
        return out
    return out, (FoldedNorm(st, M, Nout) if epi else row_stats(out))


def stat_parts(C: int) -> int:
    """CNNA_STAT_PARTS(C): row-statistics partials per row of C columns."""
    return (C + STAT_TILE - 1) // STAT_TILE


def _stats_epilogue_ok(out: torch.Tensor, rr: Optional[torch.Tensor]) -> bool:
    """The GEMM's statistics epilogue applies (bf16 / fp16, Nout % 8 == 0,
    16-byte aligned rows); otherwise the statistics come from ``row_stats``."""
    if (out.dtype not in (torch.bfloat16, torch.float16) or out.shape[1] % 8 or out.data_ptr() % 16
            or out.stride(0) % 8):
        return False
    return rr is None or (rr.data_ptr() % 16 == 0 and rr.stride(0) % 8 == 0)


class FoldedNorm:
    """A LayerNorm split for folding: the fp32 statistics partials of ``rows``
    rows of ``C`` columns ((rows, stat_parts(C), 2): each 128-column tile's
    mean and sum of squared deviations), and, once ``with_norm`` names it, the
    nn.LayerNorm whose normalisation the consuming GEMM applies."""

    def __init__(self, stats: torch.Tensor, rows: int, C: int, weight=None, bias=None, eps=1e-5):
        self.stats, self.rows, self.C = stats, rows, C
        self.weight, self.bias, self.eps = weight, bias, float(eps)

    def with_norm(self, norm: torch.nn.LayerNorm) -> "FoldedNorm":
        if tuple(norm.normalized_shape) != (self.C,):
            raise ValueError(f"cnna: LayerNorm over {tuple(norm.normalized_shape)} folded into rows of {self.C}")
        return FoldedNorm(self.stats, self.rows, self.C, norm.weight, norm.bias, norm.eps)

    def check(self, rows2d: torch.Tensor) -> None:
        n = rows2d.numel() // rows2d.shape[-1]
        if n != self.rows or rows2d.shape[-1] != self.C:
            raise ValueError(f"cnna: statistics of {self.rows} x {self.C} rows for a {n} x {rows2d.shape[-1]} "
                             "operand")
        for p in (self.weight, self.bias):
            if p is not None and p.dtype != rows2d.dtype:
                raise TypeError(f"cnna: LayerNorm parameters in {p.dtype} for {rows2d.dtype} rows")

    def struct(self) -> Ln:
        g = None if self.weight is None else self.weight.contiguous()
        b = None if self.bias is None else self.bias.contiguous()
        self._keep = (g, b)     # alive until the launch has been queued
        return Ln(self.stats.data_ptr(), None if g is None else g.data_ptr(),
                  None if b is None else b.data_ptr(), self.eps)


def row_stats(x: torch.Tensor) -> FoldedNorm:
    """Statistics partials of the rows of ``x`` (..., C) for a LayerNorm folded
    into the GEMM that consumes x (the pre-pass of the first block)."""
    xr = _rows(x)
    rows, C = xr.shape
    st = torch.empty((rows, stat_parts(C), 2), dtype=torch.float32, device=x.device)
    check(LIB.cnna_row_stats(dtype_code(x.dtype), rows, C, _ptr(xr), xr.stride(0), _ptr(st), _stream()))
    return FoldedNorm(st, rows, C)


def conv1d_branch(x, Wx, bx, conv_w, conv_b, Wo, bo, num_heads, out=None):
    """MultiHeadConv1dAttention's forward (layers.py:452-499) through the
    native kernels: W_x GEMM, per-head token Conv1d ('same'), the token-mixing
    merge, W_o GEMM.  ``out``: optional (B, N, C) view to write into."""
    x = _token_rows(x)
    B, N, C = x.shape
    ks = conv_w.shape[-1]
    if out is None:
        out = torch.empty((B, N, C), dtype=x.dtype, device=x.device)
    ldo = _out_rows(out, B, N, C)
    dt = dtype_code(x.dtype)
    nws = LIB.cnna_conv1d_branch_workspace(dt, B, N, C, num_heads, ks)
    if nws == 0:
        raise RuntimeError("cnna: unsupported Conv1d branch shape")
    ws = torch.empty((nws,), dtype=torch.uint8, device=x.device)
    c = lambda t: None if t is None else _ptr(t.to(x.dtype).contiguous())
    check(LIB.cnna_conv1d_branch(dt, B, N, C, num_heads, ks, _ptr(x), x.stride(1), c(Wx), c(bx), c(conv_w),
                                 c(conv_b), c(Wo), c(bo), _ptr(out), ldo, _ptr(ws), nws, _stream()))
    return out


def output_proj_backward(d: Desc, z, Wo, dout):
    """dz = dout @ Wo, dWo = dout^T @ z."""
    dout = dout.contiguous()
    # row-major outputs whatever the strides of z / Wo (empty_like would keep
    # a permuted layout, which the kernels do not write)
    dz = torch.empty(z.shape, dtype=z.dtype, device=z.device)
    dWo = torch.empty(Wo.shape, dtype=Wo.dtype, device=Wo.device)
    nws = LIB.cnna_output_proj_backward_workspace(ctypes.byref(d))
    ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=z.device)
    check(LIB.cnna_output_proj_backward(ctypes.byref(d), _ptr(z.contiguous()), _ptr(Wo.contiguous()),
                                        _ptr(dout), d.C, _ptr(dz), _ptr(dWo), _ptr(ws), nws,
                                        _stream()))
    return dz, dWo


def core_backward(d: Desc, x, cand, Wq, Wk, Wv, w0, w1, saved, dz, want_db=False):
    """Gradients of x, W_q, W_k, W_v and the conv weights from dz (B, N, C),
    and with ``want_db`` that of the projection biases (3C) as a seventh value
    (None otherwise).

    ``saved`` = (q, k, v, qn, kn, idx, vals, w, wmul, cols) from the forward
    stages (wmul: the multipliers applied to w before the aggregation, or None;
    cols: the sampled paths' candidate columns from ``select_cols``).
    """
    q, k, v, qn, kn, idx, vals, w, wmul, cols = saved
    x = _token_rows(x)
    dz = dz.contiguous()
    w0c = w0.to(x.dtype).contiguous()
    w1c = None if w1 is None else w1.to(x.dtype).contiguous()
    dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    dWq, dWk, dWv = (torch.empty(W.shape, dtype=x.dtype, device=x.device) for W in (Wq, Wk, Wv))
    dw0 = torch.empty(w0.shape, dtype=x.dtype, device=x.device)
    dw1 = None if w1 is None else torch.empty(w1.shape, dtype=x.dtype, device=x.device)
    db = torch.empty((3 * d.C,), dtype=x.dtype, device=x.device) if want_db else None
    sv = Saved(*(None if t is None else t.data_ptr() for t in (q, k, v, qn, kn, idx, vals, w, wmul, cols)))
    gr = Grads(*(None if t is None else t.data_ptr() for t in (dx, dWq, dWk, dWv, dw0, dw1, db)))
    nws = LIB.cnna_core_backward_workspace(ctypes.byref(d))
    ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=x.device)
    check(LIB.cnna_core_backward(ctypes.byref(d), _ptr(x), x.stride(1), _ptr(cand),
                                 _ptr(Wq.contiguous()), _ptr(Wk.contiguous()), _ptr(Wv.contiguous()),
                                 _ptr(w0c), _ptr(w1c), ctypes.byref(sv), _ptr(dz), ctypes.byref(gr),
                                 _ptr(ws), nws, _stream()))
    return dx, dWq, dWk, dWv, dw0, dw1, db


# --------------------------------------------------------------------------
# autograd
# --------------------------------------------------------------------------

class ConvNNCore(torch.autograd.Function):
    """x -> z (B, N, C): projections, neighbour selection, aggregation, head merge.

    ``reference_errors``: raise where the reference's autograd raises.  The
    reference masks the self column of the sampled euclidean distance matrix in
    place on the output of ``sqrt`` (layers.py:278, 291-292, 304-305), so its
    backward fails with RuntimeError for sampled euclidean; the kernels here
    can differentiate that case, and do when this flag is off.

    ``dmask``: optional dense keep-mask (B, H, N, Nq) of an attention dropout
    drawn over the whole score matrix (MultiHeadKvtAttention's ``attn_drop``,
    layers.py:680); the kept probabilities are multiplied by
    ``dmask[..., idx] * dscale`` (0 or 1/(1-p)); depthwise conv only.

    ``bqkv``: optional (3C) [bq | bk | bv] projection biases
    (MultiHeadKvtAttention's ``qkv_bias``, layers.py:662).
    """

    @staticmethod
    def forward(ctx, x, Wq, Wk, Wv, w0, w1, cand, d, reference_errors=False, dmask=None, dscale=1.0,
                bqkv=None):
        q, k, v, qn, kn = project_qkv(d, x, cand, Wq, Wk, Wv, bqkv=bqkv)
        idx, vals, w, cols = select_cols(d, k, q, kn, qn, cand)
        wmul = entry_multipliers(d, idx, dmask, dscale)
        z = aggregate(d, v, idx, w if wmul is None else w * wmul, w0, w1)
        ctx.d = d
        ctx.reference_errors = reference_errors
        ctx.has_bias = bqkv is not None
        ctx.save_for_backward(x, Wq, Wk, Wv, w0, w1, cand, q, k, v, qn, kn, idx, vals, w, wmul, cols)
        return z

    @staticmethod
    def backward(ctx, dz):
        d = ctx.d
        if ctx.reference_errors and d.sampled and d.metric == METRICS["euclidean"]:
            raise RuntimeError(
                "one of the variables needed for gradient computation has been modified by an "
                "inplace operation: the sampled euclidean similarity is masked in place after "
                "sqrt (layers.py:291-292, 304-305)")
        x, Wq, Wk, Wv, w0, w1, cand, q, k, v, qn, kn, idx, vals, w, wmul, cols = ctx.saved_tensors
        dx, dWq, dWk, dWv, dw0, dw1, db = core_backward(ctx.d, x, cand, Wq, Wk, Wv, w0, w1,
                                                        (q, k, v, qn, kn, idx, vals, w, wmul, cols), dz,
                                                        want_db=ctx.has_bias)
        dw0 = dw0.to(w0.dtype)
        dw1 = None if dw1 is None else dw1.to(w1.dtype)
        return dx, dWq, dWk, dWv, dw0, dw1, None, None, None, None, None, db


def entry_multipliers(d: Desc, idx, dmask, dscale):
    """Per-entry multipliers (B*H, N, K) fp32 from a dense keep-mask
    (B, H, N, Nq) at the selected columns, times the dropout scale; None
    without a mask."""
    if dmask is None:
        return None
    dm = dmask.reshape(d.B * d.H, d.N, d.Nq)
    return dm.gather(2, idx.long()).to(torch.float32) * dscale


class OutputProj(torch.autograd.Function):
    """out = z @ Wo^T."""

    @staticmethod
    def forward(ctx, z, Wo, d):
        ctx.d = d
        ctx.save_for_backward(z, Wo)
        return output_proj(d, z, Wo)

    @staticmethod
    def backward(ctx, dout):
        z, Wo = ctx.saved_tensors
        dz, dWo = output_proj_backward(ctx.d, z, Wo, dout)
        return dz, dWo, None


# --------------------------------------------------------------------------
# torch.library operators: the same C-ABI calls as custom ops with fake
# (shape-only) kernels, registered autograd and FLOP formulas, so that
# torch.compile traces the layer without graph breaks and
# torch.utils.flop_counter.FlopCounterMode counts it.  The eager path keeps
# the autograd.Function classes above (lower Python dispatch cost); the
# layers switch to these ops while compiling or under a dispatch mode.
# --------------------------------------------------------------------------

DESC_FIELDS = ("B", "N", "C", "H", "Nq", "K", "seq_length", "dtype", "metric", "conv", "softmax",
               "sampled", "coord", "merge")


def desc_list(d: Desc) -> list:
    return [int(getattr(d, f)) for f in DESC_FIELDS]


def desc_values(B, N, C, H, Nq, K, seq_length, dtype, metric, conv, softmax, sampled, coord,
                merge=MERGE_REFERENCE):
    """The descriptor as plain ints (no library call: traceable)."""
    return [B, N, C, H, Nq, K, seq_length, dtype_code(dtype), METRICS[metric], CONVS[conv],
            int(bool(softmax)), int(bool(sampled)), int(bool(coord)), int(merge)]


def _desc_of(dl, scale) -> Desc:
    d = Desc(*dl, float(scale))
    check(LIB.cnna_check_desc(ctypes.byref(d)))
    return d


def _dkp(dl) -> int:
    din = dl[2] // dl[3] + (1 if dl[12] else 0)
    return (din + 15) // 16 * 16


def use_library_ops() -> bool:
    """True while torch.compile traces or a Python dispatch mode (fake tensors,
    FlopCounterMode, ...) is active."""
    return torch.compiler.is_compiling() or _get_current_dispatch_mode() is not None


_EMPTY = lambda like: torch.empty((0,), dtype=torch.float32, device=like.device)


@torch.library.custom_op("cnna::core", mutates_args=())
def core_op(x: torch.Tensor, Wq: torch.Tensor, Wk: torch.Tensor, Wv: torch.Tensor, w0: torch.Tensor,
            w1: Optional[torch.Tensor], cand: Optional[torch.Tensor], dmask: Optional[torch.Tensor],
            desc: List[int], scale: float, reference_errors: bool, dscale: float,
            bqkv: Optional[torch.Tensor] = None
            ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                       torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """x -> (z, q, k, v, qn, kn, idx, vals, w, wmul, cols): projections (with
    the optional (3C) biases ``bqkv``), selection, aggregation, head merge
    (layers.py:261-317); qn / kn empty when unused; wmul the per-entry dropout
    multipliers of ``dmask`` (empty without); cols the sampled paths'
    candidate columns (empty for 'all')."""
    d = _desc_of(desc, scale)
    q, k, v, qn, kn = project_qkv(d, x, cand, Wq, Wk, Wv, bqkv=bqkv)
    idx, vals, w, cols = select_cols(d, k, q, kn, qn, cand)
    wmul = entry_multipliers(d, idx, dmask, dscale)
    z = aggregate(d, v, idx, w if wmul is None else w * wmul, w0, w1)
    i32 = lambda: torch.empty((0,), dtype=torch.int32, device=x.device)
    return (z, q, k, v, _EMPTY(x) if qn is None else qn, _EMPTY(x) if kn is None else kn, idx, vals, w,
            _EMPTY(x) if wmul is None else wmul, i32() if cols is None else cols)


@core_op.register_fake
def _core_fake(x, Wq, Wk, Wv, w0, w1, cand, dmask, desc, scale, reference_errors, dscale, bqkv=None):
    B, N, C, H, Nq, K = desc[:6]
    BH, dkp = B * H, _dkp(desc)
    f32 = dict(dtype=torch.float32, device=x.device)
    norms = desc[8] != METRICS["matmul"]
    return (x.new_empty((B, N, C)), x.new_empty((BH, Nq, dkp)), x.new_empty((BH, N, dkp)),
            x.new_empty((BH, N, dkp)), torch.empty((BH * Nq if norms else 0,), **f32),
            torch.empty((BH * N if norms else 0,), **f32),
            torch.empty((BH, N, K), dtype=torch.int32, device=x.device), torch.empty((BH, N, K), **f32),
            torch.empty((BH, N, K), **f32), torch.empty((BH, N, K) if dmask is not None else (0,), **f32),
            torch.empty((BH, N, K) if desc[11] else (0,), dtype=torch.int32, device=x.device))


@torch.library.custom_op("cnna::core_backward", mutates_args=())
def core_backward_op(x: torch.Tensor, Wq: torch.Tensor, Wk: torch.Tensor, Wv: torch.Tensor,
                     w0: torch.Tensor, w1: Optional[torch.Tensor], cand: Optional[torch.Tensor],
                     q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qn: torch.Tensor, kn: torch.Tensor,
                     idx: torch.Tensor, vals: torch.Tensor, w: torch.Tensor, wmul: Optional[torch.Tensor],
                     cols: Optional[torch.Tensor], dz: torch.Tensor, desc: List[int], scale: float,
                     want_db: bool = False
                     ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                torch.Tensor, torch.Tensor]:
    """Gradients (dx, dWq, dWk, dWv, dw0, dw1, dbqkv) of ``cnna::core``; dw1
    empty without w1, dbqkv empty without ``want_db``."""
    d = _desc_of(desc, scale)
    nq = None if qn.numel() == 0 else qn
    nk = None if kn.numel() == 0 else kn
    dx, dWq, dWk, dWv, dw0, dw1, db = core_backward(d, x, cand, Wq, Wk, Wv, w0, w1,
                                                    (q, k, v, nq, nk, idx, vals, w, wmul, cols), dz,
                                                    want_db=want_db)
    return (dx, dWq, dWk, dWv, dw0.to(w0.dtype), (x.new_empty((0,)) if dw1 is None else dw1.to(w1.dtype)),
            x.new_empty((0,)) if db is None else db)


@core_backward_op.register_fake
def _core_backward_fake(x, Wq, Wk, Wv, w0, w1, cand, q, k, v, qn, kn, idx, vals, w, wmul, cols, dz, desc,
                        scale, want_db=False):
    return (x.new_empty(x.shape), x.new_empty(Wq.shape), x.new_empty(Wk.shape), x.new_empty(Wv.shape),
            w0.new_empty(w0.shape), (x.new_empty((0,)) if w1 is None else w1.new_empty(w1.shape)),
            x.new_empty((3 * desc[2],) if want_db else (0,)))


def _core_setup(ctx, inputs, output):
    x, Wq, Wk, Wv, w0, w1, cand, dmask, desc, scale, reference_errors, dscale, bqkv = inputs
    z, q, k, v, qn, kn, idx, vals, w, wmul, cols = output
    wmul = None if dmask is None else wmul
    cols = cols if desc[11] else None
    ctx.desc, ctx.scale, ctx.reference_errors = desc, scale, reference_errors
    ctx.has_w1 = w1 is not None
    ctx.has_bias = bqkv is not None
    ctx.save_for_backward(x, Wq, Wk, Wv, w0, w1, cand, q, k, v, qn, kn, idx, vals, w, wmul, cols)


def _core_bwd(ctx, dz, *unused):
    dl = ctx.desc
    if ctx.reference_errors and dl[11] and dl[8] == METRICS["euclidean"]:
        raise RuntimeError(
            "one of the variables needed for gradient computation has been modified by an "
            "inplace operation: the sampled euclidean similarity is masked in place after "
            "sqrt (layers.py:291-292, 304-305)")
    x, Wq, Wk, Wv, w0, w1, cand, q, k, v, qn, kn, idx, vals, w, wmul, cols = ctx.saved_tensors
    dx, dWq, dWk, dWv, dw0, dw1, db = core_backward_op(x, Wq, Wk, Wv, w0, w1, cand, q, k, v, qn, kn, idx,
                                                       vals, w, wmul, cols, dz.contiguous(), dl, ctx.scale,
                                                       ctx.has_bias)
    return (dx, dWq, dWk, dWv, dw0, (dw1 if ctx.has_w1 else None), None, None, None, None, None, None,
            db if ctx.has_bias else None)


torch.library.register_autograd("cnna::core", _core_bwd, setup_context=_core_setup)


@torch.library.custom_op("cnna::output_proj", mutates_args=())
def output_proj_op(z: torch.Tensor, Wo: torch.Tensor, desc: List[int], scale: float) -> torch.Tensor:
    """out = z @ Wo^T (layers.py:320)."""
    return output_proj(_desc_of(desc, scale), z, Wo)


@output_proj_op.register_fake
def _output_proj_fake(z, Wo, desc, scale):
    return z.new_empty((desc[0], desc[1], desc[2]))


@torch.library.custom_op("cnna::output_proj_backward", mutates_args=())
def output_proj_backward_op(z: torch.Tensor, Wo: torch.Tensor, dout: torch.Tensor, desc: List[int],
                            scale: float) -> Tuple[torch.Tensor, torch.Tensor]:
    return output_proj_backward(_desc_of(desc, scale), z, Wo, dout)


@output_proj_backward_op.register_fake
def _output_proj_backward_fake(z, Wo, dout, desc, scale):
    return z.new_empty(z.shape), Wo.new_empty(Wo.shape)


def _oproj_setup(ctx, inputs, output):
    z, Wo, desc, scale = inputs
    ctx.desc, ctx.scale = desc, scale
    ctx.save_for_backward(z, Wo)


def _oproj_bwd(ctx, dout):
    z, Wo = ctx.saved_tensors
    dz, dWo = output_proj_backward_op(z, Wo, dout.contiguous(), ctx.desc, ctx.scale)
    return dz, dWo, None, None


torch.library.register_autograd("cnna::output_proj", _oproj_bwd, setup_context=_oproj_setup)


# ---- FLOP formulas (2 per multiply-accumulate, the work the reference's ops do)
def core_flops(desc) -> int:
    """Projections, similarity and conv of one forward (layers.py:264-313)."""
    B, N, C, H, Nq, K = desc[:6]
    conv = desc[9]
    dk = C // H
    din = dk + (1 if desc[12] else 0)
    proj = 2 * B * C * C * (2 * N + Nq)
    sim = 2 * B * N * Nq * H * din
    if conv == CONVS["depthwise"]:
        cv = 2 * B * N * H * dk * K
    elif conv == CONVS["standard"]:
        cv = 2 * B * N * H * dk * din * K
    else:
        cv = 2 * B * N * H * (din * K + dk * din)
    return proj + sim + cv


def _register_flops():
    from torch.utils.flop_counter import register_flop_formula

    @register_flop_formula(torch.ops.cnna.core)
    def _f_core(x, Wq, Wk, Wv, w0, w1, cand, dmask, desc, scale, reference_errors, dscale, *a,
                out_shape=None, **kw):
        return core_flops(desc)

    @register_flop_formula(torch.ops.cnna.core_backward)
    def _f_core_bwd(*args, out_shape=None, **kw):
        return 2 * core_flops(args[18])

    @register_flop_formula(torch.ops.cnna.output_proj)
    def _f_oproj(z, Wo, desc, scale, *a, out_shape=None, **kw):
        return 2 * desc[0] * desc[1] * desc[2] * desc[2]

    @register_flop_formula(torch.ops.cnna.output_proj_backward)
    def _f_oproj_bwd(z, Wo, dout, desc, scale, *a, out_shape=None, **kw):
        return 4 * desc[0] * desc[1] * desc[2] * desc[2]


_register_flops()
