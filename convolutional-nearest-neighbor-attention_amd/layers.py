"""Drop-in ``MultiHeadConvNNAttention`` backed by the gfx950 HIP library.

Same class name, constructor signature, defaults, parameter names and forward
contract as the reference (layers.py:132-321 of
mingikang31/Convolutional-Nearest-Neighbor-Attention), so ``vit.py``-style
callers switch by putting this directory on ``sys.path``::

    from layers import MultiHeadConvNNAttention

The forward runs on ROCm device tensors only; a CPU tensor raises (there is no
fallback path).  Arithmetic differences to the eager reference: fp32
accumulation everywhere (the reference rounds bf16 intermediates), and top-k
ties break by the lowest candidate index.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

import cnna_ops as ops


class MultiHeadConvNNAttention(nn.Module):
    def __init__(self,
                 d_hidden,
                 num_heads,
                 attention_dropout,
                 K,
                 sampling_type,
                 num_samples,
                 sample_padding,
                 magnitude_type,
                 seq_length=197,
                 coordinate_encoding=False,
                 convolution_type='depthwise',
                 softmax_topk_val=True
                 ):
        super().__init__()
        # layers.py:149
        assert d_hidden % num_heads == 0, "d_hidden must be divisible by num_heads"
        self.d_hidden = d_hidden
        self.num_heads = num_heads
        self.attention_dropout = attention_dropout
        self.d_k = d_hidden // num_heads
        self.K = K
        self.seq_length = seq_length
        self.sampling_type = sampling_type
        self.num_samples = int(num_samples)                                          # layers.py:163
        self.sample_padding = int(sample_padding) if sampling_type == 'spatial' else 0  # layers.py:164
        self.magnitude_type = magnitude_type
        self.maximum = True if self.magnitude_type in ('cosine', 'matmul') else False
        self.coordinate_encoding = coordinate_encoding
        self.coordinate_cache = {}

        # Parameters are created in the reference's order (layers.py:175-228) so
        # that a seeded construction draws the same initial weights.
        self.W_q = nn.Linear(d_hidden, d_hidden, bias=False)
        self.W_k = nn.Linear(d_hidden, d_hidden, bias=False)
        self.W_v = nn.Linear(d_hidden, d_hidden, bias=False)
        self.W_o = nn.Linear(d_hidden, d_hidden, bias=False)
        self.dropout = nn.Dropout(attention_dropout)

        self.in_channels = (d_hidden // num_heads) + 1 if coordinate_encoding else (d_hidden // num_heads)
        self.out_channels = (d_hidden // num_heads)
        self.convolution_type = convolution_type
        if convolution_type == 'standard':
            self.conv = nn.Conv1d(self.in_channels, self.out_channels, kernel_size=self.K,
                                  stride=self.K, padding=0, bias=False)
        elif convolution_type == 'depthwise':
            self.conv = nn.Conv1d(self.in_channels, self.out_channels, kernel_size=self.K,
                                  stride=self.K, padding=0, groups=self.in_channels, bias=False)
            self.conv.weight.data.fill_(1.0)                                         # layers.py:206
        elif convolution_type == 'depthwise-separable':
            self.conv = nn.Sequential(
                nn.Conv1d(self.in_channels, self.in_channels, kernel_size=self.K, stride=self.K,
                          padding=0, groups=self.in_channels, bias=False),
                nn.Conv1d(self.in_channels, self.out_channels, kernel_size=1, stride=1,
                          padding=0, bias=False))
        self.softmax_topk_val = softmax_topk_val
        self.INF = 1.1
        self.NEG_INF = -0.1

    # -- helpers ------------------------------------------------------------
    def _conv_weights(self):
        if self.convolution_type == 'depthwise-separable':
            return self.conv[0].weight, self.conv[1].weight
        if self.convolution_type in ('standard', 'depthwise'):
            return self.conv.weight, None
        raise ValueError(f"unknown convolution_type {self.convolution_type}")

    def _candidates(self, x):
        """Sampled candidate token indices, drawn exactly like layers.py:284, 297."""
        N = x.shape[1]
        if self.sampling_type == 'all':
            return None
        if self.sampling_type == 'random':
            idx = torch.randperm(N, device=x.device)[:self.num_samples]
        elif self.sampling_type == 'spatial':
            idx = torch.linspace(0 + self.sample_padding, N - self.sample_padding - 1,
                                 self.num_samples, device=x.device).long()
        else:
            raise ValueError("Invalid sampling_type. Must be one of ['all', 'random', 'spatial']")
        return idx.to(torch.int32)

    def forward(self, x):
        z, d = self.core(x)
        Wo = _amp_cast(self.W_o.weight, z.dtype)
        if isinstance(d, list):
            return torch.ops.cnna.output_proj(z, Wo, d, 0.0)
        return ops.OutputProj.apply(z, Wo, d)

    def core(self, x):
        """Everything before W_o (layers.py:261-317): returns (z, desc), z the
        merged conv output after dropout.  Under torch.autocast the layer
        computes in autocast's dtype (float16 or bfloat16); while compiling
        or under a dispatch mode it runs as the ``cnna::`` library ops and the
        descriptor is a list of ints."""
        if x.dim() != 3:
            raise RuntimeError(f"expected x of shape (B, N, C), got {tuple(x.shape)}")
        if not x.is_cuda:
            raise RuntimeError("MultiHeadConvNNAttention (cnna) runs on ROCm device tensors only")
        B, N, C = x.shape
        self.batch_size = B                                                          # layers.py:239
        cand = self._candidates(x)
        Nq = N if cand is None else int(cand.numel())
        x, Wq, Wk, Wv = _amp_inputs(x, self.W_q.weight, self.W_k.weight, self.W_v.weight)
        if Wq.dtype != x.dtype:
            raise RuntimeError(f"mat1 and mat2 must have the same dtype, but got {x.dtype} and "
                               f"{Wq.dtype}")
        w0, w1 = self._conv_weights()
        if ops.use_library_ops():
            d = ops.desc_values(B, N, C, self.num_heads, Nq, self.K, self.seq_length, x.dtype,
                                self.magnitude_type, self.convolution_type, self.softmax_topk_val,
                                cand is not None, self.coordinate_encoding)
            z = torch.ops.cnna.core(x, Wq, Wk, Wv, _amp_cast(w0, x.dtype), _amp_cast(w1, x.dtype), cand,
                                    None, d, 0.0, True, 1.0)[0]
            return self._conv_output_dropout(z), d
        d = ops.make_desc(B, N, C, self.num_heads, Nq, self.K, self.seq_length, x.dtype,
                          self.magnitude_type, self.convolution_type, self.softmax_topk_val,
                          cand is not None, self.coordinate_encoding)
        z = ops.ConvNNCore.apply(x, Wq, Wk, Wv, w0, w1, cand, d, True)
        return self._conv_output_dropout(z), d

    def core_folded(self, x, ln):
        """``core`` of LayerNorm(x) in inference with the LayerNorm folded into
        the Q/K/V projection (vit.py:262 feeding layers.py:264-265): ``ln``
        (cnna_ops.FoldedNorm) holds x's row statistics and the norm, and the
        projection GEMM normalises x as it loads it.  Eval mode: no autograd,
        dropout is the identity.  Returns (z, desc)."""
        if self.training:
            raise RuntimeError("MultiHeadConvNNAttention.core_folded is an inference path (eval mode)")
        B, N, C = x.shape
        self.batch_size = B                                                          # layers.py:239
        cand = self._candidates(x)
        Nq = N if cand is None else int(cand.numel())
        d = ops.make_desc(B, N, C, self.num_heads, Nq, self.K, self.seq_length, x.dtype,
                          self.magnitude_type, self.convolution_type, self.softmax_topk_val,
                          cand is not None, self.coordinate_encoding)
        if self.W_q.weight.dtype != x.dtype:
            raise RuntimeError(f"mat1 and mat2 must have the same dtype, but got {x.dtype} and "
                               f"{self.W_q.weight.dtype}")
        w0, w1 = self._conv_weights()
        q, k, v, qn, kn = ops.project_qkv(d, x, cand, self.W_q.weight, self.W_k.weight, self.W_v.weight,
                                          ln=ln)
        idx, _, w, _ = ops.select_cols(d, k, q, kn, qn, cand)
        return ops.aggregate(d, v, idx, w, w0, w1), d

    def _conv_output_dropout(self, z):
        """``self.dropout`` on the conv output y (B*H, d_k, N), where the reference
        applies it (layers.py:316), given the head-merged z (B, N, C).

        z is a permutation of y's elements; y is rebuilt contiguous in the
        reference's layout, dropped out there (so the mask, the random numbers
        consumed and the rounding are those of the reference's call) and merged
        again.  Eval mode and p = 0 draw nothing and return z."""
        if not self.training or self.dropout.p == 0:
            return z
        B, N, C = z.shape
        H, dk = self.num_heads, C // self.num_heads
        if H == 1:
            # layers.py:248-249, 255-256: the merge is a transpose
            y = z.transpose(1, 2).contiguous()
            return self.dropout(y).transpose(1, 2).contiguous()
        # z[b, t, h*d_k + a] = y_tok[b*H + h].flat[a*N + t], y_tok = y.transpose(1, 2)
        y = z.view(B, N, H, dk).permute(0, 2, 3, 1).reshape(B * H, N, dk).transpose(1, 2).contiguous()
        y = self.dropout(y)
        return y.transpose(1, 2).reshape(B, H, dk, N).permute(0, 3, 1, 2).reshape(B, N, C).contiguous()


def _amp_cast(t, dtype):
    return t if t is None or t.dtype == dtype else t.to(dtype)


def _amp_dtype():
    """The reduced type of the active ``torch.autocast('cuda')``: float16 (its
    default, the reference's ``--use_amp`` loop) or bfloat16."""
    dt = torch.get_autocast_dtype("cuda")
    return dt if dt in (torch.float16, torch.bfloat16) else torch.float16


def _amp_inputs(x, *weights):
    """Autocast policy of the native layers: inside ``torch.autocast('cuda')``
    (the reference's ``--use_amp`` loop, train_eval.py:137-146) x and the
    weights are cast to autocast's dtype (float16 by default, or bfloat16),
    which the kernels compute in with fp32 accumulation, as autocast runs
    ``nn.Linear`` and the reference's ``bmm``; gradients flow back through the
    casts."""
    if torch.is_autocast_enabled("cuda"):
        dt = _amp_dtype()
        return (_amp_cast(x, dt),) + tuple(_amp_cast(w, dt) for w in weights)
    return (x,) + weights


def _inference(module: nn.Module, x: torch.Tensor) -> bool:
    """Nothing to differentiate, no autocast, not tracing: the fused native
    inference kernels may run."""
    if not x.is_cuda or torch.is_autocast_enabled("cuda") or ops.use_library_ops():
        return False
    if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in module.parameters())):
        return False
    return True


class MultiHeadAttention(nn.Module):
    """Softmax multi-head attention (layers.py:88-130): the sibling branch of
    ``MultiHeadBranchingAttention`` and the ViT's ``layer="Attention"``.

    Not a ConvNN path: it runs through PyTorch.  The score / softmax / value
    products are evaluated in float32 (bfloat16 inputs are widened), so no
    batched bfloat16 product takes a transposed operand.
    """

    def __init__(self, d_hidden, num_heads, attention_dropout):
        super().__init__()
        assert d_hidden % num_heads == 0, "d_hidden must be divisible by num_heads"
        self.d_hidden = d_hidden
        self.num_heads = num_heads
        self.d_k = d_hidden // num_heads
        self.dropout = nn.Dropout(attention_dropout)
        self.W_q = nn.Linear(d_hidden, d_hidden, bias=False)
        self.W_k = nn.Linear(d_hidden, d_hidden, bias=False)
        self.W_v = nn.Linear(d_hidden, d_hidden, bias=False)
        self.W_o = nn.Linear(d_hidden, d_hidden, bias=False)

    def _heads(self, t):
        B, N, _ = t.shape
        return t.view(B, N, self.num_heads, self.d_k).transpose(1, 2).float().contiguous()

    def forward(self, x, mask=None):
        B, N, _ = x.shape
        q, k, v = self._heads(self.W_q(x)), self._heads(self.W_k(x)), self._heads(self.W_v(x))
        scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) / math.sqrt(self.d_k)
        if mask is not None:
            scores = scores.masked_fill(mask == 0, -1e9)                 # layers.py:111-112
        probs = self.dropout(torch.softmax(scores, dim=-1))
        o = torch.matmul(probs, v).to(x.dtype)
        return self.W_o(o.transpose(1, 2).reshape(B, N, self.d_hidden))


class MultiHeadConv1dAttention(nn.Module):
    """Per-head token Conv1d (layers.py:452-499): W_x, Conv1d(d_k, d_k,
    kernel_size, stride 1, padding 'same') shared by the heads, the reference's
    token-mixing reshape back to (B, N, d_hidden), W_o.

    Inference runs the native path (``cnna_conv1d_branch``: MFMA GEMMs for W_x
    and W_o with their biases, a LDS-tiled token convolution, the merge
    kernel); with gradients required it runs the same arithmetic as PyTorch
    modules so autograd applies.
    """

    def __init__(self, d_hidden, num_heads, kernel_size):
        super().__init__()
        assert d_hidden % num_heads == 0, "d_hidden must be divisible by num_heads"
        self.d_hidden = d_hidden
        self.num_heads = num_heads
        self.d_k = d_hidden // num_heads
        self.kernel_size = kernel_size
        self.stride = 1
        self.W_x = nn.Linear(d_hidden, d_hidden)
        self.W_o = nn.Linear(d_hidden, d_hidden)
        self.in_channels = d_hidden // num_heads
        self.out_channels = d_hidden // num_heads
        self.conv = nn.Conv1d(self.in_channels, self.out_channels, kernel_size=self.kernel_size,
                              stride=self.stride, padding="same")

    def forward(self, x, out=None):
        if _inference(self, x) and self.W_x.weight.dtype == x.dtype:
            return ops.conv1d_branch(x, self.W_x.weight, self.W_x.bias, self.conv.weight, self.conv.bias,
                                     self.W_o.weight, self.W_o.bias, self.num_heads, out=out)
        y = self._forward_modules(x)
        if out is not None:
            out.copy_(y)
            return out
        return y

    def _forward_modules(self, x):
        B, N, _ = x.shape
        H, dk = self.num_heads, self.d_k
        u = self.W_x(x).view(B, N, H, dk).permute(0, 2, 3, 1).reshape(B * H, dk, N)  # layers.py:476-487
        y = self.conv(u)                                                              # (B*H, d_k, N)
        # layers.py:483-497: the token-major conv output of each head, read as
        # (d_k, N) and transposed, z[b, t, h*d_k + a] = y_tok[b*H + h].flat[a*N + t]
        z = y.transpose(1, 2).reshape(B, H, dk, N).transpose(2, 3).transpose(1, 2).reshape(B, N, H * dk)
        return self.W_o(z)


class _Branching(nn.Module):
    """Shared forward of the two branching layers (layers.py:590-600, 644-652)."""

    def _both(self, x, second):
        d1 = self.d_hidden_convnn
        if not (_inference(self, x) and not self.training and
                self.pointwise_linear.weight.dtype == x.dtype):
            x1 = self.convnn(x[:, :, :d1])
            x2 = second(x[:, :, d1:])
            return self.pointwise_linear(torch.cat((x1, x2), dim=2))
        # inference: each branch writes its channel slice of one (B, N, C)
        # tensor (no concatenation copy), the ConvNN branch straight from the
        # strided input slice; then the pointwise linear with its bias
        B, N, C = x.shape
        cat = torch.empty((B, N, C), dtype=x.dtype, device=x.device)
        z, d = self.convnn.core(x[:, :, :d1])
        ops.output_proj(d, z, self.convnn.W_o.weight, out=cat[:, :, :d1])
        if isinstance(second, MultiHeadConv1dAttention):
            second(x[:, :, d1:], out=cat[:, :, d1:])
        else:
            cat[:, :, d1:] = second(x[:, :, d1:])
        return ops.linear(cat, self.pointwise_linear.weight, self.pointwise_linear.bias)


class MultiHeadBranchingConv(_Branching):
    """ConvNN on the first ``int(branch_ratio * d_hidden)`` channels, a
    ``MultiHeadConv1dAttention`` on the rest, concatenated and mixed by a
    pointwise linear (layers.py:502-600).  Same constructor, attribute and
    parameter names as the reference."""

    def __init__(self, d_hidden, num_heads, attention_dropout, kernel_size, K, sampling_type,
                 num_samples, sample_padding, magnitude_type, seq_length=197,
                 coordinate_encoding=False, convolution_type='depthwise', softmax_topk_val=True,
                 branch_ratio=0.5):
        super().__init__()
        self.d_hidden = d_hidden
        self.num_heads = num_heads
        self.attention_dropout = attention_dropout
        self.kernel_size = kernel_size
        self.K = K
        self.sampling_type = sampling_type
        self.num_samples = int(num_samples)
        self.sample_padding = int(sample_padding) if sampling_type == 'spatial' else 0
        self.magnitude_type = magnitude_type
        self.seq_length = seq_length
        self.coordinate_encoding = coordinate_encoding
        self.branch_ratio = branch_ratio
        self.d_hidden_convnn = int(self.branch_ratio * d_hidden)
        self.d_hidden_conv1d = d_hidden - self.d_hidden_convnn
        if self.branch_ratio != 0:
            self.convnn = MultiHeadConvNNAttention(
                d_hidden=self.d_hidden_convnn, num_heads=num_heads, attention_dropout=attention_dropout,
                K=K, sampling_type=sampling_type, num_samples=num_samples, sample_padding=sample_padding,
                magnitude_type=magnitude_type, seq_length=seq_length,
                coordinate_encoding=coordinate_encoding, convolution_type=convolution_type,
                softmax_topk_val=softmax_topk_val)
        if self.branch_ratio != 1:
            self.conv1d = MultiHeadConv1dAttention(d_hidden=self.d_hidden_conv1d, num_heads=num_heads,
                                                   kernel_size=kernel_size)
        self.pointwise_linear = nn.Linear(d_hidden, d_hidden)

    def forward(self, x):
        if self.branch_ratio == 0:
            return self.conv1d(x)
        if self.branch_ratio == 1:
            return self.convnn(x)
        return self._both(x, self.conv1d)


class MultiHeadBranchingAttention(_Branching):
    """ConvNN on the first ``int(branch_ratio * d_hidden)`` channels, softmax
    ``MultiHeadAttention`` on the rest, concatenated and mixed by a pointwise
    linear (layers.py:602-652).  As in the reference, ``branch_ratio`` 0 calls
    the ConvNN branch and 1 the attention branch, neither of which exists in
    that case (AttributeError, layers.py:645-648)."""

    def __init__(self, d_hidden, num_heads, attention_dropout, K, sampling_type, num_samples,
                 sample_padding, magnitude_type, seq_length=197, coordinate_encoding=False,
                 convolution_type='depthwise', softmax_topk_val=True, branch_ratio=0.5):
        super().__init__()
        self.d_hidden = d_hidden
        self.num_heads = num_heads
        self.attention_dropout = attention_dropout
        self.K = K
        self.sampling_type = sampling_type
        self.num_samples = int(num_samples)
        self.sample_padding = int(sample_padding) if sampling_type == 'spatial' else 0
        self.magnitude_type = magnitude_type
        self.seq_length = seq_length
        self.coordinate_encoding = coordinate_encoding
        self.branch_ratio = branch_ratio
        self.d_hidden_convnn = int(self.branch_ratio * d_hidden)
        self.d_hidden_attention = d_hidden - self.d_hidden_convnn
        if self.branch_ratio != 0:
            self.convnn = MultiHeadConvNNAttention(
                d_hidden=self.d_hidden_convnn, num_heads=num_heads, attention_dropout=attention_dropout,
                K=K, sampling_type=sampling_type, num_samples=num_samples, sample_padding=sample_padding,
                magnitude_type=magnitude_type, seq_length=seq_length,
                coordinate_encoding=coordinate_encoding, convolution_type=convolution_type,
                softmax_topk_val=softmax_topk_val)
        if self.branch_ratio != 1:
            self.attention = MultiHeadAttention(d_hidden=self.d_hidden_attention, num_heads=num_heads,
                                                attention_dropout=attention_dropout)
        self.pointwise_linear = nn.Linear(d_hidden, d_hidden)

    def forward(self, x):
        if self.branch_ratio == 0:
            return self.convnn(x)
        if self.branch_ratio == 1:
            return self.attention(x)
        return self._both(x, self.attention)


def dropout_keep_scale(p: float) -> float:
    """The factor nn.Dropout applies to kept elements on the GPU: 1/(1-p)
    evaluated as 1.0 / float32(1 - p) in double, then rounded to float32."""
    import numpy as np
    return float(np.float32(1.0 / float(np.float32(1.0 - p))))


class MultiHeadKvtAttention(nn.Module):
    """Top-k sparse softmax attention (layers.py:654-686) on the streaming
    top-k kernel instead of a dense (B, H, N, N) score matrix and scatter mask.

    Each query keeps the ``topk`` keys with the largest q . k * scale (ties:
    lowest key index), softmax over them, weighted sum of their values, heads
    side by side, ``proj``.  That is the operator's own select -> aggregate
    path with the roles of the projections assigned as
    ``W_k := qkv.weight[:C]`` (rows that choose) and ``W_q := qkv.weight[C:2C]``
    (candidates), unit depthwise weights, softmax weights and the concatenated
    head layout; forward and backward both run natively.  ``attn_drop`` draws
    the reference's dense (B, H, N, N) mask and applies it at the kept
    probabilities (the dropped entries of the reference's dense row are zero
    already).  Any ``topk`` runs forward (selections wider than 32 in rounds
    of 32); the backward takes ``topk`` <= 64 (NotImplementedError otherwise).
    ``qkv_bias`` adds the biases in the
    projection GEMM's epilogue; their gradient is the column sums of dQ, dK, dV.
    """

    def __init__(self, dim, num_heads=8, qkv_bias=False, qk_scale=None, attn_drop=0., proj_drop=0.,
                 topk=100):
        super().__init__()
        self.num_heads = num_heads
        head_dim = dim // num_heads
        self.scale = qk_scale or head_dim ** -0.5
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.attn_drop = nn.Dropout(attn_drop)
        self.proj = nn.Linear(dim, dim, bias=False)
        self.proj_drop = nn.Dropout(proj_drop)
        self.topk = topk

    def _dense_dropout_mask(self, B, H, N, x):
        """``attn_drop`` of the reference (layers.py:680) draws its mask over the
        dense (B, H, N, N) probability matrix; the same draw (random numbers,
        element order, dtype) on a tensor of ones gives the mask, whose entries
        at the kept positions become the per-entry multipliers.  Returns
        (mask or None, scale)."""
        p = self.attn_drop.p
        if not self.training or p == 0:
            return None, 1.0
        with torch.no_grad():
            kept = self.attn_drop(torch.ones((B, H, N, N), dtype=x.dtype, device=x.device)) != 0
        return kept, (dropout_keep_scale(p) if p < 1 else 0.0)

    def forward(self, x):
        if not x.is_cuda:
            raise RuntimeError("MultiHeadKvtAttention (cnna) runs on ROCm device tensors only")
        B, N, C = x.shape
        H = self.num_heads
        if self.topk > N:
            raise RuntimeError("selected index k out of range")                # torch.topk
        x, W, P, b = _amp_inputs(x, self.qkv.weight, self.proj.weight, self.qkv.bias)
        # qkv_bias (layers.py:662) in this operator's role order [W_q | W_k | W_v]
        bqkv = None if b is None else torch.cat((b[C:2 * C], b[:C], b[2 * C:]))
        if W.dtype != x.dtype:
            raise RuntimeError(f"mat1 and mat2 must have the same dtype, but got {x.dtype} and "
                               f"{W.dtype}")
        ones = torch.ones((C // H, 1, self.topk), dtype=x.dtype, device=x.device)
        dmask, dscale = self._dense_dropout_mask(B, H, N, x)
        if ops.use_library_ops():
            d = ops.desc_values(B, N, C, H, N, self.topk, N, x.dtype, "matmul", "depthwise", True, False,
                                False, merge=ops.MERGE_CONCAT)
            z = torch.ops.cnna.core(x, W[C:2 * C], W[:C], W[2 * C:], ones, None, None, dmask, d,
                                    float(self.scale), False, dscale, bqkv)[0]
            return self.proj_drop(torch.ops.cnna.output_proj(z, P, d, float(self.scale)))
        d = ops.make_desc(B, N, C, H, N, self.topk, N, x.dtype, "matmul", "depthwise", True, False, False,
                          merge=ops.MERGE_CONCAT, scale=self.scale)
        z = ops.ConvNNCore.apply(x, W[C:2 * C], W[:C], W[2 * C:], ones, None, None, d, False, dmask, dscale,
                                 bqkv)
        return self.proj_drop(ops.OutputProj.apply(z, P, d))
