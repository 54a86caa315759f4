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
        return ops.OutputProj.apply(z, self.W_o.weight, d)

    def core(self, x):
        """Everything before W_o (layers.py:261-317): returns (z, desc), z the
        merged conv output after dropout."""
        if x.dim() != 3:
            raise RuntimeError(f"expected x of shape (B, N, C), got {tuple(x.shape)}")
        if not x.is_cuda:
            raise RuntimeError("MultiHeadConvNNAttention (cnna) runs on ROCm device tensors only")
        B, N, C = x.shape
        self.batch_size = B                                                          # layers.py:239
        cand = self._candidates(x)
        Nq = N if cand is None else int(cand.numel())
        if self.W_q.weight.dtype != x.dtype:
            raise RuntimeError(f"mat1 and mat2 must have the same dtype, but got {x.dtype} and "
                               f"{self.W_q.weight.dtype}")
        d = ops.make_desc(B, N, C, self.num_heads, Nq, self.K, self.seq_length, x.dtype,
                          self.magnitude_type, self.convolution_type, self.softmax_topk_val,
                          cand is not None, self.coordinate_encoding)
        w0, w1 = self._conv_weights()
        z = ops.ConvNNCore.apply(x, self.W_q.weight, self.W_k.weight, self.W_v.weight, w0, w1, cand, d,
                                 True)
        # dropout on the conv output (layers.py:316); elementwise, so applying it
        # after the head merge is the same operation on permuted elements
        return self.dropout(z), d
