"""ViT harness around the MI355X ConvNN-Attention layer.

Restates the parts of the reference ViT (vit.py:22-270) that the ConvNN-ViT
configuration uses: patch embedding (Conv2d + LayerNorm), class token and
sinusoidal positional encoding, pre-norm transformer blocks, GELU MLP and the
CLS classifier.  Module and parameter names follow the reference so state
dicts carry over.  The block's attention (vit.py:186-203) is one of
``ConvNNAttention`` (the operator), ``BranchConv`` / ``BranchAttention`` (the
operator on a channel slice beside a Conv1d or softmax-attention branch),
``KvtAttention`` (top-k attention on the operator's select kernel) or
``Attention``; the reference's Local / Neighborhood / Sparse attention
families are outside this operator's scope and raise ValueError.

In inference (eval mode, no gradients, no autocast, not being traced) the
blocks run with their prologues and epilogues fused.  With ConvNN attention
both LayerNorms are folded: the GEMM that writes a residual-stream row (W_o +
residual, fc2 + residual) also writes the row's statistics in its epilogue
(bf16; fp32 takes a statistics pass over the row instead), and the GEMM that
consumes the row (the next block's Q/K/V projection, fc1) normalises it as it
loads it; the first block's statistics come from a pre-pass (cnna_row_stats,
cnna_linear_ln, cnna_project_qkv_ex).  Other layers keep a LayerNorm kernel in
front of the attention and the residual add inside the second LayerNorm.
fc1 + bias + GELU and fc2 + bias + residual are GEMM epilogues throughout.
Training and autograd use the composable modules.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn as nn

import cnna_ops as ops
from layers import (MultiHeadAttention, MultiHeadBranchingAttention, MultiHeadBranchingConv,
                    MultiHeadConvNNAttention, MultiHeadKvtAttention)


def vit_tiny_args(**overrides) -> SimpleNamespace:
    """The reference CLI defaults for ViT-Tiny (main.py:32-113); softmax_topk_val
    is True there whatever the flags say (main.py:48-49 sets the default of a
    store_true flag to True)."""
    a = dict(layer="ConvNNAttention", img_size=(3, 224, 224), patch_size=16, num_layers=12,
             num_heads=3, d_hidden=192, d_mlp=768, dropout=0.1, attention_dropout=0.1,
             num_classes=10, K=9, sampling_type="all", num_samples=-1, sample_padding=0,
             magnitude_type="matmul", coordinate_encoding=False, convolution_type="depthwise",
             softmax_topk_val=True, kernel_size=9, branch_ratio=0.5)
    a.update(overrides)
    return SimpleNamespace(**a)


class PatchEmbedding(nn.Module):
    """Conv2d(kernel = stride = patch) -> flatten -> (B, n_patches, d) -> LayerNorm (vit.py:91-111)."""

    def __init__(self, d_hidden, img_size, patch_size, n_channels=3):
        super().__init__()
        self.linear_projection = nn.Conv2d(n_channels, d_hidden, kernel_size=patch_size,
                                           stride=patch_size)
        self.norm = nn.LayerNorm(d_hidden)
        self.flatten = nn.Flatten(start_dim=2)

    def forward(self, x):
        if (x.is_cuda and not self.training and not torch.is_grad_enabled() and self.norm.weight.dtype == x.dtype
                and not torch.is_autocast_enabled("cuda") and not ops.use_library_ops()):
            # inference: the stride = kernel convolution is a GEMM over the patches
            # (one permuting copy, the MFMA GEMM with its bias, the LayerNorm kernel)
            conv = self.linear_projection
            B, cin, h, w = x.shape
            p, q = conv.kernel_size
            patches = x.view(B, cin, h // p, p, w // q, q).permute(0, 2, 4, 1, 3, 5).reshape(
                B, (h // p) * (w // q), cin * p * q)
            y = ops.linear(patches, conv.weight.reshape(conv.out_channels, -1), conv.bias)
            return ops.layernorm(y, self.norm.weight, self.norm.bias, self.norm.eps)
        x = self.flatten(self.linear_projection(x)).transpose(1, 2)
        return self.norm(x)


class PositionalEncoding(nn.Module):
    """Class token + sinusoidal table (vit.py:113-133)."""

    def __init__(self, d_hidden, max_seq_length):
        super().__init__()
        self.cls_tokens = nn.Parameter(torch.randn(1, 1, d_hidden))
        pe = torch.zeros(max_seq_length, d_hidden)
        position = torch.arange(0, max_seq_length, dtype=torch.float).unsqueeze(1)
        div_term = torch.exp(torch.arange(0, d_hidden, 2).float() * (-math.log(10000.0) / d_hidden))
        pe[:, 0::2] = torch.sin(position * div_term)
        pe[:, 1::2] = torch.cos(position * div_term)
        self.register_buffer("pe", pe.unsqueeze(0))

    def forward(self, x):
        x = torch.cat((self.cls_tokens.expand(x.shape[0], -1, -1), x), dim=1)
        return x + self.pe[:, :x.size(1)].to(x.device)


class TransformerEncoder(nn.Module):
    """Pre-norm attention and MLP with residuals (vit.py:135-270)."""

    def __init__(self, args, d_hidden, d_mlp, num_heads, dropout, attention_dropout):
        super().__init__()
        # vit.py:147-203; no seq_length is passed (default 197)
        convnn = dict(K=args.K, sampling_type=args.sampling_type, num_samples=args.num_samples,
                      sample_padding=args.sample_padding, magnitude_type=args.magnitude_type,
                      coordinate_encoding=args.coordinate_encoding,
                      convolution_type=args.convolution_type, softmax_topk_val=args.softmax_topk_val)
        if args.layer == "Attention":
            self.attention = MultiHeadAttention(d_hidden, num_heads, attention_dropout)
        elif args.layer == "ConvNNAttention":
            self.attention = MultiHeadConvNNAttention(d_hidden, num_heads, attention_dropout, **convnn)
        elif args.layer == "BranchConv":
            self.attention = MultiHeadBranchingConv(d_hidden, num_heads, attention_dropout,
                                                    kernel_size=args.kernel_size,
                                                    branch_ratio=args.branch_ratio, **convnn)
        elif args.layer == "BranchAttention":
            self.attention = MultiHeadBranchingAttention(d_hidden, num_heads, attention_dropout,
                                                         branch_ratio=args.branch_ratio, **convnn)
        elif args.layer == "KvtAttention":
            self.attention = MultiHeadKvtAttention(dim=d_hidden, num_heads=num_heads,
                                                   attn_drop=attention_dropout, topk=args.K)
        else:
            raise ValueError(f"layer {args.layer!r} is not built here; one of 'Attention', "
                             "'ConvNNAttention', 'BranchConv', 'BranchAttention', 'KvtAttention'")
        self.norm1 = nn.LayerNorm(d_hidden)
        self.norm2 = nn.LayerNorm(d_hidden)
        self.dropout1 = nn.Dropout(dropout)
        self.dropout2 = nn.Dropout(dropout)
        self.mlp = nn.Sequential(nn.Linear(d_hidden, d_mlp), nn.GELU(), nn.Dropout(dropout),
                                 nn.Linear(d_mlp, d_hidden))

    def forward(self, x):
        if self._fusable(x):
            return self._forward_fused(x)[0]
        x = x + self.dropout1(self.attention(self.norm1(x)))
        return x + self.dropout2(self.mlp(self.norm2(x)))

    def _fusable(self, x):
        """Inference on the GPU: dropout inactive and nothing to differentiate."""
        if self.training or not x.is_cuda or torch.is_autocast_enabled("cuda") or ops.use_library_ops():
            return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        return self.norm1.weight.dtype == x.dtype

    def _foldable(self, x):
        return (isinstance(self.attention, MultiHeadConvNNAttention) and x.shape[-1] <= 1024
                and self.mlp[0].in_features == x.shape[-1])

    def _forward_fused(self, x, stats=None):
        """The same block with its prologue and epilogues fused.  Returns the
        block output and, with ConvNN attention, its row statistics
        (cnna_ops.FoldedNorm) for the next block's folded norm1; ``stats``:
        those of x from the previous block (computed here when None).

        ConvNN attention: norm1 folded into the Q/K/V projection, W_o with the
        residual add and the statistics of x1 = x + attention in its epilogue,
        norm2 folded into fc1 (bias + GELU epilogue), fc2 with bias + residual
        and the output's statistics in its epilogue.  Other layers: LayerNorm
        kernel, the layer, the residual add fused into norm2, fc1 and fc2 with
        their epilogues."""
        fc1, fc2 = self.mlp[0], self.mlp[3]
        if self._foldable(x):
            if stats is None:
                stats = ops.row_stats(x)
            z, _ = self.attention.core_folded(x, stats.with_norm(self.norm1))
            x1, st1 = ops.linear(z, self.attention.W_o.weight, residual=x, want_stats=True)
            m = ops.linear(x1, fc1.weight, fc1.bias, gelu=True, ln=st1.with_norm(self.norm2))
            return ops.linear(m, fc2.weight, fc2.bias, residual=x1, want_stats=True)
        h = ops.layernorm(x, self.norm1.weight, self.norm1.bias, self.norm1.eps)
        a = self.attention(h)
        h2, x1 = ops.layernorm(a, self.norm2.weight, self.norm2.bias, self.norm2.eps, residual=x,
                               want_sum=True)
        m = ops.linear(h2, fc1.weight, fc1.bias, gelu=True)
        return ops.linear(m, fc2.weight, fc2.bias, residual=x1), None


class ViT(nn.Module):
    """ViT with ConvNN-Attention blocks (vit.py:22-80)."""

    def __init__(self, args):
        super().__init__()
        assert args.img_size[1] % args.patch_size == 0 and args.img_size[2] % args.patch_size == 0
        assert args.d_hidden % args.num_heads == 0
        self.args = args
        img = args.img_size[1:]
        patch = (args.patch_size, args.patch_size)
        n_patches = (img[0] * img[1]) // (patch[0] * patch[1])
        self.patch_embedding = PatchEmbedding(args.d_hidden, img, patch, args.img_size[0])
        self.positional_encoding = PositionalEncoding(args.d_hidden, n_patches + 1)
        self.transformer_encoder = nn.Sequential(*[
            TransformerEncoder(args, args.d_hidden, args.d_mlp, args.num_heads, args.dropout,
                               args.attention_dropout) for _ in range(args.num_layers)])
        self.classifier = nn.Linear(args.d_hidden, args.num_classes)

    def forward(self, x):
        x = self.positional_encoding(self.patch_embedding(x))
        blocks = self.transformer_encoder
        if len(blocks) and blocks[0]._fusable(x):
            # fused inference: each block hands its output's row statistics on
            stats = None
            for blk in blocks:
                x, stats = blk._forward_fused(x, stats)
        else:
            x = blocks(x)
        return self.classifier(x[:, 0])
