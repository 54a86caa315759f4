"""ViT harness around the MI355X ConvNN-Attention layer.

Restates the parts of the reference ViT (vit.py:22-270) that the ConvNN-ViT
configuration uses: patch embedding (Conv2d + LayerNorm), class token and
sinusoidal positional encoding, pre-norm transformer blocks whose attention is
``MultiHeadConvNNAttention`` (vit.py:190), GELU MLP and the CLS classifier.
Module and parameter names follow the reference so state dicts carry over.
Only ``layer="ConvNNAttention"`` is built here; the other attention families
of the reference are outside this operator's scope and raise ValueError.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn as nn

from layers import MultiHeadConvNNAttention


def vit_tiny_args(**overrides) -> SimpleNamespace:
    """The reference CLI defaults for ViT-Tiny (main.py:32-113)."""
    a = dict(layer="ConvNNAttention", img_size=(3, 224, 224), patch_size=16, num_layers=12,
             num_heads=3, d_hidden=192, d_mlp=768, dropout=0.1, attention_dropout=0.1,
             num_classes=10, K=9, sampling_type="all", num_samples=-1, sample_padding=0,
             magnitude_type="matmul", coordinate_encoding=False, convolution_type="depthwise",
             softmax_topk_val=False)
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
        if args.layer != "ConvNNAttention":
            raise ValueError(f"layer {args.layer!r} is not built here; only 'ConvNNAttention'")
        # vit.py:190 passes no seq_length (default 197)
        self.attention = MultiHeadConvNNAttention(
            d_hidden, num_heads, attention_dropout, K=args.K, sampling_type=args.sampling_type,
            num_samples=args.num_samples, sample_padding=args.sample_padding,
            magnitude_type=args.magnitude_type, coordinate_encoding=args.coordinate_encoding,
            convolution_type=args.convolution_type, softmax_topk_val=args.softmax_topk_val)
        self.norm1 = nn.LayerNorm(d_hidden)
        self.norm2 = nn.LayerNorm(d_hidden)
        self.dropout1 = nn.Dropout(dropout)
        self.dropout2 = nn.Dropout(dropout)
        self.mlp = nn.Sequential(nn.Linear(d_hidden, d_mlp), nn.GELU(), nn.Dropout(dropout),
                                 nn.Linear(d_mlp, d_hidden))

    def forward(self, x):
        x = x + self.dropout1(self.attention(self.norm1(x)))
        return x + self.dropout2(self.mlp(self.norm2(x)))


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
        x = self.transformer_encoder(x)
        return self.classifier(x[:, 0])
