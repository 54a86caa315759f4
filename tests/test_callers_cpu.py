"""Host-side checks of the callers' modules (no GPU needed).

The composable (autograd) paths of MultiHeadConv1dAttention and
MultiHeadAttention run on CPU tensors and must equal the oracle's
restatements of layers.py:452-499 and 88-130; the branching layers keep the
reference's constructor, attribute and parameter names (state dicts carry
over) and its channel split int(branch_ratio * d_hidden).
"""
import pytest
import torch

from oracle import cnna_oracle as O
from layers import (MultiHeadAttention, MultiHeadBranchingAttention, MultiHeadBranchingConv,
                    MultiHeadConv1dAttention, MultiHeadKvtAttention)


@pytest.mark.parametrize("H,ks", [(1, 9), (3, 4), (2, 1)])
def test_conv1d_module_matches_oracle(H, ks):
    torch.manual_seed(H * 10 + ks)
    m = MultiHeadConv1dAttention(12 * H, H, ks).double()
    x = torch.randn(2, 11, 12 * H, dtype=torch.float64)
    want = O.conv1d_branch(x, m.W_x.weight, m.W_x.bias, m.conv.weight, m.conv.bias, m.W_o.weight,
                           m.W_o.bias, H)
    torch.testing.assert_close(m(x), want, rtol=1e-12, atol=1e-12)


def test_mha_module_matches_oracle():
    torch.manual_seed(0)
    m = MultiHeadAttention(24, 3, 0.0).eval()
    x = torch.randn(2, 13, 24)
    want = O.mha(x.double(), *(W.weight.double() for W in (m.W_q, m.W_k, m.W_v, m.W_o)), 3)
    torch.testing.assert_close(m(x).double(), want, rtol=1e-5, atol=1e-5)


def test_branching_names_and_split():
    m = MultiHeadBranchingConv(192, 3, 0.1, kernel_size=9, K=9, sampling_type="all", num_samples=-1,
                               sample_padding=0, magnitude_type="matmul", branch_ratio=0.5)
    names = [n for n, _ in m.named_parameters()]
    assert names == ["convnn.W_q.weight", "convnn.W_k.weight", "convnn.W_v.weight", "convnn.W_o.weight",
                     "convnn.conv.weight", "conv1d.W_x.weight", "conv1d.W_x.bias", "conv1d.W_o.weight",
                     "conv1d.W_o.bias", "conv1d.conv.weight", "conv1d.conv.bias",
                     "pointwise_linear.weight", "pointwise_linear.bias"]
    assert (m.d_hidden_convnn, m.d_hidden_conv1d) == (96, 96)
    a = MultiHeadBranchingAttention(192, 3, 0.1, K=9, sampling_type="all", num_samples=-1,
                                    sample_padding=0, magnitude_type="matmul", branch_ratio=0.25)
    assert (a.d_hidden_convnn, a.d_hidden_attention) == (48, 144)
    assert not hasattr(MultiHeadBranchingConv(192, 3, 0.1, 9, 9, "all", -1, 0, "matmul",
                                              branch_ratio=1), "conv1d")


def test_kvt_names_and_scale():
    m = MultiHeadKvtAttention(192, num_heads=3, topk=9)
    assert [n for n, _ in m.named_parameters()] == ["qkv.weight", "proj.weight"]
    assert m.scale == 64 ** -0.5
    assert MultiHeadKvtAttention(192, 3, qk_scale=0.5).scale == 0.5
    with pytest.raises(RuntimeError):
        m(torch.randn(1, 20, 192))           # CPU tensors: no fallback path
