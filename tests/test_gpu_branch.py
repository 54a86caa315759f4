"""Callers of the operator on the GPU (run on an MI355X), against the oracle.

* MultiHeadConv1dAttention's native inference path (cnna_conv1d_branch);
* MultiHeadBranchingConv / MultiHeadBranchingAttention: the ConvNN branch on a
  strided channel slice, branch outputs written into slices of one tensor,
  forward and the training backward through the slice;
* MultiHeadKvtAttention on the select kernel: forward, backward, attention
  dropout with a known mask, and the ViT blocks built on each layer.
Tolerances: fp32 rtol/atol 1e-3 (2e-3 for gradients), bf16 3e-2 against the
float32 oracle on bf16-rounded inputs.
"""
import copy
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import cnna_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops
    from layers import (MultiHeadBranchingAttention, MultiHeadBranchingConv, MultiHeadConv1dAttention,
                        MultiHeadKvtAttention)
    from vit import ViT, vit_tiny_args

DEV = "cuda"


def _cpu(t):
    return None if t is None else t.detach().double().cpu()


def _tol(dtype):
    return dict(rtol=1e-3, atol=1e-3) if dtype == torch.float32 else dict(rtol=3e-2, atol=3e-2)


def _conv1d_oracle(m, x):
    return O.conv1d_branch(_cpu(x), _cpu(m.W_x.weight), _cpu(m.W_x.bias), _cpu(m.conv.weight),
                           _cpu(m.conv.bias), _cpu(m.W_o.weight), _cpu(m.W_o.bias), m.num_heads)


def _convnn_oracle(m, x):
    cfg = O.Config(d_hidden=m.d_hidden, num_heads=m.num_heads, K=m.K, sampling_type=m.sampling_type,
                   magnitude_type=m.magnitude_type, convolution_type=m.convolution_type,
                   softmax_topk_val=m.softmax_topk_val, seq_length=m.seq_length)
    p = O.Params.from_module_state({k: _cpu(v) for k, v in m.state_dict().items()}, m.convolution_type)
    return O.forward(_cpu(x), p, cfg, mode="exact")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,C,H,ks", [(4, 197, 96, 3, 9), (3, 50, 64, 1, 4), (2, 33, 48, 2, 3),
                                        (2, 70, 256, 2, 5), (1, 9, 24, 3, 1)])
def test_conv1d_branch_matches_oracle(dtype, B, N, C, H, ks):
    torch.manual_seed(N + C)
    m = MultiHeadConv1dAttention(C, H, ks).to(DEV).to(dtype).eval()
    x = torch.randn(B, N, C, device=DEV).to(dtype)
    with torch.no_grad():
        got = m(x)
    torch.testing.assert_close(got.double().cpu(), _conv1d_oracle(m, x), **_tol(dtype))
    # the autograd path of the same module agrees
    ref = m(x).detach()
    torch.testing.assert_close(got.float(), ref.float(), **_tol(dtype))


def test_conv1d_branch_into_strided_slice():
    torch.manual_seed(1)
    m = MultiHeadConv1dAttention(48, 3, 3).to(DEV).eval()
    x = torch.randn(2, 40, 100, device=DEV)
    out = torch.full((2, 40, 80), 7.0, device=DEV)
    with torch.no_grad():
        m(x[:, :, 10:58], out=out[:, :, 32:])
    torch.testing.assert_close(out[:, :, 32:].double().cpu(), _conv1d_oracle(m, x[:, :, 10:58]),
                               rtol=1e-3, atol=1e-3)
    assert torch.all(out[:, :, :32] == 7.0)


def _branch_conv(dtype, ratio=0.5, C=192, H=3, K=9, sampling="all", metric="matmul"):
    torch.manual_seed(7)
    return MultiHeadBranchingConv(C, H, 0.0, kernel_size=9, K=K, sampling_type=sampling, num_samples=-1,
                                  sample_padding=0, magnitude_type=metric, seq_length=197,
                                  convolution_type="depthwise", softmax_topk_val=True,
                                  branch_ratio=ratio).to(DEV).to(dtype).eval()


def _branch_attn(dtype, ratio=0.5, C=192, H=3):
    torch.manual_seed(8)
    return MultiHeadBranchingAttention(C, H, 0.0, K=9, sampling_type="all", num_samples=-1,
                                       sample_padding=0, magnitude_type="cosine", seq_length=197,
                                       convolution_type="standard", softmax_topk_val=False,
                                       branch_ratio=ratio).to(DEV).to(dtype).eval()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("metric", ["matmul", "euclidean"])
def test_branching_conv_matches_oracle(dtype, metric):
    m = _branch_conv(dtype, metric=metric)
    x = torch.randn(4, 197, 192, device=DEV).to(dtype)
    with torch.no_grad():
        got = m(x)
    d1 = m.d_hidden_convnn
    want = O.branching_conv(_cpu(x), lambda t: _convnn_oracle(m.convnn, t),
                            lambda t: _conv1d_oracle(m.conv1d, t), _cpu(m.pointwise_linear.weight),
                            _cpu(m.pointwise_linear.bias), d1)
    torch.testing.assert_close(got.double().cpu(), want, **_tol(dtype))


@pytest.mark.parametrize("ratio", [0.25, 0.5, 0.75])
def test_branching_attention_matches_oracle(ratio):
    m = _branch_attn(torch.float32, ratio)
    x = torch.randn(3, 197, 192, device=DEV)
    with torch.no_grad():
        got = m(x)
    a = m.attention
    want = O.branching_conv(_cpu(x), lambda t: _convnn_oracle(m.convnn, t),
                            lambda t: O.mha(t, _cpu(a.W_q.weight), _cpu(a.W_k.weight), _cpu(a.W_v.weight),
                                            _cpu(a.W_o.weight), a.num_heads),
                            _cpu(m.pointwise_linear.weight), _cpu(m.pointwise_linear.bias),
                            m.d_hidden_convnn)
    torch.testing.assert_close(got.double().cpu(), want, rtol=1e-3, atol=1e-3)


def test_branching_single_branch_ratios():
    x = torch.randn(2, 197, 192, device=DEV)
    with torch.no_grad():
        m0 = _branch_conv(torch.float32, ratio=0.0)
        torch.testing.assert_close(m0(x).double().cpu(), _conv1d_oracle(m0.conv1d, x), rtol=1e-3, atol=1e-3)
        m1 = _branch_conv(torch.float32, ratio=1.0)
        torch.testing.assert_close(m1(x).double().cpu(), _convnn_oracle(m1.convnn, x), rtol=1e-3, atol=1e-3)
        # the reference calls the branch it did not build (layers.py:645-648)
        with pytest.raises(AttributeError):
            _branch_attn(torch.float32, ratio=0.0)(x)
        with pytest.raises(AttributeError):
            _branch_attn(torch.float32, ratio=1.0)(x)


def test_branching_conv_backward_through_slice():
    m = _branch_conv(torch.float32, C=96, H=2)
    m.train()
    mc = copy.deepcopy(m).double().cpu()          # oracle network: float64 on the CPU
    x = torch.randn(2, 197, 96, device=DEV, requires_grad=True)
    m(x).square().sum().backward()
    xc = x.detach().double().cpu().requires_grad_(True)
    cv = mc.convnn
    cfg = O.Config(d_hidden=cv.d_hidden, num_heads=2, K=9, magnitude_type="matmul",
                   convolution_type="depthwise", softmax_topk_val=True, seq_length=197)
    p = O.Params(cv.W_q.weight, cv.W_k.weight, cv.W_v.weight, cv.W_o.weight, cv.conv.weight)
    y = O.branching_conv(xc, lambda t: O.forward(t, p, cfg), lambda t: mc.conv1d._forward_modules(t),
                         mc.pointwise_linear.weight, mc.pointwise_linear.bias, m.d_hidden_convnn)
    y.square().sum().backward()
    torch.testing.assert_close(x.grad.double().cpu(), xc.grad, rtol=2e-3, atol=2e-3)
    for (n, a), (_, b) in zip(m.named_parameters(), mc.named_parameters()):
        torch.testing.assert_close(a.grad.double().cpu(), b.grad, rtol=2e-3, atol=2e-3, msg=n)


def _kvt(dtype, C=192, H=3, topk=9, attn_drop=0.0, qk_scale=None, qkv_bias=False):
    torch.manual_seed(11)
    m = MultiHeadKvtAttention(C, num_heads=H, attn_drop=attn_drop, qk_scale=qk_scale, topk=topk,
                              qkv_bias=qkv_bias).to(DEV)
    if qkv_bias:
        with torch.no_grad():
            m.qkv.bias.copy_(torch.randn(3 * C, device=DEV) * 0.5)
    return m.to(dtype).eval()


def _kvt_oracle(m, x, wmul=None):
    H = m.num_heads
    return O.kvt(_cpu(x), _cpu(m.qkv.weight), _cpu(m.proj.weight), H, m.topk, m.scale,
                 wmul=None if wmul is None else wmul.double().cpu(),
                 bqkv=None if m.qkv.bias is None else _cpu(m.qkv.bias))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,C,H,topk,qs", [(8, 197, 192, 3, 9, None), (4, 256, 128, 1, 16, None),
                                             (3, 100, 96, 2, 1, 0.3), (2, 40, 64, 4, 32, None),
                                             (3, 100, 96, 2, 5, -0.3),
                                             (2, 12, 48, 3, 12, None),
                                             # the reference's default topk=100 (rounds of 32)
                                             (2, 197, 192, 3, 100, None), (2, 80, 64, 2, 50, 0.2)])
def test_kvt_forward_matches_oracle(dtype, B, N, C, H, topk, qs):
    m = _kvt(dtype, C, H, topk, qk_scale=qs)
    x = torch.randn(B, N, C, device=DEV).to(dtype)
    with torch.no_grad():
        got = m(x)
    if dtype == torch.float32:
        torch.testing.assert_close(got.double().cpu(), _kvt_oracle(m, x), **_tol(dtype))
        return
    # bf16: the projections are rounded to bf16 (as nn.Linear's output is), so
    # the oracle ranks the kernel's own q / k rows in float64; selections may
    # differ only at near ties (1e-6), the output is the float64 softmax
    # aggregation over the kernel's selection, rounded to bf16 before proj
    W = m.qkv.weight
    d = ops.make_desc(B, N, C, H, N, topk, N, dtype, "matmul", "depthwise", True, False, False,
                      merge=ops.MERGE_CONCAT, scale=m.scale)
    with torch.no_grad():
        q, k, v, _, _ = ops.project_qkv(d, x, None, W[C:2 * C], W[:C], W[2 * C:])
        idx, vals, w = ops.select(d, k, q)
    dk = C // H
    rows, cands, vv = (t[..., :dk].double().cpu() for t in (k, q, v))
    S = torch.matmul(rows, cands.transpose(1, 2)) * m.scale
    _, idx_e = O.stable_topk(S, topk, largest=True)
    idx_g = idx.long().cpu()
    cfg = O.Config(d_hidden=C, num_heads=H, K=topk)
    assert O.topk_gap_ok(S, idx_g, idx_e, cfg, tol=1e-6).all()
    p = torch.softmax(torch.gather(S, -1, idx_g), -1)
    o = (p.unsqueeze(-1) * vv[torch.arange(B * H).view(-1, 1, 1), idx_g]).sum(2)     # (BH, N, dk)
    z = o.view(B, H, N, dk).transpose(1, 2).reshape(B, N, C).to(dtype).double()
    want = z @ _cpu(m.proj.weight).T
    torch.testing.assert_close(got.double().cpu(), want, rtol=1e-2, atol=1e-2)


def test_kvt_errors():
    m = _kvt(torch.float32, 64, 2, topk=50)
    with pytest.raises(RuntimeError, match="out of range"):
        m(torch.randn(1, 20, 64, device=DEV))
    # topk above 64: the forward runs, the backward is beyond the native limit
    m = _kvt(torch.float32, 64, 2, topk=80).train()
    x = torch.randn(1, 100, 64, device=DEV, requires_grad=True)
    y = m(x)
    with pytest.raises(NotImplementedError, match="K <= 64"):
        y.sum().backward()


@pytest.mark.parametrize("H,topk", [(1, 9), (3, 9), (3, 48), (2, 64)])
def test_kvt_backward_matches_oracle(H, topk):
    m = _kvt(torch.float32, 96, H, topk=topk).train()
    x = torch.randn(3, 197, 96, device=DEV, requires_grad=True)
    m(x).square().sum().backward()
    xc = x.detach().double().cpu().requires_grad_(True)
    Wqkv = m.qkv.weight.detach().double().cpu().requires_grad_(True)
    Wp = m.proj.weight.detach().double().cpu().requires_grad_(True)
    O.kvt(xc, Wqkv, Wp, H, topk, m.scale).square().sum().backward()
    torch.testing.assert_close(x.grad.double().cpu(), xc.grad, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(m.qkv.weight.grad.double().cpu(), Wqkv.grad, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(m.proj.weight.grad.double().cpu(), Wp.grad, rtol=2e-3, atol=2e-3)


def test_kvt_attention_dropout_forward_and_backward():
    m = _kvt(torch.float32, 96, 3, topk=9, attn_drop=0.25).train()
    B, N = 2, 197
    x = torch.randn(B, N, 96, device=DEV, requires_grad=True)
    torch.manual_seed(5)
    y = m(x)
    after = torch.rand(16, device=DEV)
    # the reference's draw: attn_drop on the dense (B, H, N, N) probabilities (layers.py:680)
    torch.manual_seed(5)
    dense = F.dropout(torch.ones(B, 3, N, N, device=DEV), 0.25, True)
    assert torch.equal(torch.rand(16, device=DEV), after)      # same random numbers consumed
    assert 0 < (dense == 0).float().mean().item() < 0.5
    y.square().sum().backward()
    xc = x.detach().double().cpu().requires_grad_(True)
    Wqkv = m.qkv.weight.detach().double().cpu().requires_grad_(True)
    yo = O.kvt(xc, Wqkv, m.proj.weight.detach().double().cpu(), 3, 9, m.scale,
               dense_mult=dense.double().cpu())
    torch.testing.assert_close(y.detach().double().cpu(), yo.detach(), rtol=1e-3, atol=1e-3)
    yo.square().sum().backward()
    torch.testing.assert_close(x.grad.double().cpu(), xc.grad, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(m.qkv.weight.grad.double().cpu(), Wqkv.grad, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("layer", ["BranchConv", "BranchAttention", "KvtAttention", "Attention"])
def test_vit_layers_fused_match_composable(layer):
    torch.manual_seed(0)
    args = vit_tiny_args(layer=layer, img_size=(3, 64, 64), patch_size=8, num_layers=2, dropout=0.0,
                         attention_dropout=0.0, K=9)
    model = ViT(args).to(DEV).eval()
    for blk in model.transformer_encoder:
        for mod in blk.modules():
            if hasattr(mod, "seq_length") and hasattr(mod, "coordinate_cache"):
                mod.seq_length = 65
    imgs = torch.randn(4, 3, 64, 64, device=DEV)
    with torch.no_grad():
        fused = model(imgs)
    with torch.enable_grad():
        plain = model(imgs).detach()
    torch.testing.assert_close(fused, plain, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kvt_qkv_bias_forward(dtype):
    """qkv_bias=True (layers.py:662): the biases go into the projection GEMM's
    epilogue in the operator's role order."""
    B, N, C, H, topk = 3, 197, 96, 3, 9
    m = _kvt(dtype, C, H, topk, qkv_bias=True)
    x = torch.randn(B, N, C, device=DEV).to(dtype)
    with torch.no_grad():
        got = m(x)
    if dtype == torch.float32:
        torch.testing.assert_close(got.double().cpu(), _kvt_oracle(m, x), rtol=1e-3, atol=1e-3)
        return
    # bf16: the kernel's own projections equal x W^T + b rounded, and the
    # output is the exact aggregation over the kernel's selection
    W, b = m.qkv.weight, m.qkv.bias
    bq = torch.cat((b[C:2 * C], b[:C], b[2 * C:]))
    d = ops.make_desc(B, N, C, H, N, topk, N, dtype, "matmul", "depthwise", True, False, False,
                      merge=ops.MERGE_CONCAT, scale=m.scale)
    with torch.no_grad():
        q, k, v, _, _ = ops.project_qkv(d, x, None, W[C:2 * C], W[:C], W[2 * C:], bqkv=bq)
    dk = C // H
    ref_k = (x.float() @ W[:C].float().t() + b[:C].float()).view(B, N, H, dk).transpose(1, 2).reshape(B * H, N, dk)
    torch.testing.assert_close(k[..., :dk].float(), ref_k, rtol=1e-2, atol=1e-2)
    with torch.no_grad():
        idx, vals, w = ops.select(d, k, q)
    rows, cands, vv = (t[..., :dk].double().cpu() for t in (k, q, v))
    S = torch.matmul(rows, cands.transpose(1, 2)) * m.scale
    _, idx_e = O.stable_topk(S, topk, largest=True)
    idx_g = idx.long().cpu()
    assert O.topk_gap_ok(S, idx_g, idx_e, O.Config(d_hidden=C, num_heads=H, K=topk), tol=1e-6).all()
    pr = torch.softmax(torch.gather(S, -1, idx_g), -1)
    o = (pr.unsqueeze(-1) * vv[torch.arange(B * H).view(-1, 1, 1), idx_g]).sum(2)
    z = o.view(B, H, N, dk).transpose(1, 2).reshape(B, N, C).to(dtype).double()
    torch.testing.assert_close(got.double().cpu(), z @ _cpu(m.proj.weight).T, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("topk", [9, 40])
def test_kvt_qkv_bias_backward(topk):
    m = _kvt(torch.float32, 96, 3, topk=topk, qkv_bias=True).train()
    x = torch.randn(2, 197, 96, device=DEV, requires_grad=True)
    m(x).square().sum().backward()
    xc = x.detach().double().cpu().requires_grad_(True)
    Wqkv = m.qkv.weight.detach().double().cpu().requires_grad_(True)
    bqkv = m.qkv.bias.detach().double().cpu().requires_grad_(True)
    Wp = m.proj.weight.detach().double().cpu().requires_grad_(True)
    O.kvt(xc, Wqkv, Wp, 3, topk, m.scale, bqkv=bqkv).square().sum().backward()
    torch.testing.assert_close(x.grad.double().cpu(), xc.grad, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(m.qkv.weight.grad.double().cpu(), Wqkv.grad, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(m.qkv.bias.grad.double().cpu(), bqkv.grad, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(m.proj.weight.grad.double().cpu(), Wp.grad, rtol=2e-3, atol=2e-3)


def test_kvt_qkv_bias_compiled_matches_eager():
    m = _kvt(torch.float32, 96, 3, topk=9, qkv_bias=True).train()
    x = torch.randn(2, 100, 96, device=DEV, requires_grad=True)
    y = m(x)
    y.square().sum().backward()
    g_eager = (x.grad.clone(), m.qkv.bias.grad.clone())
    x.grad = None
    m.zero_grad()
    mc = torch.compile(m, fullgraph=True)
    yc = mc(x)
    yc.square().sum().backward()
    torch.testing.assert_close(yc, y, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(x.grad, g_eager[0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(m.qkv.bias.grad, g_eager[1], rtol=1e-5, atol=1e-5)
