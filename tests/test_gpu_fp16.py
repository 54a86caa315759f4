"""float16 kernels (run on an MI355X): the reference's AMP loop runs under
``torch.autocast('cuda')`` whose default type is float16 (train_eval.py:137-146).

Each stage in float16 against the oracle on the kernel's own intermediates
(the selection rule and tolerances of the bf16 tests; float16 keeps 10
mantissa bits, so its tolerances are tighter: 1e-2 relative), the backward
against oracle autograd on the GPU's selection, the ViT block's fused float16
path against its composable modules, and autocast: the layer computes in
autocast's own type and its gradients reach the fp32 weights.
"""
import copy

import pytest
import torch
import torch.nn.functional as F

from oracle import cnna_oracle as O

from test_gpu_parity import check_select, make, run_stages
from test_gpu_backward import NAMES, gpu_grads, oracle_grads, rel_l2

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops
    from layers import MultiHeadConvNNAttention, MultiHeadKvtAttention
    from vit import ViT, vit_tiny_args

DEV = "cuda"
H16 = torch.float16


def test_projection_headsplit_fp16():
    cfg = O.Config(d_hidden=192, num_heads=3, K=4, seq_length=65)
    p, x = make(cfg, 4, 65, H16, seed=11)
    _, r = run_stages(cfg, p, x, None)
    for name, W in (("q", p.W_q), ("k", p.W_k), ("v", p.W_v)):
        ref = O.split_heads(x.float() @ W.float().t(), 3).transpose(1, 2)
        torch.testing.assert_close(r[name][..., :64].float(), ref, rtol=2e-3, atol=2e-3)


FP16_CASES = [
    ("matmul_N1024", dict(d_hidden=384, num_heads=3, K=9, seq_length=1024), 2, 1024),
    ("cosine_N197", dict(d_hidden=192, num_heads=3, K=9, magnitude_type="cosine", seq_length=197), 4, 197),
    ("euclid_dw", dict(d_hidden=64, num_heads=2, K=5, magnitude_type="euclidean", seq_length=150), 3, 150),
    ("k16_d256_std", dict(d_hidden=768, num_heads=3, K=16, convolution_type="standard", seq_length=300), 1, 300),
    ("random_dws", dict(d_hidden=192, num_heads=3, K=9, sampling_type="random", num_samples=64, convolution_type="depthwise-separable", seq_length=197), 2, 197),
    ("k40_wide", dict(d_hidden=96, num_heads=3, K=40, seq_length=120), 2, 120),
]


@pytest.mark.parametrize("name,kw,B,N", FP16_CASES, ids=[c[0] for c in FP16_CASES])
def test_stages_fp16(name, kw, B, N):
    cfg = O.Config(**kw)
    p, x = make(cfg, B, N, H16, seed=5)
    cand = None
    if cfg.sampling_type != "all":
        cand = O.sample_indices(cfg, N, generator=torch.Generator().manual_seed(2))
    _, r = run_stages(cfg, p, x, cand)
    check_select(cfg, r, cand, B)
    z_exp = O.aggregate_exact(r["v"], r["idx"], r["vals"], p, cfg, B, cand is not None)
    torch.testing.assert_close(r["z"].double(), z_exp, rtol=1e-2, atol=1e-2 * z_exp.abs().max().item())
    out_exp = r["z"].double().to(H16).double() @ p.W_o.double().t()
    torch.testing.assert_close(r["out"].double(), out_exp, rtol=1e-2, atol=1e-2 * out_exp.abs().max().item())


def test_forward_fp16_end_to_end_c3_shape():
    """Config-3 shape (B reduced): end-to-end against the exact oracle on the
    same float16 inputs, as the bf16 test, at half its tolerance."""
    cfg = O.Config(d_hidden=384, num_heads=3, K=9, seq_length=1024)
    B, N = 2, 1024
    p, x = make(cfg, B, N, H16, seed=1, rand_conv=False)
    _, r = run_stages(cfg, p, x, None)
    check_select(cfg, r, None, B)
    ref = O.forward(x, p, cfg, mode="exact")
    rms = ref.double().pow(2).mean().sqrt().item()
    err = (r["out"].double() - ref.double()).pow(2).mean().sqrt().item()
    assert err < 1e-2 * rms * 3, (err, rms)


@pytest.mark.parametrize("conv,N,C,K", [("standard", 256, 384, 16), ("depthwise", 197, 192, 9),
                                        ("depthwise-separable", 100, 96, 5)])
def test_backward_fp16(conv, N, C, K):
    cfg = O.Config(d_hidden=C, num_heads=3, K=K, convolution_type=conv, seq_length=N)
    B = 2
    p, x = make(cfg, B, N, H16, seed=11)
    dout = torch.randn(B, N, C, generator=torch.Generator().manual_seed(13)).to(H16)
    out, got, cols = gpu_grads(cfg, p, x, None, dout)
    out_e, exp = oracle_grads(cfg, p, x, None, dout, cols)
    assert rel_l2(out, out_e) < 1e-2
    for n in NAMES:
        if exp[n] is None:
            continue
        err = rel_l2(got[n], exp[n])
        assert err < 1e-2, (n, err)


@pytest.mark.parametrize("amp", [torch.float16, torch.bfloat16])
def test_autocast_computes_in_autocast_dtype(amp):
    torch.manual_seed(0)
    m = MultiHeadConvNNAttention(96, 3, 0.0, 7, "all", -1, 0, "matmul", seq_length=128).to(DEV)
    m16 = copy.deepcopy(m).to(amp)
    x = torch.randn(2, 128, 96, device=DEV, requires_grad=True)
    with torch.autocast("cuda", dtype=amp):
        y = m(x)
    assert y.dtype == amp
    y.float().square().sum().backward()
    assert m.W_q.weight.grad.dtype == torch.float32 and x.grad.dtype == torch.float32
    # exactly the reduced-type layer on the rounded inputs and weights
    x16 = x.detach().to(amp).requires_grad_(True)
    y16 = m16(x16)
    y16.float().square().sum().backward()
    assert torch.equal(y, y16)
    for (n, a), (_, b) in zip(m.named_parameters(), m16.named_parameters()):
        assert torch.equal(a.grad, b.grad.float()), n


@pytest.mark.parametrize("mode", ["plain", "bias_gelu", "bias_res"])
def test_linear_and_layernorm_fp16(mode):
    torch.manual_seed(3)
    M, Nout, Kd = 1000, 768, 192
    a = torch.randn(M, Kd, device=DEV).to(H16)
    W = (torch.randn(Nout, Kd, device=DEV) / Kd ** 0.5).to(H16)
    bias = torch.randn(Nout, device=DEV).to(H16) if mode.startswith("bias") else None
    res = torch.randn(M, Nout, device=DEV).to(H16) if mode.endswith("res") else None
    out = ops.linear(a, W, bias, gelu=mode == "bias_gelu", residual=res)
    ref = F.linear(a.float(), W.float(), None if bias is None else bias.float()).to(H16)
    if mode == "bias_gelu":
        ref = F.gelu(ref.float()).to(H16)
    if res is not None:
        ref = (ref.float() + res.float()).to(H16)
    torch.testing.assert_close(out.float(), ref.float(), rtol=5e-3, atol=5e-3)
    g = (torch.rand(Kd, device=DEV) + 0.5).to(H16)
    b = torch.randn(Kd, device=DEV).to(H16)
    y = ops.layernorm(a, g, b, 1e-5)
    torch.testing.assert_close(y.float(), F.layer_norm(a.float(), (Kd,), g.float(), b.float(), 1e-5),
                               rtol=2e-3, atol=2e-3)
    # folded LayerNorm and the statistics epilogue in float16
    norm = torch.nn.LayerNorm(Kd).to(DEV).to(H16)
    with torch.no_grad():
        norm.weight.copy_(g)
        norm.bias.copy_(b)
    got = ops.linear(a, W, bias, ln=ops.row_stats(a).with_norm(norm))
    want = ops.linear(ops.layernorm(a, g, b, 1e-5), W, bias)
    torch.testing.assert_close(got.float(), want.float(), rtol=5e-3, atol=5e-3)
    o, st = ops.linear(a, W, bias, residual=res, want_stats=True)
    assert ops._stats_epilogue_ok(o.view(M, Nout), res)
    torch.testing.assert_close(st.stats, ops.row_stats(o).stats, rtol=1e-5, atol=1e-4)


def test_vit_fused_blocks_fp16_as_accurate_as_composable():
    torch.manual_seed(0)
    args = vit_tiny_args(img_size=(3, 64, 64), patch_size=8, num_layers=3, dropout=0.0, attention_dropout=0.0)
    model32 = ViT(args).to(DEV).eval()
    for blk in model32.transformer_encoder:
        blk.attention.seq_length = 65
    model16 = copy.deepcopy(model32).to(H16)
    imgs = torch.randn(16, 3, 64, 64, device=DEV)
    with torch.no_grad():
        ref = model32(imgs)
        fused = model16(imgs.to(H16)).float()
    with torch.enable_grad():
        plain = model16(imgs.to(H16)).float().detach()
    err_f = ((fused - ref).norm() / ref.norm()).item()
    err_p = ((plain - ref).norm() / ref.norm()).item()
    assert err_f <= 1.5 * err_p + 0.01, (err_f, err_p)


def test_kvt_fp16_matches_oracle_on_own_projections():
    torch.manual_seed(11)
    B, N, C, H, topk = 4, 197, 192, 3, 9
    m = MultiHeadKvtAttention(C, num_heads=H, topk=topk).to(DEV).to(H16).eval()
    x = torch.randn(B, N, C, device=DEV).to(H16)
    with torch.no_grad():
        got = m(x)
    W = m.qkv.weight
    d = ops.make_desc(B, N, C, H, N, topk, N, H16, "matmul", "depthwise", True, False, False,
                      merge=ops.MERGE_CONCAT, scale=m.scale)
    with torch.no_grad():
        q, k, v, _, _ = ops.project_qkv(d, x, None, W[C:2 * C], W[:C], W[2 * C:])
        idx, vals, w = ops.select(d, k, q)
    dk = C // H
    rows, cands, vv = (t[..., :dk].double().cpu() for t in (k, q, v))
    S = torch.matmul(rows, cands.transpose(1, 2)) * m.scale
    _, idx_e = O.stable_topk(S, topk, largest=True)
    idx_g = idx.long().cpu()
    assert O.topk_gap_ok(S, idx_g, idx_e, O.Config(d_hidden=C, num_heads=H, K=topk), tol=1e-6).all()
    pr = torch.softmax(torch.gather(S, -1, idx_g), -1)
    o = (pr.unsqueeze(-1) * vv[torch.arange(B * H).view(-1, 1, 1), idx_g]).sum(2)
    z = o.view(B, H, N, dk).transpose(1, 2).reshape(B, N, C).to(H16).double()
    want = z @ m.proj.weight.detach().double().cpu().T
    torch.testing.assert_close(got.double().cpu(), want, rtol=5e-3, atol=5e-3)


@pytest.mark.parametrize("topk,bias", [(9, True), (48, False)])
def test_kvt_fp16_backward(topk, bias):
    """float16 KVT training step (qkv_bias, and a selection wider than one
    32-entry list) against oracle autograd in float64 (relative L2 1e-2)."""
    torch.manual_seed(11)
    C, H = 96, 3
    m = MultiHeadKvtAttention(C, num_heads=H, topk=topk, qkv_bias=bias).to(DEV)
    if bias:
        with torch.no_grad():
            m.qkv.bias.normal_(0, 0.5)
    m = m.to(H16).train()
    x = torch.randn(2, 197, C, device=DEV).to(H16).requires_grad_(True)
    m(x).float().square().sum().backward()
    xc = x.detach().double().cpu().requires_grad_(True)
    Wqkv = m.qkv.weight.detach().double().cpu().requires_grad_(True)
    bq = None if not bias else m.qkv.bias.detach().double().cpu().requires_grad_(True)
    Wp = m.proj.weight.detach().double().cpu().requires_grad_(True)
    O.kvt(xc, Wqkv, Wp, H, topk, m.scale, bqkv=bq).square().sum().backward()
    pairs = [(x.grad, xc.grad), (m.qkv.weight.grad, Wqkv.grad), (m.proj.weight.grad, Wp.grad)]
    if bias:
        pairs.append((m.qkv.bias.grad, bq.grad))
    for g, e in pairs:
        assert rel_l2(g.cpu(), e) < 2e-2, rel_l2(g.cpu(), e)
