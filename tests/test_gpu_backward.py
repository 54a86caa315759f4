"""GPU parity of the backward pass (run on an MI355X).

The HIP backward (cnna_core_backward + cnna_output_proj_backward) is compared
with torch autograd through the CPU oracle in float64, on the *same* neighbour
selection: the oracle is given the candidate columns the GPU selected
(``cols``), so gradients are compared on one fixed piecewise-smooth branch of
the function (the reference's own autograd differentiates exactly that branch).

Tolerances: fp32 rtol 1e-3 with an absolute floor of 1e-3 x RMS of the
expected gradient; bf16 element-wise rtol 2e-2 with an absolute floor of
2e-2 x RMS, and relative L2 error 2e-2 per gradient tensor.
"""
import pytest
import torch

from oracle import cnna_oracle as O

from test_gpu_parity import DEV, E2E_CASES, cand_for, desc_for, make

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops
    from layers import MultiHeadConvNNAttention

NAMES = ("x", "W_q", "W_k", "W_v", "W_o", "conv0", "conv1")


def columns(idx, cand, N, cols=None):
    """The candidate columns the GPU selected, for the oracle to use: token
    indices for sampling 'all', the select kernel's own column output for the
    sampled paths (slot 0, the token itself, dropped)."""
    if cand is None:
        return idx.long()
    c = cols[..., 1:].long()
    assert ((c >= 0) & (c < cand.numel())).all()
    assert torch.equal(cand[c], idx[..., 1:].long())     # each column holds the selected token
    return c


def gpu_grads(cfg, p, x, cand, dout):
    B, N, C = x.shape
    Nq = N if cand is None else cand.numel()
    d = desc_for(cfg, B, N, Nq, x.dtype)
    cg = None if cand is None else cand.to(torch.int32).to(DEV)
    ts = [None if t is None else t.to(DEV).requires_grad_(True)
          for t in (x, p.W_q, p.W_k, p.W_v, p.W_o, p.conv0, p.conv1)]
    xg, Wq, Wk, Wv, Wo, w0, w1 = ts
    z = ops.ConvNNCore.apply(xg, Wq, Wk, Wv, w0, w1, cg, d)
    out = ops.OutputProj.apply(z, Wo, d)
    out.backward(dout.to(DEV))
    # the selection the forward made (kernels are deterministic)
    with torch.no_grad():
        q, k, v, qn, kn = ops.project_qkv(d, xg.detach(), cg, Wq.detach(), Wk.detach(), Wv.detach())
        idx, vals, w, cols = ops.select_cols(d, k, q, kn, qn, cg)
    torch.cuda.synchronize()
    grads = {n: (None if t is None else t.grad.detach().cpu()) for n, t in zip(NAMES, ts)}
    return out.detach().cpu(), grads, columns(idx.cpu(), cand, N, None if cols is None else cols.cpu())


def oracle_grads(cfg, p, x, cand, dout, cols):
    ts = [None if t is None else t.detach().double().requires_grad_(True)
          for t in (x, p.W_q, p.W_k, p.W_v, p.W_o, p.conv0, p.conv1)]
    pp = O.Params(*ts[1:])
    out = O.forward(ts[0], pp, cfg, cand=cand, mode="exact", cols=cols)
    out.backward(dout.double())
    return out.detach(), {n: (None if t is None else t.grad) for n, t in zip(NAMES, ts)}


def assert_grads_fp32(got, exp):
    for n in NAMES:
        if exp[n] is None:
            assert got[n] is None
            continue
        e = exp[n]
        g = got[n].double()
        rms = e.pow(2).mean().sqrt().item()
        torch.testing.assert_close(g, e, rtol=1e-3, atol=1e-3 * rms + 1e-12, msg=lambda m: f"{n}: {m}")


def assert_close_bf16(got, exp, name, tol=2e-2):
    """Element-wise bf16 contract: |got - exp| <= tol * |exp| + tol * RMS(exp)."""
    got, exp = got.double().cpu(), exp.double().cpu()
    rms = exp.pow(2).mean().sqrt().item()
    torch.testing.assert_close(got, exp, rtol=tol, atol=tol * rms + 1e-12, msg=lambda m: f"{name}: {m}")


def rel_l2(g, e):
    return ((g.double() - e).norm() / e.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("name,kw,B,N", E2E_CASES, ids=[c[0] for c in E2E_CASES])
def test_backward_fp32(name, kw, B, N):
    cfg = O.Config(**kw)
    p, x = make(cfg, B, N, torch.float32, seed=5)
    cand = cand_for(cfg, N)
    dout = torch.randn(B, N, cfg.d_hidden, generator=torch.Generator().manual_seed(7))
    out, got, cols = gpu_grads(cfg, p, x, cand, dout)
    out_e, exp = oracle_grads(cfg, p, x, cand, dout, cols)
    torch.testing.assert_close(out.double(), out_e, rtol=1e-3, atol=1e-4)
    assert_grads_fp32(got, exp)


BWD_EXTRA = [
    ("cosine_std_softmax_h3", dict(d_hidden=96, num_heads=3, K=6, magnitude_type="cosine", convolution_type="standard", seq_length=50), 2, 50),
    ("matmul_dws_coord", dict(d_hidden=64, num_heads=2, K=5, coordinate_encoding=True, convolution_type="depthwise-separable", seq_length=33), 2, 33),
    ("euclid_all_raw_dw", dict(d_hidden=48, num_heads=3, K=4, magnitude_type="euclidean", softmax_topk_val=False, seq_length=40), 2, 40),
    ("cosine_random_raw_dws", dict(d_hidden=64, num_heads=2, K=6, sampling_type="random", num_samples=16, magnitude_type="cosine", softmax_topk_val=False, convolution_type="depthwise-separable", seq_length=48), 2, 48),
    ("spatial_dup_columns", dict(d_hidden=48, num_heads=3, K=5, sampling_type="spatial", num_samples=40, seq_length=24), 2, 24),
    # duplicate columns whose q rows differ (coordinate channel over the columns),
    # cosine normalisation over that channel: the backward must use the selected column
    ("spatial_dup_cosine_coord", dict(d_hidden=48, num_heads=3, K=6, sampling_type="spatial", num_samples=40, magnitude_type="cosine", coordinate_encoding=True, convolution_type="standard", seq_length=24), 2, 24),
    ("spatial_dup_matmul_coord_dws", dict(d_hidden=32, num_heads=2, K=5, sampling_type="spatial", num_samples=30, coordinate_encoding=True, convolution_type="depthwise-separable", seq_length=17), 2, 17),
    ("k32_dk128", dict(d_hidden=256, num_heads=2, K=32, seq_length=80), 2, 80),
    ("dk128_std_k16", dict(d_hidden=256, num_heads=2, K=16, convolution_type="standard", seq_length=64), 1, 64),
    # depthwise with 20-channel heads: the vector weight-gradient path (fp32, 5 vectors per row)
    ("matmul_dw_dk20", dict(d_hidden=60, num_heads=3, K=7, seq_length=45), 2, 45),
    # K above one select list (rounds of 32) up to the backward's 64
    ("k48_dw_dk64", dict(d_hidden=128, num_heads=2, K=48, seq_length=90), 2, 90),
    ("k64_std_dk32", dict(d_hidden=64, num_heads=2, K=64, convolution_type="standard", seq_length=100), 1, 100),
    ("k40_random_cosine_dws", dict(d_hidden=64, num_heads=2, K=40, sampling_type="random", num_samples=60, magnitude_type="cosine", convolution_type="depthwise-separable", seq_length=80), 2, 80),
]


@pytest.mark.parametrize("name,kw,B,N", BWD_EXTRA, ids=[c[0] for c in BWD_EXTRA])
def test_backward_fp32_more(name, kw, B, N):
    test_backward_fp32(name, kw, B, N)


@pytest.mark.parametrize("conv,N,C,K", [("standard", 512, 768, 16), ("depthwise", 1024, 384, 9),
                                        ("depthwise", 256, 768, 32), ("depthwise", 197, 192, 9),
                                        ("depthwise", 64, 60, 7), ("depthwise", 197, 192, 64)])
def test_backward_bf16(conv, N, C, K):
    """bf16 at config-5 / config-3 / ViT head sizes (batch reduced); 20-channel
    heads take the element-wise weight-gradient path (rows not whole 16-byte
    vectors)."""
    cfg = O.Config(d_hidden=C, num_heads=3, K=K, convolution_type=conv, seq_length=N)
    B = 2
    p, x = make(cfg, B, N, torch.bfloat16, seed=11)
    dout = torch.randn(B, N, C, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    out, got, cols = gpu_grads(cfg, p, x, None, dout)
    out_e, exp = oracle_grads(cfg, p, x, None, dout, cols)
    assert_close_bf16(out, out_e, "out")
    assert rel_l2(out, out_e) < 2e-2
    for n in NAMES:
        if exp[n] is None:
            continue
        # element-wise at the bf16 contract (rtol 2e-2, absolute floor 2e-2 x RMS)
        assert_close_bf16(got[n], exp[n], n)
        err = rel_l2(got[n], exp[n])
        assert err < 2e-2, (n, err)


def test_backward_deterministic():
    cfg = O.Config(d_hidden=192, num_heads=3, K=9, seq_length=197, convolution_type="standard")
    p, x = make(cfg, 3, 197, torch.float32, seed=2)
    dout = torch.randn(3, 197, 192, generator=torch.Generator().manual_seed(1))
    _, g1, _ = gpu_grads(cfg, p, x, None, dout)
    _, g2, _ = gpu_grads(cfg, p, x, None, dout)
    for n in NAMES:
        if g1[n] is not None:
            assert torch.equal(g1[n], g2[n]), n


def test_module_training_step():
    """The drop-in module trains: loss.backward() fills every parameter's grad
    with the oracle's values (dropout 0, sampling 'all')."""
    torch.manual_seed(0)
    m = MultiHeadConvNNAttention(192, 3, 0.0, 9, "all", -1, 0, "matmul", seq_length=65).to(DEV)
    x = torch.randn(4, 65, 192, device=DEV, requires_grad=True)
    out = m(x)
    loss = out.float().pow(2).mean()
    loss.backward()
    torch.cuda.synchronize()
    sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    cfg = O.Config(d_hidden=192, num_heads=3, K=9, seq_length=65)
    p = O.Params.from_module_state(sd, "depthwise")
    d = desc_for(cfg, 4, 65, 65, torch.float32)
    with torch.no_grad():
        q, k, v, qn, kn = ops.project_qkv(d, x.detach(), None, m.W_q.weight, m.W_k.weight, m.W_v.weight)
        idx, _, _ = ops.select(d, k, q, kn, qn, None)
    ts = [t.double().requires_grad_(True) for t in (x.detach().cpu(), p.W_q, p.W_k, p.W_v, p.W_o, p.conv0)]
    ref = O.forward(ts[0], O.Params(*ts[1:]), cfg, mode="exact", cols=idx.cpu().long())
    ref.pow(2).mean().backward()
    pairs = [(x.grad, ts[0]), (m.W_q.weight.grad, ts[1]), (m.W_k.weight.grad, ts[2]),
             (m.W_v.weight.grad, ts[3]), (m.W_o.weight.grad, ts[4]), (m.conv.weight.grad, ts[5])]
    for g, t in pairs:
        e = t.grad
        rms = e.pow(2).mean().sqrt().item()
        torch.testing.assert_close(g.cpu().double(), e, rtol=1e-3, atol=1e-3 * rms + 1e-12)


def test_module_sampled_euclidean_backward_raises_like_reference():
    """The reference's backward fails for sampled euclidean (in-place self mask
    on the sqrt output); the drop-in raises the same RuntimeError there, while
    the C-ABI differentiates it (covered by the fp32 cases above)."""
    m = MultiHeadConvNNAttention(48, 3, 0.0, 4, "random", 8, 0, "euclidean", seq_length=20).to(DEV)
    x = torch.randn(2, 20, 48, device=DEV, requires_grad=True)
    out = m(x)
    with pytest.raises(RuntimeError):
        out.sum().backward()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_output_proj_backward_with_noncontiguous_z(dtype):
    """z reaching W_o may be a permuted view (the dropout re-layout of the
    training path): the gradients come back row-major and correct."""
    B, N, C = 2, 40, 96
    d = ops.make_desc(B, N, C, 3, N, 9, N, dtype, "matmul", "depthwise", True, False, False)
    base = torch.randn(B, C, N, device=DEV).to(dtype)
    z = base.transpose(1, 2).requires_grad_(True)            # (B, N, C), strides (C*N, 1, N)
    z.retain_grad()
    assert not z.is_contiguous()
    Wo = (torch.randn(C, C, device=DEV) / C ** 0.5).to(dtype).requires_grad_(True)
    g = torch.randn(B, N, C, device=DEV).to(dtype)
    out = ops.OutputProj.apply(z, Wo, d)
    out.backward(g)
    zz, WW, gg = (t.detach().double().cpu() for t in (z, Wo, g))
    tol = dict(rtol=1e-4, atol=1e-4) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(out.detach().double().cpu(), zz @ WW.T, **tol)
    torch.testing.assert_close(z.grad.double().cpu(), gg @ WW, **tol)
    torch.testing.assert_close(Wo.grad.double().cpu(), gg.reshape(-1, C).T @ zz.reshape(-1, C),
                               rtol=tol["rtol"], atol=tol["atol"] * 10)
