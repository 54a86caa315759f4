"""GPU: the drop-in layer's attention dropout is the reference's draw.

The reference applies ``self.dropout`` to the conv output y (B*H, d_k, N)
(layers.py:316), after the ``randperm`` of the sampled paths (layers.py:284).
With the same seed, the drop-in module in training mode must consume the same
random numbers and produce the output of the reference's forward with the
mask that draw gives at y.  The expected output is the oracle (float64) on the
kernel's own neighbour selection with that mask applied at y; gradients are
compared the same way.  Tolerances: fp32 rtol 1e-3, bf16 rtol 2e-2 (absolute
floors at the same fraction of the expected RMS).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import cnna_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops
    from layers import MultiHeadConvNNAttention, dropout_keep_scale

DEV = "cuda"

CASES = [
    # (dtype, H, dk, N, K, sampling, num_samples, conv, p)
    (torch.float32, 3, 32, 64, 9, "all", -1, "depthwise", 0.1),
    (torch.bfloat16, 3, 64, 197, 9, "all", -1, "depthwise", 0.1),
    (torch.float16, 3, 64, 197, 9, "all", -1, "depthwise", 0.1),
    (torch.float32, 1, 24, 50, 5, "all", -1, "standard", 0.3),
    (torch.float32, 2, 16, 40, 6, "random", 20, "depthwise-separable", 0.2),
]


def _tol(dtype, e):
    f = 1e-3 if dtype == torch.float32 else 2e-2
    rms = e.pow(2).mean().sqrt().item()
    return dict(rtol=f, atol=f * rms + 1e-12)


@pytest.mark.parametrize("dtype,H,dk,N,K,sampling,ns,conv,p", CASES)
def test_training_forward_and_backward_use_the_reference_dropout_draw(dtype, H, dk, N, K, sampling, ns, conv, p):
    B, C = 2, H * dk
    torch.manual_seed(0)
    m = MultiHeadConvNNAttention(C, H, p, K, sampling, ns, 0, "matmul", seq_length=N,
                                 convolution_type=conv).to(DEV).to(dtype).train()
    if conv != "depthwise":
        with torch.no_grad():
            for n, t in m.named_parameters():
                if n.startswith("conv"):
                    t.normal_(0, 0.5)
    x = torch.randn(B, N, C, device=DEV).to(dtype).requires_grad_(True)
    dout = torch.randn(B, N, C, device=DEV).to(dtype)
    torch.manual_seed(123)
    out = m(x)
    after = torch.rand(16, device=DEV)
    out.backward(dout)

    # the reference's draws under the same seed: randperm (sampled), then the
    # dropout of y (B*H, d_k, N) in y's dtype (fp32 for sampled paths, whose
    # fp32 ``ones`` promote the gathered tensor, layers.py:374-376)
    torch.manual_seed(123)
    cand = torch.randperm(N, device=DEV)[:ns] if sampling == "random" else None
    ydt = torch.float32 if sampling != "all" else dtype
    kept = F.dropout(torch.ones(B * H, dk, N, device=DEV, dtype=ydt), p, True) != 0
    assert torch.equal(torch.rand(16, device=DEV), after)         # same random numbers consumed
    assert 0 < (~kept).float().mean().item() < 2 * p
    mult = kept.double().cpu() * dropout_keep_scale(p)

    # the kernel's own selection, for the oracle to use (cols)
    Nq = N if cand is None else ns
    d = ops.make_desc(B, N, C, H, Nq, K, N, dtype, "matmul", conv, True, cand is not None, False)
    cg = None if cand is None else cand.to(torch.int32)
    with torch.no_grad():
        q, k, v, qn, kn = ops.project_qkv(d, x.detach(), cg, m.W_q.weight, m.W_k.weight, m.W_v.weight)
        idx, _, _ = ops.select(d, k, q, kn, qn, cg)
    idx = idx.long().cpu()
    if cand is None:
        cols = idx
    else:
        inv = torch.full((N,), -1, dtype=torch.long)
        for j in reversed(range(ns)):
            inv[int(cand[j])] = j
        cols = inv[idx[..., 1:]]
    cfg = O.Config(d_hidden=C, num_heads=H, K=K, sampling_type=sampling, num_samples=ns, seq_length=N,
                   convolution_type=conv)
    w0, w1 = m._conv_weights()
    ts = [None if t is None else t.detach().double().cpu().requires_grad_(True)
          for t in (x, m.W_q.weight, m.W_k.weight, m.W_v.weight, m.W_o.weight, w0, w1)]
    ref = O.forward(ts[0], O.Params(*ts[1:]), cfg, cand=None if cand is None else cand.cpu(), mode="exact",
                    cols=cols, y_dropout=lambda y: y * mult)
    torch.testing.assert_close(out.detach().double().cpu(), ref.detach(), **_tol(dtype, ref.detach()))
    ref.backward(dout.double().cpu())
    got = [x.grad, m.W_q.weight.grad, m.W_k.weight.grad, m.W_v.weight.grad, m.W_o.weight.grad,
           w0.grad, None if w1 is None else w1.grad]
    for name, g, t in zip(("x", "W_q", "W_k", "W_v", "W_o", "conv0", "conv1"), got, ts):
        if t is None:
            continue
        e = t.grad
        if dtype == torch.float32:
            torch.testing.assert_close(g.double().cpu(), e, **_tol(dtype, e), msg=lambda s: f"{name}: {s}")
        else:
            # bf16 gradients: sums of many bf16-rounded products; per-tensor relative L2
            err = ((g.double().cpu() - e).norm() / e.norm()).item()
            assert err < 2e-2, (name, err)


def test_eval_mode_and_zero_p_draw_nothing():
    torch.manual_seed(0)
    m = MultiHeadConvNNAttention(96, 3, 0.0, 9, "all", -1, 0, "matmul", seq_length=64).to(DEV).train()
    x = torch.randn(2, 64, 96, device=DEV)
    torch.manual_seed(1)
    m(x)
    r = torch.rand(4, device=DEV)
    torch.manual_seed(1)
    assert torch.equal(torch.rand(4, device=DEV), r)
    m2 = MultiHeadConvNNAttention(96, 3, 0.5, 9, "all", -1, 0, "matmul", seq_length=64).to(DEV).eval()
    m2.load_state_dict(m.state_dict())
    with torch.no_grad():
        assert torch.equal(m2(x), m(x))
