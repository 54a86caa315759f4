"""torch.compile / autocast / FLOP-counter integration on the GPU (run on an MI355X).

* ``torch.compile(..., fullgraph=True)`` traces the layers through the
  ``cnna::`` library ops (no graph break) and the compiled forward and
  backward equal eager;
* the reference loop's ``torch.compile(model, fullgraph=False)`` with the
  default backend on a small ViT equals eager;
* FlopCounterMode counts the registered formulas, forward and backward;
* under ``torch.autocast('cuda')`` (fp16 by default, as in the reference loop)
  the layer computes in float16 and its gradients reach the fp32 weights.
"""
import pytest
import torch

from oracle import cnna_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops
    from layers import MultiHeadConvNNAttention, MultiHeadKvtAttention
    from vit import ViT, vit_tiny_args

DEV = "cuda"


def _layer(sampling="all", ns=-1, metric="matmul", conv="depthwise", dtype=torch.float32, N=128):
    torch.manual_seed(0)
    return MultiHeadConvNNAttention(96, 3, 0.0, 7, sampling, ns, 0, metric, seq_length=N,
                                    convolution_type=conv).to(DEV).to(dtype)


def _grads(m, x):
    m.zero_grad(set_to_none=True)
    xg = x.clone().requires_grad_(True)
    y = m(xg)
    y.backward(torch.ones_like(y))
    return y.detach(), xg.grad, {n.replace("_orig_mod.", ""): p.grad.clone() for n, p in m.named_parameters()}


@pytest.mark.parametrize("sampling,ns,metric,conv", [("all", -1, "matmul", "depthwise"),
                                                     ("spatial", 32, "cosine", "standard"),
                                                     ("all", -1, "euclidean", "depthwise-separable")])
def test_compile_fullgraph_matches_eager(sampling, ns, metric, conv):
    torch._dynamo.reset()
    m = _layer(sampling, ns, metric, conv)
    x = torch.randn(2, 128, 96, device=DEV)
    y0, gx0, gp0 = _grads(m, x)
    mc = torch.compile(m, backend="aot_eager", fullgraph=True)
    y1, gx1, gp1 = _grads(mc, x)
    torch.testing.assert_close(y1, y0, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(gx1, gx0, rtol=1e-5, atol=1e-5)
    for n in gp0:
        torch.testing.assert_close(gp1[n], gp0[n], rtol=1e-5, atol=1e-5, msg=n)


def test_compile_kvt_fullgraph_matches_eager():
    torch._dynamo.reset()
    torch.manual_seed(1)
    m = MultiHeadKvtAttention(96, num_heads=3, topk=9).to(DEV)
    x = torch.randn(2, 100, 96, device=DEV)
    y0, gx0, gp0 = _grads(m, x)
    y1, gx1, gp1 = _grads(torch.compile(m, backend="aot_eager", fullgraph=True), x)
    torch.testing.assert_close(y1, y0, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(gx1, gx0, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(gp1["qkv.weight"], gp0["qkv.weight"], rtol=1e-5, atol=1e-5)


def test_compile_vit_default_backend_like_the_reference_loop():
    pytest.importorskip("triton")
    torch._dynamo.reset()
    torch.manual_seed(0)
    args = vit_tiny_args(img_size=(3, 32, 32), patch_size=8, num_layers=2, dropout=0.0,
                         attention_dropout=0.0)
    model = ViT(args).to(DEV)
    for blk in model.transformer_encoder:
        blk.attention.seq_length = 17
    imgs = torch.randn(4, 3, 32, 32, device=DEV)
    y0 = model(imgs)
    y0.sum().backward()
    g0 = model.transformer_encoder[0].attention.W_q.weight.grad.clone()
    model.zero_grad(set_to_none=True)
    mc = torch.compile(model, fullgraph=False, dynamic=False)
    y1 = mc(imgs)
    y1.sum().backward()
    torch.testing.assert_close(y1, y0, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(model.transformer_encoder[0].attention.W_q.weight.grad, g0,
                               rtol=1e-3, atol=1e-4)


def test_flop_counter_counts_forward_and_backward():
    from torch.utils.flop_counter import FlopCounterMode
    m = _layer(N=256)
    x = torch.randn(4, 256, 96, device=DEV, requires_grad=True)
    fc = FlopCounterMode(display=False)
    with fc:
        y = m(x)
        y.sum().backward()
    counts = {str(k): v for k, v in fc.get_flop_counts()["Global"].items()}
    B, N, C, K = 4, 256, 96, 7
    fwd = 2 * B * C * C * 3 * N + 2 * B * N * N * C + 2 * B * N * C * K
    assert counts["cnna.core"] == fwd
    assert counts["cnna.core_backward"] == 2 * fwd
    assert counts["cnna.output_proj"] == 2 * B * N * C * C
    assert counts["cnna.output_proj_backward"] == 4 * B * N * C * C
    # the flop-counted run is the native one: same output as the eager path
    torch.testing.assert_close(y.detach(), m(x).detach(), rtol=1e-5, atol=1e-5)


def test_autocast_runs_fp16_and_reaches_fp32_weights():
    import copy
    m = _layer(N=128)
    m16 = copy.deepcopy(m).to(torch.float16)
    x = torch.randn(2, 128, 96, device=DEV, requires_grad=True)
    with torch.autocast("cuda"):                     # fp16 autocast, as the reference loop
        y = m(x)
    assert y.dtype == torch.float16
    y.float().square().sum().backward()
    assert m.W_q.weight.grad.dtype == torch.float32 and x.grad.dtype == torch.float32
    # the autocast run is exactly the float16 layer on the rounded inputs and weights
    x16 = x.detach().to(torch.float16).requires_grad_(True)
    y16 = m16(x16)
    y16.float().square().sum().backward()
    assert torch.equal(y, y16)
    for (n, a), (_, b) in zip(m.named_parameters(), m16.named_parameters()):
        assert torch.equal(a.grad, b.grad.float()), n
    assert torch.equal(x.grad, x16.grad.float())
    # (the float16 layer's own parity is covered by tests/test_gpu_fp16.py; it
    # is not compared with the float32 layer here: rounding q and k flips
    # near-tied neighbour choices, which moves whole rows)


@pytest.mark.parametrize("layer", ["ConvNNAttention", "KvtAttention"])
def test_forward_replays_from_a_hip_graph(layer):
    # the inference forward launches no memset and allocates nothing inside the
    # library, so it can be captured; every replay (with eager work and
    # synchronisations between replays) equals the eager forward
    torch.manual_seed(0)
    args = vit_tiny_args(layer=layer, img_size=(3, 64, 64), patch_size=8, num_layers=2, dropout=0.0,
                         attention_dropout=0.0)
    model = ViT(args).to(DEV).to(torch.bfloat16).eval()
    for blk in model.transformer_encoder:
        if hasattr(blk.attention, "seq_length"):
            blk.attention.seq_length = 65
    imgs = torch.randn(8, 3, 64, 64, device=DEV).to(torch.bfloat16)
    static_in = imgs.clone()
    with torch.no_grad():
        ref = model(imgs)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                model(static_in)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            static_out = model(static_in)
        for _ in range(4):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, ref)
            model(torch.randn_like(imgs))          # eager work between replays
            torch.cuda.synchronize()
