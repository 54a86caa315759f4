"""Attention dropout drawn where the reference draws it (CPU, no GPU needed).

The reference applies ``self.dropout`` to the conv output y (B*H, d_k, N)
before the head merge (layers.py:316) and KVT's ``attn_drop`` to the dense
(B, H, N, N) probabilities (layers.py:680).  The same seed must give the same
mask, so the draw has to happen on a tensor of the reference's shape, layout
and dtype, in the reference's order relative to the sampling draw.

* the oracle with ``y_dropout`` = ``nn.Dropout`` (and KVT with the dense mask
  of ``nn.Dropout`` on ones) reproduces training-mode outputs and gradients
  the reference itself wrote (tests/golden/dropout_*.npz, seeded CPU runs);
* the drop-in's re-layout (head-merged z -> y -> dropout -> z) equals the
  merge of the dropped-out y under the same seed, for H = 1 and H > 1;
* KVT's mask helper returns the mask of that same draw.
"""
import glob
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cnna_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = sorted(glob.glob(os.path.join(HERE, "golden", "dropout_*.npz")))
CONVNN = [p for p in CASES if "_convnn_" in p]
KVT = [p for p in CASES if "_kvt_" in p]


def load(path):
    z = np.load(path, allow_pickle=False)
    kw = json.loads(bytes(z["ctor"]).decode())
    return z, kw


def test_fixtures_present():
    assert len(CONVNN) >= 6 and len(KVT) >= 4


@pytest.mark.parametrize("path", CONVNN, ids=[os.path.basename(p) for p in CONVNN])
def test_oracle_dropout_site_matches_reference(path):
    z, kw = load(path)
    p_drop = kw.pop("attention_dropout")
    cfg = O.Config(**kw, attention_dropout=p_drop)
    sd = {k[len("param:"):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param:")}
    p = O.Params.from_module_state(sd, cfg.convolution_type)
    x = torch.from_numpy(z["x"])
    names = ["W_q", "W_k", "W_v", "W_o", "conv0", "conv1"]
    ts = [None if t is None else t.clone().requires_grad_(True)
          for t in (x, p.W_q, p.W_k, p.W_v, p.W_o, p.conv0, p.conv1)]
    torch.manual_seed(int(z["fwd_seed"][0]))
    # cand drawn by the oracle from the default generator (randperm, as layers.py:284)
    out = O.forward(ts[0], O.Params(*ts[1:]), cfg, mode="reference",
                    y_dropout=lambda y: F.dropout(y, p_drop, training=True))
    tol = dict(rtol=1e-11, atol=1e-11) if x.dtype == torch.float64 else dict(rtol=2e-5, atol=2e-5)
    torch.testing.assert_close(out.detach(), torch.from_numpy(z["out"]), **tol)
    out.backward(torch.from_numpy(z["dout"]))
    gtol = dict(rtol=1e-9, atol=1e-10) if x.dtype == torch.float64 else dict(rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(ts[0].grad, torch.from_numpy(z["grad:x"]), **gtol)
    ref_names = {"W_q": "W_q.weight", "W_k": "W_k.weight", "W_v": "W_v.weight", "W_o": "W_o.weight"}
    if cfg.convolution_type == "depthwise-separable":
        ref_names.update(conv0="conv.0.weight", conv1="conv.1.weight")
    else:
        ref_names.update(conv0="conv.weight")
    for n, t in zip(names, ts[1:]):
        if t is not None:
            torch.testing.assert_close(t.grad, torch.from_numpy(z["grad:" + ref_names[n]]), **gtol)


def test_dropout_after_merge_would_differ():
    """The site matters: the same seed applied to the head-merged tensor gives
    a different output (so the test above can tell the two apart)."""
    z, kw = load([p for p in CONVNN if "h3_matmul" in p and p.endswith("_f64.npz")][0])
    p_drop = kw.pop("attention_dropout")
    cfg = O.Config(**kw)
    sd = {k[len("param:"):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param:")}
    p = O.Params.from_module_state(sd, cfg.convolution_type)
    x = torch.from_numpy(z["x"])
    _, it = O.forward(x, p, cfg, mode="reference", return_intermediates=True)
    torch.manual_seed(int(z["fwd_seed"][0]))
    wrong = F.linear(F.dropout(it.z, p_drop, training=True), p.W_o)
    assert not torch.allclose(wrong, torch.from_numpy(z["out"]))


@pytest.mark.parametrize("H", [1, 2, 3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_dropin_relayout_draws_on_the_conv_output(H, dtype):
    from layers import MultiHeadConvNNAttention
    B, N, dk = 2, 11, 4
    C = H * dk
    m = MultiHeadConvNNAttention(C, H, 0.4, 3, "all", -1, 0, "matmul", seq_length=N).train()
    y = torch.randn(B * H, dk, N, dtype=torch.float64).to(dtype)
    zm = O.head_merge(y, B, H, N)
    torch.manual_seed(3)
    got = m._conv_output_dropout(zm)
    torch.manual_seed(3)
    want = O.head_merge(F.dropout(y, 0.4, training=True), B, H, N)
    assert torch.equal(got, want)
    # eval and p = 0 draw nothing
    m.eval()
    assert m._conv_output_dropout(zm) is zm


@pytest.mark.parametrize("path", KVT, ids=[os.path.basename(p) for p in KVT])
def test_oracle_kvt_dense_dropout_matches_reference(path):
    z, kw = load(path)
    x = torch.from_numpy(z["x"])
    B, N, C = x.shape
    H, topk = kw["num_heads"], kw["topk"]
    scale = kw.get("qk_scale") or (C // H) ** -0.5
    Wqkv, Wp = torch.from_numpy(z["param:qkv.weight"]), torch.from_numpy(z["param:proj.weight"])
    torch.manual_seed(int(z["fwd_seed"][0]))
    dense = F.dropout(torch.ones(B, H, N, N, dtype=x.dtype), kw["attn_drop"], training=True)
    got = O.kvt(x, Wqkv, Wp, H, topk, scale, dense_mult=dense)
    tol = dict(rtol=1e-10, atol=1e-10) if x.dtype == torch.float64 else dict(rtol=2e-5, atol=2e-5)
    torch.testing.assert_close(got, torch.from_numpy(z["out"]), **tol)


def test_kvt_mask_helper_is_the_dense_draw():
    from layers import MultiHeadKvtAttention
    m = MultiHeadKvtAttention(12, 3, attn_drop=0.3, topk=4).train()
    x = torch.randn(2, 10, 12)
    torch.manual_seed(9)
    mask, scale = m._dense_dropout_mask(2, 3, 10, x)
    torch.manual_seed(9)
    dense = F.dropout(torch.ones(2, 3, 10, 10), 0.3, training=True)
    assert torch.equal(mask, dense != 0)
    assert abs(scale - 1 / 0.7) < 1e-6
    m.eval()
    assert m._dense_dropout_mask(2, 3, 10, x) == (None, 1.0)
