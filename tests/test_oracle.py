"""Pin the CPU oracle (oracle/cnna_oracle.py) before trusting it.

* golden vectors written by the reference itself (tests/golden/*.npz);
* closed forms and textbook reductions a plausible mistake would break;
* brute force on tiny inputs.
"""
import glob
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cnna_oracle as O

# eval-mode fixtures (make_golden.py); the training-mode dropout fixtures
# (make_golden_dropout.py, dropout_*.npz) are checked in test_dropout_cpu.py
GOLDEN = sorted(p for p in glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz"))
                if not os.path.basename(p).startswith("dropout_"))


def load_case(path):
    z = np.load(path, allow_pickle=False)
    kw = json.loads(bytes(z["ctor"]).decode())
    cfg = O.Config(**kw)
    sd = {k[len("param:"):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param:")}
    p = O.Params.from_module_state(sd, cfg.convolution_type)
    cand = torch.from_numpy(z["cand"]) if "cand" in z.files else None
    return cfg, p, torch.from_numpy(z["x"]), cand, torch.from_numpy(z["out"])


def test_golden_present():
    assert len(GOLDEN) >= 20


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_oracle_matches_reference_golden(path):
    cfg, p, x, cand, out = load_case(path)
    got = O.forward(x, p, cfg, cand=cand, mode="reference")
    tol = 1e-11 if x.dtype == torch.float64 else 2e-5
    torch.testing.assert_close(got, out, rtol=tol, atol=tol)


@pytest.mark.parametrize("path", [p for p in GOLDEN if p.endswith("_f64.npz")],
                         ids=lambda p: os.path.basename(p))
def test_exact_mode_matches_reference_in_f64(path):
    cfg, p, x, cand, out = load_case(path)
    got = O.forward(x, p, cfg, cand=cand, mode="exact")
    torch.testing.assert_close(got, out, rtol=1e-11, atol=1e-11)


def test_head_merge_closed_form():
    torch.manual_seed(0)
    for (B, H, dk, N) in [(2, 3, 4, 7), (1, 2, 5, 3), (3, 4, 2, 9)]:
        y = torch.randn(B * H, dk, N, dtype=torch.float64)
        torch.testing.assert_close(O.head_merge(y, B, H, N), O.head_merge_closed_form(y, B, H))


def test_head_merge_h1_is_transpose():
    y = torch.randn(3, 5, 7, dtype=torch.float64)
    torch.testing.assert_close(O.head_merge(y, 3, 1, 197), y.transpose(1, 2))


def test_head_merge_seq_length_mismatch_raises():
    y = torch.randn(2 * 3, 4, 8)
    with pytest.raises(RuntimeError):
        O.head_merge(y, 2, 3, 9)
    with pytest.raises(RuntimeError):
        O.head_merge(torch.randn(2 * 3, 4, 16), 2, 3, 8)   # divisible but wrong


def test_split_heads_index_formula():
    x = torch.randn(2, 5, 6)
    s = O.split_heads(x, 3)
    for b in range(2):
        for h in range(3):
            for c in range(2):
                for n in range(5):
                    assert s[b * 3 + h, c, n] == x[b, n, h * 2 + c]


def test_stable_topk_bruteforce_with_ties():
    g = torch.Generator().manual_seed(1)
    S = torch.randint(0, 4, (6, 5, 11), generator=g).to(torch.float64)
    S[0, 0, 3] = float("nan")
    for largest in (True, False):
        vals, idx = O.stable_topk(S, 4, largest)
        for a in range(6):
            for b in range(5):
                row = S[a, b].tolist()
                def key(j):
                    v = row[j]
                    if math.isnan(v):
                        return (1, 0, j)
                    return (0, -v if largest else v, j)
                exp = sorted(range(11), key=key)[:4]
                assert idx[a, b].tolist() == exp


def test_torch_topk_is_not_index_stable():
    # the reason the oracle uses a stable sort (CPU kernel, ties)
    v, i = torch.topk(torch.tensor([1.0, 3, 3, 2, 3, 0]), 3)
    _, si = O.stable_topk(torch.tensor([1.0, 3, 3, 2, 3, 0]), 3, True)
    assert si.tolist() == [1, 2, 4]
    assert sorted(i.tolist()) == [1, 2, 4]


def test_euclidean_is_cdist():
    cfg = O.Config(d_hidden=8, num_heads=2, K=3, magnitude_type="euclidean")
    k = torch.randn(4, 4, 9, dtype=torch.float64)
    q = torch.randn(4, 4, 7, dtype=torch.float64)
    S = O.similarity(k, q, cfg)
    torch.testing.assert_close(S, torch.cdist(k.transpose(1, 2), q.transpose(1, 2)))


def test_cosine_bounded_and_self_one():
    cfg = O.Config(d_hidden=8, num_heads=2, K=3, magnitude_type="cosine")
    k = torch.randn(4, 4, 9, dtype=torch.float64)
    S = O.similarity(k, k, cfg)
    assert S.abs().max() <= 1 + 1e-12
    torch.testing.assert_close(torch.diagonal(S, dim1=1, dim2=2), torch.ones(4, 9, dtype=torch.float64))


def test_matmul_symmetric_when_same_projection():
    cfg = O.Config(d_hidden=8, num_heads=2, K=3)
    k = torch.randn(4, 4, 9, dtype=torch.float64)
    S = O.similarity(k, k, cfg)
    torch.testing.assert_close(S, S.transpose(1, 2))
    torch.testing.assert_close(S[0, 1, 2], (k[0, :, 1] @ k[0, :, 2]) / 2.0)


def test_full_k_reduces_to_softmax_attention():
    """K == Nq, unit depthwise weight, softmax: the conv sums softmax(S) * v over
    all candidates -- textbook attention with query=k, key=q, value=v."""
    B, N, C, H = 2, 7, 8, 2
    cfg = O.Config(d_hidden=C, num_heads=H, K=N, seq_length=N)
    p = O.init_params(cfg, seed=3, dtype=torch.float64)
    x = torch.randn(B, N, C, dtype=torch.float64)
    out, it = O.forward(x, p, cfg, mode="exact", return_intermediates=True)
    att = F.scaled_dot_product_attention(it.k.transpose(1, 2), it.q.transpose(1, 2), it.v.transpose(1, 2))
    torch.testing.assert_close(it.y, att.transpose(1, 2))


def test_standard_conv_is_einsum():
    B, N, C, H, K = 2, 6, 8, 2, 3
    cfg = O.Config(d_hidden=C, num_heads=H, K=K, seq_length=N, convolution_type="standard")
    p = O.init_params(cfg, seed=4, dtype=torch.float64)
    x = torch.randn(B, N, C, dtype=torch.float64)
    _, it = O.forward(x, p, cfg, mode="exact", return_intermediates=True)
    g = torch.stack([it.v[b][:, it.idx[b]] for b in range(B * H)])        # (BH, c, N, K)
    ref = torch.einsum("ocr,bcnr->bon", p.conv0, g * it.w.unsqueeze(1))
    torch.testing.assert_close(it.y, ref)


def test_sampled_hand_worked():
    """N=5, Ns=3, K=3, H=1, d=2, matmul, no softmax, depthwise weight 1."""
    cfg = O.Config(d_hidden=2, num_heads=1, K=3, sampling_type="random", num_samples=3,
                   softmax_topk_val=False)
    eye = torch.eye(2, dtype=torch.float64)
    p = O.Params(eye, eye, eye, eye, torch.ones(2, 1, 3, dtype=torch.float64))
    x = torch.tensor([[[1., 0.], [0., 1.], [2., 0.], [0., 3.], [1., 1.]]], dtype=torch.float64)
    cand = torch.tensor([4, 0, 2])
    out, it = O.forward(x, p, cfg, cand=cand, mode="reference", return_intermediates=True)
    s2 = math.sqrt(2)
    # S[i, j] = x_i . x_cand[j] / sqrt(2), then S[cand[j], j] = -0.1
    # token 0: [1, -0.1(self), 2]/s2 -> top2 cols {2, 0} -> tokens [2, 4]
    assert it.idx[0, 0].tolist() == [0, 2, 4]
    torch.testing.assert_close(it.vals[0, 0], torch.tensor([1.0, 2 / s2, 1 / s2], dtype=torch.float64))
    # token 4 (a candidate itself): [-0.1(self), 1/s2, 2/s2] -> cols {2, 1} -> tokens [2, 0]
    assert it.idx[0, 4].tolist() == [4, 2, 0]
    y0 = 1.0 * x[0, 0] + (2 / s2) * x[0, 2] + (1 / s2) * x[0, 4]
    torch.testing.assert_close(out[0, 0], y0)


def test_spatial_indices_are_1d_linspace():
    cfg = O.Config(d_hidden=192, num_heads=3, K=9, sampling_type="spatial", num_samples=8)
    assert O.sample_indices(cfg, 197).tolist() == [0, 28, 56, 84, 112, 140, 168, 196]


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_oracle_grads_match_reference_golden(path):
    """Backward: torch autograd through the oracle equals the reference's own
    autograd (fixtures hold grad:x and grad:<param> for an upstream dout)."""
    z = np.load(path, allow_pickle=False)
    if "grad_error" in z.files:
        # the reference cannot differentiate sampled euclidean (in-place self
        # mask on the output of sqrt, layers.py:278-305); nothing to pin
        assert "modified by an inplace operation" in bytes(z["grad_error"]).decode()
        return
    cfg, p, x, cand, _ = load_case(path)
    dout = torch.from_numpy(z["dout"])
    names = ["W_q", "W_k", "W_v", "W_o", "conv0", "conv1"]
    ts = [None if t is None else t.clone().requires_grad_(True)
          for t in (x, p.W_q, p.W_k, p.W_v, p.W_o, p.conv0, p.conv1)]
    out = O.forward(ts[0], O.Params(*ts[1:]), cfg, cand=cand, mode="reference")
    out.backward(dout)
    ref_names = {"W_q": "W_q.weight", "W_k": "W_k.weight", "W_v": "W_v.weight",
                 "W_o": "W_o.weight"}
    if cfg.convolution_type == "depthwise-separable":
        ref_names.update(conv0="conv.0.weight", conv1="conv.1.weight")
    else:
        ref_names.update(conv0="conv.weight")
    tol = dict(rtol=1e-9, atol=1e-10) if x.dtype == torch.float64 else dict(rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(ts[0].grad, torch.from_numpy(z["grad:x"]), **tol)
    for n, t in zip(names, ts[1:]):
        if t is None:
            continue
        torch.testing.assert_close(t.grad, torch.from_numpy(z["grad:" + ref_names[n]]), **tol,
                                   msg=lambda m: f"{n}: {m}")


def test_oracle_cols_hook_reproduces_topk():
    """Passing the top-k's own columns back as ``cols`` changes nothing."""
    for sampling in ("all", "random"):
        cfg = O.Config(d_hidden=12, num_heads=3, K=4, sampling_type=sampling, num_samples=7,
                       seq_length=15, magnitude_type="cosine")
        p = O.init_params(cfg, seed=3, dtype=torch.float64)
        x = torch.randn(2, 15, 12, dtype=torch.float64)
        cand = O.sample_indices(cfg, 15, generator=torch.Generator().manual_seed(1))
        out, it = O.forward(x, p, cfg, cand=cand, mode="exact", return_intermediates=True)
        if cand is None:
            cols = it.idx
        else:
            inv = {int(t): j for j, t in enumerate(cand.tolist())}
            cols = torch.tensor([[[inv[int(t)] for t in row[1:]] for row in bh] for bh in it.idx])
        out2 = O.forward(x, p, cfg, cand=cand, mode="exact", cols=cols)
        assert torch.equal(out, out2)


def test_gradcheck_oracle_f64():
    B, N, C, H = 1, 6, 4, 2
    cfg = O.Config(d_hidden=C, num_heads=H, K=3, seq_length=N, convolution_type="standard")
    p = O.init_params(cfg, seed=5, dtype=torch.float64)
    x = torch.randn(B, N, C, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda t: O.forward(t, p, cfg, mode="exact"), (x,))


# ---------------------------------------------------------------- callers
def _rand(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64) * scale


@pytest.mark.parametrize("H,ks", [(1, 3), (2, 3), (2, 4), (3, 1), (1, 6)])
def test_conv1d_branch_elementwise_loop(H, ks):
    """'same' padding puts (ks-1)//2 zeros in front; the merge mixes tokens
    for every H: z[b, t, h*dk + a] = y_tok[b*H + h].flat[a*N + t]."""
    B, N, dk = 2, 7, 2
    C = H * dk
    x = _rand(B, N, C, seed=1)
    Wx, bx = _rand(C, C, seed=2), _rand(C, seed=3)
    cw, cb = _rand(dk, dk, ks, seed=4), _rand(dk, seed=5)
    Wo, bo = _rand(C, C, seed=6), _rand(C, seed=7)
    got = O.conv1d_branch(x, Wx, bx, cw, cb, Wo, bo, H)
    u = x @ Wx.T + bx
    pl = (ks - 1) // 2
    ytok = torch.zeros(B * H, N, dk, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            for t in range(N):
                for o in range(dk):
                    s = float(cb[o])
                    for r in range(ks):
                        tt = t + r - pl
                        if 0 <= tt < N:
                            for c in range(dk):
                                s += float(cw[o, c, r]) * float(u[b, tt, h * dk + c])
                    ytok[b * H + h, t, o] = s
    z = torch.empty(B, N, C, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            flat = ytok[b * H + h].reshape(-1)
            for t in range(N):
                for a in range(dk):
                    z[b, t, h * dk + a] = flat[a * N + t]
    torch.testing.assert_close(got, z @ Wo.T + bo, rtol=1e-12, atol=1e-12)


def test_mha_rowwise_softmax_loop():
    B, N, H, dk = 2, 5, 2, 3
    C = H * dk
    x = _rand(B, N, C, seed=8)
    Ws = [_rand(C, C, seed=9 + i, scale=0.5) for i in range(4)]
    mask = (torch.rand(B, 1, N, N, generator=torch.Generator().manual_seed(0)) > 0.3).long()
    mask[..., 0] = 1
    got = O.mha(x, *Ws, H, mask=mask)
    q, k, v = (x @ W.T for W in Ws[:3])
    o = torch.empty(B, N, C, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            sl = slice(h * dk, (h + 1) * dk)
            for i in range(N):
                s = [(float(q[b, i, sl] @ k[b, j, sl]) / math.sqrt(dk)) if mask[b, 0, i, j] else -1e9
                     for j in range(N)]
                m = max(s)
                e = [math.exp(t - m) for t in s]
                o[b, i, sl] = sum(e[j] / sum(e) * v[b, j, sl] for j in range(N))
    torch.testing.assert_close(got, o @ Ws[3].T, rtol=1e-12, atol=1e-12)


def _kvt_loop(x, Wqkv, Wproj, H, topk, scale, wmul=None):
    B, N, C = x.shape
    dk = C // H
    qkv = x @ Wqkv.T
    q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
    o = torch.empty(B, N, C, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            sl = slice(h * dk, (h + 1) * dk)
            for i in range(N):
                s = [float(q[b, i, sl] @ k[b, j, sl]) * scale for j in range(N)]
                keep = sorted(range(N), key=lambda j: (-s[j], j))[:topk]
                m = max(s[j] for j in keep)
                e = [math.exp(s[j] - m) for j in keep]
                p = [t / sum(e) for t in e]
                if wmul is not None:
                    p = [p[r] * float(wmul[b * H + h, i, r]) for r in range(topk)]
                o[b, i, sl] = sum(p[r] * v[b, keep[r], sl] for r in range(topk))
    return o @ Wproj.T


@pytest.mark.parametrize("H,topk", [(1, 3), (2, 1), (3, 4)])
def test_kvt_rowwise_loop(H, topk):
    B, N, dk = 2, 6, 2
    C = H * dk
    x = _rand(B, N, C, seed=20)
    Wqkv, Wp = _rand(3 * C, C, seed=21), _rand(C, C, seed=22)
    wmul = (torch.rand(B * H, N, topk, generator=torch.Generator().manual_seed(1)) > 0.25).double() / 0.75
    for wm in (None, wmul):
        got = O.kvt(x, Wqkv, Wp, H, topk, 0.37, wmul=wm)
        torch.testing.assert_close(got, _kvt_loop(x, Wqkv, Wp, H, topk, 0.37, wm), rtol=1e-12, atol=1e-12)


def test_kvt_with_all_keys_is_softmax_attention():
    B, N, H, dk = 2, 9, 3, 4
    C = H * dk
    x = _rand(B, N, C, seed=30)
    Wqkv, Wp = _rand(3 * C, C, seed=31, scale=0.3), _rand(C, C, seed=32)
    got = O.kvt(x, Wqkv, Wp, H, N, dk ** -0.5)
    qkv = (x @ Wqkv.T).reshape(B, N, 3, H, dk).permute(2, 0, 3, 1, 4)
    o = F.scaled_dot_product_attention(qkv[0], qkv[1], qkv[2])
    torch.testing.assert_close(got, o.transpose(1, 2).reshape(B, N, C) @ Wp.T, rtol=1e-10, atol=1e-10)


def test_kvt_is_the_operator_with_concat_heads_at_h1():
    """With one head the operator's merge is the concatenation, so KVT equals
    the ConvNN restatement with W_k := q rows, W_q := k rows, unit depthwise
    weights, softmax weights and K = topk."""
    B, N, C, topk = 2, 11, 5, 4
    x = _rand(B, N, C, seed=40)
    Wqkv, Wp = _rand(3 * C, C, seed=41), _rand(C, C, seed=42)
    cfg = O.Config(d_hidden=C, num_heads=1, K=topk, magnitude_type="matmul",
                   convolution_type="depthwise", softmax_topk_val=True, seq_length=N)
    p = O.Params(Wqkv[C:2 * C], Wqkv[:C], Wqkv[2 * C:], Wp, torch.ones(C, 1, topk, dtype=torch.float64))
    ref = O.forward(x, p, cfg)
    torch.testing.assert_close(O.kvt(x, Wqkv, Wp, 1, topk, C ** -0.5), ref, rtol=1e-12, atol=1e-12)


def test_branching_is_concat_of_branches():
    B, N, C, d1 = 2, 4, 6, 2
    x = _rand(B, N, C, seed=50)
    Wp, bp = _rand(C, C, seed=51), _rand(C, seed=52)
    f1 = lambda t: t * 2.0
    f2 = lambda t: t - 1.0
    got = O.branching_conv(x, f1, f2, Wp, bp, d1)
    want = torch.cat((x[..., :d1] * 2.0, x[..., d1:] - 1.0), -1) @ Wp.T + bp
    torch.testing.assert_close(got, want)
