"""ViT block prologue/epilogue fusion on the GPU (run on an MI355X).

* cnna_layernorm equals torch.nn.functional.layer_norm (with the residual
  sum rounded to the storage type first, as the unfused x + y is);
* cnna_linear's bias / GELU / residual epilogues equal the unfused
  nn.Linear -> nn.GELU -> + residual sequence;
* a ViT whose blocks run fused (eval, no gradients) equals the same ViT run
  through the composable modules;
* the folded LayerNorm: cnna_row_stats's per-tile (mean, M2) partials equal
  the float64 ones; the GEMMs' LayerNorm prologue equals LayerNorm -> GEMM
  (cnna_linear_ln, cnna_project_qkv_ex, also on the sampled Q rows); the
  statistics epilogue equals the statistics pass over the stored output; a
  folded ViT block runs no LayerNorm kernel.
"""
import copy

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops
    from vit import ViT, vit_tiny_args

DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("C", [192, 384, 1000])
@pytest.mark.parametrize("with_res", [False, True])
def test_layernorm_matches_torch(dtype, C, with_res):
    torch.manual_seed(C)
    rows = 777
    x = (torch.randn(rows, C, device=DEV) * 3 + 0.5).to(dtype)
    res = torch.randn(rows, C, device=DEV).to(dtype) if with_res else None
    g = (torch.rand(C, device=DEV) + 0.5).to(dtype)
    b = torch.randn(C, device=DEV).to(dtype)
    y, s = ops.layernorm(x, g, b, 1e-5, residual=res, want_sum=True)
    s_ref = x if res is None else x + res          # rounded to dtype like the unfused add
    assert torch.equal(s, s_ref)
    ref = F.layer_norm(s_ref.float(), (C,), g.float(), b.float(), 1e-5)
    if dtype == torch.float32:
        torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)
    else:
        # one bf16 rounding of the same fp32 value, up to an ulp from the statistics' order
        torch.testing.assert_close(y.float(), ref, rtol=8e-3, atol=8e-3)


def test_layernorm_strided_rows_and_no_affine():
    torch.manual_seed(0)
    base = torch.randn(64, 300, device=DEV)
    x = base[:, :192]                               # row stride 300
    y = ops.layernorm(x, None, None, 1e-6)
    torch.testing.assert_close(y, F.layer_norm(x, (192,), eps=1e-6), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,Nout,Kd", [(1000, 768, 192), (1000, 192, 768), (257, 200, 64), (25216, 192, 192)])
@pytest.mark.parametrize("mode", ["plain", "bias_gelu", "bias_res", "res"])
def test_linear_epilogues(dtype, M, Nout, Kd, mode):
    torch.manual_seed(M + Nout)
    a = torch.randn(M, Kd, device=DEV).to(dtype)
    W = (torch.randn(Nout, Kd, device=DEV) / Kd ** 0.5).to(dtype)
    bias = torch.randn(Nout, device=DEV).to(dtype) if mode.startswith("bias") else None
    res = torch.randn(M, Nout, device=DEV).to(dtype) if mode.endswith("res") else None
    out = ops.linear(a, W, bias, gelu=mode == "bias_gelu", residual=res)
    # the unfused sequence: nn.Linear (rounded to dtype) -> nn.GELU -> + residual
    ref = F.linear(a.float(), W.float(), None if bias is None else bias.float()).to(dtype)
    if mode == "bias_gelu":
        ref = F.gelu(ref.float()).to(dtype)
    if res is not None:
        ref = (ref.float() + res.float()).to(dtype)
    if dtype == torch.float32:
        torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-4)
    else:
        torch.testing.assert_close(out.float(), ref.float(), rtol=2e-2, atol=2e-2)



@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_linear_gelu_values(dtype):
    """The GELU epilogue as a function: with A = 0 the GEMM output is the bias,
    so every column checks GELU at one input (a sweep over [-20, 20], values
    near 0 and the special values) against nn.GELU's erf form in float64.
    Bounds: the erf approximation's 1.5e-7 plus float32 rounding; in bf16 one
    rounding of the same value (an ulp apart where it falls near a tie)."""
    sweep = torch.linspace(-20.0, 20.0, 4000, dtype=torch.float64)
    small = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 1e-7, -1e-7, 3e-3, -3e-3], dtype=torch.float64)
    special = torch.tensor([float("inf"), float("-inf"), float("nan"), 3e38, -3e38], dtype=torch.float64)
    xs = torch.cat([sweep, small, special]).to(dtype)
    n = ((xs.numel() + 7) // 8) * 8
    bias = torch.cat([xs, torch.zeros(n - xs.numel(), dtype=dtype)]).to(DEV)
    a = torch.zeros(64, 64, device=DEV, dtype=dtype)
    W = torch.zeros(n, 64, device=DEV, dtype=dtype)
    out = ops.linear(a, W, bias, gelu=True)
    ref = F.gelu(bias.double())                    # erf form, float64
    for row in (0, 63):
        got = out[row].double()
        fin = torch.isfinite(ref)
        # the special values: +inf -> +inf, -inf and NaN -> NaN, as the erf form gives
        assert torch.equal(torch.isnan(got), torch.isnan(ref))
        assert torch.equal(got[torch.isinf(ref)], ref[torch.isinf(ref)])
        if dtype == torch.float32:
            torch.testing.assert_close(got[fin], ref[fin], rtol=1e-6, atol=1e-6)
        else:
            torch.testing.assert_close(got[fin], ref[fin].to(dtype).double(), rtol=8e-3, atol=1e-6)


def _tiny_vit(dtype):
    torch.manual_seed(0)
    args = vit_tiny_args(img_size=(3, 64, 64), patch_size=8, num_layers=3, dropout=0.0,
                         attention_dropout=0.0)
    model = ViT(args).to(DEV).to(dtype).eval()
    for blk in model.transformer_encoder:
        blk.attention.seq_length = 65
    return model


def test_vit_fused_blocks_match_composable_fp32():
    model = _tiny_vit(torch.float32)
    imgs = torch.randn(8, 3, 64, 64, device=DEV)
    with torch.no_grad():
        fused = model(imgs)
    with torch.enable_grad():                       # parameters require grad -> composable path
        assert not model.transformer_encoder[0]._fusable(imgs.new_zeros(1, 65, 192, device=DEV))
        plain = model(imgs).detach()
    torch.testing.assert_close(fused, plain, rtol=1e-4, atol=1e-4)


def test_vit_fused_blocks_bf16_as_accurate_as_composable():
    # bf16: LayerNorm / GEMM roundings differ by an ulp here and there, which can
    # flip near-tied neighbours, so both bf16 paths are measured against the
    # float32 network with the same weights and the fused one may not be worse
    model32 = _tiny_vit(torch.float32)
    model16 = _tiny_vit(torch.bfloat16)
    model16.load_state_dict({k: v.to(torch.bfloat16) for k, v in model32.state_dict().items()})
    imgs = torch.randn(16, 3, 64, 64, device=DEV)
    with torch.no_grad():
        ref = model32(imgs)
        fused = model16(imgs.to(torch.bfloat16)).float()
    with torch.enable_grad():
        plain = model16(imgs.to(torch.bfloat16)).float().detach()
    err_f = ((fused - ref).norm() / ref.norm()).item()
    err_p = ((plain - ref).norm() / ref.norm()).item()
    assert err_f <= 1.5 * err_p + 0.02, (err_f, err_p)


def test_vit_fused_block_is_the_one_that_runs():
    model = _tiny_vit(torch.bfloat16)
    blk = model.transformer_encoder[0]
    x = torch.randn(2, 65, 192, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        assert blk._fusable(x)
    model.train()
    with torch.no_grad():
        assert not blk._fusable(x)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_patch_embedding_gemm_matches_conv(dtype):
    from vit import PatchEmbedding
    torch.manual_seed(3)
    pe = PatchEmbedding(192, (64, 64), (8, 8)).to(DEV).to(dtype).eval()
    x = torch.randn(5, 3, 64, 64, device=DEV).to(dtype)
    with torch.no_grad():
        fused = pe(x).float()                         # GEMM + LayerNorm kernels
    with torch.enable_grad():
        ref = pe(x).float().detach()                  # Conv2d + nn.LayerNorm
    tol = 1e-4 if dtype == torch.float32 else 3e-2
    torch.testing.assert_close(fused, ref, rtol=tol, atol=tol)


# ---------------------------------------------------------------- folded LayerNorm
def _tile_stats64(x):
    """Float64 (mean, M2) of each 128-column tile of each row."""
    x = x.double()
    rows, C = x.shape
    out = torch.zeros(rows, (C + 127) // 128, 2, dtype=torch.float64, device=x.device)
    for t in range(out.shape[1]):
        seg = x[:, 128 * t:min(C, 128 * t + 128)]
        mu = seg.mean(1)
        out[:, t, 0] = mu
        out[:, t, 1] = ((seg - mu[:, None]) ** 2).sum(1)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("C", [64, 192, 200, 768, 1000])
def test_row_stats_partials(dtype, C):
    torch.manual_seed(C)
    base = (torch.randn(333, C + 8, device=DEV) * 2 + 3).to(dtype)
    x = base[:, 4:4 + C]                              # row stride C + 8, offset start
    st = ops.row_stats(x)
    assert st.stats.shape == (333, (C + 127) // 128, 2) and st.rows == 333 and st.C == C
    torch.testing.assert_close(st.stats.double(), _tile_stats64(x), rtol=1e-5, atol=1e-4)


def _ln_ref(x, norm):
    """nn.LayerNorm's output in x's dtype (fp32 statistics of the same x)."""
    return F.layer_norm(x.float(), norm.normalized_shape, None if norm.weight is None else norm.weight.float(),
                        None if norm.bias is None else norm.bias.float(), norm.eps).to(x.dtype)


def _norm(C, dtype, affine=True, seed=0):
    torch.manual_seed(seed)
    n = torch.nn.LayerNorm(C, elementwise_affine=affine).to(DEV)
    if affine:
        with torch.no_grad():
            n.weight.copy_(torch.rand(C) + 0.5)
            n.bias.copy_(torch.randn(C) * 0.3)
    return n.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,Nout,Kd", [(1000, 768, 192), (1000, 192, 768), (257, 200, 200), (300, 136, 1000)])
@pytest.mark.parametrize("mode", ["plain", "bias_gelu", "bias_res"])
def test_linear_layernorm_prologue(dtype, M, Nout, Kd, mode):
    """linear(ln=row statistics + norm) == linear(LayerNorm(a)): Kd % 64 == 0
    takes the vector loader, 200 and 1000 the element-wise one."""
    torch.manual_seed(M + Kd)
    a = (torch.randn(M, Kd, device=DEV) * 1.5 + 0.7).to(dtype)
    W = (torch.randn(Nout, Kd, device=DEV) / Kd ** 0.5).to(dtype)
    bias = torch.randn(Nout, device=DEV).to(dtype) if mode.startswith("bias") else None
    res = torch.randn(M, Nout, device=DEV).to(dtype) if mode.endswith("res") else None
    norm = _norm(Kd, dtype, seed=Kd)
    out = ops.linear(a, W, bias, gelu=mode == "bias_gelu", residual=res, ln=ops.row_stats(a).with_norm(norm))
    h = _ln_ref(a, norm)
    ref = ops.linear(h, W, bias, gelu=mode == "bias_gelu", residual=res)
    if dtype == torch.float32:
        torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-4)
    else:
        # h may differ by one bf16 ulp where the statistics' summation order
        # moves a value across a rounding boundary
        torch.testing.assert_close(out.float(), ref.float(), rtol=2e-2, atol=2e-2)
        assert (out.float() - ref.float()).abs().mean() < 2e-3


def test_linear_layernorm_prologue_without_affine():
    torch.manual_seed(5)
    a = torch.randn(500, 192, device=DEV) * 4 - 2
    W = torch.randn(384, 192, device=DEV) / 14
    norm = _norm(192, torch.float32, affine=False)
    out = ops.linear(a, W, ln=ops.row_stats(a).with_norm(norm))
    ref = F.linear(F.layer_norm(a, (192,)), W)
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("M,Nout,Kd", [(1000, 192, 192), (257, 200, 768), (25216, 192, 768), (64, 1024, 64)])
@pytest.mark.parametrize("mode", ["plain", "bias_res", "res", "bias_gelu"])
def test_linear_statistics_epilogue(M, Nout, Kd, mode):
    """bf16: the epilogue's partials are those of the stored output rows (the
    residual sum as rounded to bf16), and the output is unchanged."""
    torch.manual_seed(M + Nout + Kd)
    a = torch.randn(M, Kd, device=DEV).to(torch.bfloat16)
    W = (torch.randn(Nout, Kd, device=DEV) / Kd ** 0.5).to(torch.bfloat16)
    bias = torch.randn(Nout, device=DEV).to(torch.bfloat16) if mode.startswith("bias") else None
    res = (torch.randn(M, Nout, device=DEV) * 3).to(torch.bfloat16) if mode.endswith("res") else None
    out, st = ops.linear(a, W, bias, gelu=mode == "bias_gelu", residual=res, want_stats=True)
    assert ops._stats_epilogue_ok(out.view(M, Nout), None if res is None else res)
    ref = ops.linear(a, W, bias, gelu=mode == "bias_gelu", residual=res)
    assert torch.equal(out, ref)
    assert st.rows == M and st.C == Nout
    torch.testing.assert_close(st.stats.double(), _tile_stats64(out), rtol=1e-5, atol=1e-4)


def test_linear_statistics_fp32_from_pass():
    """fp32 (no statistics epilogue): want_stats falls back to the statistics
    pass over the output."""
    torch.manual_seed(2)
    a = torch.randn(300, 192, device=DEV)
    W = torch.randn(192, 192, device=DEV) / 14
    out, st = ops.linear(a, W, residual=a, want_stats=True)
    torch.testing.assert_close(st.stats.double(), _tile_stats64(out), rtol=1e-5, atol=1e-4)


def _qkv_desc(dtype, sampled, coord=False, metric="matmul", B=2, N=197, C=192, H=3, Nq=None):
    Nq = N if not sampled else Nq
    return ops.make_desc(B, N, C, H, Nq, 9, N, dtype, metric, "standard", True, sampled, coord)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", ["all", "sampled", "coord_cosine", "strided"])
def test_project_qkv_layernorm_prologue(dtype, case):
    """project_qkv(x, ln) == project_qkv(LayerNorm(x)); the sampled Q rows read
    the statistics of their source rows x[b, cand]."""
    torch.manual_seed(11)
    B, N, C = 2, 197, 192
    xb = (torch.randn(B, N, C + 64, device=DEV) * 2 - 1).to(dtype)
    x = xb[..., :C] if case == "strided" else xb[..., :C].contiguous()
    cand = None
    if case == "sampled":
        cand = torch.randperm(N, device=DEV)[:40].to(torch.int32)
    d = _qkv_desc(dtype, case == "sampled", coord=case == "coord_cosine",
                  metric="cosine" if case == "coord_cosine" else "matmul", Nq=40)
    Wq, Wk, Wv = [(torch.randn(C, C, device=DEV) / C ** 0.5).to(dtype) for _ in range(3)]
    norm = _norm(C, dtype, seed=1)
    got = ops.project_qkv(d, x, cand, Wq, Wk, Wv, ln=ops.row_stats(x).with_norm(norm))
    ref = ops.project_qkv(d, _ln_ref(x, norm), cand, Wq, Wk, Wv)
    for g, r in zip(got, ref):
        if r is None:
            assert g is None
            continue
        if dtype == torch.float32:
            torch.testing.assert_close(g, r, rtol=1e-4, atol=1e-4)
        else:
            torch.testing.assert_close(g.float(), r.float(), rtol=2e-2, atol=2e-2)


def test_folded_vit_block_runs_no_layernorm_kernel(monkeypatch):
    """With ConvNN attention both LayerNorms of a fused block are folded into
    the GEMMs: the LayerNorm kernel is never called, the first block's
    statistics come from one pre-pass and the others from the epilogues."""
    model = _tiny_vit(torch.bfloat16)
    imgs = torch.randn(4, 3, 64, 64, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        expect = model(imgs)
    calls = {"ln": 0, "stats": 0}
    real_ln, real_stats = ops.layernorm, ops.row_stats

    def ln_spy(*a, **k):
        calls["ln"] += 1
        return real_ln(*a, **k)

    def stats_spy(*a, **k):
        calls["stats"] += 1
        return real_stats(*a, **k)

    monkeypatch.setattr(ops, "layernorm", ln_spy)
    monkeypatch.setattr(ops, "row_stats", stats_spy)
    with torch.no_grad():
        got = model(imgs)
    assert torch.equal(got, expect)
    assert calls["stats"] == 1
    # the patch embedding's own LayerNorm (vit.py PatchEmbedding.norm) is the one kernel left
    assert calls["ln"] == 1
