"""ViT block prologue/epilogue fusion on the GPU (run on an MI355X).

* cnna_layernorm equals torch.nn.functional.layer_norm (with the residual
  sum rounded to the storage type first, as the unfused x + y is);
* cnna_linear's bias / GELU / residual epilogues equal the unfused
  nn.Linear -> nn.GELU -> + residual sequence;
* a ViT whose blocks run fused (eval, no gradients) equals the same ViT run
  through the composable modules.
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
