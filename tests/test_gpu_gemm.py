"""GPU: the MFMA GEMM at the workloads' sizes (c3 / c5 projections, ViT MLP,
W_o, dP-like wide outputs), against float32 torch on the same bf16 operands:
plain rows, partial edge tiles, the Q/K/V head split, and the ViT block
epilogues (bias, bias + GELU, residual).  Tolerance: bf16 output rounding,
rtol 1e-2 with an absolute floor of 1e-2 x the output RMS."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops

DEV = "cuda"


def _close(got, want):
    rms = want.pow(2).mean().sqrt().item()
    torch.testing.assert_close(got.float(), want, rtol=1e-2, atol=1e-2 * rms)


@pytest.mark.parametrize("M,N,K", [(32768, 1152, 384), (25216, 768, 192), (30001, 1000, 256),
                                   (65536, 384, 384), (24000, 4096, 64)])
@pytest.mark.parametrize("epi", ["none", "bias", "gelu", "residual"])
def test_linear_large(M, N, K, epi):
    g = torch.Generator(device=DEV).manual_seed(M + N)
    a = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(torch.bfloat16)
    b = torch.randn(N, device=DEV, generator=g).to(torch.bfloat16) if epi in ("bias", "gelu", "residual") else None
    res = torch.randn(M, N, device=DEV, generator=g).to(torch.bfloat16) if epi == "residual" else None
    out = ops.linear(a, W, b, gelu=(epi == "gelu"), residual=res)
    ref = a.float() @ W.float().t()
    if b is not None:
        ref = (ref + b.float()).to(torch.bfloat16).float()
    if epi == "gelu":
        ref = F.gelu(ref)
    if res is not None:
        ref = ref + res.float()
    torch.cuda.synchronize()
    _close(out, ref)


@pytest.mark.parametrize("B,N,C,H", [(32, 1024, 384, 3), (8, 4096, 768, 3), (64, 197, 192, 3)])
def test_projection_headsplit_large(B, N, C, H):
    torch.manual_seed(0)
    d = ops.make_desc(B, N, C, H, N, 9, N, torch.bfloat16, "matmul", "depthwise", True, False, False)
    x = torch.randn(B, N, C, device=DEV).to(torch.bfloat16)
    Ws = [(torch.randn(C, C, device=DEV) / C ** 0.5).to(torch.bfloat16) for _ in range(3)]
    q, k, v, _, _ = ops.project_qkv(d, x, None, *Ws)
    dk = C // H
    for t, W in zip((q, k, v), Ws):
        ref = (x.float() @ W.float().t()).view(B, N, H, dk).transpose(1, 2).reshape(B * H, N, dk)
        _close(t[..., :dk], ref)


def test_staged_tiles_exact_selection():
    """A GEMM with a ramp A and a 0/1 selection W isolates every element of the
    staged operand tiles: any misplaced 16-byte chunk shows up as a wrong
    element (the result is exact in bf16)."""
    M, N, K = 256 * 40, 128 * 12, 64
    a = (torch.arange(M * K, device=DEV) % 251).view(M, K).to(torch.bfloat16)
    W = torch.zeros(N, K, device=DEV)
    W[torch.arange(N), torch.arange(N) % K] = 1.0
    out = ops.linear(a, W.to(torch.bfloat16))
    torch.cuda.synchronize()
    ref = a.float()[:, torch.arange(N, device=DEV) % K]
    assert torch.equal(out.float(), ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(128 * 33 + 5, 192 * 5 + 8, 192), (4099, 384, 384), (1000, 200, 64)])
def test_direct_tiles_exact_selection(dtype, M, N, K):
    """The 16-bit row GEMM loads its operand tiles straight into LDS with the
    16-byte chunks of each row permuted.  A ramp A against a 0/1 selection W
    (column n picks A column (7 n + 3) % K) makes every output one exact A
    element, so a misplaced chunk, row or k-tile shows up as a wrong value;
    partial row and column tiles are included."""
    a = (torch.arange(M * K, device=DEV) % 251).view(M, K).to(dtype)
    pick = (torch.arange(N, device=DEV) * 7 + 3) % K
    W = torch.zeros(N, K, device=DEV)
    W[torch.arange(N, device=DEV), pick] = 1.0
    out = ops.linear(a, W.to(dtype))
    torch.cuda.synchronize()
    assert torch.equal(out.float(), a.float()[:, pick])
