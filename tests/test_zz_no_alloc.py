"""GPU: cnna_forward_noalloc (static device scratch, no workspace) returns what
cnna_forward (caller workspace) returns, bit for bit, on consecutive calls
whose sizes shrink, so a call that leaves larger intermediates in the shared
scratch does not disturb the next one."""
import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops

DEV = "cuda"


def _case(B, N, C, H, K, dtype, metric, conv, seed):
    g = torch.Generator().manual_seed(seed)
    d = ops.make_desc(B, N, C, H, N, K, N, dtype, metric, conv, True, False, False)
    x = torch.randn(B, N, C, generator=g).to(dtype).to(DEV)
    W = [(torch.randn(C, C, generator=g) / C ** 0.5).to(dtype).to(DEV) for _ in range(4)]
    dk = C // H
    if conv == "standard":
        w0, w1 = (torch.randn(dk, dk, K, generator=g) * 0.3).to(dtype).to(DEV), None
    elif conv == "depthwise":
        w0, w1 = (torch.randn(dk, 1, K, generator=g)).to(dtype).to(DEV), None
    else:
        w0 = torch.randn(dk, 1, K, generator=g).to(dtype).to(DEV)
        w1 = (torch.randn(dk, dk, 1, generator=g) * 0.3).to(dtype).to(DEV)
    return d, x, W, w0, w1


# consecutive calls, each smaller than the one before (the first near the c3 size)
CASES = [
    (16, 1024, 384, 3, 9, torch.bfloat16, "matmul", "depthwise", 1),
    (4, 512, 384, 3, 9, torch.bfloat16, "matmul", "depthwise", 2),
    (2, 197, 192, 3, 9, torch.float32, "cosine", "standard", 3),
    (2, 150, 128, 2, 40, torch.float16, "matmul", "depthwise", 5),
    (1, 65, 96, 2, 5, torch.float32, "euclidean", "depthwise-separable", 4),
]


def test_noalloc_forward_matches_workspace_forward_on_shrinking_calls():
    outs = []
    for case in CASES:
        d, x, W, w0, w1 = _case(*case)
        assert ops.LIB.cnna_forward_workspace(__import__("ctypes").byref(d)) <= ops.NOALLOC_SCRATCH_BYTES
        ref = ops.forward_fused(d, x, None, *W, w0, w1)
        out = torch.full_like(ref, float("nan"))
        got = ops.forward_noalloc(d, x, None, *W, w0, w1, out=out)
        torch.cuda.synchronize()
        print(f"case {case[:8]}: max |noalloc - workspace| "
              f"{(got.float() - ref.float()).abs().max().item():.3g}", flush=True)
        assert torch.equal(got, ref), case
        outs.append((d, x, W, w0, w1, ref))
    # again, in the same order: the scratch still holds the last (smallest) call's data
    for d, x, W, w0, w1, ref in outs:
        assert torch.equal(ops.forward_noalloc(d, x, None, *W, w0, w1), ref)


def test_noalloc_rejects_a_call_beyond_the_scratch():
    d = ops.make_desc(8, 4096, 768, 3, 4096, 16, 4096, torch.bfloat16, "matmul", "standard", True, False, False)
    x = torch.zeros(1, device=DEV)
    with pytest.raises(RuntimeError, match="static scratch"):
        ops.check(ops.LIB.cnna_forward_noalloc(__import__("ctypes").byref(d), ops._ptr(x), 768, None, ops._ptr(x),
                                               ops._ptr(x), ops._ptr(x), ops._ptr(x), ops._ptr(x), None,
                                               ops._ptr(x), 768, ops._stream()))
