"""Host-side checks of the C-ABI library (no GPU needed).

* libcnna.so loads and exports every entry point include/cnna.h declares;
* descriptor validation returns the error codes that map to the exceptions the
  reference raises (layers.py:149, 251, 310, torch.topk range, Conv1d groups).
"""
import ctypes
import os
import re

import pytest
import torch

import cnna_ops as ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "cnna.h")).read()
    return sorted(set(re.findall(r"\b(cnna_[a-z_0-9]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 10
    for n in names:
        assert hasattr(ops.LIB, n), n
    assert set(names) == set(ops.EXPORTED)


def test_abi_version():
    assert ops.LIB.cnna_abi_version() == 4


def desc(**kw):
    base = dict(B=2, N=16, C=12, H=3, Nq=16, K=4, seq_length=16, dtype=ops.CNNA_F32, metric=0, conv=1,
                softmax=1, sampled=0, coord=0, merge=0, scale=0.0)
    base.update(kw)
    return ops.Desc(*[base[f] for f, _ in ops.Desc._fields_])


def status(**kw):
    d = desc(**kw)
    return ops.LIB.cnna_check_desc(ctypes.byref(d))


def test_check_desc_ok():
    assert status() == 0
    assert status(sampled=1, Nq=5, K=6) == 0


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=7), ops.ERR_DTYPE),
    (dict(C=13), ops.ERR_SHAPE),                       # d_hidden % num_heads
    (dict(metric=5), ops.ERR_OPTION),
    (dict(conv=9), ops.ERR_OPTION),
    (dict(coord=1), ops.ERR_GROUPS),                   # depthwise + coordinate encoding
    (dict(K=17), ops.ERR_K_RANGE),                     # K > candidates
    (dict(sampled=1, Nq=4, K=6), ops.ERR_K_RANGE),     # K-1 > num_samples
    (dict(merge=2), ops.ERR_OPTION),                   # unknown head layout
    (dict(metric=1, scale=0.5), ops.ERR_OPTION),       # a scale only for matmul
    (dict(scale=float("inf")), ops.ERR_OPTION),
    (dict(seq_length=197), ops.ERR_SEQ),               # H > 1 and seq_length != N
    (dict(K=0), ops.ERR_K_RANGE),
    # valid for the reference, beyond the kernels' limits: NotImplementedError, not a range error
    (dict(C=3 * 264, dtype=ops.CNNA_BF16), ops.ERR_UNSUPPORTED),   # bf16 head width > 256
    (dict(C=3 * 264), ops.ERR_UNSUPPORTED),                        # f32 head width > 256
    (dict(C=2 * 256, H=2, conv=0, coord=1), ops.ERR_UNSUPPORTED),  # 256 + coordinate channel
    (dict(N=70000, Nq=70000, seq_length=70000), ops.ERR_UNSUPPORTED),
])
def test_check_desc_errors(kw, code):
    assert status(**kw) == code


def test_negative_matmul_scale_accepted():
    # KVT's qk_scale may be negative (layers.py:662): the kernels rank k.q * scale
    assert status(scale=-0.25) == 0
    assert status(scale=-0.25, merge=1, seq_length=5) == 0


def test_concat_merge_ignores_seq_length():
    # KVT's head layout has no reshape by seq_length
    assert status(seq_length=5) == ops.ERR_SEQ
    assert status(seq_length=5, merge=1, scale=0.25) == 0


def test_h1_ignores_seq_length():
    assert status(H=1, seq_length=197) == 0


def test_error_strings_and_exception_types():
    with pytest.raises(RuntimeError):
        ops.check(ops.ERR_K_RANGE)
    with pytest.raises(RuntimeError):
        ops.check(ops.ERR_SEQ)
    with pytest.raises(ValueError):
        ops.check(ops.ERR_GROUPS)
    with pytest.raises(TypeError):
        ops.check(ops.ERR_DTYPE)
    with pytest.raises(NotImplementedError, match="K <= 64"):
        ops.check(ops.ERR_UNSUPPORTED)
    assert b"workspace" in ops.LIB.cnna_error_string(ops.ERR_WS)


def test_head_stride_padding():
    d = desc(C=384, H=3, N=8, Nq=8, seq_length=8)
    assert ops.LIB.cnna_head_stride(ctypes.byref(d)) == 128
    d = desc(C=12, H=3)
    assert ops.LIB.cnna_head_stride(ctypes.byref(d)) == 16
    d = desc(C=128, H=2, conv=0, coord=1)
    assert ops.LIB.cnna_head_stride(ctypes.byref(d)) == 80


def test_workspace_size_positive():
    d = desc()
    assert ops.LIB.cnna_forward_workspace(ctypes.byref(d)) > 0
    bad = desc(K=99)
    assert ops.LIB.cnna_forward_workspace(ctypes.byref(bad)) == 0


def test_module_rejects_cpu_tensors():
    from layers import MultiHeadConvNNAttention
    m = MultiHeadConvNNAttention(12, 3, 0.0, 4, "all", -1, 0, "matmul", seq_length=16)
    with pytest.raises(RuntimeError, match="ROCm"):
        m(torch.randn(2, 16, 12))


def test_module_matches_reference_parameter_names_and_init():
    """Same parameter names/shapes and the same seeded initial values as the
    oracle's restatement of the reference init order."""
    from layers import MultiHeadConvNNAttention
    from oracle import cnna_oracle as O
    for conv in ("standard", "depthwise", "depthwise-separable"):
        torch.manual_seed(0)
        m = MultiHeadConvNNAttention(12, 3, 0.1, 4, "all", -1, 0, "matmul", seq_length=16,
                                     convolution_type=conv)
        names = sorted(m.state_dict().keys())
        exp = ["W_k.weight", "W_o.weight", "W_q.weight", "W_v.weight"]
        exp += ["conv.0.weight", "conv.1.weight"] if conv == "depthwise-separable" else ["conv.weight"]
        assert names == sorted(exp)
        p = O.Params.from_module_state(m.state_dict(), conv)
        assert p.W_q.shape == (12, 12)
        if conv == "depthwise":
            assert torch.all(p.conv0 == 1.0) and p.conv0.shape == (4, 1, 4)


def test_noalloc_scratch_limit():
    """cnna_forward_noalloc works in a static 128 MiB device array: the c3
    layer fits, the c5 one is rejected with CNNA_ERR_SCRATCH before any device
    call (so this runs without a GPU)."""
    c3 = desc(B=32, N=1024, Nq=1024, C=384, H=3, K=9, seq_length=1024, dtype=ops.CNNA_BF16)
    assert ops.LIB.cnna_forward_workspace(ctypes.byref(c3)) <= ops.NOALLOC_SCRATCH_BYTES
    c5 = desc(B=8, N=4096, Nq=4096, C=768, H=3, K=16, seq_length=4096, dtype=ops.CNNA_BF16, conv=0)
    assert ops.LIB.cnna_forward_workspace(ctypes.byref(c5)) > ops.NOALLOC_SCRATCH_BYTES
    st = ops.LIB.cnna_forward_noalloc(ctypes.byref(c5), None, 768, None, None, None, None, None, None, None,
                                      None, 768, None)
    assert st == ops.ERR_SCRATCH
    assert b"128 MiB" in ops.LIB.cnna_error_string(ops.ERR_SCRATCH)


def test_folded_layernorm_limits():
    """The LayerNorm folding entry points reject what their kernels do not do
    before any device call: fp32 statistics epilogue, Nout % 8 != 0, rows
    wider than 1024 for the prologue, misaligned statistics, a missing ln."""
    fake = ctypes.c_void_p(1 << 20)              # never dereferenced: rejected first
    st = ctypes.c_void_p(1 << 20)
    ln = ops.Ln(1 << 20, None, None, 1e-5)
    lin = ops.LIB.cnna_linear_ln
    # fp32 output statistics come from cnna_row_stats, not the GEMM epilogue
    assert lin(ops.CNNA_F32, 64, 192, 192, fake, 192, None, fake, None, 0, None, 0, fake, 192, st,
               None) == ops.ERR_UNSUPPORTED
    assert lin(ops.CNNA_BF16, 64, 196, 192, fake, 192, None, fake, None, 0, None, 0, fake, 196, st,
               None) == ops.ERR_UNSUPPORTED
    assert lin(ops.CNNA_BF16, 64, 192, 2048, fake, 2048, ctypes.byref(ln), fake, None, 0, None, 0, fake, 192,
               None, None) == ops.ERR_UNSUPPORTED
    assert lin(ops.CNNA_BF16, 64, 192, 192, fake, 192, None, fake, None, 0, None, 0, fake, 192,
               ctypes.c_void_p((1 << 20) + 4), None) == ops.ERR_SHAPE
    bad = ops.Ln(None, None, None, 1e-5)
    assert lin(ops.CNNA_BF16, 64, 192, 192, fake, 192, ctypes.byref(bad), fake, None, 0, None, 0, fake, 192,
               None, None) == ops.ERR_NULL
    d = desc(dtype=ops.CNNA_BF16)
    assert ops.LIB.cnna_project_qkv_ex(ctypes.byref(d), fake, 12, ctypes.byref(bad), None, fake, fake, fake,
                                       None, fake, fake, fake, None, None, None) == ops.ERR_NULL
    assert ops.LIB.cnna_row_stats(ops.CNNA_BF16, 4, 192, fake, 100, st, None) == ops.ERR_SHAPE
    assert ops.LIB.cnna_row_stats(ops.CNNA_BF16, 0, 192, None, 192, None, None) == 0
    assert b"folded LayerNorm" in ops.LIB.cnna_error_string(ops.ERR_UNSUPPORTED)


def test_wide_k_forward_accepted_backward_limited():
    """K > 32 runs forward (rounds of 32 in the select kernel); the backward
    holds a token's entries one per lane and refuses K > 64 before any device
    call (NotImplementedError naming the limit)."""
    assert status(N=200, Nq=200, seq_length=200, K=100) == 0
    assert status(N=200, Nq=200, seq_length=200, K=200) == 0
    d = desc(N=200, Nq=200, seq_length=200, K=65)
    fake = ctypes.c_void_p(1 << 20)
    sv, gr = ops.Saved(*([1 << 20] * 10)), ops.Grads(*([1 << 20] * 6))
    st = ops.LIB.cnna_core_backward(ctypes.byref(d), fake, 12, None, fake, fake, fake, fake, None,
                                    ctypes.byref(sv), fake, ctypes.byref(gr), fake, 1 << 30, None)
    assert st == ops.ERR_UNSUPPORTED
    assert b"K <= 64" in ops.LIB.cnna_error_string(ops.ERR_UNSUPPORTED)


def test_wide_float32_heads_accepted():
    # float32 heads up to 256 channels (the wide select instances), as for 16-bit types
    assert status(C=2 * 256, H=2) == 0
    assert status(C=2 * 192, H=2) == 0
    assert status(C=2 * 255, H=2, conv=0, coord=1) == 0
