"""torch.library registration of the operator, checked without a GPU.

Under a fake-tensor mode the layers route through ``cnna::core`` /
``cnna::output_proj`` (the path torch.compile traces): the fake kernels give
the shapes and dtypes of the native ones, and FlopCounterMode counts the
registered formulas.  Backward needs a device and is covered by the GPU tests.
"""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.utils.flop_counter import FlopCounterMode

import cnna_ops as ops
from layers import MultiHeadConvNNAttention, MultiHeadKvtAttention


def test_eager_path_is_the_default():
    assert not ops.use_library_ops()


@pytest.mark.parametrize("sampling,ns,metric,conv,coord", [
    ("all", -1, "matmul", "depthwise", False),
    ("random", 64, "euclidean", "standard", False),
    ("spatial", 16, "cosine", "depthwise-separable", True),
])
def test_fake_forward_shapes_and_flops(sampling, ns, metric, conv, coord):
    B, N, C, H, K = 2, 256, 192, 3, 9
    with FakeTensorMode(), torch.device("cuda"):
        m = MultiHeadConvNNAttention(C, H, 0.0, K, sampling, ns, 0, metric, seq_length=N,
                                     coordinate_encoding=coord, convolution_type=conv)
        x = torch.randn(B, N, C)
        fc = FlopCounterMode(display=False)
        with fc:
            y = m(x)
        assert y.shape == (B, N, C) and y.dtype == torch.float32
        counts = {str(k): v for k, v in fc.get_flop_counts()["Global"].items()}
    Nq = N if sampling == "all" else ns
    dk = C // H
    din = dk + int(coord)
    proj = 2 * B * C * C * (2 * N + Nq)
    sim = 2 * B * N * Nq * H * din
    cv = {"depthwise": 2 * B * N * C * K, "standard": 2 * B * N * H * dk * din * K,
          "depthwise-separable": 2 * B * N * H * (din * K + dk * din)}[conv]
    assert counts == {"cnna.core": proj + sim + cv, "cnna.output_proj": 2 * B * N * C * C}


def test_fake_core_outputs():
    with FakeTensorMode(), torch.device("cuda"):
        x = torch.randn(2, 100, 96, dtype=torch.bfloat16)
        W = [torch.randn(96, 96, dtype=torch.bfloat16) for _ in range(3)]
        w0 = torch.ones(32, 1, 5, dtype=torch.bfloat16)
        d = ops.desc_values(2, 100, 96, 3, 100, 5, 100, torch.bfloat16, "cosine", "depthwise", True,
                            False, False)
        z, q, k, v, qn, kn, idx, vals, w, wm, cols = torch.ops.cnna.core(x, *W, w0, None, None, None, d, 0.0, True, 1.0)
    assert z.shape == (2, 100, 96) and z.dtype == torch.bfloat16
    assert q.shape == k.shape == v.shape == (6, 100, 32)
    assert qn.shape == kn.shape == (600,)
    assert idx.dtype == torch.int32 and idx.shape == vals.shape == w.shape == (6, 100, 5)


def test_fake_kvt_forward():
    with FakeTensorMode(), torch.device("cuda"):
        m = MultiHeadKvtAttention(192, 3, topk=9)
        fc = FlopCounterMode(display=False)
        with fc:
            y = m(torch.randn(4, 197, 192))
        assert y.shape == (4, 197, 192)
        assert fc.get_total_flops() > 0
