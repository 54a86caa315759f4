"""Write golden vectors of the reference's attention dropout (training mode).

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden_dropout.py [/root/reference]

It imports the reference's ``layers.py`` and runs, on the CPU with a seeded
generator, in training mode:

* ``MultiHeadConvNNAttention.forward`` with ``attention_dropout`` > 0: the
  mask is drawn on the conv output y (B*H, d_k, N) (layers.py:316), before
  the head merge; for sampled paths after the ``randperm`` draw
  (layers.py:284);
* ``MultiHeadKvtAttention.forward`` with ``attn_drop`` > 0: the mask is drawn
  on the dense (B, H, N, N) probabilities (layers.py:680).

Each case is written as ``dropout_<name>_<dtype>.npz`` holding data only: x,
the parameters (reference names), the forward seed, the output, an upstream
gradient ``dout`` with the reference's autograd gradients, and the
constructor arguments as JSON.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

CONVNN = [
    # name, ctor kwargs, (B, N)
    ("convnn_h3_matmul_dw", dict(d_hidden=12, num_heads=3, attention_dropout=0.3, K=4, sampling_type="all",
                                 num_samples=-1, sample_padding=0, magnitude_type="matmul", seq_length=13,
                                 convolution_type="depthwise", softmax_topk_val=True), (2, 13)),
    ("convnn_h1_cosine_std", dict(d_hidden=8, num_heads=1, attention_dropout=0.5, K=3, sampling_type="all",
                                  num_samples=-1, sample_padding=0, magnitude_type="cosine", seq_length=197,
                                  convolution_type="standard", softmax_topk_val=True), (2, 9)),
    ("convnn_h2_random_dws", dict(d_hidden=8, num_heads=2, attention_dropout=0.2, K=3, sampling_type="random",
                                  num_samples=5, sample_padding=0, magnitude_type="matmul", seq_length=10,
                                  convolution_type="depthwise-separable", softmax_topk_val=True), (2, 10)),
]
KVT = [
    ("kvt_h3", dict(dim=12, num_heads=3, attn_drop=0.3, topk=4), (2, 10)),
    ("kvt_h2_scale", dict(dim=8, num_heads=2, attn_drop=0.5, qk_scale=0.7, topk=3), (2, 7)),
]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import layers  # the reference module (layers.py)

    for dtype in (torch.float64, torch.float32):
        tag = "f64" if dtype == torch.float64 else "f32"
        for i, (name, kw, (B, N)) in enumerate(CONVNN + KVT):
            seed = 2000 + i
            torch.manual_seed(seed)
            if name.startswith("kvt"):
                mod = layers.MultiHeadKvtAttention(**kw).to(dtype).train()
                C = kw["dim"]
            else:
                mod = layers.MultiHeadConvNNAttention(**kw).to(dtype).train()
                C = kw["d_hidden"]
                with torch.no_grad():
                    for name_p, p in mod.named_parameters():
                        if name_p.startswith("conv"):
                            p.copy_(torch.randn_like(p))
            x = torch.randn(B, N, C, dtype=dtype)
            dout = torch.randn(B, N, C, dtype=dtype)
            fwd_seed = 50 + i
            torch.manual_seed(fwd_seed)
            xr = x.clone().requires_grad_(True)
            out = mod(xr)
            out.backward(dout)
            arrays = {"x": x.numpy(), "out": out.detach().numpy(), "dout": dout.numpy(),
                      "fwd_seed": np.array([fwd_seed], dtype=np.int64), "grad:x": xr.grad.numpy()}
            for name_p, p in mod.state_dict().items():
                arrays["param:" + name_p] = p.numpy()
            for name_p, p in mod.named_parameters():
                arrays["grad:" + name_p] = p.grad.numpy()
            arrays["ctor"] = np.frombuffer(json.dumps(kw).encode(), dtype=np.uint8)
            path = os.path.join(HERE, f"dropout_{name}_{tag}.npz")
            np.savez_compressed(path, **arrays)
            print("wrote", path, tuple(out.shape))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
