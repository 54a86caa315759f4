"""Write golden vectors for the compositions no closed form pins.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden.py [/root/reference]

It imports the reference's ``layers.py`` and runs
``MultiHeadConvNNAttention.forward`` at tiny shapes for the parts of the
operator whose composition only the reference itself can pin:

* sampled paths ``_prime_N`` / ``_prime_softmax_N`` (layers.py:361-437):
  self at rank 0, fp32 ``ones`` logits, self-mask constants
  (layers.py:291-292, 304-305);
* ``batch_split`` / ``combine_heads`` head merge (layers.py:247-259, 317);
* coordinate encoding on sampled queries (layers.py:286-287, 439-450);
* the euclidean ``_prime`` division (layers.py:352-353, 382-383).

Each case is written as ``<name>.npz`` holding only data: the input ``x``,
the module's parameters (by their reference names), the sampled candidate
indices (when any), the output, the constructor arguments as JSON, and the
reference's autograd gradients for an upstream gradient ``dout``:
``grad:x`` and ``grad:<parameter name>``.
Cases run in float64 (tight comparison) and float32.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = [
    # name, ctor kwargs, (B, N), dtype
    ("all_cosine_softmax_dw_h3", dict(d_hidden=12, num_heads=3, K=4, sampling_type="all", num_samples=-1,
                                      sample_padding=0, magnitude_type="cosine", seq_length=13,
                                      convolution_type="depthwise", softmax_topk_val=True), (2, 13)),
    ("all_matmul_softmax_dws_h3", dict(d_hidden=12, num_heads=3, K=3, sampling_type="all", num_samples=-1,
                                       sample_padding=0, magnitude_type="matmul", seq_length=11,
                                       convolution_type="depthwise-separable", softmax_topk_val=True), (2, 11)),
    ("all_matmul_raw_std_h1", dict(d_hidden=8, num_heads=1, K=3, sampling_type="all", num_samples=-1,
                                   sample_padding=0, magnitude_type="matmul", seq_length=197,
                                   convolution_type="standard", softmax_topk_val=False), (2, 9)),
    ("all_euclid_raw_dw_h2", dict(d_hidden=8, num_heads=2, K=3, sampling_type="all", num_samples=-1,
                                  sample_padding=0, magnitude_type="euclidean", seq_length=10,
                                  convolution_type="depthwise", softmax_topk_val=False), (2, 10)),
    ("all_euclid_softmax_std_h2", dict(d_hidden=8, num_heads=2, K=4, sampling_type="all", num_samples=-1,
                                       sample_padding=0, magnitude_type="euclidean", seq_length=10,
                                       convolution_type="standard", softmax_topk_val=True), (2, 10)),
    ("random_matmul_softmax_dw_h3", dict(d_hidden=12, num_heads=3, K=4, sampling_type="random", num_samples=6,
                                         sample_padding=0, magnitude_type="matmul", seq_length=13,
                                         convolution_type="depthwise", softmax_topk_val=True), (2, 13)),
    ("random_cosine_raw_std_h3", dict(d_hidden=12, num_heads=3, K=3, sampling_type="random", num_samples=5,
                                      sample_padding=0, magnitude_type="cosine", seq_length=12,
                                      convolution_type="standard", softmax_topk_val=False), (2, 12)),
    ("random_euclid_softmax_dws_h1", dict(d_hidden=6, num_heads=1, K=3, sampling_type="random", num_samples=5,
                                          sample_padding=0, magnitude_type="euclidean", seq_length=197,
                                          convolution_type="depthwise-separable", softmax_topk_val=True), (3, 9)),
    ("spatial_cosine_raw_dw_h3", dict(d_hidden=12, num_heads=3, K=4, sampling_type="spatial", num_samples=5,
                                      sample_padding=1, magnitude_type="cosine", seq_length=14,
                                      convolution_type="depthwise", softmax_topk_val=False), (2, 14)),
    ("spatial_euclid_raw_std_h2", dict(d_hidden=8, num_heads=2, K=3, sampling_type="spatial", num_samples=4,
                                       sample_padding=0, magnitude_type="euclidean", seq_length=11,
                                       convolution_type="standard", softmax_topk_val=False), (2, 11)),
    ("random_matmul_softmax_std_coord_h2", dict(d_hidden=8, num_heads=2, K=3, sampling_type="random",
                                                num_samples=5, sample_padding=0, magnitude_type="matmul",
                                                seq_length=10, coordinate_encoding=True,
                                                convolution_type="standard", softmax_topk_val=True), (2, 10)),
    ("all_cosine_softmax_dws_coord_h2", dict(d_hidden=8, num_heads=2, K=3, sampling_type="all", num_samples=-1,
                                             sample_padding=0, magnitude_type="cosine", seq_length=9,
                                             coordinate_encoding=True, convolution_type="depthwise-separable",
                                             softmax_topk_val=True), (2, 9)),
]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import layers  # the reference module (layers.py)

    for dtype in (torch.float64, torch.float32):
        tag = "f64" if dtype == torch.float64 else "f32"
        for i, (name, kw, (B, N)) in enumerate(CASES):
            seed = 1000 + i
            torch.manual_seed(seed)
            mod = layers.MultiHeadConvNNAttention(attention_dropout=0.0, **kw).to(dtype).eval()
            # non-unit depthwise weights so tap order matters
            with torch.no_grad():
                for name_p, p in mod.named_parameters():
                    if name_p.startswith("conv"):
                        p.copy_(torch.randn_like(p))
            x = torch.randn(B, N, kw["d_hidden"], dtype=dtype)
            dout = torch.randn(B, N, kw["d_hidden"], dtype=dtype)
            fwd_seed = 7 + i
            torch.manual_seed(fwd_seed)
            xr = x.clone().requires_grad_(True)
            out = mod(xr)
            grad_error = None
            try:
                out.backward(dout)
            except RuntimeError as e:   # the reference's own autograd failure
                grad_error = str(e).split("\n")[0]
            out = out.detach()
            cand = None
            if kw["sampling_type"] == "random":
                torch.manual_seed(fwd_seed)
                cand = torch.randperm(N)[: kw["num_samples"]]
            elif kw["sampling_type"] == "spatial":
                pad = kw["sample_padding"]
                cand = torch.linspace(pad, N - pad - 1, kw["num_samples"]).long()
            arrays = {"x": x.numpy(), "out": out.numpy(), "dout": dout.numpy()}
            for name_p, p in mod.state_dict().items():
                arrays["param:" + name_p] = p.numpy()
            if grad_error is None:
                arrays["grad:x"] = xr.grad.numpy()
                for name_p, p in mod.named_parameters():
                    arrays["grad:" + name_p] = p.grad.numpy()
            else:
                arrays["grad_error"] = np.frombuffer(grad_error.encode(), dtype=np.uint8)
            if cand is not None:
                arrays["cand"] = cand.numpy()
            arrays["ctor"] = np.frombuffer(json.dumps(kw).encode(), dtype=np.uint8)
            path = os.path.join(HERE, f"{name}_{tag}.npz")
            np.savez_compressed(path, **arrays)
            print("wrote", path, tuple(out.shape))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
