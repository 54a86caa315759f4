"""ViT-Tiny harness on the GPU (run on an MI355X).

* parity: a 2-block ViT with the HIP ConvNN-Attention equals the same network
  whose attention blocks run the CPU oracle's restatement (fp32, exact mode);
* the config-2 target: the 12-block ViT-Tiny forward (B=128, 224x224, bf16)
  is faster than the reference's own GPU path, i.e. the same network with the
  reference op sequence (oracle reference mode) run eagerly on ROCm tensors.
"""
import copy
import time

import pytest
import torch

from oracle import cnna_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from vit import ViT, vit_tiny_args

DEV = "cuda"


class OracleAttention(torch.nn.Module):
    """Attention block running the oracle with the module's own parameters."""

    def __init__(self, attn, cfg, mode, device):
        super().__init__()
        sd = {k: v.detach().to(device) for k, v in attn.state_dict().items()}
        self.p = O.Params.from_module_state(sd, cfg.convolution_type)
        self.cfg, self.mode = cfg, mode

    def forward(self, x):
        out = O.forward(x, self.p, self.cfg, mode=self.mode)
        return out.to(x.dtype)


def oracle_vit(model, mode, device):
    ref = copy.deepcopy(model).to(device)
    a = model.args
    N = (a.img_size[1] // a.patch_size) * (a.img_size[2] // a.patch_size) + 1
    cfg = O.Config(d_hidden=a.d_hidden, num_heads=a.num_heads, K=a.K, sampling_type=a.sampling_type,
                   num_samples=a.num_samples, magnitude_type=a.magnitude_type, seq_length=N,
                   convolution_type=a.convolution_type, softmax_topk_val=a.softmax_topk_val)
    for blk in ref.transformer_encoder:
        blk.attention = OracleAttention(blk.attention, cfg, mode, device)
    return ref


def test_vit_matches_oracle_fp32():
    torch.manual_seed(0)
    # N = 65: the seq_length the attention layers need is the patch count + 1
    args = vit_tiny_args(img_size=(3, 32, 32), patch_size=4, num_layers=2, dropout=0.0,
                         attention_dropout=0.0, softmax_topk_val=True)
    model = ViT(args).to(DEV).eval()
    for blk in model.transformer_encoder:
        blk.attention.seq_length = 65
    x = torch.randn(4, 3, 32, 32, device=DEV)
    with torch.no_grad():
        out = model(x).cpu().double()
        ref = oracle_vit(model, "exact", "cpu").double()(x.cpu().double())
    torch.testing.assert_close(out, ref, rtol=1e-3, atol=1e-4)


def test_vit_tiny_faster_than_reference_gpu_path():
    torch.manual_seed(0)
    model = ViT(vit_tiny_args()).to(DEV).to(torch.bfloat16).eval()
    imgs = torch.randn(128, 3, 224, 224, device=DEV).to(torch.bfloat16)
    ref = oracle_vit(model, "reference", DEV)

    def timed(m, reps=3):
        with torch.no_grad():
            m(imgs)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                m(imgs)
            torch.cuda.synchronize()
        return (time.perf_counter() - t0) / reps

    t_ours, t_ref = timed(model), timed(ref)
    print(f"ViT-Tiny B=128 bf16 forward: ours {t_ours * 1e3:.2f} ms, reference GPU path "
          f"{t_ref * 1e3:.2f} ms, speed-up {t_ref / t_ours:.1f}x")
    assert t_ours < t_ref
