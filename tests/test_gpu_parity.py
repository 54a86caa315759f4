"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Stage by stage (each kernel on the *same* inputs as the oracle):
  projection  -> torch fp32 GEMM of the same operands, within output rounding;
  select      -> oracle stable top-k on float64 S of the kernel's own k, q:
                 indices exact except where |S gap| < 1e-6 (north-star rule);
  aggregate   -> oracle float64 weights/gather/conv on the kernel's v/idx/vals;
  output proj -> oracle head merge (the reference's reshapes) + W_o.
End to end: fp32 within rtol 1e-3; bf16 within rtol 2e-2 (of the output RMS)
against the oracle's exact mode fed the same bf16 projections.
"""
import math

import pytest
import torch

from oracle import cnna_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cnna_ops as ops
    from layers import MultiHeadConvNNAttention

DEV = "cuda"
TOL_IDX = 1e-6


def make(cfg: O.Config, B, N, dtype, seed=0, rand_conv=True):
    g = torch.Generator().manual_seed(seed)
    p = O.init_params(cfg, seed=seed, dtype=torch.float32)
    if rand_conv:
        p.conv0 = torch.randn(p.conv0.shape, generator=g) * 0.5
        if p.conv1 is not None:
            p.conv1 = torch.randn(p.conv1.shape, generator=g) * 0.5
    p = p.to(dtype=dtype)
    x = torch.randn(B, N, cfg.d_hidden, generator=g).to(dtype)
    return p, x


def desc_for(cfg, B, N, Nq, dtype):
    return ops.make_desc(B, N, cfg.d_hidden, cfg.num_heads, Nq, cfg.K, cfg.seq_length, dtype,
                         cfg.magnitude_type, cfg.convolution_type, cfg.softmax_topk_val,
                         cfg.sampling_type != "all", cfg.coordinate_encoding)


def cand_for(cfg, N, seed=2):
    if cfg.sampling_type == "all":
        return None
    g = torch.Generator().manual_seed(seed)
    return O.sample_indices(cfg, N, generator=g)


def gpu(t):
    return None if t is None else t.to(DEV)


def run_stages(cfg, p, x, cand):
    B, N, C = x.shape
    Nq = N if cand is None else cand.numel()
    d = desc_for(cfg, B, N, Nq, x.dtype)
    cg = None if cand is None else cand.to(torch.int32).to(DEV)
    xg = x.to(DEV)
    q, k, v, qn, kn = ops.project_qkv(d, xg, cg, gpu(p.W_q), gpu(p.W_k), gpu(p.W_v))
    idx, vals, w = ops.select(d, k, q, kn, qn, cg)
    z = ops.aggregate(d, v, idx, w, gpu(p.conv0), gpu(p.conv1))
    out = ops.output_proj(d, z, gpu(p.W_o))
    torch.cuda.synchronize()
    return d, dict(q=q.cpu(), k=k.cpu(), v=v.cpu(), idx=idx.cpu().long(), vals=vals.cpu(), w=w.cpu(),
                   z=z.cpu(), out=out.cpu())


def check_select(cfg, r, cand, B):
    din = cfg.in_channels
    idx_e, vals_e, S = O.topk_exact(r["k"], r["q"], cfg, cand, kvalid=din, normalized_inputs=True)
    ok = O.topk_gap_ok(S, r["idx"], idx_e, cfg, cand, tol=TOL_IDX)
    bad = (~ok).sum().item()
    assert bad == 0, f"{bad} rows with top-k mismatch beyond the 1e-6 gap rule"
    # values: the selected similarity values (self = 1.0 for sampled)
    got = r["vals"].double()
    exp = vals_e
    fin = torch.isfinite(exp)
    torch.testing.assert_close(got[fin], exp[fin], rtol=1e-5, atol=1e-5)
    return idx_e


# --------------------------------------------------------------------------- projection

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 13, 12, 3), (4, 65, 192, 3), (2, 200, 384, 3), (3, 40, 64, 1)])
def test_projection_headsplit(dtype, shape):
    B, N, C, H = shape
    cfg = O.Config(d_hidden=C, num_heads=H, K=4, seq_length=N)
    p, x = make(cfg, B, N, dtype, seed=11)
    d, r = run_stages(cfg, p, x, None)
    dk = C // H
    for name, W in (("q", p.W_q), ("k", p.W_k), ("v", p.W_v)):
        ref = O.split_heads(x.float() @ W.float().t(), H).transpose(1, 2)     # (BH, N, dk)
        got = r[name][..., :dk].float()
        tol = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=8e-3, atol=8e-3)
        torch.testing.assert_close(got, ref, **tol)
        if r[name].shape[-1] > dk:
            assert torch.all(r[name][..., dk:] == 0)


# --------------------------------------------------------------------------- select

SELECT_CASES = [
    # (name, cfg kwargs, B, N, dtype)
    ("c1_cosine_f32", dict(d_hidden=192, num_heads=3, K=9, magnitude_type="cosine", seq_length=65), 8, 65, torch.float32),
    ("matmul_f32_N197", dict(d_hidden=192, num_heads=3, K=9, seq_length=197), 4, 197, torch.float32),
    ("matmul_bf16_N1024", dict(d_hidden=384, num_heads=3, K=9, seq_length=1024), 2, 1024, torch.bfloat16),
    # long rows (more than 16 tiles: the pass-1 bound from three quarters of the
    # row, mid-sweep drains of raw keys into float-key lists) in float32, and
    # cosine on a row of 19 tiles
    ("matmul_f32_N1024", dict(d_hidden=192, num_heads=3, K=9, seq_length=1024), 1, 1024, torch.float32),
    ("cosine_bf16_N600", dict(d_hidden=256, num_heads=2, K=7, magnitude_type="cosine", seq_length=600), 2, 600, torch.bfloat16),
    ("euclid_f32", dict(d_hidden=64, num_heads=2, K=5, magnitude_type="euclidean", seq_length=150), 3, 150, torch.float32),
    ("k16_bf16_d256", dict(d_hidden=768, num_heads=3, K=16, seq_length=300), 1, 300, torch.bfloat16),
    ("k32_f32", dict(d_hidden=32, num_heads=1, K=32, seq_length=90), 2, 90, torch.float32),
    ("tiny_k_eq_n", dict(d_hidden=12, num_heads=3, K=13, seq_length=13), 2, 13, torch.float32),
    ("random_matmul_f32", dict(d_hidden=192, num_heads=3, K=9, sampling_type="random", num_samples=64, seq_length=197), 4, 197, torch.float32),
    ("spatial_cosine_f32", dict(d_hidden=192, num_heads=3, K=9, sampling_type="spatial", num_samples=8, magnitude_type="cosine", seq_length=197), 4, 197, torch.float32),
    ("random_euclid_f32", dict(d_hidden=64, num_heads=2, K=6, sampling_type="random", num_samples=20, magnitude_type="euclidean", seq_length=70), 2, 70, torch.float32),
    # float32 heads wider than 128 (key rows of 128 registers, one block per CU):
    # d_k = 256 exactly, and guarded chunks for d_k = 192 / 200
    ("d256_f32", dict(d_hidden=512, num_heads=2, K=9, seq_length=300), 2, 300, torch.float32),
    ("d256_k16_random_euclid_f32", dict(d_hidden=768, num_heads=3, K=16, sampling_type="random", num_samples=100, magnitude_type="euclidean", seq_length=197), 2, 197, torch.float32),
    ("d192_cosine_f32", dict(d_hidden=384, num_heads=2, K=9, magnitude_type="cosine", seq_length=150), 2, 150, torch.float32),
    ("d200_k40_f32", dict(d_hidden=400, num_heads=2, K=40, seq_length=120), 2, 120, torch.float32),
]


@pytest.mark.parametrize("name,kw,B,N,dtype", SELECT_CASES, ids=[c[0] for c in SELECT_CASES])
def test_select_topk_exact(name, kw, B, N, dtype):
    cfg = O.Config(**kw)
    p, x = make(cfg, B, N, dtype, seed=5)
    cand = cand_for(cfg, N)
    d, r = run_stages(cfg, p, x, cand)
    check_select(cfg, r, cand, B)


def test_select_ties_break_by_lowest_index():
    # identical candidate rows -> every key ties; lowest indices must win, in order
    cfg = O.Config(d_hidden=16, num_heads=1, K=7, seq_length=100)
    B, N = 1, 100
    d = desc_for(cfg, B, N, N, torch.float32)
    k = torch.zeros(1, N, 16)
    k[..., 0] = 1.0
    q = torch.zeros(1, N, 16)
    q[..., 0] = 0.5
    q[0, 40, 0] = 0.75          # one clear winner
    idx, vals, _ = ops.select(d, k.to(DEV), q.to(DEV))
    torch.cuda.synchronize()
    exp = [40, 0, 1, 2, 3, 4, 5]
    assert (idx.cpu()[0] == torch.tensor(exp, dtype=torch.int32)).all()


# --------------------------------------------------------------------------- aggregate + merge

AGG_CASES = [
    ("dw_softmax_f32", dict(d_hidden=192, num_heads=3, K=9, seq_length=65), 4, 65, torch.float32),
    ("std_softmax_f32", dict(d_hidden=96, num_heads=3, K=5, seq_length=50, convolution_type="standard"), 2, 50, torch.float32),
    ("dws_raw_f32", dict(d_hidden=64, num_heads=2, K=4, seq_length=33, convolution_type="depthwise-separable", softmax_topk_val=False), 2, 33, torch.float32),
    ("euclid_raw_dw_f32", dict(d_hidden=48, num_heads=3, K=3, seq_length=20, magnitude_type="euclidean", softmax_topk_val=False), 2, 20, torch.float32),
    ("dw_bf16_h3", dict(d_hidden=384, num_heads=3, K=9, seq_length=256), 2, 256, torch.bfloat16),
    ("dw_f32_h1", dict(d_hidden=64, num_heads=1, K=6, seq_length=197), 3, 40, torch.float32),
    ("std_coord_f32", dict(d_hidden=64, num_heads=2, K=4, seq_length=30, convolution_type="standard", coordinate_encoding=True), 2, 30, torch.float32),
]


@pytest.mark.parametrize("name,kw,B,N,dtype", AGG_CASES, ids=[c[0] for c in AGG_CASES])
def test_aggregate_and_merge(name, kw, B, N, dtype):
    cfg = O.Config(**kw)
    p, x = make(cfg, B, N, dtype, seed=7)
    cand = cand_for(cfg, N)
    d, r = run_stages(cfg, p, x, cand)
    # aggregate on the kernel's own v / idx / vals
    z_exp = O.aggregate_exact(r["v"], r["idx"], r["vals"], p, cfg, B, cand is not None)
    z_got = r["z"].double()
    # the weights the select kernel emitted
    w_exp = O.neighbour_weights(r["vals"].double(), cfg, cand is not None)
    torch.testing.assert_close(r["w"].double(), w_exp, rtol=1e-5, atol=1e-6)
    if dtype == torch.float32:
        torch.testing.assert_close(z_got, z_exp, rtol=1e-4, atol=1e-5)
    else:
        torch.testing.assert_close(z_got, z_exp, rtol=1e-2, atol=1e-2 * z_exp.abs().max().item())
    # output projection with the in-place head merge
    out_exp = (z_got.to(dtype).double() @ p.W_o.double().t())
    tol = (1e-5, 1e-5) if dtype == torch.float32 else (1e-2, 1e-2 * out_exp.abs().max().item())
    torch.testing.assert_close(r["out"].double(), out_exp, rtol=tol[0], atol=tol[1])


# --------------------------------------------------------------------------- end to end

E2E_CASES = [
    ("c1_tiny", dict(d_hidden=192, num_heads=3, K=9, magnitude_type="cosine", seq_length=65), 8, 65),
    ("matmul_dw_h3", dict(d_hidden=96, num_heads=3, K=9, seq_length=100), 3, 100),
    ("matmul_std_raw", dict(d_hidden=64, num_heads=2, K=5, seq_length=70, convolution_type="standard", softmax_topk_val=False), 2, 70),
    ("euclid_dws", dict(d_hidden=64, num_heads=2, K=4, seq_length=40, magnitude_type="euclidean", convolution_type="depthwise-separable"), 2, 40),
    ("random_c4a_small", dict(d_hidden=192, num_heads=3, K=9, sampling_type="random", num_samples=64, seq_length=197), 4, 197),
    ("spatial_c4b_small", dict(d_hidden=192, num_heads=3, K=9, sampling_type="spatial", num_samples=8, seq_length=197), 4, 197),
    ("spatial_pad_euclid_raw", dict(d_hidden=48, num_heads=3, K=4, sampling_type="spatial", num_samples=6, sample_padding=2, magnitude_type="euclidean", softmax_topk_val=False, seq_length=30), 2, 30),
    ("coord_std_random", dict(d_hidden=64, num_heads=2, K=5, sampling_type="random", num_samples=12, coordinate_encoding=True, convolution_type="standard", seq_length=40), 2, 40),
    ("h1", dict(d_hidden=48, num_heads=1, K=7, seq_length=197), 2, 60),
    # float32 heads wider than 128
    ("d256_dw_f32", dict(d_hidden=512, num_heads=2, K=9, seq_length=120), 2, 120),
    ("d256_std_k16_f32", dict(d_hidden=768, num_heads=3, K=16, convolution_type="standard", seq_length=100), 1, 100),
    ("d192_coord_std_random_f32", dict(d_hidden=384, num_heads=2, K=5, sampling_type="random", num_samples=40, coordinate_encoding=True, convolution_type="standard", seq_length=60), 2, 60),
]


@pytest.mark.parametrize("name,kw,B,N", E2E_CASES, ids=[c[0] for c in E2E_CASES])
def test_forward_fp32_end_to_end(name, kw, B, N):
    cfg = O.Config(**kw)
    p, x = make(cfg, B, N, torch.float32, seed=3)
    cand = cand_for(cfg, N)
    d, r = run_stages(cfg, p, x, cand)
    ref = O.forward(x.double(), p.to(dtype=torch.float64), cfg, cand=cand, mode="exact")
    torch.testing.assert_close(r["out"].double(), ref, rtol=1e-3, atol=1e-4)


def test_forward_bf16_c3_shape():
    """Config-3 shape (B reduced to 4): staged parity on the kernel's own
    intermediates plus an end-to-end RMS check against the exact oracle."""
    cfg = O.Config(d_hidden=384, num_heads=3, K=9, seq_length=1024)
    B, N = 4, 1024
    p, x = make(cfg, B, N, torch.bfloat16, seed=1, rand_conv=False)
    d, r = run_stages(cfg, p, x, None)
    check_select(cfg, r, None, B)
    z_exp = O.aggregate_exact(r["v"], r["idx"], r["vals"], p, cfg, B, False)
    out_exp = z_exp.to(torch.bfloat16).double() @ p.W_o.double().t()
    rms = out_exp.pow(2).mean().sqrt().item()
    torch.testing.assert_close(r["out"].double(), out_exp, rtol=2e-2, atol=2e-2 * rms)
    # end to end against the exact oracle on the same bf16 inputs
    ref = O.forward(x, p, cfg, mode="exact")
    err = (r["out"].double() - ref.double()).pow(2).mean().sqrt().item()
    assert err < 2e-2 * rms * 3, (err, rms)


def test_cnna_forward_single_entry_matches_stages():
    cfg = O.Config(d_hidden=192, num_heads=3, K=9, seq_length=197)
    B, N = 4, 197
    p, x = make(cfg, B, N, torch.bfloat16, seed=9)
    d, r = run_stages(cfg, p, x, None)
    out = ops.forward_fused(d, x.to(DEV), None, gpu(p.W_q), gpu(p.W_k), gpu(p.W_v), gpu(p.W_o),
                            gpu(p.conv0), gpu(p.conv1))
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), r["out"])


# --------------------------------------------------------------------------- drop-in module

@pytest.mark.parametrize("sampling", ["all", "random", "spatial"])
def test_module_drop_in(sampling):
    torch.manual_seed(0)
    kw = dict(K=9, sampling_type=sampling, num_samples=32 if sampling == "random" else 8,
              sample_padding=0, magnitude_type="cosine", seq_length=65)
    m = MultiHeadConvNNAttention(192, 3, 0.1, **kw).to(DEV).eval()
    x = torch.randn(8, 65, 192, device=DEV)
    torch.cuda.manual_seed(123)
    out = m(x)
    torch.cuda.synchronize()
    cand = None
    if sampling == "random":
        torch.cuda.manual_seed(123)
        cand = torch.randperm(65, device=DEV)[:32].cpu()
    elif sampling == "spatial":
        cand = torch.linspace(0, 64, 8).long()
    cfg = O.Config(d_hidden=192, num_heads=3, **kw)
    p = O.Params.from_module_state({k: v.cpu() for k, v in m.state_dict().items()}, "depthwise")
    ref = O.forward(x.cpu().double(), p.to(dtype=torch.float64), cfg, cand=cand, mode="exact")
    torch.testing.assert_close(out.cpu().double(), ref, rtol=1e-3, atol=1e-4)
    assert m.batch_size == 8


def test_module_errors_match_reference():
    m = MultiHeadConvNNAttention(12, 3, 0.0, 4, "bogus", -1, 0, "matmul", seq_length=16).to(DEV)
    with pytest.raises(ValueError):
        m(torch.randn(2, 16, 12, device=DEV))
    m = MultiHeadConvNNAttention(12, 3, 0.0, 4, "all", -1, 0, "matmul", seq_length=15).to(DEV)
    with pytest.raises(RuntimeError):
        m(torch.randn(2, 16, 12, device=DEV))
    m = MultiHeadConvNNAttention(12, 3, 0.0, 17, "all", -1, 0, "matmul", seq_length=16).to(DEV)
    with pytest.raises(RuntimeError):
        m(torch.randn(2, 16, 12, device=DEV))


# --------------------------------------------------------------------------- K wider than one list

WIDE_K_CASES = [
    # (name, cfg kwargs, B, N, dtype): K > 32 runs the select kernel in rounds of 32
    ("k33_f32", dict(d_hidden=64, num_heads=2, K=33, seq_length=120), 2, 120, torch.float32),
    ("k64_bf16_N1024", dict(d_hidden=384, num_heads=3, K=64, seq_length=1024), 1, 1024, torch.bfloat16),
    ("k100_bf16_vit", dict(d_hidden=192, num_heads=3, K=100, seq_length=197), 2, 197, torch.bfloat16),
    ("k197_eq_n_f32", dict(d_hidden=192, num_heads=3, K=197, seq_length=197), 1, 197, torch.float32),
    ("k70_random_euclid_f32", dict(d_hidden=64, num_heads=2, K=70, sampling_type="random", num_samples=90, magnitude_type="euclidean", seq_length=150), 2, 150, torch.float32),
    ("k41_spatial_cosine_f32", dict(d_hidden=96, num_heads=2, K=41, sampling_type="spatial", num_samples=60, magnitude_type="cosine", seq_length=100), 2, 100, torch.float32),
    # d_k = 48: no exact-width instance, the guarded-chunk kernel in rounds
    ("k45_dk48_bf16", dict(d_hidden=96, num_heads=2, K=45, seq_length=300), 2, 300, torch.bfloat16),
]


@pytest.mark.parametrize("name,kw,B,N,dtype", WIDE_K_CASES, ids=[c[0] for c in WIDE_K_CASES])
def test_select_wide_k(name, kw, B, N, dtype):
    cfg = O.Config(**kw)
    p, x = make(cfg, B, N, dtype, seed=5)
    cand = cand_for(cfg, N)
    d, r = run_stages(cfg, p, x, cand)
    check_select(cfg, r, cand, B)
    # the weights of all K entries (written after the last round)
    v = r["vals"].double()
    if cfg.softmax_topk_val:
        exp_w = torch.softmax(-v if cfg.magnitude_type == "euclidean" else v, dim=-1)
    else:
        exp_w = 1.0 / (v + 1e-8) if cfg.magnitude_type == "euclidean" else v
    torch.testing.assert_close(r["w"].double(), exp_w, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("K", [33, 50, 64, 70])
def test_select_wide_k_ties_continue_in_index_order(K):
    """Every key ties except one: the rounds must hand the tie over at the
    32-entry boundary and continue with the next lowest index."""
    cfg = O.Config(d_hidden=16, num_heads=1, K=K, seq_length=100)
    B, N = 1, 100
    d = desc_for(cfg, B, N, N, torch.float32)
    k = torch.zeros(1, N, 16)
    k[..., 0] = 1.0
    q = torch.zeros(1, N, 16)
    q[..., 0] = 0.5
    q[0, 40, 0] = 0.75
    idx, vals, w = ops.select(d, k.to(DEV), q.to(DEV))
    torch.cuda.synchronize()
    exp = [40] + [j for j in range(N) if j != 40][:K - 1]
    assert (idx.cpu()[0] == torch.tensor(exp, dtype=torch.int32)).all()
    assert torch.all(vals.cpu()[0, :, 1:] == 0.5 / 4.0)


WIDE_K_E2E = [
    ("k40_dw_f32", dict(d_hidden=96, num_heads=3, K=40, seq_length=100), 2, 100),
    ("k36_std_random_f32", dict(d_hidden=64, num_heads=2, K=36, sampling_type="random", num_samples=50, convolution_type="standard", seq_length=80), 2, 80),
]


@pytest.mark.parametrize("name,kw,B,N", WIDE_K_E2E, ids=[c[0] for c in WIDE_K_E2E])
def test_forward_wide_k_end_to_end(name, kw, B, N):
    test_forward_fp32_end_to_end(name, kw, B, N)
