"""Benchmark: ConvNN-Attention layer throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]

One step = one forward of ``MultiHeadConvNNAttention`` (eval mode) over one
batch of synthetic input already resident in HBM.  The default workload is
B=32, N=1024, C=384, H=3, K=9, bf16, matmul similarity,
depthwise conv, sampling 'all'.  ``--config c5`` times a training step
instead: forward + backward (loss gradient dout fixed, all parameter and
input gradients) at B=8, N=4096, C=768, H=3, K=16, standard conv.

Prints one JSON line with tokens/s, the roofline of the dominant forward
kernel (timed with HIP events on the launch stream) and the CPU baseline (the
oracle's restatement of the reference op sequence on a bounded sample, timed
on this host's cores).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "convolutional-nearest-neighbor-attention_amd")
sys.path.insert(0, ROOT)
sys.path.insert(0, PKG)

PEAK_BF16_TFLOPS = 2500.0
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # name: (B, N, C, H, K, dtype, metric, conv, sampling, num_samples, seed)
    "c3": (32, 1024, 384, 3, 9, torch.bfloat16, "matmul", "depthwise", "all", -1, 1),
    "c2layer": (128, 197, 192, 3, 9, torch.bfloat16, "matmul", "depthwise", "all", -1, 0),
    "c1": (64, 65, 192, 3, 9, torch.float32, "cosine", "depthwise", "all", -1, 0),
    "c4a": (128, 197, 192, 3, 9, torch.float32, "matmul", "depthwise", "random", 64, 2),
    "c4b": (128, 197, 192, 3, 9, torch.float32, "matmul", "depthwise", "spatial", 8, 2),
    "c5": (8, 4096, 768, 3, 16, torch.bfloat16, "matmul", "standard", "all", -1, 3),
    # c2: the whole ViT-Tiny (12 blocks, N = 197) in run_vit; the layer shape is c2layer
    "c2": (128, 197, 192, 3, 9, torch.bfloat16, "matmul", "depthwise", "all", -1, 0),
    # callers at the ViT-Tiny block shape (run_callers): KVT top-k attention
    # (topk = K) and the branching Conv1d layer (ConvNN on half the channels)
    "kvt": (128, 197, 192, 3, 9, torch.bfloat16, "matmul", "depthwise", "all", -1, 0),
    "branch": (128, 197, 192, 3, 9, torch.bfloat16, "matmul", "depthwise", "all", -1, 0),
}
CALLERS = {"kvt", "branch"}
TRAIN = {"c5"}


STAGE_KERNELS = {  # bench stage -> substring of the HIP kernel name
    "select": "select_kernel",
    "aggregate": "agg_kernel",
    "project": "gemm_dl_kernel<unsigned short, 1",
    "output_proj": "gemm_dl_kernel<unsigned short, 0",
}


def summarize_pmc(config, fetch_dir, write_dir):
    """Turn two ``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE`` runs of this
    script into HBM bytes per launch (profiles/traffic.json).  Each counter is
    scaled by what it reads for the calibration copy of COPY_BYTES (the largest
    copy kernel of the run)."""
    import csv
    import glob

    def load(d, counter):
        per = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                per.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]) * 1024.0)
        return per

    out = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        per = load(d, counter)
        copies = [max(v) for k, v in per.items() if "copy" in k.lower()]
        if not copies:
            raise SystemExit(f"no copy kernel in the {counter} run")
        factor = max(copies) / COPY_BYTES
        for stage, pat in STAGE_KERNELS.items():
            vals = [x for k, v in per.items() if pat in k for x in v]
            if not vals:
                continue
            e = out.setdefault(stage, {"kernel": pat})
            e[counter.lower() + "_bytes"] = sorted(vals)[len(vals) // 2] / factor
            e[counter.lower() + "_factor"] = round(factor, 4)
    for e in out.values():
        e["bytes_per_launch"] = round(e.get("fetch_size_bytes", 0.0) + e.get("write_size_bytes", 0.0))
    try:
        with open(TRAFFIC_FILE) as f:
            allt = json.load(f)
    except (OSError, ValueError):
        allt = {}
    allt[config] = out
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(allt, f, indent=1, sort_keys=True)
    print(json.dumps(out, indent=1))


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-also", action="store_true",
                    help="c3 only: skip the short c2 / c5 measurements carried on the line")
    ap.add_argument("--cpu-sample-batch", type=int, default=8)
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/traffic.json from two rocprofv3 --pmc runs of this script")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
COPY_BYTES = 256 << 20   # calibration copy: reads and writes exactly this many bytes


def calibration_copy(dev):
    """One plain device copy of COPY_BYTES, run before the timed region so a
    ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` pass over this script sees a
    kernel of known traffic next to the operator's kernels (the scale factor
    for the counters)."""
    src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def measured_traffic(config, kernel):
    """HBM bytes per launch of the dominant kernel from the committed counter
    summary (profiles/traffic.json), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t[config][kernel]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def flops_of(B, N, Nq, C, H, K, conv):
    dk = C // H
    proj = 2 * B * C * C * (3 * N + Nq)
    sim = 2 * B * N * Nq * C
    cv = {"depthwise": 2 * B * N * C * K, "standard": 2 * B * N * C * dk * K,
          "depthwise-separable": 2 * B * N * C * (K + dk)}[conv]
    return proj, sim, cv


def vit_cpu_baseline(model, imgs, args):
    """The ViT on the host cores with every attention block replaced by the
    oracle's restatement of the reference op sequence (bounded sample)."""
    import copy

    from oracle import cnna_oracle as O

    class OracleAttention(torch.nn.Module):
        def __init__(self, attn, cfg):
            super().__init__()
            self.p = O.Params.from_module_state({k: v.detach() for k, v in attn.state_dict().items()},
                                                cfg.convolution_type)
            self.cfg = cfg

        def forward(self, x):
            return O.forward(x, self.p, self.cfg, mode="reference")

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    cpu = copy.deepcopy(model).cpu()
    a = cpu.args
    cfg = O.Config(d_hidden=a.d_hidden, num_heads=a.num_heads, K=a.K, sampling_type=a.sampling_type,
                   num_samples=a.num_samples, magnitude_type=a.magnitude_type, seq_length=197,
                   convolution_type=a.convolution_type, softmax_topk_val=a.softmax_topk_val)
    for blk in cpu.transformer_encoder:
        blk.attention = OracleAttention(blk.attention, cfg)
    bs = max(1, min(args.cpu_sample_batch, imgs.shape[0]))
    x = imgs[:bs].cpu()
    with torch.no_grad():
        cpu(x)
        reps, t = 0, 0.0
        while reps < 3 or (t < 10.0 and reps < 20):
            c0 = time.perf_counter()
            cpu(x)
            t += time.perf_counter() - c0
            reps += 1
    n_tok = bs * 197 * reps
    return {"value": round(n_tok / t, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{reps} ViT forwards of {bs} of {imgs.shape[0]} images in bf16, "
                                      "attention = oracle reference-mode op sequence",
            "affinity_cores": ncores, "os_cpu_count": os.cpu_count(), "torch": torch.__version__}


def run_vit(args):
    """c2: full ViT-Tiny forward (12 ConvNN-Attention blocks, B=128, 224x224, bf16)."""
    import cnna_ops as ops
    from vit import ViT, vit_tiny_args

    torch.manual_seed(0)
    model = ViT(vit_tiny_args()).to("cuda").to(torch.bfloat16).eval()
    B = 128
    imgs = torch.randn(B, 3, 224, 224, device="cuda").to(torch.bfloat16)
    calibration_copy("cuda")
    with torch.no_grad():
        for _ in range(args.warmup):
            model(imgs)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            model(imgs)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    tokens = B * 197
    # dominant operator stage at the block shape, timed with HIP events
    blk = model.transformer_encoder[0].attention
    x = torch.randn(B, 197, 192, device="cuda").to(torch.bfloat16)
    d = ops.make_desc(B, 197, 192, 3, 197, 9, 197, torch.bfloat16, "matmul", "depthwise",
                      blk.softmax_topk_val, False, False)
    ts = []
    with torch.no_grad():
        q, k, v, qn, kn = ops.project_qkv(d, x, None, blk.W_q.weight, blk.W_k.weight, blk.W_v.weight)
        # back to back, one synchronisation at the end: the host runs ahead of the
        # GPU, so each event pair brackets the kernel alone (a synchronisation per
        # launch would add the host's launch latency to every interval)
        evs = []
        for it in range(args.warmup + args.steps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            ops.select(d, k, q, kn, qn, None)
            e1.record()
            if it >= args.warmup:
                evs.append((e0, e1))
        torch.cuda.synchronize()
        ts = [e0.elapsed_time(e1) for e0, e1 in evs]
    t_sel = sorted(ts)[len(ts) // 2] / 1e3
    f_sim = 2 * B * 197 * 197 * 192
    achieved = f_sim / t_sel / 1e12
    # ViT-Tiny forward flops: patch embedding + 12 x (layer + MLP) + classifier
    f_layer = 2 * B * 192 * 192 * 4 * 197 + f_sim + 2 * B * 197 * 192 * 9
    f_mlp = 2 * 2 * B * 197 * 192 * 768
    f_total = 2 * B * 196 * 192 * 768 + 12 * (f_layer + f_mlp) + 2 * B * 192 * 10
    cpu = None if args.no_cpu else vit_cpu_baseline(model, imgs, args)
    rec = {
        "metric": "ConvNN-ViT-Tiny forward tokens/s (12 blocks, N=197, C=192, K=9, bf16)",
        "value": round(tokens / (ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: images ~ N(0,1), random-init weights (seed 0)",
        "config": {"workload": "c2: ViT-Tiny forward, 12 ConvNN-Attention blocks (matmul, depthwise, "
                               "K=9, sampling all, softmax_topk_val=True as main.py:48-49 forces), "
                               "B=128 images 224x224, patch 16",
                   "B": B, "N": 197, "C": 192, "H": 3, "K": 9, "layers": 12},
        "roofline": {"kernel": "select", "bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic("c2", "select")},
        "model": {"flops": f_total, "tflops": round(f_total / (ms / 1e3) / 1e12, 2)},
        "cpu_baseline": cpu,
    }
    return rec


def kvt_dense(x, Wqkv, Wproj, H, topk, scale):
    """The reference's dense KVT forward (layers.py:668-686) as plain torch ops
    on the GPU: full (B, H, N, N) scores, torch.topk, a dense 0/1 mask filled by
    scatter_, -inf fill, softmax over N, dense probabilities @ v.  Operands of
    the batched products are made contiguous first."""
    B, N, C = x.shape
    qkv = torch.nn.functional.linear(x, Wqkv).reshape(B, N, 3, H, C // H).permute(2, 0, 3, 1, 4)
    q, k, v = qkv[0].contiguous(), qkv[1].transpose(-2, -1).contiguous(), qkv[2].contiguous()
    attn = torch.matmul(q, k) * scale
    mask = torch.zeros(B, H, N, N, device=x.device)
    index = torch.topk(attn, k=topk, dim=-1, largest=True)[1]
    mask.scatter_(-1, index, 1.0)
    attn = torch.where(mask > 0, attn, torch.full_like(attn, float("-inf"))).softmax(dim=-1)
    o = torch.matmul(attn, v).transpose(1, 2).reshape(B, N, C)
    return torch.nn.functional.linear(o, Wproj)


def run_callers(args):
    """kvt / branch: one forward of the caller layer at the ViT-Tiny block
    shape (B=128, N=197, C=192, H=3, K = topk = 9, bf16), inference path."""
    import cnna_ops as ops
    from layers import MultiHeadBranchingConv, MultiHeadKvtAttention

    B, N, C, H, K, dtype, metric, conv, sampling, ns, seed = CONFIGS[args.config]
    torch.manual_seed(seed)
    if args.config == "kvt":
        m = MultiHeadKvtAttention(C, num_heads=H, attn_drop=0.0, topk=K)
        C1 = C
    else:
        m = MultiHeadBranchingConv(C, H, 0.0, kernel_size=9, K=K, sampling_type="all", num_samples=-1,
                                   sample_padding=0, magnitude_type=metric, seq_length=N,
                                   convolution_type=conv, softmax_topk_val=True, branch_ratio=0.5)
        C1 = m.d_hidden_convnn
    m = m.to("cuda").to(dtype).eval()
    x = torch.randn(B, N, C, device="cuda").to(dtype)
    calibration_copy("cuda")

    def timed(fn):
        with torch.no_grad():
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / args.steps

    ms = timed(lambda: m(x))
    ref_ms = None
    if args.config == "kvt":
        ref_ms = timed(lambda: kvt_dense(x, m.qkv.weight, m.proj.weight, H, K, m.scale))
    # dominant stage: the select kernel at the operator's shape, HIP events on the launch stream
    dk = C1 // H
    if args.config == "kvt":
        d = ops.make_desc(B, N, C, H, N, K, N, dtype, "matmul", "depthwise", True, False, False,
                          merge=ops.MERGE_CONCAT, scale=m.scale)
        W = m.qkv.weight
        Wq, Wk, Wv = W[C:2 * C], W[:C], W[2 * C:]
    else:
        d = ops.make_desc(B, N, C1, H, N, K, N, dtype, metric, conv, True, False, False)
        cv = m.convnn
        Wq, Wk, Wv = cv.W_q.weight, cv.W_k.weight, cv.W_v.weight
    ts = []
    with torch.no_grad():
        q, k, v, qn, kn = ops.project_qkv(d, x[:, :, :C1], None, Wq, Wk, Wv)
        # back to back, one synchronisation at the end: the host runs ahead of the
        # GPU, so each event pair brackets the kernel alone (a synchronisation per
        # launch would add the host's launch latency to every interval)
        evs = []
        for it in range(args.warmup + args.steps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            ops.select(d, k, q, kn, qn, None)
            e1.record()
            if it >= args.warmup:
                evs.append((e0, e1))
        torch.cuda.synchronize()
        ts = [e0.elapsed_time(e1) for e0, e1 in evs]
    t_sel = sorted(ts)[len(ts) // 2] / 1e3
    f_sim = 2 * B * N * N * C1
    achieved = f_sim / t_sel / 1e12
    cpu = None
    if not args.no_cpu:
        from oracle import cnna_oracle as O
        ncores = len(os.sched_getaffinity(0))
        torch.set_num_threads(ncores)
        bs = max(1, min(args.cpu_sample_batch, B))
        xc = x[:bs].float().cpu()
        if args.config == "kvt":
            Wc, Pc = m.qkv.weight.float().cpu(), m.proj.weight.float().cpu()
            fn = lambda: O.kvt(xc, Wc, Pc, H, K, m.scale)
        else:
            mc = __import__("copy").deepcopy(m).float().cpu()
            cv = mc.convnn
            cfg = O.Config(d_hidden=C1, num_heads=H, K=K, magnitude_type=metric, seq_length=N,
                           convolution_type=conv, softmax_topk_val=True)
            p = O.Params(cv.W_q.weight, cv.W_k.weight, cv.W_v.weight, cv.W_o.weight, cv.conv.weight)
            c1 = mc.conv1d
            fn = lambda: O.branching_conv(
                xc, lambda t: O.forward(t, p, cfg),
                lambda t: O.conv1d_branch(t, c1.W_x.weight, c1.W_x.bias, c1.conv.weight, c1.conv.bias,
                                          c1.W_o.weight, c1.W_o.bias, H),
                mc.pointwise_linear.weight, mc.pointwise_linear.bias, C1)
        with torch.no_grad():
            fn()
            reps, t_cpu = 0, 0.0
            while reps < 3 or (t_cpu < 10.0 and reps < 20):
                c0 = time.perf_counter()
                fn()
                t_cpu += time.perf_counter() - c0
                reps += 1
        cpu = {"value": round(bs * N * reps / t_cpu, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
               "kind": "port", "sample": f"{reps} forwards of {bs} of {B} sequences (N={N}) in f32, "
                                         "oracle restatement", "affinity_cores": ncores}
    name = {"kvt": "KVT top-k attention forward tokens/s (N=197, C=192, H=3, topk=9, bf16)",
            "branch": "BranchConv layer forward tokens/s (N=197, C=192, ratio 0.5, K=9, ks=9, bf16)"}
    rec = {
        "metric": name[args.config], "value": round(B * N / (ms / 1e3), 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: x ~ N(0,1), random-init weights (seeded)",
        "config": {"workload": f"{args.config}: caller layer forward at the ViT-Tiny block shape",
                   "B": B, "N": N, "C": C, "H": H, "K": K},
        "roofline": {"kernel": "select", "bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": None},
        "reference_gpu_ms": None if ref_ms is None else round(ref_ms, 4),
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


def summary(rec):
    """The figures of a secondary workload carried on the primary JSON line."""
    out = {k: rec[k] for k in ("metric", "value", "unit", "ms_per_step", "steps", "warmup") if k in rec}
    out["roofline"] = {k: rec["roofline"][k] for k in ("kernel", "bound", "achieved", "unit", "frac")}
    for k in ("stages_ms", "gather_stage", "stage_roofline"):
        if rec.get(k) is not None:
            out[k] = rec[k]
    return out


def main():
    args = parse()
    if args.summarize_pmc:
        summarize_pmc(args.config, *args.summarize_pmc)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU figures are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.config == "c2":
        print(json.dumps(run_vit(args)), flush=True)
        return
    if args.config in CALLERS:
        run_callers(args)
        return
    rec = run_layer(args)
    if args.config == "c3" and not args.no_also:
        # the other GPU workloads, timed in the same run with short step counts
        # (their own bench lines: --config c2 / --config c5)
        import copy
        also = {}
        a2 = copy.copy(args)
        a2.steps, a2.warmup, a2.no_cpu, a2.config = 10, 3, True, "c2"
        also["c2"] = summary(run_vit(a2))
        a5 = copy.copy(args)
        a5.steps, a5.warmup, a5.no_cpu, a5.config = 5, 2, True, "c5"
        also["c5"] = summary(run_layer(a5))
        rec["also"] = also
    print(json.dumps(rec), flush=True)


def run_layer(args):
    """One MultiHeadConvNNAttention config (forward, or a training step for c5)."""
    import cnna_ops as ops
    from layers import MultiHeadConvNNAttention

    B, N, C, H, K, dtype, metric, conv, sampling, ns, seed = CONFIGS[args.config]
    train = args.config in TRAIN
    dev = "cuda"
    torch.manual_seed(seed)
    m = MultiHeadConvNNAttention(C, H, 0.0, K, sampling, ns, 0, metric, seq_length=N,
                                 convolution_type=conv).to(dev).to(dtype)
    m.train(train)
    x = torch.randn(B, N, C, device=dev).to(dtype)
    Nq = N if sampling == "all" else ns
    calibration_copy(dev)

    # ---- whole-layer timing
    if train:
        xg = x.clone().requires_grad_(True)
        dout = torch.randn(B, N, C, device=dev).to(dtype)

        def step():
            m.zero_grad(set_to_none=True)
            xg.grad = None
            m(xg).backward(dout)
    else:
        def step():
            with torch.no_grad():
                m(x)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    tokens = B * N
    value = tokens / (ms / 1e3)

    # ---- per-stage timing with HIP events on the launch stream
    cand = m._candidates(x)
    d = ops.make_desc(B, N, C, H, Nq, K, N, dtype, metric, conv, True, cand is not None, False)
    w0, w1 = m._conv_weights()
    Wq, Wk, Wv, Wo = m.W_q.weight, m.W_k.weight, m.W_v.weight, m.W_o.weight
    stages = {"project": [], "select": [], "aggregate": [], "output_proj": []}
    with torch.no_grad():
        # back to back, one synchronisation at the end (see run_vit)
        evl = []
        for it in range(args.warmup + args.steps):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
            ev[0].record()
            q, k, v, qn, kn = ops.project_qkv(d, x, cand, Wq, Wk, Wv)
            ev[1].record()
            idx, vals, w = ops.select(d, k, q, kn, qn, cand)
            ev[2].record()
            z = ops.aggregate(d, v, idx, w, w0, w1)
            ev[3].record()
            ops.output_proj(d, z, Wo)
            ev[4].record()
            if it >= args.warmup:
                evl.append(ev)
        torch.cuda.synchronize()
        for ev in evl:
            for i, name in enumerate(stages):
                stages[name].append(ev[i].elapsed_time(ev[i + 1]))
    st_ms = {k_: sorted(v_)[len(v_) // 2] for k_, v_ in stages.items()}

    proj_f, sim_f, conv_f = flops_of(B, N, Nq, C, H, K, conv)
    es = 2 if dtype == torch.bfloat16 else 4
    peak_mfma = PEAK_BF16_TFLOPS if dtype == torch.bfloat16 else PEAK_F32_TFLOPS
    # algorithmic work per launch of each stage
    work = {
        "project": ("mfma", 2 * B * C * C * (2 * N + Nq)),
        "select": ("mfma", sim_f),
        # depthwise: read V, write y, read int32 index + fp32 value per neighbour
        # (HBM-bound); standard / depthwise-separable: the conv GEMM (MFMA)
        "aggregate": (("hbm", 2 * B * N * C * es + B * H * N * K * 8) if conv == "depthwise"
                      else ("mfma", conv_f)),
        "output_proj": ("mfma", 2 * B * N * C * C),
    }
    dom = max(st_ms, key=st_ms.get)
    bound, amount = work[dom]
    t_s = st_ms[dom] / 1e3
    if bound == "mfma":
        achieved = amount / t_s / 1e12
        roof = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": peak_mfma,
                "unit": "TFLOP/s", "frac": round(achieved / peak_mfma, 4),
                "traffic": measured_traffic(args.config, dom)}
    else:
        achieved = amount / t_s / 1e9
        roof = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": measured_traffic(args.config, dom)}

    # every stage against its own roof (HIP-event medians above); the gather /
    # conv stage is HBM-bound: v read, z written, int32 index + fp32 weight read
    stage_roof = {}
    for name, (bnd, amt) in work.items():
        t_st = st_ms[name] / 1e3
        if bnd == "mfma":
            ach = amt / t_st / 1e12
            stage_roof[name] = {"bound": "mfma", "achieved_TFLOPs": round(ach, 1), "frac": round(ach / peak_mfma, 4)}
        else:
            ach = amt / t_st / 1e9
            stage_roof[name] = {"bound": "hbm", "achieved_GBs": round(ach, 1), "frac": round(ach / PEAK_HBM_GBS, 4)}
    gather = None
    if conv == "depthwise":
        agg_bytes = work["aggregate"][1]
        gather = {"kernel": "aggregate", "bound": "hbm", "bytes": agg_bytes, "ms": round(st_ms["aggregate"], 4),
                  "achieved_GBs": round(agg_bytes / (st_ms["aggregate"] / 1e3) / 1e9, 1), "peak_GBs": PEAK_HBM_GBS,
                  "frac": round(agg_bytes / (st_ms["aggregate"] / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
                  "traffic": measured_traffic(args.config, "aggregate"),
                  "l2_gather_bytes": B * H * N * K * (C // H) * es}
    total_flops = proj_f + sim_f + conv_f
    if train:
        # backward: twice the projection and conv GEMM work plus the sparse
        # similarity / softmax / gather terms over the K selected entries
        total_flops += 2 * (proj_f + conv_f) + 8 * B * N * K * C
    layer_tflops = total_flops / (ms / 1e3) / 1e12

    # ---- CPU baseline: the oracle's reference-mode op sequence on a bounded sample
    cpu = None
    if not args.no_cpu:
        from oracle import cnna_oracle as O
        ncores = len(os.sched_getaffinity(0))
        torch.set_num_threads(ncores)
        bs = 1 if train else max(1, min(args.cpu_sample_batch, B))
        cfg = O.Config(d_hidden=C, num_heads=H, K=K, sampling_type=sampling, num_samples=ns,
                       magnitude_type=metric, seq_length=N, convolution_type=conv)
        p = O.Params.from_module_state({k_: v_.detach().cpu() for k_, v_ in m.state_dict().items()}, conv)
        xc = x[:bs].cpu()
        cdt = dtype
        try:
            O.forward(xc[:1], p, cfg, cand=None if cand is None else cand.cpu().long(), mode="reference")
        except RuntimeError:
            cdt = torch.float32
        xc, p = xc.to(cdt), p.to(dtype=cdt)
        cc = None if cand is None else cand.cpu().long()

        def cpu_step():
            if not train:
                with torch.no_grad():
                    O.forward(xc, p, cfg, cand=cc, mode="reference")
                return
            ts = [t.clone().requires_grad_(True) for t in (xc, p.W_q, p.W_k, p.W_v, p.W_o, p.conv0)]
            out = O.forward(ts[0], O.Params(*ts[1:], p.conv1), cfg, cand=cc, mode="reference")
            out.backward(torch.ones_like(out))

        cpu_step()                                                 # warm-up
        reps, t_cpu = 0, 0.0
        while reps < 3 or (t_cpu < 10.0 and reps < 20):
            c0 = time.perf_counter()
            cpu_step()
            t_cpu += time.perf_counter() - c0
            reps += 1
        cpu = {"value": round(bs * N * reps / t_cpu, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{reps} {'training steps' if train else 'forwards'} of {bs} of {B} sequences (N={N}) in "
                         f"{str(cdt).replace('torch.', '')}, oracle reference-mode op sequence",
               "affinity_cores": ncores, "os_cpu_count": os.cpu_count(), "torch": torch.__version__}

    metric_name = "ConvNN-Attn layer tokens/s (N=1024,C=384,K=9,bf16); % MFMA/HBM roofline"
    if train:
        metric_name = "ConvNN-Attn training-step tokens/s (N=4096,C=768,K=16,standard conv,bf16)"
    rec = {
        "metric": metric_name,
        "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16" if dtype == torch.bfloat16 else "f32",
        "data": "synthetic: x ~ N(0,1), random-init weights (seeded)",
        "config": {"workload": f"{args.config}: MultiHeadConvNNAttention "
                               f"{'forward+backward' if train else 'forward'} B={B} N={N} C={C} "
                               f"H={H} K={K} {metric} {conv} sampling={sampling}",
                   "B": B, "N": N, "C": C, "H": H, "K": K, "sampling": sampling},
        "roofline": roof,
        "gather_stage": gather,
        "stage_roofline": stage_roof,
        "layer": {"flops": total_flops, "tflops": round(layer_tflops, 2),
                  "frac_of_mfma_peak": round(layer_tflops / peak_mfma, 4)},
        "stages_ms": {k_: round(v_, 4) for k_, v_ in st_ms.items()},
        "cpu_baseline": cpu,
    }
    return rec


if __name__ == "__main__":
    main()
