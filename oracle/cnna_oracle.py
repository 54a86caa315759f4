"""CPU oracle for the ConvNN-Attention operator (test infrastructure only).

This module restates, on the CPU and in plain PyTorch, the arithmetic of
``MultiHeadConvNNAttention`` from the reference repository
(``layers.py:132-450``).  It is the *checker* for the HIP path and the CPU
baseline that ``bench.py`` times; it is never on the product path.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import it.

Two evaluation modes
--------------------
``mode="reference"``
    follows the reference op sequence in the input dtype (rounding after every
    op the way eager PyTorch does).  Used against the golden fixtures written
    by ``tests/golden/make_golden.py`` and as the CPU baseline.
``mode="exact"``
    the projections are rounded to the input dtype exactly like the reference
    (``nn.Linear`` output), then similarity, top-k, softmax, gather and the
    convolution run in float64, and the head-merged tensor is rounded to the
    input dtype before ``W_o``.  This is the well-defined target of the HIP
    kernels, which keep fp32 accumulators where the reference rounds to bf16
    (the reference ranks bf16 rows on a twice-rounded similarity, so its bf16
    top-k is ill-defined at near ties).

Top-k ties are broken by the lowest candidate index (``stable_topk``), which
``torch.topk`` does not guarantee.

Pinning (what checks this restatement, see ``tests/test_oracle.py``):
  * golden vectors produced by the reference itself at tiny shapes
    (sampled paths, head merge, coordinate encoding, euclidean division,
    all three conv types) -> ``tests/golden/*.npz``;
  * closed forms: head merge == index formula; H=1 merge == transpose;
    euclidean similarity == ``torch.cdist``; cosine within [-1, 1];
    K == Nq with unit depthwise weight == softmax attention
    (``scaled_dot_product_attention``); standard conv == einsum;
  * brute-force python sort for ``stable_topk``;
  * fp64 ``gradcheck`` of the differentiable restatement.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as F

# Constants of the reference (layers.py:234-235).
INF_MASK = 1.1
NEG_INF_MASK = -0.1


@dataclass
class Config:
    """Constructor arguments of the reference module (layers.py:133-146)."""

    d_hidden: int
    num_heads: int
    K: int
    sampling_type: str = "all"
    num_samples: int = -1
    sample_padding: int = 0
    magnitude_type: str = "matmul"
    seq_length: int = 197
    coordinate_encoding: bool = False
    convolution_type: str = "depthwise"
    softmax_topk_val: bool = True
    attention_dropout: float = 0.0

    @property
    def d_k(self) -> int:
        return self.d_hidden // self.num_heads

    @property
    def maximum(self) -> bool:
        # layers.py:168
        return self.magnitude_type in ("cosine", "matmul")

    @property
    def in_channels(self) -> int:
        # layers.py:181
        return self.d_k + 1 if self.coordinate_encoding else self.d_k

    @property
    def padding(self) -> int:
        # layers.py:164: padding only applies to spatial sampling
        return int(self.sample_padding) if self.sampling_type == "spatial" else 0


@dataclass
class Params:
    """Parameters with the reference's names and shapes (layers.py:175-228)."""

    W_q: torch.Tensor
    W_k: torch.Tensor
    W_v: torch.Tensor
    W_o: torch.Tensor
    conv0: torch.Tensor                    # standard / depthwise weight, or dw part of dw-separable
    conv1: Optional[torch.Tensor] = None   # pointwise weight of depthwise-separable

    @staticmethod
    def from_module_state(sd: dict, convolution_type: str) -> "Params":
        if convolution_type == "depthwise-separable":
            return Params(sd["W_q.weight"], sd["W_k.weight"], sd["W_v.weight"], sd["W_o.weight"],
                          sd["conv.0.weight"], sd["conv.1.weight"])
        return Params(sd["W_q.weight"], sd["W_k.weight"], sd["W_v.weight"], sd["W_o.weight"],
                      sd["conv.weight"])

    def to(self, **kw) -> "Params":
        return Params(*[None if t is None else t.to(**kw) for t in
                        (self.W_q, self.W_k, self.W_v, self.W_o, self.conv0, self.conv1)])


def init_params(cfg: Config, seed: int = 0, dtype=torch.float32) -> Params:
    """Default PyTorch init of the reference layer (nn.Linear / nn.Conv1d
    kaiming-uniform; depthwise weight filled with 1.0, layers.py:206).

    Draw order follows module construction order (layers.py:175-228):
    W_q, W_k, W_v, W_o, conv.
    """
    g = torch.Generator().manual_seed(seed)
    C, dk, cin = cfg.d_hidden, cfg.d_k, cfg.in_channels

    def kaiming(shape, fan_in):
        bound = 1.0 / math.sqrt(fan_in)
        return (torch.rand(shape, generator=g, dtype=torch.float32) * 2 - 1) * bound

    Wq = kaiming((C, C), C)
    Wk = kaiming((C, C), C)
    Wv = kaiming((C, C), C)
    Wo = kaiming((C, C), C)
    conv1 = None
    if cfg.convolution_type == "standard":
        conv0 = kaiming((dk, cin, cfg.K), cin * cfg.K)
    elif cfg.convolution_type == "depthwise":
        if dk % cin != 0:
            raise ValueError("out_channels must be divisible by groups")
        conv0 = torch.ones((dk, 1, cfg.K))
    elif cfg.convolution_type == "depthwise-separable":
        conv0 = kaiming((cin, 1, cfg.K), cfg.K)
        conv1 = kaiming((dk, cin, 1), cin)
    else:
        raise ValueError(f"unknown convolution_type {cfg.convolution_type}")
    return Params(Wq, Wk, Wv, Wo, conv0, conv1).to(dtype=dtype)


# --------------------------------------------------------------------------
# index helpers
# --------------------------------------------------------------------------

def sample_indices(cfg: Config, N: int, generator=None, device="cpu") -> Optional[torch.Tensor]:
    """Candidate indices of the sampled paths.

    random:  ``torch.randperm(N)[:num_samples]`` (layers.py:284); one draw per
             forward, shared by the whole batch.
    spatial: ``linspace(pad, N - pad - 1, num_samples).long()`` over token
             indices (layers.py:297) -- 1-D, CLS included.
    """
    if cfg.sampling_type == "all":
        return None
    if cfg.sampling_type == "random":
        perm = torch.randperm(N, device=device, generator=generator)
        return perm[: cfg.num_samples]
    if cfg.sampling_type == "spatial":
        p = cfg.padding
        return torch.linspace(0 + p, N - p - 1, cfg.num_samples, device=device).long()
    raise ValueError("Invalid sampling_type. Must be one of ['all', 'random', 'spatial']")


def stable_topk(S: torch.Tensor, k: int, largest: bool):
    """Top-k along the last dim, sorted, ties broken by the lowest index.

    NaN ranks last in both directions (``torch.topk(largest=False)`` never
    prefers a NaN; the reference's euclidean ``sqrt`` can produce one,
    layers.py:333).
    """
    key = S.to(torch.float64)
    nan = torch.isnan(key)
    if largest:
        key = torch.where(nan, torch.full_like(key, -math.inf), key)
        order = torch.sort(-key, dim=-1, stable=True).indices
    else:
        key = torch.where(nan, torch.full_like(key, math.inf), key)
        order = torch.sort(key, dim=-1, stable=True).indices
    idx = order[..., :k]
    return torch.gather(S, -1, idx), idx


def split_heads(t: torch.Tensor, H: int) -> torch.Tensor:
    """(B, N, C) -> (B*H, d_k, N), channel-major per head.

    Restates ``split_head`` + ``batch_combine`` (layers.py:237-245):
    ``out[b*H + h, c, n] = t[b, n, h*d_k + c]``.
    """
    B, N, C = t.shape
    dk = C // H
    return t.reshape(B, N, H, dk).permute(0, 2, 3, 1).reshape(B * H, dk, N)


def head_merge(y: torch.Tensor, B: int, H: int, seq_length: int) -> torch.Tensor:
    """Conv output (B*H, d_k, N) -> (B, N, C), the reference's own reshapes.

    Restates ``permute`` + ``batch_split`` + ``combine_heads``
    (layers.py:317, 247-259).  When H > 1 this *mixes tokens*:
    ``out[b, n, h*d_k + a] = y[b*H + h, f % d_k, f // d_k]`` with
    ``f = a*N + n`` (closed form checked in tests).  H == 1 is a transpose.
    Raises RuntimeError when ``seq_length != N`` and H > 1, like the
    reference's reshape/view.
    """
    BH, dk, N = y.shape
    x = y.permute(0, 2, 1)                                  # (BH, N, d_k) view
    if H == 1:
        x = x.unsqueeze(1)                                   # layers.py:248-249
        return x.squeeze(1)                                  # layers.py:255-256
    x = x.reshape(B, -1, dk, seq_length).permute(0, 1, 3, 2).contiguous()   # layers.py:251-252
    b, _, sl, d = x.size()
    return x.transpose(1, 2).contiguous().view(b, sl, H * dk)               # layers.py:259


def head_merge_closed_form(y: torch.Tensor, B: int, H: int) -> torch.Tensor:
    """Independent index-arithmetic statement of ``head_merge`` (H > 1)."""
    BH, dk, N = y.shape
    out = torch.empty(B, N, H * dk, dtype=y.dtype)
    n = torch.arange(N).view(N, 1)
    a = torch.arange(dk).view(1, dk)
    f = a * N + n
    for b in range(B):
        for h in range(H):
            out[b, :, h * dk:(h + 1) * dk] = y[b * H + h][f % dk, f // dk]
    return out


def coordinate_channel(t: torch.Tensor) -> torch.Tensor:
    """Append ``linspace(-1, 1, t)`` as an extra channel (layers.py:439-450)."""
    b, c, n = t.shape
    # linspace in the default dtype (float32), then promoted by cat, exactly as
    # the reference does (its float64 models see float32-rounded coordinates)
    coords = torch.linspace(-1, 1, n).view(1, 1, n).expand(b, 1, n)
    return torch.cat([t, coords.to(t.dtype)], dim=1)


# --------------------------------------------------------------------------
# similarity (layers.py:323-340)
# --------------------------------------------------------------------------

def similarity(k: torch.Tensor, q: torch.Tensor, cfg: Config) -> torch.Tensor:
    """S[bh, i, j] between key i (rows) and candidate query j (columns).

    k: (BH, c, N), q: (BH, c, Nq) in the reference's channel-major layout.
    """
    if cfg.magnitude_type == "matmul":
        # layers.py:323-325
        return torch.matmul(k.transpose(1, 2), q) / cfg.d_k ** 0.5
    if cfg.magnitude_type == "cosine":
        # layers.py:336-340: F.normalize(p=2, dim=1, eps=1e-12)
        kn = k / k.norm(p=2, dim=1, keepdim=True).clamp_min(1e-12)
        qn = q / q.norm(p=2, dim=1, keepdim=True).clamp_min(1e-12)
        return torch.matmul(kn.transpose(1, 2), qn)
    if cfg.magnitude_type == "euclidean":
        # layers.py:327-334 with sqrt=True
        ksq = torch.sum(k ** 2, dim=1, keepdim=True)
        qsq = torch.sum(q ** 2, dim=1, keepdim=True)
        dot = torch.bmm(k.transpose(1, 2), q)
        return torch.sqrt(ksq.transpose(1, 2) + qsq - 2 * dot)
    raise ValueError(f"unknown magnitude_type {cfg.magnitude_type}")


def mask_self(S: torch.Tensor, cand: torch.Tensor, cfg: Config) -> torch.Tensor:
    """Sampled paths: ``S[:, cand[j], j] = INF/NEG_INF`` (layers.py:291-292, 304-305)."""
    S = S.clone()
    val = INF_MASK if cfg.magnitude_type == "euclidean" else NEG_INF_MASK
    S[:, cand, torch.arange(cand.numel())] = val
    return S


# --------------------------------------------------------------------------
# neighbour selection and weights (layers.py:342-437)
# --------------------------------------------------------------------------

def select_neighbours(S: torch.Tensor, cfg: Config, cand: Optional[torch.Tensor],
                      cols: Optional[torch.Tensor] = None):
    """Returns (idx (BH,N,K) int64 token indices, vals (BH,N,K) logits/values).

    all:     top-K of S along candidates (layers.py:344, 391).
    sampled: top-(K-1) over Ns candidates, mapped through ``cand``, with the
             token itself prepended at rank 0 with value 1.0
             (layers.py:363-376, 410-423).  ``K - 1`` candidates must exist.
    ``cols`` (BH, N, K or K-1) replaces the top-k search by a given choice of
    candidate columns (test hook: gradients on a fixed selection).
    """
    BH, N, Nq = S.shape
    ksel = cfg.K if cand is None else cfg.K - 1
    if ksel > Nq:
        raise RuntimeError("selected index k out of range")
    if cols is not None:
        tk = cols.to(torch.int64)
        vals = torch.gather(S, -1, tk)
    else:
        vals, tk = stable_topk(S, ksel, cfg.maximum)
    if cand is None:
        return tk, vals
    mapped = cand[tk]
    self_idx = torch.arange(N).view(1, N, 1).expand(BH, N, 1)
    idx = torch.cat([self_idx, mapped], dim=-1)
    # fp32 ones: layers.py:374-375 promote bf16 values to fp32
    ones = torch.ones((BH, N, 1), dtype=torch.float32)
    vals = torch.cat([ones, vals.to(torch.promote_types(vals.dtype, torch.float32))], dim=-1)
    return idx, vals


def neighbour_weights(vals: torch.Tensor, cfg: Config, sampled: bool) -> torch.Tensor:
    """Per-neighbour multiplier applied to the gathered V rows.

    softmax_topk_val: softmax(vals) or softmax(-vals) for euclidean
                      (layers.py:394-397, 426-429).
    otherwise:        vals for cosine/matmul; 1/(vals + 1e-8) for euclidean
                      (layers.py:352-355, 382-385).
    """
    if cfg.softmax_topk_val:
        return torch.softmax(vals if cfg.maximum else -vals, dim=-1)
    if cfg.maximum:
        return vals
    return 1.0 / (vals + 1e-8)


def gather_prime(v: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, cfg: Config) -> torch.Tensor:
    """prime[bh, c, i*K + r] = w[bh,i,r] * v[bh, c, idx[bh,i,r]] (layers.py:348-358, 402-405).

    Euclidean without softmax divides by (val + 1e-8) instead of multiplying,
    which ``neighbour_weights`` turned into a reciprocal; ``reference`` mode
    below performs the division literally.
    """
    BH, c, N = v.shape
    K = idx.shape[-1]
    g = torch.gather(v.unsqueeze(-1).expand(BH, c, N, K), 2,
                     idx.unsqueeze(1).expand(BH, c, N, K))
    return (w.unsqueeze(1) * g).reshape(BH, c, N * K)


def conv(prime: torch.Tensor, p: Params, cfg: Config) -> torch.Tensor:
    """Kernel K, stride K convolution over the gathered neighbours (layers.py:187-228, 313)."""
    K = cfg.K
    if cfg.convolution_type == "standard":
        return F.conv1d(prime, p.conv0.to(prime.dtype), stride=K)
    if cfg.convolution_type == "depthwise":
        return F.conv1d(prime, p.conv0.to(prime.dtype), stride=K, groups=cfg.in_channels)
    if cfg.convolution_type == "depthwise-separable":
        t = F.conv1d(prime, p.conv0.to(prime.dtype), stride=K, groups=cfg.in_channels)
        return F.conv1d(t, p.conv1.to(prime.dtype))
    raise ValueError(cfg.convolution_type)


# --------------------------------------------------------------------------
# whole forward
# --------------------------------------------------------------------------

@dataclass
class Intermediates:
    k: torch.Tensor = None       # (BH, c, N) after projection (+coords)
    q: torch.Tensor = None       # (BH, c, Nq)
    v: torch.Tensor = None       # (BH, c, N)
    S: torch.Tensor = None       # (BH, N, Nq)
    idx: torch.Tensor = None     # (BH, N, K) token indices
    vals: torch.Tensor = None    # (BH, N, K) selected values (self = 1.0 for sampled)
    w: torch.Tensor = None       # (BH, N, K) neighbour multipliers
    y: torch.Tensor = None       # (BH, d_k, N) conv output
    z: torch.Tensor = None       # (B, N, C) head-merged, input to W_o
    cand: Optional[torch.Tensor] = None
    extra: dict = field(default_factory=dict)


def forward(x: torch.Tensor, p: Params, cfg: Config, cand: Optional[torch.Tensor] = None,
            mode: str = "reference", generator=None, return_intermediates: bool = False,
            cols: Optional[torch.Tensor] = None, y_dropout=None):
    """Restatement of ``MultiHeadConvNNAttention.forward`` (layers.py:261-321).

    ``cand`` injects the sampled candidate indices; when None they are drawn
    with ``sample_indices`` (randperm on ``generator``).  Dropout is the
    identity (eval mode) unless ``y_dropout`` is given: a function applied to
    the conv output y (B*H, d_k, N) where the reference applies
    ``self.dropout`` (layers.py:316), e.g. ``nn.Dropout`` in training mode or
    a multiplication by a given mask.  ``cols`` fixes the selected candidate
    columns (see ``select_neighbours``); the function stays differentiable in
    x and p.
    """
    if mode not in ("reference", "exact"):
        raise ValueError(mode)
    if cfg.sampling_type not in ("all", "random", "spatial"):
        raise ValueError("Invalid sampling_type. Must be one of ['all', 'random', 'spatial']")
    B, N, C = x.shape
    H = cfg.num_heads
    dt = x.dtype
    it = Intermediates()

    # 1. projections + head split (layers.py:264-265, 274, 286, 299)
    k = split_heads(F.linear(x, p.W_k.to(dt)), H)
    v = split_heads(F.linear(x, p.W_v.to(dt)), H)
    if cfg.coordinate_encoding:                                     # layers.py:269-270
        k, v = coordinate_channel(k), coordinate_channel(v)
    if cfg.sampling_type == "all":
        xs = x
        cand = None
    else:
        if cand is None:
            cand = sample_indices(cfg, N, generator=generator)
        xs = x[:, cand, :]
    q = split_heads(F.linear(xs, p.W_q.to(dt)), H)
    if cfg.coordinate_encoding:
        q = coordinate_channel(q)

    # 2. similarity (+ self mask for sampled paths)
    wk = torch.float64 if mode == "exact" else dt
    S = similarity(k.to(wk), q.to(wk), cfg)
    if cand is not None:
        S = mask_self(S, cand, cfg)

    # 3. neighbours, weights, gather, conv
    idx, vals = select_neighbours(S, cfg, cand, cols)
    vv = v.to(wk)
    if mode == "reference" and not cfg.softmax_topk_val and not cfg.maximum:
        # literal division, layers.py:352-353 / 382-383
        BHc, c, Nt = vv.shape
        Kk = idx.shape[-1]
        g = torch.gather(vv.unsqueeze(-1).expand(BHc, c, Nt, Kk), 2,
                         idx.unsqueeze(1).expand(BHc, c, Nt, Kk))
        w = vals
        prime = (g / (vals.unsqueeze(1) + 1e-8)).reshape(BHc, c, Nt * Kk)
    else:
        w = neighbour_weights(vals, cfg, cand is not None)
        prime = gather_prime(vv, idx, w.to(prime_dtype(vv, w)), cfg)
    y = conv(prime, p.to(dtype=prime.dtype), cfg)

    # 4. dropout on y (layers.py:316), head merge and W_o (layers.py:317-320)
    if y_dropout is not None:
        y = y_dropout(y)
    z = head_merge(y, B, H, cfg.seq_length)
    z = z.to(dt)
    out = F.linear(z, p.W_o.to(dt))
    if return_intermediates:
        it.k, it.q, it.v, it.S, it.idx, it.vals, it.w, it.y, it.z, it.cand = (
            k, q, v, S, idx, vals, w, y, z, cand)
        return out, it
    return out


def prime_dtype(v: torch.Tensor, w: torch.Tensor):
    # sampled paths promote to fp32 through the fp32 ``ones`` (layers.py:374-376)
    return torch.promote_types(v.dtype, w.dtype)


# --------------------------------------------------------------------------
# stage oracles used by kernel-level parity tests
# --------------------------------------------------------------------------

def topk_exact(k_tok: torch.Tensor, q_tok: torch.Tensor, cfg: Config,
               cand: Optional[torch.Tensor] = None, kvalid: Optional[int] = None,
               normalized_inputs: bool = False):
    """Top-k of the similarity between token-major k (BH,N,c) and q (BH,Nq,c),
    computed in float64 from the given (already rounded) operands.

    Returns (idx int64 (BH,N,K), vals float64 (BH,N,K), S float64 (BH,N,Nq)).
    ``kvalid`` limits the channels used (padding channels are ignored).
    ``normalized_inputs``: cosine operands were already normalised (and rounded)
    by the projection stage, so S is their plain dot product.
    """
    c = kvalid if kvalid is not None else k_tok.shape[-1]
    k = k_tok[..., :c].to(torch.float64).transpose(1, 2)
    q = q_tok[..., :c].to(torch.float64).transpose(1, 2)
    if normalized_inputs and cfg.magnitude_type == "cosine":
        S = torch.matmul(k.transpose(1, 2), q)
    else:
        S = similarity(k, q, cfg)
    if cand is not None:
        S = mask_self(S, cand, cfg)
    idx, vals = select_neighbours(S, cfg, cand)
    return idx, vals.to(torch.float64), S


def topk_gap_ok(S: torch.Tensor, idx_got: torch.Tensor, idx_exp: torch.Tensor, cfg: Config,
                cand: Optional[torch.Tensor] = None, tol: float = 1e-6) -> torch.Tensor:
    """Per-row boolean: the kernel's selection is acceptable.

    A row passes when indices match exactly, or when every rank where they
    differ has |S[got] - S[exp]| < ``tol`` (a near tie, exempt by contract).
    Sampled rows compare positions 1.. through the candidate map.
    """
    if cand is not None:
        # map token index back to candidate column
        inv = torch.full((max(int(cand.max()) + 1, 1),), -1, dtype=torch.long)
        inv[cand] = torch.arange(cand.numel())
        got_c = inv[idx_got[..., 1:]]
        exp_c = inv[idx_exp[..., 1:]]
        selfok = (idx_got[..., 0] == idx_exp[..., 0])
        sg = torch.gather(S, -1, got_c.clamp_min(0))
        se = torch.gather(S, -1, exp_c)
        same = got_c == exp_c
        close = (sg - se).abs() < tol
        return selfok & (same | close).all(-1) & (got_c >= 0).all(-1)
    sg = torch.gather(S, -1, idx_got)
    se = torch.gather(S, -1, idx_exp)
    same = idx_got == idx_exp
    close = (sg - se).abs() < tol
    return (same | close).all(-1)


def aggregate_exact(v_tok: torch.Tensor, idx: torch.Tensor, vals: torch.Tensor, p: Params,
                    cfg: Config, B: int, sampled: bool) -> torch.Tensor:
    """Weights + gather + conv + head merge in float64 from token-major v (BH,N,c).

    Returns z (B, N, C) float64 -- the tensor that enters W_o.
    """
    v = v_tok.to(torch.float64).transpose(1, 2)[:, : cfg.in_channels]
    w = neighbour_weights(vals.to(torch.float64), cfg, sampled)
    prime = gather_prime(v, idx, w, cfg)
    y = conv(prime, p.to(dtype=torch.float64), cfg)
    return head_merge(y, B, cfg.num_heads, cfg.seq_length)


def flops(cfg: Config, B: int, N: int) -> dict:
    """Algorithmic flops of one forward (2 per multiply-accumulate)."""
    C, dk, K = cfg.d_hidden, cfg.d_k, cfg.K
    Nq = N if cfg.sampling_type == "all" else cfg.num_samples
    proj = 2 * B * C * C * (3 * N + Nq)
    sim = 2 * B * N * Nq * C
    if cfg.convolution_type == "depthwise":
        cv = 2 * B * N * C * K
    elif cfg.convolution_type == "standard":
        cv = 2 * B * N * C * dk * K
    else:
        cv = 2 * B * N * C * (K + dk)
    return {"proj": proj, "sim": sim, "conv": cv, "total": proj + sim + cv}


# ---------------------------------------------------------------------------
# Callers of the operator (layers.py:452-686).  Pinning, in tests/test_oracle.py:
#   conv1d_branch   == an element-by-element loop (padding placement, merge);
#   mha             == a per-row softmax loop;
#   kvt             == a per-row python sort + softmax loop; == full softmax
#                      attention at topk == N; == the ConvNN restatement above
#                      with H == 1 and the projections assigned as in
#                      MultiHeadKvtAttention's docstring;
#   branching_*     == the concatenation of the two branches by construction
#                      (each branch pinned on its own).
# ---------------------------------------------------------------------------

def conv1d_branch(x: torch.Tensor, Wx, bx, conv_w, conv_b, Wo, bo, H: int) -> torch.Tensor:
    """MultiHeadConv1dAttention.forward (layers.py:495-499).

    W_x, split_head + batch_combine to (B*H, d_k, N), Conv1d with padding
    'same' ((ks-1)//2 zeros in front, the rest behind), then permute +
    batch_split + combine_heads: the token-major conv output of each head read
    as (d_k, N) and transposed, which mixes tokens for every H
    (``z[b, t, h*d_k + a] = y_tok[b*H + h].flat[a*N + t]``), then W_o.
    """
    B, N, C = x.shape
    dk = C // H
    u = F.linear(x, Wx, bx)
    u = u.view(B, N, H, dk).transpose(1, 2).permute(0, 1, 3, 2).contiguous().view(-1, dk, N)
    y = F.conv1d(u, conv_w, conv_b, stride=1, padding="same")            # (B*H, d_k, N)
    y = y.permute(0, 2, 1).reshape(B, -1, dk, N).permute(0, 1, 3, 2).contiguous()
    z = y.transpose(1, 2).contiguous().view(B, N, C)
    return F.linear(z, Wo, bo)


def mha(x: torch.Tensor, Wq, Wk, Wv, Wo, H: int, mask=None) -> torch.Tensor:
    """MultiHeadAttention.forward in eval mode (layers.py:106-130)."""
    B, N, C = x.shape
    dk = C // H
    sh = lambda t: t.view(B, N, H, dk).transpose(1, 2)
    q, k, v = sh(F.linear(x, Wq)), sh(F.linear(x, Wk)), sh(F.linear(x, Wv))
    s = torch.matmul(q, k.transpose(-2, -1).contiguous()) / math.sqrt(dk)
    if mask is not None:
        s = s.masked_fill(mask == 0, -1e9)
    o = torch.matmul(torch.softmax(s, dim=-1), v.contiguous())
    return F.linear(o.transpose(1, 2).contiguous().view(B, N, C), Wo)


def kvt(x: torch.Tensor, Wqkv, Wproj, H: int, topk: int, scale: float, wmul=None,
        bqkv=None, dense_mult=None) -> torch.Tensor:
    """MultiHeadKvtAttention.forward (layers.py:668-686), eval mode.

    attn = q k^T * scale; keep the ``topk`` largest of each row (ties: lowest
    key index, see ``stable_topk``), -inf elsewhere; softmax; @ v; heads side
    by side; proj.  ``wmul`` (B*H, N, topk): multipliers on the kept
    probabilities in rank order (attention dropout with a given mask).
    ``dense_mult`` (B, H, N, N): ``attn_drop`` as the reference applies it
    (layers.py:680), a multiplier on the whole probability row (the
    probabilities outside the top-k are zero).
    """
    B, N, C = x.shape
    dk = C // H
    qkv = F.linear(x, Wqkv, bqkv).reshape(B, N, 3, H, dk).permute(2, 0, 3, 1, 4)
    q, k, v = qkv[0], qkv[1], qkv[2]
    attn = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale
    vals, idx = stable_topk(attn, topk, largest=True)
    p = torch.softmax(vals, dim=-1)                                  # == masked dense softmax
    if wmul is not None:
        p = p * wmul.view(B, H, N, topk).to(p.dtype)
    if dense_mult is not None:
        p = p * torch.gather(dense_mult.to(p.dtype), -1, idx)
    vg = torch.gather(v.unsqueeze(2).expand(B, H, N, N, dk), 3,
                      idx.unsqueeze(-1).expand(B, H, N, topk, dk))   # (B, H, N, topk, dk)
    o = (p.unsqueeze(-1) * vg).sum(3)
    return F.linear(o.transpose(1, 2).reshape(B, N, C), Wproj)


def branching_conv(x: torch.Tensor, convnn_fn, conv1d_fn, Wp, bp, d1: int) -> torch.Tensor:
    """MultiHeadBranchingConv / MultiHeadBranchingAttention forward with both
    branches (layers.py:590-600, 644-652): branch 1 on channels [0, d1),
    branch 2 on the rest, concatenated, pointwise linear with bias."""
    x1 = convnn_fn(x[:, :, :d1])
    x2 = conv1d_fn(x[:, :, d1:])
    return F.linear(torch.cat((x1, x2), dim=2), Wp, bp)
