"""Seeded synthetic hot-tier workloads (the five benchmark configurations).

Every tensor is drawn in fp32 from a seeded torch.Generator and then cast to
the configuration dtype, so a CPU checker and the GPU see the same bytes.

  * q_pre, k_pre, v ~ N(0,1); q_post/k_post = RoPE(pre, positions 0..S-1)
    with theta = 500000 and the rotate_half convention (split halves).
  * needles: `needles` prompt offsets drawn uniformly from [0, S-W); the
    needle's post-RoPE key is set to 3*sqrt(D)*u + N(0,1), u the unit mean of
    the window's post-RoPE queries of that KV-head group; its pre-RoPE key is
    the inverse rotation, so the cold tier stores consistent pre-RoPE keys.
  * outliers: `outliers` seeded channels of k_pre scaled x20 before RoPE.
  * decode steps draw a fresh N(0,1) token (q_pre, k_pre, v) per layer.

Seeds: layer l of a run with seed s uses seed s*1000 + l; with
per_sequence_seeds every batch row b additionally uses its own generator
seeded (s*1000 + l)*64 + b, so rows are independent sequences.
"""

import dataclasses
import math

import torch


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    layers: int
    batch: int
    seq_len: int
    dtype: torch.dtype
    budget: int
    window: int
    pool: int
    decode_steps: int
    held: int = 0
    retrieve_every: int = 0
    prefill_retrieval: int = 0
    needles: int = 0
    outliers: int = 0
    per_sequence_seeds: bool = False
    hq: int = 32
    hk: int = 8
    head_dim: int = 128
    theta: float = 500000.0

    @property
    def group(self):
        return self.hq // self.hk

    @property
    def scaling(self):
        return 1.0 / math.sqrt(self.head_dim)

    @property
    def hot_capacity(self):
        return self.held + self.budget + self.decode_steps


WORKLOADS = {
    "plumbing_fp32_2k_b512": Workload("plumbing_fp32_2k_b512", layers=1, batch=1, seq_len=2048, dtype=torch.float32,
                                 budget=512, window=32, pool=7, decode_steps=64),
    "llama8b_8k_b512": Workload("llama8b_8k_b512", layers=32, batch=1, seq_len=8192, dtype=torch.float16,
                                   budget=512, window=32, pool=7, decode_steps=63, needles=16),
    "llama8b_16k_b1024_held64": Workload("llama8b_16k_b1024_held64", layers=32, batch=1, seq_len=16384,
                                            dtype=torch.float16, budget=1024, window=32, pool=7, decode_steps=128,
                                            held=64, retrieve_every=16, needles=16),
    "b16_32k_b2048_held128": Workload("b16_32k_b2048_held128", layers=32, batch=16, seq_len=32768,
                                         dtype=torch.float16, budget=2048, window=64, pool=7, decode_steps=256,
                                         held=128, retrieve_every=16, needles=16, per_sequence_seeds=True),
    "bf16_b4_64k_b4096_held256": Workload("bf16_b4_64k_b4096_held256", layers=32, batch=4, seq_len=65536,
                                             dtype=torch.bfloat16, budget=4096, window=64, pool=7,
                                             decode_steps=128, held=256, retrieve_every=8, prefill_retrieval=256,
                                             needles=16, outliers=4, per_sequence_seeds=True),
}


def inv_freq(head_dim, theta, device=None):
    """Default RoPE inverse frequencies, fp32 (1 / theta^(2i/D))."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))


def rope(x, pos, inv, inverse=False):
    """Rotate x (..., S, D) fp32 to positions pos (S,) with rotate_half."""
    freqs = pos.float()[:, None] * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos(), emb.sin()
    if inverse:
        sin = -sin
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    rot = torch.cat((-x2, x1), dim=-1)
    return x * cos + rot * sin


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def make_prompt(w: Workload, layer=0, seed=0, device="cpu", seq_len=None, batch=None):
    """Prompt tensors of one layer: dict of q_pre/q_post (B,Hq,S,D),
    k_pre/k_post/v (B,Hk,S,D) in w.dtype, positions (B,S) int64 and the needle
    offsets (B,Hk,n) int64."""
    S = seq_len or w.seq_len
    B = batch or w.batch
    D, Hq, Hk, G, W = w.head_dim, w.hq, w.hk, w.group, min(w.window, S)
    base = seed * 1000 + layer
    rows = []
    for b in range(B if w.per_sequence_seeds else 1):
        g = _gen(base * 64 + b if w.per_sequence_seeds else base, device)
        nb = 1 if w.per_sequence_seeds else B
        q = torch.randn((nb, Hq, S, D), generator=g, device=device)
        k = torch.randn((nb, Hk, S, D), generator=g, device=device)
        v = torch.randn((nb, Hk, S, D), generator=g, device=device)
        if w.outliers:
            ch = torch.randperm(D, generator=g, device=device)[: w.outliers]
            k[..., ch] *= 20.0
        needle_pos = None
        if w.needles:
            needle_pos = torch.randint(0, max(1, S - W), (nb, Hk, w.needles), generator=g, device=device)
            noise = torch.randn((nb, Hk, w.needles, D), generator=g, device=device)
        rows.append((q, k, v, needle_pos, noise if w.needles else None))
    q = torch.cat([r[0] for r in rows], 0)
    k = torch.cat([r[1] for r in rows], 0)
    v = torch.cat([r[2] for r in rows], 0)
    pos = torch.arange(S, device=device)
    inv = inv_freq(D, w.theta, device)
    q_post = rope(q, pos, inv)
    k_post = rope(k, pos, inv)
    needles = None
    if w.needles:
        needles = torch.cat([r[3] for r in rows], 0)
        noise = torch.cat([r[4] for r in rows], 0)
        qw = q_post[:, :, S - W:, :].reshape(B, Hk, G * W, D).mean(dim=2)     # (B,Hk,D)
        u = qw / qw.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        nk = 3.0 * math.sqrt(D) * u[:, :, None, :] + noise                    # (B,Hk,n,D)
        idx = needles[..., None].expand(B, Hk, w.needles, D)
        k_post.scatter_(2, idx, nk)
        # inverse rotation of each needle key at its own position
        npos = needles.reshape(-1)
        freqs = npos.float()[:, None] * inv[None, :]
        emb = torch.cat((freqs, freqs), dim=-1)
        cos, sin = emb.cos(), -emb.sin()
        x = nk.reshape(-1, D)
        x1, x2 = x[:, : D // 2], x[:, D // 2:]
        pre = x * cos + torch.cat((-x2, x1), dim=-1) * sin
        k.scatter_(2, idx, pre.view(B, Hk, w.needles, D))
    dt = w.dtype
    return dict(q_pre=q.to(dt), q_post=q_post.to(dt), k_pre=k.to(dt), k_post=k_post.to(dt), v=v.to(dt),
                positions=pos[None, :].expand(B, S).contiguous(), needles=needles)


def make_decode_token(w: Workload, layer, step, seed=0, device="cpu", batch=None, position=None):
    """One decode token of one layer: q_pre/q_post (B,Hq,1,D), k_pre/k_post/v
    (B,Hk,1,D) in w.dtype, position (B,1) int64."""
    B = batch or w.batch
    D = w.head_dim
    g = _gen((seed * 1000 + layer) * 100003 + 7919 * (step + 1), device)
    q = torch.randn((B, w.hq, 1, D), generator=g, device=device)
    k = torch.randn((B, w.hk, 1, D), generator=g, device=device)
    v = torch.randn((B, w.hk, 1, D), generator=g, device=device)
    p = int(position if position is not None else w.seq_len + step)
    pos = torch.full((1,), p, device=device, dtype=torch.int64)
    inv = inv_freq(D, w.theta, device)
    dt = w.dtype
    return dict(q_pre=q.to(dt), q_post=rope(q, pos, inv).to(dt), k_pre=k.to(dt), k_post=rope(k, pos, inv).to(dt),
                v=v.to(dt), position=pos.view(1, 1).expand(B, 1).contiguous())
