"""Writes tests/golden/window_scores.npz: seeded inputs, importance scores and
kept indices under the scoring contract (window QK^T in fp64, exact-sum
softmax, fp32 importance, max-pool, top-k with ties to the lower index).

The reference ships no numeric fixtures (its tests check shapes and
invariants only), so these vectors come from the oracle after it has been
pinned by the closed-form, brute-force and literal-fp32 checks in
tests/test_oracle.py; they freeze its output so that a later change to the
oracle or to the kernels cannot drift silently.  Only the window rows of q are
stored (the other rows do not enter the scores); the test pads them with
zeros.

    python tests/golden/make_golden.py
"""

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import reference as ref  # noqa: E402

# name: (B, Hq, Hk, S, D, window, pool, budget, dtype, needles)
CASES = {
    "small_fp32": (2, 8, 2, 200, 16, 16, 7, 64, torch.float32, 0),
    "gqa4_fp16": (1, 32, 8, 600, 128, 32, 7, 128, torch.float16, 4),
    "ties_fp16": (1, 4, 4, 300, 64, 8, 5, 40, torch.float16, 0),
    "bf16_w64": (1, 16, 4, 700, 64, 64, 9, 200, torch.bfloat16, 2),
}


def make_case(name, B, Hq, Hk, S, D, W, pool, budget, dtype, needles, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((B, Hk, S, D), generator=g)
    qw = torch.randn((B, Hq, W, D), generator=g)
    if needles:
        # planted keys aligned with the group's mean window query
        qm = qw.view(B, Hk, Hq // Hk, W, D).mean(dim=(2, 3))
        u = qm / qm.norm(dim=-1, keepdim=True)
        pos = torch.randperm(S - W, generator=g)[:needles]
        for p in pos.tolist():
            k[:, :, p] += 3 * math.sqrt(D) * u
    if name.startswith("ties"):
        # coarse values: many equal logits and equal pooled scores
        k = torch.round(k)
        qw = torch.round(qw)
    k, qw = k.to(dtype), qw.to(dtype)
    q = torch.zeros((B, Hq, S, D), dtype=dtype)
    q[:, :, S - W:] = qw
    scale = 1.0 / math.sqrt(D)
    scores = ref.window_scores(q, k, W, scale, pool, "maxpool")
    keep = ref.keep_index(scores, W, budget)
    f = lambda t: t.float().numpy() if t.dtype == torch.bfloat16 else t.numpy()
    return {
        f"{name}__q": f(qw), f"{name}__k": f(k),
        f"{name}__dtype": np.array(str(dtype).split(".")[-1]),
        f"{name}__meta": np.array([W, pool, budget], dtype=np.int64),
        f"{name}__scaling": np.array(scale, dtype=np.float64),
        f"{name}__scores": scores.numpy(), f"{name}__keep": keep.numpy(),
    }


def main():
    out = {}
    for i, (name, c) in enumerate(CASES.items()):
        out.update(make_case(name, *c, seed=1234 + i))
    path = os.path.join(HERE, "window_scores.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
