"""SnapKV / H2O scoring and selection with the reference's function names
(src/hotcold_kv/baselines/scoring.py).

snapkv_importance, h2o_prefill_scores, keep_index and gather_kv run on the
gfx950 kernels (device tensors only).  The small layout helpers (repeat_kv, the GQA
reductions, pool1d, gather_scores) are plain tensor ops that the kernels
fuse; they are kept for API compatibility.
"""

import torch.nn.functional as F

from .. import ops


def repeat_kv(x, n_rep):
    """(B,Hk,S,D) -> (B,Hk*n_rep,S,D) (scoring.py:9-14)."""
    if n_rep == 1:
        return x
    B, Hk, S, D = x.shape
    return x[:, :, None].expand(B, Hk, n_rep, S, D).reshape(B, Hk * n_rep, S, D)


def _group_query_to_kv(q, Hk):
    """Mean of each GQA group (scoring.py:17-26)."""
    B, Hq, T, D = q.shape
    if Hq == Hk:
        return q
    if Hq % Hk == 0:
        return q.view(B, Hk, Hq // Hk, T, D).mean(dim=2)
    return q.mean(dim=1, keepdim=True).expand(B, Hk, T, D)


def _reduce_probs_to_kv(probs, Hk):
    """(B,Hq,T,S) -> (B,Hk,T,S) mean over each group (scoring.py:29-37)."""
    B, Hq, T, S = probs.shape
    if Hq == Hk:
        return probs
    if Hq % Hk == 0:
        return probs.view(B, Hk, Hq // Hk, T, S).mean(dim=2)
    return probs.mean(dim=1, keepdim=True).expand(B, Hk, T, S)


def pool1d(x, kernel_size, pooling):
    """Length-preserving 1-D pooling over the last dim (scoring.py:40-47)."""
    if kernel_size is None or kernel_size <= 1:
        return x
    pad = kernel_size // 2
    if pooling == "avgpool":
        return F.avg_pool1d(x, kernel_size=kernel_size, stride=1, padding=pad)
    return F.max_pool1d(x, kernel_size=kernel_size, stride=1, padding=pad)


def snapkv_importance(q_post, keys, window_size, scaling, kernel_size, pooling):
    """SnapKV per-KV-head importance (B,Hk,S) float32 (scoring.py:50-79):
    GQA-mean window queries, causal window logits, softmax over keys, sum over
    the window, pooling -- one fused pipeline on the device."""
    return ops.snapkv_scores(q_post, keys, window_size, scaling, kernel_size, pooling)


def h2o_prefill_scores(q_post, keys, scaling, chunk=512):
    """H2O accumulated attention over the whole prefill per KV head (B,Hk,S)
    float32 (scoring.py:82-107): causal softmax of every query row summed per
    query head, then averaged over the query heads of each KV head.  `chunk`
    is the reference's query-row chunking; the device pipeline needs none."""
    return ops.h2o_prefill_scores(q_post, keys, scaling)


def keep_index(scores, window_size, budget):
    """Top prefix tokens (score desc, ties to the lower index), ascending,
    followed by the recent window: (B,Hk,keep) int64 (scoring.py:110-132)."""
    return ops.keep_index(scores, window_size, budget)


def gather_kv(t, keep):
    """Gather (B,H,S,D) along S with per-head indices (B,H,k) (scoring.py:135-139)."""
    return ops.gather_kv(t, keep)


def gather_scores(s, keep):
    """Gather (B,H,S) along S (scoring.py:142-144)."""
    return s.gather(2, keep)
