"""Decode attention entry point with the reference's signature.

triton_evict_attention_forward keeps the name, arguments, validation and
return tuple of src/hotcold_kv/kernels.py:77-137 so existing callers work
unchanged; the work is done by the gfx950 split-K decode kernel
(hc_decode_attn).  Differences from the reference, by design:
  * the softmax is max-stabilised (the reference exponentiates raw logits,
    kernels.py:57, and overflows past ~88.7); outputs agree wherever the
    reference is finite;
  * K/V are read once per KV head, not once per query head;
  * the eviction score (kernels.py:66-67, 134-136) is computed only when
    asked for (compute_evict, default True to keep the return value).
"""

import torch

from . import ops


def triton_evict_attention_forward(query, key, value, attention_mask, num_key_value_groups, scaling,
                                   dropout=0.0, block_s=64, compute_evict=True):
    """Single-token GQA attention.

    query (B,Hq,1,D), key/value (B,Hk,S,D), attention_mask (B,S) bool (True =
    attend).  Returns (attn_out (B,1,Hq,D) in query's dtype, evict_idx (B,)
    int64 or None when compute_evict is False).  block_s is accepted for
    signature compatibility; tiling is chosen by the kernel.
    """
    assert query.is_cuda and key.is_cuda and value.is_cuda and attention_mask.is_cuda
    if dropout != 0.0:
        raise ValueError("dropout must be 0.0 , because we are not in training")
    B, Hq, _, D = query.shape
    _, Hk, S, _ = key.shape
    if Hq // num_key_value_groups != Hk:
        raise ValueError(f"Hq({Hq})//N_REP({num_key_value_groups}) must equal Hk({Hk})")
    out = torch.empty((B, 1, Hq, D), dtype=query.dtype, device=query.device)
    res = ops.decode_attention(query, key, value, scaling, mask=attention_mask, out=out[:, 0],
                               with_evict=compute_evict)
    if compute_evict:
        _, _, evict_idx = res
        return out, evict_idx
    return out, None


def decode_attention_forward(query, key, value, attention_mask, num_key_value_groups, scaling, dropout=0.0):
    """Same as triton_evict_attention_forward without the eviction score."""
    out, _ = triton_evict_attention_forward(query, key, value, attention_mask, num_key_value_groups, scaling,
                                            dropout=dropout, compute_evict=False)
    return out
