"""Transfer objects between the hot tier and the cold store, and the shape
canonicalisers of the reference (src/hotcold_kv/datatypes.py:8-63)."""

from dataclasses import dataclass

import torch


def _squeeze_to(x, ndim, name, layout):
    """Drop singleton dims after the batch dim until x has `ndim` dims
    (datatypes.py:8-44: the batch dim is never squeezed, so B == 1 survives)."""
    if not isinstance(x, torch.Tensor):
        raise RuntimeError(f"{name} must be a Tensor")
    while x.dim() > ndim:
        singles = [d for d in range(1, x.dim()) if x.shape[d] == 1]
        if not singles:
            break
        x = x.squeeze(singles[0])
    if x.dim() != ndim:
        raise RuntimeError(f"{name} must be {ndim}D {layout}; got {tuple(x.shape)}")
    return x


def _canon_kv_4d(x, name):
    """Return x as (B,Hk,R,D) (datatypes.py:8-27)."""
    return _squeeze_to(x, 4, name, "(B,Hk,R,D)")


def _canon_br_2d(x, name):
    """Return x as (B,R) (datatypes.py:29-44)."""
    return _squeeze_to(x, 2, name, "(B,R)")


@dataclass
class RetrievedKV:
    """Retrieved cold tokens staged on the device (datatypes.py:50-56).

    k_pre/v are (B,Hk,R,D) pre-RoPE keys and values; pos/valid are (B,R)
    (one position set per batch row) or (B,Hk,R) when retrieval runs per KV
    head.  ready is True once the host-to-device copy has completed."""

    k_pre: torch.Tensor
    v: torch.Tensor
    pos: torch.Tensor
    valid: torch.Tensor
    ready: bool = False
    # rotary tables at pos, first D/2 dims in the cache dtype ((B,R,D/2) or
    # (B,Hk,R,D/2)), computed with the retrieval when the rotary parameters
    # are known; None otherwise (not fields of the reference)
    cos: torch.Tensor = None
    sin: torch.Tensor = None


@dataclass
class EvictedKV:
    """Tokens leaving the hot tier (datatypes.py:58-63): pinned fp32 host
    copies (B,Hk,Te,D), int64 positions (B,Te) and the evicted hot-buffer
    indices padded with -1 (B,Te)."""

    k_pre_cpu: torch.Tensor
    v_cpu: torch.Tensor
    pos_cpu: torch.Tensor
    evicted_idx: torch.Tensor
