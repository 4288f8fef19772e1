"""Per-layer SnapKV / PyramidKV state machine on the MI355X hot tier
(src/hotcold_kv/baselines/layer_state.py:68-117).

prefill: the prompt's own causal attention (the model's attention, torch
SDPA), then window scoring -> kept indices -> gather of K/V into a
fixed-capacity hot buffer, all on the gfx950 kernels.  decode: the new token
is written into the next free row (no torch.cat of the whole cache) and GQA
decode attention runs over the hot buffer.  Stored keys are post-RoPE, so a
kept token keeps its original position (layer_state.py:1-10).
"""

import torch
import torch.nn.functional as F

from .. import ops
from ..hot_buffer import HotBuffer
from .scoring import repeat_kv


class PressLayerState:
    def __init__(self, method: str, budget: int, window_size: int, kernel_size: int, pooling: str,
                 decode_reserve: int = 256):
        if method == "h2o":
            raise NotImplementedError("H2O is not part of the MI355X hot tier (SnapKV / PyramidKV only)")
        if method not in ("snapkv", "pyramidkv"):
            raise ValueError(f"unknown method {method}")
        self.method = method
        self.budget = int(budget)
        self.window_size = int(window_size)
        self.kernel_size = int(kernel_size)
        self.pooling = pooling
        self.decode_reserve = int(decode_reserve)
        self.buf = None
        self.scores = None  # H2O accumulator slot of the reference; unused here

    # -- introspection -------------------------------------------------------
    @property
    def keys(self):
        return None if self.buf is None else self.buf.keys

    @property
    def values(self):
        return None if self.buf is None else self.buf.values

    def get_seq_length(self) -> int:
        return 0 if self.buf is None else self.buf.n

    # -- attention -------------------------------------------------------------
    @staticmethod
    def _attn(q, k, v, n_rep, scaling, causal):
        """The prompt's own attention (layer_state.py:49-53)."""
        out = F.scaled_dot_product_attention(q, repeat_kv(k, n_rep), repeat_kv(v, n_rep), is_causal=causal,
                                             scale=scaling)
        return out.to(q.dtype)

    def _new_buffer(self, k_post, rows):
        B, Hk, _, D = k_post.shape
        self.buf = HotBuffer(B, Hk, D, k_post.dtype, k_post.device, rows + self.decode_reserve)

    # -- forward paths -----------------------------------------------------------
    def prefill(self, q_post, k_post, v, n_rep, scaling):
        """Attend over the full prompt, then compress the prompt KV to the budget."""
        out = self._attn(q_post, k_post, v, n_rep, scaling, causal=True)
        S = int(k_post.shape[2])
        if S <= self.budget:
            self._new_buffer(k_post, S)
            self.buf.set_from(k_post, v)
            return out
        scores = ops.snapkv_scores(q_post, k_post, self.window_size, scaling, self.kernel_size, self.pooling)
        keep = ops.keep_index(scores, self.window_size, self.budget)
        self._new_buffer(k_post, int(keep.shape[-1]))
        self.buf.gather_from(k_post, v, keep)
        return out

    def decode(self, q_post, k_post, v, n_rep, scaling):
        """Single-token decode: append, then attend over the compressed cache
        (one fused launch for one token)."""
        if self.buf is None:
            raise RuntimeError("decode before prefill")
        if k_post.shape[2] == 1:
            out = self.buf.append_attend(q_post, k_post, v, scaling)
        else:
            self.buf.append(k_post, v)
            out = ops.decode_attention(q_post, self.buf.keys, self.buf.values, scaling)
        return out.unsqueeze(2)  # (B,Hq,1,D)
