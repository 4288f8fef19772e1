"""Per-layer SnapKV / PyramidKV / H2O state machine on the MI355X hot tier
(src/hotcold_kv/baselines/layer_state.py:29-117).

prefill: the prompt's own causal attention (the model's attention, torch
SDPA), then scoring -> kept indices -> gather of K/V into a fixed-capacity
hot buffer, all on the gfx950 kernels.  SnapKV / PyramidKV score with the
observation window; H2O with the whole prompt's accumulated attention.
decode: the new token is written into the next free row (no torch.cat of the
whole cache) and GQA decode attention runs over the hot buffer.  H2O also
adds each key's attention probability (mean over the query heads of its KV
head) to its score and re-evicts to the budget every step.  Stored keys are
post-RoPE, so a kept token keeps its original position (layer_state.py:1-10).
"""

import torch
import torch.nn.functional as F

from .. import ops
from ..hot_buffer import HotBuffer
from .scoring import repeat_kv


class PressLayerState:
    def __init__(self, method: str, budget: int, window_size: int, kernel_size: int, pooling: str,
                 decode_reserve: int = 256):
        if method not in ("snapkv", "pyramidkv", "h2o"):
            raise ValueError(f"unknown method {method}")
        self.method = method
        self.budget = int(budget)
        self.window_size = int(window_size)
        self.kernel_size = int(kernel_size)
        self.pooling = pooling
        self.decode_reserve = int(decode_reserve)
        self.buf = None
        self._h2o = None        # H2O scores [B][Hk][buffer capacity] fp32, aligned with the hot rows
        self._h2o_spare = None

    # -- introspection -------------------------------------------------------
    @property
    def keys(self):
        return None if self.buf is None else self.buf.keys

    @property
    def values(self):
        return None if self.buf is None else self.buf.values

    @property
    def scores(self):
        """H2O accumulated scores (B,Hk,n) of the resident tokens (None for
        the window methods), as the reference's `scores` attribute."""
        if self.method != "h2o" or self.buf is None or self._h2o is None:
            return None
        return self._h2o[:, :, : self.buf.n]

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

    # -- H2O score rows ------------------------------------------------------------
    def _h2o_storage(self):
        """Score rows sized to the hot buffer's capacity (kept on growth)."""
        cap = self.buf.cap
        if self._h2o is None or self._h2o.shape[2] != cap:
            new = torch.zeros((self.buf.B, self.buf.H, cap), dtype=torch.float32, device=self.buf.device)
            if self._h2o is not None:
                n = min(self._h2o.shape[2], cap)
                new[:, :, :n].copy_(self._h2o[:, :, :n])
            self._h2o = new
            self._h2o_spare = torch.empty_like(new)

    def _h2o_keep(self, scores_src, keep):
        """Score rows keep (B,Hk,n) of scores_src (B,Hk,S) into the score buffer."""
        self._h2o_storage()
        ops.gather_rows(keep, [(scores_src.unsqueeze(-1), self._h2o_spare.unsqueeze(-1))])
        self._h2o, self._h2o_spare = self._h2o_spare, self._h2o

    # -- forward paths -----------------------------------------------------------
    def prefill(self, q_post, k_post, v, n_rep, scaling):
        """Attend over the full prompt, then compress the prompt KV to the budget."""
        out = self._attn(q_post, k_post, v, n_rep, scaling, causal=True)
        S = int(k_post.shape[2])
        h2o = self.method == "h2o"
        scores = ops.h2o_prefill_scores(q_post, k_post, scaling) if h2o else None
        if S <= self.budget:
            self._new_buffer(k_post, S)
            self.buf.set_from(k_post, v)
            if h2o:
                self._h2o_storage()
                self._h2o[:, :, :S].copy_(scores)
            return out
        if not h2o:
            scores = ops.snapkv_scores(q_post, k_post, self.window_size, scaling, self.kernel_size, self.pooling)
        keep = ops.keep_index(scores, self.window_size, self.budget)
        self._new_buffer(k_post, int(keep.shape[-1]))
        self.buf.gather_from(k_post, v, keep)
        if h2o:
            self._h2o_keep(scores, keep)
        return out

    def decode(self, q_post, k_post, v, n_rep, scaling):
        """Single-token decode: append, then attend over the compressed cache
        (one fused launch for one token)."""
        if self.buf is None:
            raise RuntimeError("decode before prefill")
        if self.method == "h2o":
            return self._decode_h2o(q_post, k_post, v, scaling)
        if k_post.shape[2] == 1:
            out = self.buf.append_attend(q_post, k_post, v, scaling)
        else:
            self.buf.append(k_post, v)
            out = ops.decode_attention(q_post, self.buf.keys, self.buf.values, scaling)
        return out.unsqueeze(2)  # (B,Hq,1,D)

    def _decode_h2o(self, q_post, k_post, v, scaling):
        """layer_state.py:102-114: append, attend while adding each key's
        attention probability (mean over the query heads of its KV head) to
        its score, then keep the budget by score (window kept) when over it."""
        if k_post.shape[2] != 1:
            raise RuntimeError("H2O decode takes one token per step")
        n = self.buf.n + 1
        if (n > self.budget and not self.buf.with_pre and not self.buf.with_pos
                and ops.h2o_evicts_one(n, self.window_size, self.budget)):
            # one row over budget: append, attention, score update and the
            # one-row eviction in one call, written into the second buffers
            self.buf.ensure(n)
            self._h2o_storage()
            lo = self.buf.held
            out = ops.decode_attention_h2o_evict(q_post, self.buf.st["k"][:, :, lo:lo + n],
                                                 self.buf.st["v"][:, :, lo:lo + n], scaling,
                                                 self._h2o[:, :, :n], self.window_size, self.budget,
                                                 self.buf.spare_rows("k"), self.buf.spare_rows("v"),
                                                 self._h2o_spare, k_new=k_post, v_new=v)
            self.buf.adopt_spare(n - 1)
            self._h2o, self._h2o_spare = self._h2o_spare, self._h2o
            return out.unsqueeze(2)  # (B,Hq,1,D)
        self.buf.append(k_post, v)
        self._h2o_storage()
        n = self.buf.n
        out = ops.decode_attention_h2o(q_post, self.buf.keys, self.buf.values, scaling, self._h2o[:, :, :n])
        if n > self.budget:
            keep = ops.keep_index(self._h2o[:, :, :n], self.window_size, self.budget)
            self.buf.compact(keep)
            self._h2o_keep(self._h2o[:, :, :n], keep)
        return out.unsqueeze(2)  # (B,Hq,1,D)
