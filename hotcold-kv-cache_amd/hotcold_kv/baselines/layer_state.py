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
from ..hot_buffer import HotBuffer, kv_rows
from .scoring import repeat_kv


class DeferredCompaction:
    """The prompt compactions of many layers, run together in one launch set.

    A model's prefill visits its layers in turn, and each layer's SnapKV /
    PyramidKV compaction (layer_state.py:82-94) depends only on that layer's
    own prompt queries and keys; no prompt attention reads a compacted cache.
    So a layer's compaction can wait until the prompt has passed every layer,
    and all pending layers then compact together: one scoring launch set over
    every layer's keys (per-layer row tables, no copies), one top-k launch and
    one gather into every layer's hot buffer per budget.  The kept indices are
    the ones each layer would get on its own, bit for bit.

    Pending layers keep their prompt K/V (and a copy of their window's query
    rows) alive until then; past max_pending_bytes the pending layers are
    compacted early.  By default that limit is an eighth of the device's
    memory, at most 16 GiB, so deferring cannot take a device that fitted the
    per-layer compaction far past its memory.
    """

    DEFAULT_MAX_BYTES = 16 << 30

    def __init__(self, max_pending_bytes=None):
        self.max_pending_bytes = None if max_pending_bytes is None else int(max_pending_bytes)
        self.pending = []
        self.pending_bytes = 0

    def _limit(self, device):
        if self.max_pending_bytes is None:
            total = torch.cuda.get_device_properties(device).total_memory
            self.max_pending_bytes = min(self.DEFAULT_MAX_BYTES, total // 8)
        return self.max_pending_bytes

    def add(self, state, q_post, k_post, v, scaling):
        """Hold one layer's prompt until flush: its keys and values as they
        are, and a copy of the query's window rows (the only query rows the
        scores read)."""
        W = min(state.window_size, int(q_post.shape[2]))
        q_win = q_post[:, :, q_post.shape[2] - W:].contiguous()
        self.pending.append((state, q_win, k_post, v, float(scaling)))
        self.pending_bytes += sum(t.numel() * t.element_size() for t in (q_win, k_post, v))
        state._deferred = self
        if self.pending_bytes > self._limit(k_post.device):
            self.flush()

    def flush(self):
        """Compact every pending layer: per group of layers with one shape and
        knob set, one hot storage for all of them, one copy of every row
        table, and the scoring, top-k and gather launches."""
        pending, self.pending, self.pending_bytes = self.pending, [], 0
        groups = {}
        for item in pending:
            st, q, k, v, sc = item
            key = (k.device, k.dtype, tuple(q.shape), q.stride()[1:], tuple(k.shape), k.stride()[1:],
                   tuple(v.shape), v.stride()[1:], st.window_size, st.kernel_size, st.pooling, st.budget, sc)
            groups.setdefault(key, []).append(item)
        for items in groups.values():
            st0, q0, k0, _, sc = items[0]
            B, Hk, S, D = k0.shape
            window, _, keep_prefix = ops.keep_counts(S, st0.window_size, st0.budget)
            n = keep_prefix + window
            cap = n + st0.decode_reserve
            kst, vst = kv_rows((len(items), B, Hk), cap, D, k0.dtype, k0.device)
            for i, it in enumerate(items):
                it[0].buf = HotBuffer(B, Hk, D, k0.dtype, k0.device, cap, storage=(kst[i], vst[i]))
            qs, ks, vs = [it[1] for it in items], [it[2] for it in items], [it[3] for it in items]
            kd, vd = [it[0].buf.st["k"] for it in items], [it[0].buf.st["v"] for it in items]
            q_t, k_t, v_t, kd_t, vd_t = ops.device_tables(*[ops.row_addresses(x) for x in (qs, ks, vs, kd, vd)],
                                                          device=k0.device)
            scores = ops.snapkv_scores_rows(qs, ks, st0.window_size, sc, st0.kernel_size, st0.pooling,
                                            tables=(q_t, k_t))
            keep = ops.keep_index(scores, st0.window_size, st0.budget)
            ops.gather_rows_tab(keep, ks, vs, kd, vd, dst_row0=0, tables=(k_t, v_t, kd_t, vd_t))
            for it in items:
                it[0].buf.n = n
                it[0]._deferred = None


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
        self._deferred = None   # the DeferredCompaction holding this layer's prompt, until it runs

    def _settle(self):
        """Run this layer's deferred compaction (with every other pending layer)."""
        if self._deferred is not None:
            self._deferred.flush()

    # -- introspection -------------------------------------------------------
    @property
    def keys(self):
        self._settle()
        return None if self.buf is None else self.buf.keys

    @property
    def values(self):
        self._settle()
        return None if self.buf is None else self.buf.values

    @property
    def scores(self):
        """H2O accumulated scores (B,Hk,n) of the resident tokens (None for
        the window methods), as the reference's `scores` attribute."""
        if self.method != "h2o" or self.buf is None or self._h2o is None:
            return None
        return self._h2o[:, :, : self.buf.n]

    def get_seq_length(self) -> int:
        self._settle()
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
    def prefill(self, q_post, k_post, v, n_rep, scaling, deferred=None):
        """Attend over the full prompt, then compress the prompt KV to the budget
        -- or, with a DeferredCompaction, leave the compression to it."""
        out = self._attn(q_post, k_post, v, n_rep, scaling, causal=True)
        self.compact_prompt(q_post, k_post, v, scaling, deferred)
        return out

    def compact_prompt(self, q_post, k_post, v, scaling, deferred=None):
        """The compression half of prefill (layer_state.py:82-94 after the
        attention): score the prompt, keep the budget, gather it into the hot
        buffer.  With a DeferredCompaction (SnapKV / PyramidKV over budget)
        the layer joins it and is compacted when it runs."""
        S = int(k_post.shape[2])
        h2o = self.method == "h2o"
        if deferred is not None and not h2o and S > self.budget:
            self.buf = None
            deferred.add(self, q_post, k_post, v, scaling)
            return
        scores = ops.h2o_prefill_scores(q_post, k_post, scaling) if h2o else None
        if S <= self.budget:
            self._new_buffer(k_post, S)
            self.buf.set_from(k_post, v)
            if h2o:
                self._h2o_storage()
                self._h2o[:, :, :S].copy_(scores)
            return
        if not h2o:
            scores = ops.snapkv_scores(q_post, k_post, self.window_size, scaling, self.kernel_size, self.pooling)
        keep = ops.keep_index(scores, self.window_size, self.budget)
        self._new_buffer(k_post, int(keep.shape[-1]))
        self.buf.gather_from(k_post, v, keep)
        if h2o:
            self._h2o_keep(scores, keep)

    def decode(self, q_post, k_post, v, n_rep, scaling):
        """Single-token decode: append, then attend over the compressed cache
        (one fused launch for one token)."""
        if self._deferred is not None:
            self._deferred.flush()
        buf = self.buf
        if buf is None:
            raise RuntimeError("decode before prefill")
        if self.method != "h2o" and k_post.shape[2] == 1:                   # the per-step call
            return buf.append_attend(q_post, k_post, v, scaling, None, None, True)     # (B,Hq,1,D)
        if self.method == "h2o":
            return self._decode_h2o(q_post, k_post, v, scaling)
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
            # (rows addressed by offset in the two storages: no views per step)
            self.buf.ensure(n)
            self._h2o_storage()
            lo = self.buf.held
            out = ops.decode_h2o_evict_rows(q_post, self.buf.st, lo, n, k_post, v, scaling, self._h2o,
                                            self.window_size, self.budget, self.buf.spare(), self._h2o_spare, lo)
            self.buf.adopt_spare(n - 1)
            self._h2o, self._h2o_spare = self._h2o_spare, self._h2o
            return out  # (B,Hq,1,D)
        self.buf.append(k_post, v)
        self._h2o_storage()
        n = self.buf.n
        out = ops.decode_attention_h2o(q_post, self.buf.keys, self.buf.values, scaling, self._h2o[:, :, :n])
        if n > self.budget:
            keep = ops.keep_index(self._h2o[:, :, :n], self.window_size, self.budget)
            self.buf.compact(keep)
            self._h2o_keep(self._h2o[:, :, :n], keep)
        return out.unsqueeze(2)  # (B,Hq,1,D)
