"""HotColdLayer: the hot tier as a transformers cache layer
(src/hotcold_kv/cache.py:12-173).

The layer keeps post-RoPE keys, values, pre-RoPE keys and absolute positions
in a fixed-capacity HotBuffer whose first lookahead_k rows are the held
retrieved slot.  When the resident length exceeds max_capacity_prompt it is
compressed like cache.py:37-128: the last min(recent, stashed) post-RoPE
queries score every key (raw q.k/sqrt(D) summed over the queries, mean over
KV heads), the top int(max_capacity_prompt * topk_ratio) prefix tokens plus
the recent window are kept (one index set for every head, ties to the lower
index), and the evicted prefix tokens go to the cold store as fp32 copies
staged through reusable pinned memory.  Scoring, selection, the gathers and
the eviction gather (with its fp32 upcast) run on the gfx950 kernels.

get_seq_length() reports the number of tokens processed (the absolute
position of the next token) so that transformers' default position ids stay
absolute after compression; hot_length() is the resident length.
"""

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from . import ops
from .controller import KVController
from .datatypes import EvictedKV
from .hot_buffer import HotBuffer


class HotColdLayer(CacheLayerMixin):
    is_compileable = False

    def __init__(self, kvctrl: KVController, decode_reserve: int = 256):
        super().__init__()
        self.kvctrl = kvctrl
        self.decode_reserve = int(decode_reserve)
        self.buf = None
        self.seen_tokens = 0
        self.is_initialized = False
        self._last_q_post = None

    # -- tensors of the reference's layout ----------------------------------------------
    @property
    def keys(self):
        return None if self.buf is None else self.buf.keys

    @keys.setter
    def keys(self, value):  # CacheLayerMixin.__init__ assigns None
        if value is not None:
            raise AttributeError("HotColdLayer.keys is a view of the hot buffer")

    @property
    def values(self):
        return None if self.buf is None else self.buf.values

    @values.setter
    def values(self, value):
        if value is not None:
            raise AttributeError("HotColdLayer.values is a view of the hot buffer")

    @property
    def pre_keys(self):
        return None if self.buf is None else self.buf.pre_keys

    @property
    def positions(self):
        return None if self.buf is None else self.buf.positions

    def set_last_query_post(self, q_post):
        self._last_q_post = q_post

    def hot_length(self) -> int:
        return 0 if self.buf is None else self.buf.n

    # -- lifecycle -------------------------------------------------------------------------
    def lazy_initialization(self, key_states, value_states=None):
        B, Hk, T, D = key_states.shape
        held = max(0, self.kvctrl.lookahead_k)
        # the resident length is T after the first update and at most
        # max(max_capacity_prompt, T) + steps later; HotBuffer grows on demand
        cap = T + self.decode_reserve
        self.buf = HotBuffer(B, Hk, D, key_states.dtype, key_states.device, cap, held=held, with_pre=True,
                             with_pos=True)
        self.is_initialized = True

    def update(self, key_states=None, value_states=None, *args, layer_idx=None, cache_kwargs=None, **kwargs):
        """Append this step's tokens and compress if over capacity.  Accepts the
        reference's keyword form update(layer_idx=, key_states=, value_states=,
        cache_kwargs={"pre_key_states", "positions", ...}) (cache.py:130)."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        pre_k = pos = None
        if cache_kwargs is not None:
            pre_k = cache_kwargs.get("pre_key_states")
            pos = cache_kwargs.get("positions")
        B, Hk, T, D = key_states.shape
        if pre_k is None or pos is None:
            pre_k = torch.zeros_like(key_states)
            pos = torch.zeros((B, T), device=key_states.device, dtype=torch.long)
        self.buf.append(key_states, value_states, pre_k.to(key_states.dtype), pos.to(torch.long))
        self.seen_tokens += T
        self._compress_if_needed(layer_idx if layer_idx is not None else 0)
        return self.buf.keys, self.buf.values

    # -- one-token decode: append and attend in one launch -------------------------------------
    def decode_fusable(self) -> bool:
        """True when this step's one-token append cannot trigger a compression
        (cache.py:44): the append can then run inside the decode launch."""
        return self.buf is not None and (self._last_q_post is None
                                         or self.buf.n + 1 <= self.kvctrl.max_capacity_prompt)

    def append_attend(self, q_post, k_post, v, k_pre, positions, scaling, held=None):
        """update() of one token (cache.py:130-151) fused with the decode
        attention over [held slot | hot rows | the token] (patch.py:241-305):
        one launch writes the token's post-RoPE key, value, pre-RoPE key and
        position into the next hot row and attends.  held = (pos, valid, R)
        of the held retrieved slot, or None.  Returns (B,Hq,1,D)."""
        buf = self.buf
        if positions.shape[-1] != 1:
            raise RuntimeError("HotColdLayer.append_attend: one token per step, positions (B,1)")
        n = buf.n + 1
        if n > buf.cap:
            buf.ensure(n)
        R = int(held[2]) if held is not None else 0
        # one-token step: positions is (B,1), so its first element is the
        # current position the held-slot mask compares against
        if R:
            out = ops.decode_append_rows(q_post, buf.st, buf.held - R, R + n, k_post, v, scaling, k_pre, positions,
                                         held, positions, True)
        else:
            out = ops.decode_append_rows(q_post, buf.st, buf.held, n, k_post, v, scaling, k_pre, positions, None,
                                         None, True)
        buf.n = n
        self.seen_tokens += 1
        return out

    # -- compression (cache.py:37-128) ------------------------------------------------------
    def _compress_if_needed(self, layer_idx):
        ctrl = self.kvctrl
        if self._last_q_post is None or self.buf is None:
            return
        S = self.buf.n
        if S <= ctrl.max_capacity_prompt:
            return
        recent = min(ctrl.recent_size, ctrl.max_capacity_prompt, S)
        prefix = S - recent
        if prefix <= 0:
            return
        topk = max(1, min(int(ctrl.max_capacity_prompt * ctrl.topk_ratio), prefix))
        q = self._last_q_post
        tq = min(recent, int(q.shape[2]))
        per_head = ops.snapkv_scores(q[:, :, -tq:, :], self.buf.keys, tq, 0.0, mode="rawsum")
        scores = ops.head_mean(per_head)                                   # (B,S)
        keep, evicted = ops.keep_index(scores, recent, topk + recent, return_evicted=True)
        if evicted.shape[-1] > 0:
            self._evict(layer_idx, evicted)
        self.buf.compact(keep)

    def _evict(self, layer_idx, evicted):
        """Gather the evicted prefix tokens' pre-RoPE keys, values (upcast to
        fp32) and positions in one kernel, copy the packed block to reusable
        pinned host memory in one hipMemcpyAsync, and hand it to the cold
        store (cache.py:86-125)."""
        ctrl = self.kvctrl
        B, Hk, D = self.buf.B, self.buf.H, self.buf.D
        te = int(evicted.shape[-1])
        stage = ctrl.evict_stage(self.buf.keys.device, B, Hk, te, D)
        kp_cpu, v_cpu, pos_cpu = ops.gather_evict(evicted, self.buf.pre_keys, self.buf.values, self.buf.positions,
                                                  dev_out=stage.dev, host_out=stage.host)
        idx_cpu = evicted.to("cpu")  # synchronising copy: the staged block is complete after it
        ctrl.dbg["compress_calls"] += 1
        ctrl.dbg["evicted_tokens"] += int(B * te)
        # the cold store copies the tokens on the library's worker threads while
        # the prefill goes on; the stage is reused once those adds are done
        ctrl.add_evicted_to_cold_store(layer_idx, EvictedKV(k_pre_cpu=kp_cpu, v_cpu=v_cpu, pos_cpu=pos_cpu,
                                                            evicted_idx=idx_cpu), stage=stage)

    # -- transformers cache interface -------------------------------------------------------
    def get_mask_sizes(self, query_length):
        q = query_length if isinstance(query_length, int) else int(query_length.shape[0])
        return self.seen_tokens + q, 0

    def get_seq_length(self) -> int:
        return self.seen_tokens

    def get_max_length(self) -> int:
        return int(self.kvctrl.max_capacity_prompt)

    def get_max_cache_shape(self) -> int:
        return int(self.kvctrl.max_capacity_prompt)


def build_hotcold_cache(model, kvctrl: KVController) -> Cache:
    n_layers = int(model.config.num_hidden_layers)
    return Cache(layers=[HotColdLayer(kvctrl) for _ in range(n_layers)])
