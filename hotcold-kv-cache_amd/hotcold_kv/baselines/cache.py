"""HuggingFace cache layers for the compression baselines
(src/hotcold_kv/baselines/cache.py:12-71), written against the installed
transformers CacheLayerMixin (lazy_initialization(key, value),
get_mask_sizes(query_length), get_max_length).

get_seq_length() reports the number of tokens the layer has processed (the
absolute position of the next token), so transformers' default position ids
stay absolute after compression; the physical hot length is
state.get_seq_length().
"""

from transformers.cache_utils import Cache, CacheLayerMixin

from .config import PressConfig, pyramid_layer_budget
from .layer_state import DeferredCompaction, PressLayerState


class PressCacheLayer(CacheLayerMixin):
    """A cache layer backed by a PressLayerState; the patched attention drives
    prefill/decode directly, this class carries the bookkeeping."""

    is_compileable = False

    def __init__(self, cfg: PressConfig, layer_idx: int, deferred: DeferredCompaction = None):
        super().__init__()
        self.cfg = cfg
        self.layer_idx = layer_idx
        self.deferred = deferred
        if cfg.method == "pyramidkv":
            budget = pyramid_layer_budget(layer_idx, cfg.num_layers, cfg.max_capacity, cfg.pyramid_beta)
        else:
            budget = cfg.max_capacity
        self.budget = budget
        self.state = PressLayerState(method=cfg.method, budget=budget, window_size=cfg.window_size,
                                     kernel_size=cfg.kernel_size, pooling=cfg.pooling)
        self.seen_tokens = 0

    def prefill(self, q_post, k_post, v, n_rep, scaling):
        out = self.state.prefill(q_post, k_post, v, n_rep, scaling, deferred=self.deferred)
        self.seen_tokens = int(k_post.shape[2])
        self.is_initialized = True
        if self.deferred is not None and self.layer_idx == self.cfg.num_layers - 1:
            self.deferred.flush()   # the prompt has passed every layer
        return out

    def decode(self, q_post, k_post, v, n_rep, scaling):
        out = self.state.decode(q_post, k_post, v, n_rep, scaling)
        self.seen_tokens += int(k_post.shape[2])
        return out

    # -- transformers cache interface --------------------------------------------
    def lazy_initialization(self, key_states, value_states=None):
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        return self.state.keys, self.state.values

    def get_seq_length(self) -> int:
        return self.seen_tokens

    def get_mask_sizes(self, query_length):
        q = query_length if isinstance(query_length, int) else int(query_length.shape[0])
        return self.seen_tokens + q, 0

    def get_max_length(self) -> int:
        return int(self.budget)

    def get_max_cache_shape(self) -> int:
        return int(self.budget)


def build_press_cache(model, cfg: PressConfig) -> Cache:
    """One PressCacheLayer per decoder layer.  With cfg.defer_compaction the
    layers' prompt compactions run together after the last layer's prefill
    (DeferredCompaction), with the same kept indices."""
    n_layers = int(model.config.num_hidden_layers)
    cfg.num_layers = n_layers
    deferred = DeferredCompaction(cfg.defer_max_bytes) if cfg.defer_compaction else None
    return Cache(layers=[PressCacheLayer(cfg, layer_idx=i, deferred=deferred) for i in range(n_layers)])
