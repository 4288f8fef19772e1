"""hotcold-kv-cache on MI355X: the GPU hot tier of the two-tier (GPU hot /
CPU cold) KV cache as hand-written gfx950 HIP kernels, behind the reference
package's API (src/hotcold_kv/__init__.py)."""

from .datatypes import RetrievedKV, EvictedKV
from .kernels import triton_evict_attention_forward, decode_attention_forward
from .controller import KVController
from .cache import HotColdLayer, build_hotcold_cache
from .patch import (
    set_active_kvctrl,
    set_active_rotary_emb,
    install_monkeypatch,
    uninstall_monkeypatch,
)
from . import ops

__all__ = [
    "RetrievedKV",
    "EvictedKV",
    "triton_evict_attention_forward",
    "decode_attention_forward",
    "KVController",
    "HotColdLayer",
    "build_hotcold_cache",
    "set_active_kvctrl",
    "set_active_rotary_emb",
    "install_monkeypatch",
    "uninstall_monkeypatch",
    "ops",
]
