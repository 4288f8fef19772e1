"""KV-cache compression baselines on the MI355X hot tier: SnapKV and PyramidKV
(src/hotcold_kv/baselines/__init__.py).  Each is a prompt compressor exposed
as a transformers Cache plus an attention monkeypatch."""

from .config import PressConfig, pyramid_layer_budget
from .layer_state import PressLayerState
from .cache import PressCacheLayer, build_press_cache
from .patch import set_active_press_cache, install_press_patch, uninstall_press_patch

__all__ = [
    "PressConfig",
    "pyramid_layer_budget",
    "PressLayerState",
    "PressCacheLayer",
    "build_press_cache",
    "set_active_press_cache",
    "install_press_patch",
    "uninstall_press_patch",
]
