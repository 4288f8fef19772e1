"""Knobs of the compression baselines (src/hotcold_kv/baselines/config.py:4-48)."""

from dataclasses import dataclass
from typing import Optional


@dataclass
class PressConfig:
    """KV-cache compression settings.

    method: "snapkv" (observation-window importance + pooling, compressed at
        prefill), "pyramidkv" (SnapKV importance, per-layer pyramidal budget)
        or "h2o" (accumulated attention, re-evicted every decode step).
    max_capacity: KV budget per layer including the recent window (the mean
        budget for PyramidKV).
    window_size: observation window; also the recent window that is kept.
    kernel_size, pooling: 1-D pooling of the importance ("maxpool"/"avgpool").
    pyramid_beta: spread of the PyramidKV budgets.
    defer_compaction: compact every layer's prompt together after the last
        layer's prefill, in one launch set, instead of one layer at a time
        (same kept indices; prompt K/V stay alive until then, up to
        defer_max_bytes, by default an eighth of the device's memory and at
        most 16 GiB).  Not a knob of the reference.
    """

    method: str = "snapkv"
    max_capacity: int = 512
    window_size: int = 32
    kernel_size: int = 7
    pooling: str = "maxpool"
    pyramid_beta: int = 20
    num_layers: int = 32
    defer_compaction: bool = True
    defer_max_bytes: Optional[int] = None

    def __post_init__(self):
        assert self.method in ("snapkv", "pyramidkv", "h2o"), f"unknown method {self.method}"
        assert self.pooling in ("maxpool", "avgpool"), f"unknown pooling {self.pooling}"
        assert self.window_size < self.max_capacity, "window_size must be < max_capacity"


def pyramid_layer_budget(layer_idx: int, num_layers: int, max_capacity: int, beta: int) -> int:
    """PyramidKV budget of one layer: linear from 2*max_capacity - max_capacity//beta
    at layer 0 down to max_capacity//beta at the last layer (config.py:39-48)."""
    low = max(1, max_capacity // beta)
    high = max_capacity * 2 - low
    if num_layers <= 1:
        return max_capacity
    step = (high - low) / (num_layers - 1)
    return max(int(round(high - layer_idx * step)), low)
