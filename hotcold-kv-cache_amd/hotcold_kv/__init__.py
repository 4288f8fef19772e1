"""hotcold_kv on MI355X: the GPU hot tier of hotcold-kv-cache as gfx950 HIP
kernels behind the reference package's API."""

from . import ops  # noqa: F401

__all__ = ["ops"]
