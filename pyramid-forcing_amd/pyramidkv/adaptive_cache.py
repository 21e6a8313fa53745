"""``AdaptiveKVCache``: the name of the reference's per-head strategy cache
(reference: pyramidkv/adaptive_cache.py:85), imported by
pipeline/causal_inference.py:7 for ``isinstance`` dispatch.  Constructing
it raises the ``PyramidKVCache`` out-of-scope error; the cache of this
build is the MegaCache path."""
from __future__ import annotations

from .cache import PyramidKVCache


class AdaptiveKVCache(PyramidKVCache):
    pass
