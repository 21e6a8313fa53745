"""``PyramidKVCache``: the name the reference's model and pipeline import
(wan/modules/causal_model.py:2, pipeline/causal_inference.py:7) for its
Python sliding-window cache (reference: pyramidkv/cache.py:7-232).

This package implements the MegaCache path (``_mega_cache.build_mega_caches``,
the reference's ``PYRAMIDKV_USE_MEGA_CACHE=1`` branch at
pipeline/causal_inference.py:764-803).  The Python-side caches are outside
it: the class exists so that imports and ``isinstance`` checks in the
caller resolve, and constructing one raises ``NotImplementedError`` naming
the path to use instead.
"""
from __future__ import annotations

_OUT_OF_SCOPE = ("{name} (the reference's Python-side per-head cache) is not part of this MI355X build; "
                 "use pyramidkv._mega_cache.build_mega_caches (the MegaCache path, "
                 "PYRAMIDKV_USE_MEGA_CACHE=1 in the reference's pipeline).")


class PyramidKVCache:
    def __init__(self, *args, **kwargs):
        raise NotImplementedError(_OUT_OF_SCOPE.format(name=type(self).__name__))
