"""MI355X (gfx950) implementation of Pyramid Forcing's per-step pyramid
KV-cache path behind the reference's ``pyramidkv`` API.

The exported names are the reference package's (pyramidkv/__init__.py:16-46).
Importing the package needs no GPU and does not load the native library;
the ops load it on first use (``_ops.ops()``) and raise when it is missing.
"""
from .base import FrameAnchor, HeadComposition, MiddleStrategy
from .cyclic import CyclicStrategy
from .lag import LagStrategy
from .stride import StrideStrategy
from .merge import MergeStrategy
from .recent import RecentStrategy
from .factory import HEAD_LABEL_MAP, build_compositions, load_head_labels
from .config import PyramidKVConfig
from .cache import PyramidKVCache
from .adaptive_cache import AdaptiveKVCache

__all__ = [
    "FrameAnchor", "HeadComposition", "MiddleStrategy", "CyclicStrategy", "LagStrategy", "StrideStrategy",
    "MergeStrategy", "RecentStrategy", "HEAD_LABEL_MAP", "build_compositions", "load_head_labels",
    "PyramidKVConfig", "PyramidKVCache", "AdaptiveKVCache",
]
