"""Veil heads: spatiotemporal merging (reference parameters: pyramidkv/merge.py:44-48).

Blocks of patch_size**2 consecutive frames are folded into one anchor of
patch x patch spatial means; ``capacity`` finalized anchors are kept (-1:
the builder's default).  The accumulation runs on the device
(``merge_accum_kernel``)."""
from __future__ import annotations

from . import _mega_state_ref as ref
from .base import MiddleStrategy


class MergeStrategy(MiddleStrategy):
    def __init__(self, patch_size: int = 2, capacity: int = 1, dynamic_rope: bool = True):
        self.patch_size = max(1, int(patch_size))
        self.capacity = -1 if int(capacity) < 0 else max(1, int(capacity))
        self.dynamic_rope = bool(dynamic_rope)

    @property
    def block_frames(self) -> int:
        return self.patch_size * self.patch_size

    def state_record(self) -> ref.PerHeadState:
        """Veil record: blocks of patch_size**2 frames (at most
        MAX_MERGE_BLOCK_FRAMES), capacity finalized anchors (1 to
        MAX_MERGE_BLOCKS; the builder's -1 is rejected, as in the reference)."""
        return ref.make_merge(int(getattr(self, "patch_size", 2)), int(getattr(self, "capacity", ref.MAX_MERGE_BLOCKS)))
