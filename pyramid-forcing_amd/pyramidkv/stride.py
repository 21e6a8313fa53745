"""Anchor heads: strided windows (reference parameters: pyramidkv/stride.py:27-30).

Frames with t % interval == 0 enter a FIFO of ``capacity`` frames (a
capacity <= 0 means unbounded: the state record keeps its MAX_T_KEYED
frames).  The device state machine (``update_stride``) keeps the FIFO in
the per-head state record."""
from __future__ import annotations

from . import _mega_state_ref as ref
from .base import MiddleStrategy


class StrideStrategy(MiddleStrategy):
    def __init__(self, interval: int = 6, capacity: int = -1, dynamic_rope: bool = True):
        self.interval = max(1, int(interval))
        self.capacity = int(capacity)
        self.dynamic_rope = bool(dynamic_rope)

    def state_record(self) -> ref.PerHeadState:
        """Anchor record: an unbounded (<= 0) or oversized capacity becomes the
        record's MAX_T_KEYED-entry FIFO (the reference's rule); the FIFO's
        eviction handles the rest at run time."""
        cap = int(self.capacity)
        if cap <= 0 or cap > ref.MAX_T_KEYED:
            cap = ref.MAX_T_KEYED
        return ref.make_stride(int(self.interval), cap)
