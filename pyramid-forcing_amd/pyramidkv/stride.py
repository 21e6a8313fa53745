"""Anchor heads: strided windows (reference parameters: pyramidkv/stride.py:27-30).

Frames with t % interval == 0 enter a FIFO of ``capacity`` frames (a
negative capacity is resolved by the composition builder).  The device
state machine (``update_stride``) keeps the FIFO in the per-head state
record."""
from __future__ import annotations

from .base import MiddleStrategy


class StrideStrategy(MiddleStrategy):
    def __init__(self, interval: int = 6, capacity: int = -1, dynamic_rope: bool = True):
        self.interval = max(1, int(interval))
        self.capacity = int(capacity)
        self.dynamic_rope = bool(dynamic_rope)
