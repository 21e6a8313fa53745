"""Fixed-lag anchors (reference parameters: pyramidkv/lag.py:25-33).

Every frame enters a FIFO of ``history_frames``; ``offsets`` (positive,
de-duplicated, sorted) are carried for the record but the planner does not
read them (mega_plan.cc emits the whole FIFO)."""
from __future__ import annotations

from .base import MiddleStrategy


class LagStrategy(MiddleStrategy):
    def __init__(self, offsets: list[int] | None = None, history_frames: int = 21, dynamic_rope: bool = False):
        self.offsets = sorted({int(o) for o in (offsets if offsets is not None else [6]) if int(o) > 0})
        self.history_frames = max(1, int(history_frames))
        self.dynamic_rope = bool(dynamic_rope)
