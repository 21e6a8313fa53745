"""Fixed-lag anchors (reference parameters: pyramidkv/lag.py:25-33).

Every frame enters a FIFO of ``history_frames``; ``offsets`` (positive,
de-duplicated, sorted) are carried for the record but the planner does not
read them (mega_plan.cc emits the whole FIFO)."""
from __future__ import annotations

from . import _mega_state_ref as ref
from .base import MiddleStrategy


class LagStrategy(MiddleStrategy):
    def __init__(self, offsets: list[int] | None = None, history_frames: int = 21, dynamic_rope: bool = False):
        self.offsets = sorted({int(o) for o in (offsets if offsets is not None else [6]) if int(o) > 0})
        self.history_frames = max(1, int(history_frames))
        self.dynamic_rope = bool(dynamic_rope)

    def state_record(self) -> ref.PerHeadState:
        """Lag record: a FIFO of min(history_frames, MAX_T_KEYED) frames and up
        to MAX_LAG_OFFSETS offsets."""
        hist = min(int(getattr(self, "history_frames", ref.MAX_T_KEYED)), ref.MAX_T_KEYED)
        return ref.make_lag(hist, list(getattr(self, "offsets", []) or []))
