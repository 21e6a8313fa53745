"""Heads with no middle anchors: sink + recent only (reference: pyramidkv/recent.py:12)."""
from __future__ import annotations

from . import _mega_state_ref as ref
from .base import MiddleStrategy


class RecentStrategy(MiddleStrategy):
    def __init__(self):
        self.dynamic_rope = False

    def state_record(self) -> ref.PerHeadState:
        """Sink + recent only: no middle segments."""
        return ref.make_recent()
