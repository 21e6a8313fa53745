"""Heads with no middle anchors: sink + recent only (reference: pyramidkv/recent.py:12)."""
from __future__ import annotations

from .base import MiddleStrategy


class RecentStrategy(MiddleStrategy):
    def __init__(self):
        self.dynamic_rope = False
