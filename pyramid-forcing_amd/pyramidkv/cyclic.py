"""Wave heads: periodic sampling (reference parameters: pyramidkv/cyclic.py:25-28).

Frame t falls in phase t % period; each phase keeps a ring of
``bucket_cap`` frames.  The device state machine (``update_cyclic``) keeps
the ring in the per-head state record."""
from __future__ import annotations

from . import _mega_state_ref as ref
from .base import MiddleStrategy


class CyclicStrategy(MiddleStrategy):
    def __init__(self, period: int = 6, bucket_cap: int = 1, dynamic_rope: bool = True):
        self.period = max(1, int(period))
        self.bucket_cap = max(1, int(bucket_cap))
        self.dynamic_rope = bool(dynamic_rope)

    def state_record(self) -> ref.PerHeadState:
        """Wave record: the phase ring of period x bucket_cap slots (at most
        MAX_PHASE x MAX_BUCKET); slot i of phase q is middle slot q * MAX_BUCKET + i."""
        return ref.make_cyclic(int(self.period), int(self.bucket_cap))
