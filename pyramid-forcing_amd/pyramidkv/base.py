"""Per-head cache composition records.

``HeadComposition`` is the reference's per-head record (pyramidkv/base.py:79-110):
sink frames, a union of middle strategies and recent frames.  The middle
strategies (cyclic.py, stride.py, lag.py, merge.py, recent.py) are
parameter records: the device path encodes them into the 600-byte per-head
state record, and the state machine on the GPU does the per-frame work the
reference's Python strategy objects do in its AdaptiveKVCache path.
``FrameAnchor`` is the reference's raw-anchor payload type
(pyramidkv/base.py:16-23), kept for callers that construct or annotate with it.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class FrameAnchor:
    """One stored frame: raw K, V, positions and its latent time t."""

    k: torch.Tensor
    v: torch.Tensor
    pos: torch.Tensor
    t: int


class MiddleStrategy:
    """Base of the middle-segment parameter records.  ``dynamic_rope``: the
    frames' temporal RoPE index is remapped at readout.

    ``state_record()`` encodes the strategy into the per-head state record
    that the device state machine and planner read (the reference's
    _mega_cache.py:572-628 translation, one strategy kind per head); it
    raises ValueError when the parameters do not fit the record's bounds."""

    dynamic_rope: bool = True

    def state_record(self):
        raise NotImplementedError(f"{type(self).__name__} has no state-record encoding")


class HeadComposition:
    def __init__(self, name: str, label: int, sink_frames: int, recent_frames: int,
                 middle_strategies: list | None = None, policy_type: str = "osc", capacity: int = 32768):
        self.name = name
        self.label = label
        self.sink_frames = max(0, int(sink_frames))
        self.recent_frames = max(1, int(recent_frames))
        self.middle_strategies = middle_strategies or []
        self.policy_type = policy_type
        self.capacity = int(capacity)

    @property
    def has_middle(self) -> bool:
        return len(self.middle_strategies) > 0

    def __repr__(self) -> str:
        return (f"<HeadComposition {self.name} label={self.label} "
                f"middle={[type(s).__name__ for s in self.middle_strategies]}>")
