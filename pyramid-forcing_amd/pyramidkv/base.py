"""Head compositions and middle-strategy parameter records.

``HeadComposition`` mirrors the reference's per-head record
(pyramidkv/base.py:79-110): sink frames + middle strategies + recent
frames.  The strategy classes carry the parameters the device path encodes
into the per-head state record (pyramidkv/cyclic.py:25-28, stride.py:27-30,
lag.py:25-33, merge.py:44-48, recent.py:12); the reference's Python-side
per-frame update/collect of the non-MegaCache cache is not part of this
package.
"""
from __future__ import annotations


class MiddleStrategy:
    dynamic_rope: bool = True


class CyclicStrategy(MiddleStrategy):
    """Wave: periodic sampling, one ring of ``bucket_cap`` frames per phase."""

    def __init__(self, period: int = 6, bucket_cap: int = 1, dynamic_rope: bool = True):
        self.period = max(1, int(period))
        self.bucket_cap = max(1, int(bucket_cap))
        self.dynamic_rope = bool(dynamic_rope)


class StrideStrategy(MiddleStrategy):
    """Anchor: keep frames with t % interval == 0 in a FIFO of ``capacity``."""

    def __init__(self, interval: int = 6, capacity: int = -1, dynamic_rope: bool = True):
        self.interval = max(1, int(interval))
        self.capacity = int(capacity)
        self.dynamic_rope = bool(dynamic_rope)


class LagStrategy(MiddleStrategy):
    def __init__(self, offsets: list[int] | None = None, history_frames: int = 21, dynamic_rope: bool = False):
        raw = offsets if offsets is not None else [6]
        self.offsets = sorted(set(o for o in raw if o > 0))
        self.history_frames = max(1, int(history_frames))
        self.dynamic_rope = bool(dynamic_rope)


class MergeStrategy(MiddleStrategy):
    """Veil: fold blocks of patch_size**2 frames into patch x patch means."""

    def __init__(self, patch_size: int = 2, capacity: int = 1, dynamic_rope: bool = True):
        self.patch_size = max(1, int(patch_size))
        self.capacity = -1 if int(capacity) < 0 else max(1, int(capacity))
        self.dynamic_rope = bool(dynamic_rope)
        self.block_frames = self.patch_size * self.patch_size


class RecentStrategy(MiddleStrategy):
    """No middle anchors: sink + recent only."""

    def __init__(self):
        self.dynamic_rope = False


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
