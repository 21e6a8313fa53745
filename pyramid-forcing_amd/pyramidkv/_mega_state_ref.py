"""Per-head state record types and builders (reference:
pyramidkv/_mega_state_ref.py:24-113, 339-366).

Constants, the dataclass mirror of the 600-byte record and the builders
used to compile a policy.  The state machine itself runs on the GPU
(torch.ops.adahead.mega_state_update); its CPU restatement is test
infrastructure in oracle/ and is not part of this package.
"""
from __future__ import annotations

from dataclasses import dataclass, field

SK_RECENT, SK_CYCLIC, SK_STRIDE, SK_LAG, SK_MERGE = 0, 1, 2, 3, 4
MAX_PHASE, MAX_BUCKET, MAX_T_KEYED, MAX_LAG_OFFSETS = 6, 4, 24, 4
MAX_MERGE_BLOCKS, MAX_MERGE_ACTIVE, MAX_MERGE_BLOCK_FRAMES = 6, 2, 4
DST_KIND_SINK, DST_KIND_MIDDLE, DST_KIND_RECENT, DST_KIND_SKIP, DST_KIND_MERGE_ACCUM = 0, 1, 2, -1, 5


class MergeDuplicateError(ValueError):
    """A merge block saw the same local frame twice (the device skips it)."""


@dataclass
class PerHeadState:
    kind: int = SK_RECENT
    sink_capacity: int = 0
    period: int = 0
    bucket_cap: int = 0
    interval: int = 0
    capacity: int = 0
    patch_size: int = 0
    block_frames: int = 0
    lag_offsets: list = field(default_factory=lambda: [0] * MAX_LAG_OFFSETS)
    lag_offset_count: int = 0
    cyclic_slot: list = field(default_factory=lambda: [-1] * (MAX_PHASE * MAX_BUCKET))
    cyclic_t: list = field(default_factory=lambda: [0] * (MAX_PHASE * MAX_BUCKET))
    cyclic_cursor: list = field(default_factory=lambda: [0] * MAX_PHASE)
    tkey_slot: list = field(default_factory=lambda: [-1] * MAX_T_KEYED)
    tkey_t: list = field(default_factory=lambda: [0] * MAX_T_KEYED)
    tkey_count: int = 0
    tkey_head: int = 0
    merge_completed_slot: list = field(default_factory=lambda: [-1] * MAX_MERGE_BLOCKS)
    merge_completed_block_id: list = field(default_factory=lambda: [-1] * MAX_MERGE_BLOCKS)
    merge_completed_count: int = 0
    merge_active_block_id: list = field(default_factory=lambda: [-1] * MAX_MERGE_ACTIVE)
    merge_active_seen: list = field(
        default_factory=lambda: [[False] * MAX_MERGE_BLOCK_FRAMES for _ in range(MAX_MERGE_ACTIVE)])
    merge_active_complete_count: list = field(default_factory=lambda: [0] * MAX_MERGE_ACTIVE)
    cached_num_groups: int = 0
    # fields of the byte record the reference's dataclass does not carry
    merge_completed_start_t: list = field(default_factory=lambda: [0] * MAX_MERGE_BLOCKS)
    merge_completed_end_t: list = field(default_factory=lambda: [0] * MAX_MERGE_BLOCKS)
    merge_completed_median_t: list = field(default_factory=lambda: [0] * MAX_MERGE_BLOCKS)


def _check(cond, msg):
    if not cond:
        raise ValueError(msg)


def make_cyclic(period: int, bucket_cap: int) -> PerHeadState:
    _check(1 <= period <= MAX_PHASE and 1 <= bucket_cap and period * bucket_cap <= MAX_PHASE * MAX_BUCKET,
           f"cyclic period {period} x bucket_cap {bucket_cap} exceeds the {MAX_PHASE}x{MAX_BUCKET} record")
    return PerHeadState(kind=SK_CYCLIC, period=period, bucket_cap=bucket_cap)


def make_stride(interval: int, capacity: int) -> PerHeadState:
    _check(interval >= 1 and 1 <= capacity <= MAX_T_KEYED, f"stride capacity must be in [1, {MAX_T_KEYED}]")
    return PerHeadState(kind=SK_STRIDE, interval=interval, capacity=capacity)


def make_lag(history_frames: int, offsets=None) -> PerHeadState:
    _check(1 <= history_frames <= MAX_T_KEYED, f"lag history must be in [1, {MAX_T_KEYED}]")
    s = PerHeadState(kind=SK_LAG, capacity=history_frames)
    if offsets is not None:
        for i, off in enumerate(list(offsets)[:MAX_LAG_OFFSETS]):
            s.lag_offsets[i] = off
        s.lag_offset_count = min(len(offsets), MAX_LAG_OFFSETS)
    return s


def make_recent() -> PerHeadState:
    return PerHeadState(kind=SK_RECENT)


def make_merge(patch_size: int = 2, capacity: int = 6) -> PerHeadState:
    _check(1 <= patch_size * patch_size <= MAX_MERGE_BLOCK_FRAMES and 1 <= capacity <= MAX_MERGE_BLOCKS,
           f"merge needs patch_size**2 <= {MAX_MERGE_BLOCK_FRAMES} and capacity in [1, {MAX_MERGE_BLOCKS}]")
    return PerHeadState(kind=SK_MERGE, patch_size=patch_size, capacity=capacity, block_frames=patch_size * patch_size)
