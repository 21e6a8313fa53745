"""Label matrix -> per-head compositions (the policy compiler).

Restates pyramidkv/factory.py:105-407 of the reference: each CSV label
(-1 Wave / oscillating, 1 Anchor / stable, 2 Veil / stable_sparse) is
resolved through the per-label maps into sink frames, recent frames and at
most one middle strategy.  ``PYRAMID_FORCING_POLICY`` holds the shipped
inference policy (configs/pyramid-forcing.yaml:84-139 of the reference) and
``SHIPPED_LABELS_CSV`` the shipped 30x12 label matrix.
"""
from __future__ import annotations

import csv
import os
from collections.abc import Mapping, Sequence

from .base import HeadComposition
from .cyclic import CyclicStrategy
from .lag import LagStrategy
from .merge import MergeStrategy
from .stride import StrideStrategy

HEAD_LABEL_MAP = {-1: "oscillating", 1: "stable", 2: "stable_sparse"}

SHIPPED_LABELS_CSV = os.path.join(os.path.dirname(os.path.abspath(__file__)), "configs", "best_labels.csv")

PYRAMID_FORCING_POLICY = dict(
    cyclic_enabled=True, cyclic_period=6, cyclic_bucket_cap=4, cyclic_osc_only=True, cyclic_dynamic_rope=True,
    stride_enabled=True, stride_interval=6, stride_capacity=4, stride_dynamic_rope=True,
    merge_enabled=True, merge_patch_size=2, merge_capacity=4, merge_dynamic_rope=True,
    lag_enabled=False, lag_offsets=[], lag_history=21, lag_dynamic_rope=False,
    osc_sink_frames=1, stable_sink_frames=3, recent_frames=4, stable_recent_frames=4,
    label_phase_bucket_map={"-1": 4, "1": 0, "2": 0},
    label_stride_enabled_map={"1": True, "2": False},
    label_stride_interval_map={"1": 6},
    label_merge_enabled_map={"-1": False, "1": False, "2": True},
    label_merge_patch_size_map={"2": 2},
    label_merge_capacity_map={"2": 4},
    label_sink_frames_map={"-1": 1, "1": 3, "2": 3},
    label_recent_frames_map={"-1": 4, "1": 4, "2": 4},
)

# dynamic-RoPE remap of the shipped policy (configs/pyramid-forcing.yaml:73-79)
PYRAMID_FORCING_REMAP = dict(sink_time_mapping_mode="window_clamp", sink_time_clamp_min=18, sink_time_clamp_max=21,
                             decoupled_sink_time_lag=0, history_time_mapping_mode="none",
                             history_relative_t_max=21, history_time_soft_factor=1.0)


def _key(k) -> str:
    raw = str(k).strip()
    if not raw:
        return ""
    try:
        return str(int(raw))
    except (TypeError, ValueError):
        return raw


def _items(m):
    return m.items() if isinstance(m, Mapping) else ()


def _int_map(m, min_value: int) -> dict[str, int]:
    out = {}
    for k, v in _items(m):
        n = _key(k)
        if not n:
            continue
        try:
            out[n] = max(min_value, int(v))
        except (TypeError, ValueError):
            continue
    return out


def _capacity_map(m) -> dict[str, int]:
    out = {}
    for k, v in _items(m):
        n = _key(k)
        if not n:
            continue
        try:
            p = int(v)
        except (TypeError, ValueError):
            continue
        out[n] = -1 if p < 0 else max(1, p)
    return out


def _bool_map(m) -> dict[str, bool]:
    return {_key(k): bool(v) for k, v in _items(m) if _key(k)}


def _offsets_map(m) -> dict[str, list[int]]:
    out = {}
    for k, v in _items(m):
        n = _key(k)
        if not n:
            continue
        vals = list(v) if isinstance(v, Sequence) and not isinstance(v, (str, bytes)) else [v]
        offs = []
        for x in vals:
            try:
                o = int(x)
            except (TypeError, ValueError):
                continue
            if o > 0:
                offs.append(o)
        out[n] = sorted(set(offs))
    return out


def load_head_labels(csv_path: str, num_layers: int, num_heads: int) -> list[list[int]]:
    """Rows = layers, columns = heads; missing entries default to 1."""
    labels = [[1] * num_heads for _ in range(num_layers)]
    if not csv_path or not os.path.exists(csv_path):
        return labels
    with open(csv_path, encoding="utf-8") as f:
        rows = [r for r in csv.reader(f) if r]
    for li in range(min(num_layers, len(rows))):
        for hi in range(min(num_heads, len(rows[li]))):
            try:
                labels[li][hi] = int(str(rows[li][hi]).strip())
            except ValueError:
                continue
    return labels


def build_compositions(num_layers: int, num_heads: int, capacities=None, csv_path: str | None = None, *,
                       cyclic_enabled=False, cyclic_period=6, cyclic_bucket_cap=1, cyclic_dynamic_rope=True,
                       cyclic_osc_only=True, lag_enabled=False, lag_offsets=None, lag_history=21,
                       lag_dynamic_rope=False, stride_enabled=False, stride_interval=6, stride_capacity=-1,
                       stride_dynamic_rope=True, merge_enabled=False, merge_patch_size=2, merge_capacity=1,
                       merge_dynamic_rope=True, osc_sink_frames=None, stable_sink_frames=None, recent_frames=4,
                       stable_recent_frames=None, label_sink_frames_map=None, label_recent_frames_map=None,
                       label_stride_enabled_map=None, label_stride_interval_map=None, label_phase_bucket_map=None,
                       label_lag_offsets_map=None, label_merge_enabled_map=None, label_merge_patch_size_map=None,
                       label_merge_capacity_map=None, labels=None) -> list[list[HeadComposition]]:
    """[layer][head] compositions (reference factory.py:220-407).  ``labels``
    may be given directly instead of ``csv_path``."""
    if labels is None:
        labels = load_head_labels(csv_path, num_layers, num_heads) if csv_path else [
            [1] * num_heads for _ in range(num_layers)]
    sink_map = _int_map(label_sink_frames_map, 1)
    recent_map = _int_map(label_recent_frames_map, 1)
    stride_map = _bool_map(label_stride_enabled_map)
    interval_map = _int_map(label_stride_interval_map, 1)
    phase_map = _int_map(label_phase_bucket_map, 0)
    lag_map = _offsets_map(label_lag_offsets_map)
    merge_map = _bool_map(label_merge_enabled_map)
    patch_map = _int_map(label_merge_patch_size_map, 1)
    mcap_map = _capacity_map(label_merge_capacity_map)
    out = []
    for li in range(num_layers):
        row = []
        for hi in range(num_heads):
            label = int(labels[li][hi])
            key = _key(label)
            cap = 32760 if capacities is None else int(capacities[li][hi])
            is_osc = label == -1
            policy = "osc" if is_osc else ("recent_only" if label == 2 else "stride")
            if key in sink_map:
                sink = sink_map[key]
            elif is_osc:
                sink = osc_sink_frames if osc_sink_frames is not None else 1
            else:
                sink = stable_sink_frames if stable_sink_frames is not None else 1
            recent = recent_map.get(key, recent_frames)
            if key not in recent_map and not is_osc and stable_recent_frames is not None:
                recent = stable_recent_frames
            # cyclic (factory.py:138-159)
            use_cyclic, bcap = False, 0
            if cyclic_enabled:
                if key in phase_map:
                    bcap = phase_map[key]
                    use_cyclic = bcap > 0
                elif cyclic_osc_only and not is_osc:
                    use_cyclic = False
                else:
                    raise ValueError(f"Missing explicit cyclic resolution for label {key}: "
                                     "set pyramidkv_label_phase_bucket_map to 0 or a positive capacity.")
            # lag (factory.py:162-182)
            head_lag = []
            if lag_enabled:
                if key in lag_map:
                    head_lag = lag_map[key]
                elif cyclic_osc_only and not is_osc:
                    head_lag = []
                elif lag_offsets and (is_osc or not cyclic_osc_only):
                    raise ValueError(f"Missing explicit lag resolution for label {key}: "
                                     "set pyramidkv_label_lag_offsets_map to [] or a non-empty list.")
                else:
                    head_lag = list(lag_offsets or [])
            # stride (factory.py:185-201)
            use_stride = False
            if not is_osc:
                if key in stride_map:
                    use_stride = stride_map[key]
                elif stride_enabled:
                    raise ValueError(f"Missing explicit stride resolution for label {key}: "
                                     "set pyramidkv_label_stride_enabled_map to true or false.")
            # merge (factory.py:204-217)
            if key in merge_map:
                use_merge = merge_map[key]
            elif merge_enabled:
                raise ValueError(f"Missing explicit merge resolution for label {key}: "
                                 "set pyramidkv_label_merge_enabled_map to true or false.")
            else:
                use_merge = False
            active = [n for n, on in (("cyclic", use_cyclic), ("stride", use_stride), ("merge", use_merge)) if on]
            if len(active) > 1:
                raise ValueError(f"Middle strategies must be mutually exclusive for label {key}, got {active}.")
            strategies = []
            if use_cyclic:
                strategies.append(CyclicStrategy(cyclic_period, bcap, cyclic_dynamic_rope))
                policy = "osc"
            if lag_enabled and head_lag:
                strategies.append(LagStrategy(head_lag, lag_history, lag_dynamic_rope))
            if use_stride:
                if key not in interval_map and stride_interval <= 0:
                    raise ValueError(f"Invalid stride interval for label {key}.")
                strategies.append(StrideStrategy(interval_map.get(key, stride_interval), stride_capacity,
                                                 stride_dynamic_rope))
                policy = "stride"
            if use_merge:
                if key not in patch_map:
                    raise ValueError(f"Missing explicit merge patch size for label {key}: "
                                     "set pyramidkv_label_merge_patch_size_map.")
                if key not in mcap_map:
                    raise ValueError(f"Missing explicit merge capacity for label {key}: "
                                     "set pyramidkv_label_merge_capacity_map.")
                strategies.append(MergeStrategy(patch_map.get(key, merge_patch_size),
                                                mcap_map.get(key, merge_capacity), merge_dynamic_rope))
                policy = "merge"
            row.append(HeadComposition(f"L{li}_H{hi}_{policy}", label, sink, recent, strategies, policy, cap))
        out.append(row)
    return out


def shipped_compositions(num_layers: int = 30, num_heads: int = 12, labels=None):
    """The released Pyramid Forcing policy over the shipped (or given) labels."""
    if labels is not None:
        return build_compositions(num_layers, num_heads, labels=labels, **PYRAMID_FORCING_POLICY)
    return build_compositions(num_layers, num_heads, None, SHIPPED_LABELS_CSV, **PYRAMID_FORCING_POLICY)
