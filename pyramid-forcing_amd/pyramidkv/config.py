"""PyramidKVConfig: the per-(layer, head) metadata holder the reference's
pipeline builds before choosing a cache (reference: pyramidkv/config.py:14-357;
caller pipeline/causal_inference.py:707-762).

It owns no device memory.  What it holds:

* ``capacity_map`` [L, H] int32 and ``label_map`` [L, H] int32, read from a
  CSV that is either a label matrix (rows of more than three cells: each
  cell a head label resolved to a capacity through ``code_map``; labels the
  map lacks get ``default_capacity``) or explicit ``layer, head, capacity``
  triples;
* ``compositions`` (alias ``policies``): per-head HeadComposition lists
  compiled by ``factory.build_compositions`` from the head-type CSV, or
  None; the pipeline overwrites both with its own compile;
* ``drop_head_mask`` / ``soft_ablate_head_mask`` [L, H] bool from
  ``layer, head`` lists;
* ``af_group_map``: the optional A-F head taxonomy, from a matrix CSV or
  from a manifest / per-group directory of ``layer, head`` files.

The MegaCache path reads ``capacity_map`` and ``compositions``; the rest is
carried for callers that read it.
"""
from __future__ import annotations

import csv
import os
from typing import Optional

import torch

_AF_GROUPS = ("A", "B", "C", "D", "E", "F")
# consensus class ids of the taxonomy manifest -> group letter
_AF_CLASS_IDS = {"A_RECENT_TRACKER": "A", "B_RHYTHM_DRIVER": "B", "C_WINDOW_SMOOTHER": "C",
                 "D_CYCLE_ATTENDER": "D", "E_ANCHOR_SPARSE": "E", "F_BROAD_LOCAL": "F"}
_announced: set = set()


def _csv_rows(path: str):
    with open(path, newline="", encoding="utf-8") as f:
        return [row for row in csv.reader(f) if row]


def _int_or_none(cell) -> int | None:
    try:
        return int(str(cell).strip())
    except ValueError:
        return None


def _head_pairs(path: str, num_layers: int, num_heads: int):
    """(layer, head) pairs of a CSV list; header and non-numeric rows skipped."""
    pairs = []
    for row in _csv_rows(path):
        if len(row) < 2:
            continue
        l, h = _int_or_none(row[0]), _int_or_none(row[1])
        if l is not None and h is not None and 0 <= l < num_layers and 0 <= h < num_heads:
            pairs.append((l, h))
    return pairs


class PyramidKVConfig:
    def __init__(self, config_path: Optional[str], num_layers: int, num_heads: int, default_capacity: int = 32768,
                 strategy_reduction_factor: int = 3, code_map: Optional[dict] = None,
                 head_type_csv_path: Optional[str] = None, drop_heads_csv_path: Optional[str] = None,
                 soft_ablate_heads_csv_path: Optional[str] = None, af_policy_enabled: bool = False,
                 af_csv_path: Optional[str] = None, af_group_dir: Optional[str] = None,
                 af_manifest_path: Optional[str] = None, frame_seq_length: Optional[int] = None):
        L, H = int(num_layers), int(num_heads)
        self.num_layers, self.num_heads = L, H
        self.frame_seq_length = frame_seq_length
        if code_map is None:
            code_map = {"-1": max(1, default_capacity // max(1, strategy_reduction_factor)), "1": default_capacity}
        self.code_map = {str(k): int(v) for k, v in code_map.items()}
        self.head_type_csv_path = head_type_csv_path
        self.drop_heads_csv_path = drop_heads_csv_path
        self.soft_ablate_heads_csv_path = soft_ablate_heads_csv_path
        self.af_policy_enabled = bool(af_policy_enabled)
        self.af_csv_path, self.af_group_dir, self.af_manifest_path = af_csv_path, af_group_dir, af_manifest_path

        self.capacity_map = torch.full((L, H), int(default_capacity), dtype=torch.int32)
        self.label_map = torch.ones((L, H), dtype=torch.int32)
        self.drop_head_mask = torch.zeros((L, H), dtype=torch.bool)
        self.soft_ablate_head_mask = torch.zeros((L, H), dtype=torch.bool)
        self.af_group_map = [[""] * H for _ in range(L)]

        if config_path and os.path.exists(config_path):
            if config_path not in _announced:
                _announced.add(config_path)
                print(f"PyramidKVConfig: capacities from {config_path}")
            self._load_capacities(config_path, int(default_capacity))
        elif config_path:
            print(f"Warning: {config_path} does not exist; every head keeps capacity {default_capacity}.")

        self.compositions = self._compile(head_type_csv_path)
        self.policies = self.compositions

        for path, mask, what in ((drop_heads_csv_path, self.drop_head_mask, "drop-head"),
                                 (soft_ablate_heads_csv_path, self.soft_ablate_head_mask, "soft-ablate")):
            if not path:
                continue
            if not os.path.exists(path):
                print(f"Warning: {what} list {path} does not exist; none applied.")
                continue
            before = int(mask.sum())
            for l, h in _head_pairs(path, L, H):
                mask[l, h] = True
            print(f"PyramidKVConfig: {what} list {path}: {int(mask.sum()) - before} heads")

        if self.af_policy_enabled:
            self._load_af_groups()

    # -- capacities / labels ------------------------------------------------
    def _load_capacities(self, path: str, default_capacity: int) -> None:
        matrix = []
        for row in _csv_rows(path):
            if len(row) > 3:  # a label matrix row (one cell per head)
                matrix.append([c.strip() for c in row if c.strip() != ""])
                continue
            if len(row) < 3:
                continue
            l, h, cap = (_int_or_none(c) for c in row[:3])
            if None in (l, h, cap):
                continue
            if 0 <= l < self.num_layers and 0 <= h < self.num_heads:
                self.capacity_map[l, h] = cap
        if not matrix:
            return
        if len(matrix) != self.num_layers:
            print(f"Warning: {path} has {len(matrix)} label rows for {self.num_layers} layers; "
                  "missing layers keep the default capacity.")
        unknown = set()
        for l in range(self.num_layers):
            cells = matrix[l] if l < len(matrix) else []
            if cells and len(cells) != self.num_heads:
                print(f"Warning: label row {l} has {len(cells)} cells for {self.num_heads} heads.")
            for h in range(self.num_heads):
                label = cells[h] if h < len(cells) else "1"
                as_int = _int_or_none(label)
                self.label_map[l, h] = 1 if as_int is None else as_int
                if label in self.code_map:
                    self.capacity_map[l, h] = self.code_map[label]
                else:  # a class id is not a capacity
                    self.capacity_map[l, h] = default_capacity
                    unknown.add(label)
        if unknown:
            print(f"Warning: labels {sorted(unknown)} are not in code_map; those heads get capacity "
                  f"{default_capacity}.")

    def _compile(self, head_type_csv_path):
        path = head_type_csv_path
        if not path:
            fallback = os.path.join("configs", "head_configs", "best_labels.csv")
            path = fallback if os.path.exists(fallback) else None
        if not path or not os.path.exists(path):
            return None
        from .factory import build_compositions
        try:
            return build_compositions(num_layers=self.num_layers, num_heads=self.num_heads,
                                      capacities=self.capacity_map, csv_path=path)
        except Exception as e:  # the pipeline compiles its own compositions afterwards
            print(f"Warning: head compositions from {path} failed: {e}")
            return None

    # -- A-F taxonomy -----------------------------------------------------------
    def _set_group(self, l: int, h: int, group: str) -> bool:
        if 0 <= l < self.num_layers and 0 <= h < self.num_heads and group in _AF_GROUPS:
            changed = self.af_group_map[l][h] != group
            self.af_group_map[l][h] = group
            return changed
        return False

    def _load_af_groups(self) -> None:
        counts = dict.fromkeys(_AF_GROUPS, 0)
        if self.af_csv_path and os.path.exists(self.af_csv_path):
            source = self.af_csv_path
            with open(self.af_csv_path, newline="", encoding="utf-8") as f:
                for l, row in enumerate(csv.reader(f)):
                    for h, cell in enumerate(row[:self.num_heads]):
                        g = str(cell).strip().upper()
                        if self._set_group(l, h, g):
                            counts[g] += 1
        else:
            group_dir, manifest = self.af_group_dir, self.af_manifest_path
            if not group_dir and manifest:
                group_dir = os.path.dirname(manifest)
            if not manifest and group_dir and os.path.exists(os.path.join(group_dir, "taxonomy_heads_manifest.csv")):
                manifest = os.path.join(group_dir, "taxonomy_heads_manifest.csv")
            files = []
            if manifest and os.path.exists(manifest):
                with open(manifest, newline="", encoding="utf-8") as f:
                    for row in csv.DictReader(f):
                        cid, name = str(row.get("consensus_class_id", "")).strip(), str(row.get("file_name", "")).strip()
                        if cid and name:
                            files.append((cid, name))
            elif group_dir and os.path.isdir(group_dir):
                files = [(n[:-len("_heads.csv")], n) for n in os.listdir(group_dir) if n.endswith("_heads.csv")]
            else:
                print(f"Warning: A-F policy enabled without a taxonomy source (dir={group_dir}, manifest={manifest}).")
            source = manifest or group_dir
            for cid, name in files:
                g = _AF_CLASS_IDS.get(cid)
                path = name if os.path.isabs(name) else os.path.join(group_dir or "", name)
                if not g or not os.path.exists(path):
                    continue
                with open(path, newline="", encoding="utf-8") as f:
                    for row in csv.DictReader(f):
                        l, h = _int_or_none(row.get("layer", "")), _int_or_none(row.get("head", ""))
                        if l is not None and h is not None and self._set_group(l, h, g):
                            counts[g] += 1
        total = sum(counts.values())
        if total:
            print(f"PyramidKVConfig: A-F groups from {source}: " + ", ".join(f"{g}={counts[g]}" for g in _AF_GROUPS))
        else:
            print(f"Warning: A-F policy enabled but {source} assigned no heads.")

    # -- per-layer views --------------------------------------------------------
    def get_layer_capacities(self, layer_idx: int) -> list[int]:
        return self.capacity_map[layer_idx].tolist()

    def get_layer_labels(self, layer_idx: int) -> list[int]:
        return self.label_map[layer_idx].tolist()

    def get_layer_drop_mask(self, layer_idx: int) -> list[bool]:
        return self.drop_head_mask[layer_idx].tolist()

    def get_layer_soft_ablate_mask(self, layer_idx: int) -> list[bool]:
        return self.soft_ablate_head_mask[layer_idx].tolist()

    def get_layer_af_groups(self, layer_idx: int) -> list[str]:
        return list(self.af_group_map[layer_idx])
