"""PyramidKVConfig: the per-(layer, head) metadata the pipeline builds before
it builds the cache (reference interface: pyramidkv/config.py:56-84; caller
pipeline/causal_inference.py:707-762).

The MegaCache branch of the caller reads one thing from it, ``capacity_map``,
which it hands to ``factory.build_compositions`` before it builds the caches;
``label_map``, ``code_map``, ``compositions`` (alias ``policies``) and the
``get_layer_*`` views are kept for callers that inspect them.

Head table format (the per-head classification CSV, e.g. the shipped
``best_labels.csv``):

* a row of more than three cells is one layer of a label matrix; blank cells
  are ignored, so row i gives the labels of heads 0, 1, ... of layer i;
* a row of at most three cells is an explicit ``layer, head, capacity``
  entry; rows that do not parse, or name a head outside the model, are
  ignored;
* when the file holds a label matrix, every head's capacity is
  ``code_map[label]`` -- a label the map lacks (or a head the matrix does not
  cover, whose label is "1") falls back to ``default_capacity`` when "1" is
  not in the map either -- and ``label_map`` holds the label as an integer
  (1 for labels that are not integers).

``drop_heads_csv_path``, ``soft_ablate_heads_csv_path`` and the A-F
taxonomy arguments are accepted, because the caller passes them, but their
lists are not loaded: only the reference's per-chunk attention path
(wan/modules/attention/core.py:260-266,323-350) applies them, and the
MegaCache path does not.  Passing one of them warns once and leaves
``drop_head_mask`` / ``soft_ablate_head_mask`` all False and ``af_group_map``
all "".
"""
from __future__ import annotations

import csv
import os
import warnings
from typing import NamedTuple, Optional

import numpy as np
import torch

_DEFAULT_LABEL = "1"
_warned: set = set()


class HeadTable(NamedTuple):
    """A parsed head CSV: the label-matrix rows (cells as strings, blanks
    removed) and the explicit (layer, head, capacity) entries, in file
    order."""
    matrix: list
    entries: list


def read_head_table(path: str) -> HeadTable:
    matrix, entries = [], []
    with open(path, newline="", encoding="utf-8") as f:
        for cells in csv.reader(f):
            if len(cells) > 3:
                matrix.append([c.strip() for c in cells if c.strip()])
                continue
            try:
                entries.append(tuple(int(c) for c in cells[:3]) if len(cells) == 3 else None)
            except ValueError:
                entries.append(None)
    return HeadTable(matrix, [e for e in entries if e is not None])


def _label_value(label: str) -> int:
    try:
        return int(label)
    except ValueError:
        return 1


def _warn_once(key: str, message: str) -> None:
    if key not in _warned:
        _warned.add(key)
        warnings.warn(message, stacklevel=3)


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
        self.default_capacity = int(default_capacity)
        if code_map is None:
            # oscillating heads (label -1) get a reduced window
            code_map = {"-1": max(1, self.default_capacity // max(1, int(strategy_reduction_factor))),
                        "1": self.default_capacity}
        self.code_map = {str(k): int(v) for k, v in code_map.items()}
        self.head_type_csv_path = head_type_csv_path
        self.drop_heads_csv_path = drop_heads_csv_path
        self.soft_ablate_heads_csv_path = soft_ablate_heads_csv_path
        self.af_policy_enabled = bool(af_policy_enabled)
        self.af_csv_path, self.af_group_dir, self.af_manifest_path = af_csv_path, af_group_dir, af_manifest_path

        caps = np.full((L, H), self.default_capacity, np.int64)
        labels = np.ones((L, H), np.int64)
        if config_path and os.path.exists(config_path):
            self._apply_head_table(read_head_table(config_path), caps, labels, config_path)
        elif config_path:
            _warn_once(f"missing:{config_path}", f"PyramidKVConfig: {config_path} does not exist; every head keeps "
                                                 f"capacity {self.default_capacity}")
        self.capacity_map = torch.from_numpy(caps.astype(np.int32))
        self.label_map = torch.from_numpy(labels.astype(np.int32))

        self.drop_head_mask = torch.zeros((L, H), dtype=torch.bool)
        self.soft_ablate_head_mask = torch.zeros((L, H), dtype=torch.bool)
        self.af_group_map = [[""] * H for _ in range(L)]
        for what, given in (("drop_heads_csv_path", drop_heads_csv_path),
                            ("soft_ablate_heads_csv_path", soft_ablate_heads_csv_path),
                            ("af_policy_enabled", self.af_policy_enabled)):
            if given:
                _warn_once(what, f"PyramidKVConfig: {what} is applied only by the per-chunk attention path, which "
                                 f"this build does not include; the MegaCache path ignores it (masks stay empty)")
        self._compositions = None
        self._compiled = False

    # -- head table -----------------------------------------------------------
    def _apply_head_table(self, table: HeadTable, caps: np.ndarray, labels: np.ndarray, path: str) -> None:
        L, H = caps.shape
        for l, h, cap in table.entries:
            if 0 <= l < L and 0 <= h < H:
                caps[l, h] = cap
        if not table.matrix:
            return
        if len(table.matrix) != L or any(len(r) != H for r in table.matrix[:L]):
            _warn_once(f"shape:{path}", f"PyramidKVConfig: {path} holds {len(table.matrix)} label rows of "
                                        f"{sorted({len(r) for r in table.matrix})} cells for {L} layers x {H} "
                                        f"heads; uncovered heads take label {_DEFAULT_LABEL}")
        grid = np.full((L, H), _DEFAULT_LABEL, dtype=object)
        for l, row in enumerate(table.matrix[:L]):
            grid[l, :min(H, len(row))] = row[:H]
        unknown = sorted({str(x) for x in grid.ravel()} - set(self.code_map))
        caps[:] = np.vectorize(lambda s: self.code_map.get(s, self.default_capacity), otypes=[np.int64])(grid)
        labels[:] = np.vectorize(_label_value, otypes=[np.int64])(grid)
        if unknown:
            _warn_once(f"labels:{path}", f"PyramidKVConfig: labels {unknown} of {path} are not in code_map; those "
                                         f"heads get capacity {self.default_capacity}")

    # -- compositions (compiled on first read; the pipeline assigns its own) --
    @property
    def compositions(self):
        if not self._compiled:
            self._compiled = True
            path = self.head_type_csv_path
            if path and os.path.exists(path):
                from .factory import build_compositions
                try:
                    self._compositions = build_compositions(num_layers=self.num_layers, num_heads=self.num_heads,
                                                            capacities=self.capacity_map, csv_path=path)
                except Exception as e:  # the pipeline compiles its own from the same file next
                    _warn_once(f"compile:{path}", f"PyramidKVConfig: head compositions from {path}: {e}")
        return self._compositions

    @compositions.setter
    def compositions(self, value):
        self._compiled = True
        self._compositions = value

    policies = compositions

    # -- per-layer views ----------------------------------------------------------
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
