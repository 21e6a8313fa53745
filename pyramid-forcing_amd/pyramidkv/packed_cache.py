"""PyramidKVPackedCache: the legacy FIFO-recent cache over the manager and
the plan / update / pack ops (reference: pyramidkv/packed_cache.py:28-160).

Every incoming frame goes to the recent pool as a ring of max_recent
slots; the legacy plan covers slots 0..valid_count-1 of each pool for
every (layer, head).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _ops


@dataclass
class _PackedReadout:
    k_flat: torch.Tensor        # [total_tokens, 1, head_dim]
    v_flat: torch.Tensor        # [total_tokens, 1, head_dim]
    cu_seqlens_k: torch.Tensor  # [num_layers * num_heads + 1] int32
    total_tokens: int


class PyramidKVPackedCache:
    def __init__(self, num_layers: int, num_heads: int, head_dim: int, frame_seqlen: int,
                 max_recent_frames: int = 4, max_sink_frames: int = 1, max_middle_frames: int = 1,
                 device: str = "cuda:0", kv_dtype: str = "bfloat16"):
        if not _ops.available():
            raise RuntimeError("adahead C++ extension not available")
        self.num_layers, self.num_heads, self.head_dim = num_layers, num_heads, head_dim
        self.frame_seqlen = frame_seqlen
        self.max_recent, self.max_sink, self.max_middle = max_recent_frames, max_sink_frames, max_middle_frames
        self._mgr = torch.classes.adahead.PyramidKVCacheManager(
            num_layers, num_heads, head_dim, frame_seqlen, max_sink_frames, max_middle_frames, max_recent_frames,
            device, kv_dtype, num_layers)
        self._next_slot = [[0] * num_heads for _ in range(num_layers)]

    @property
    def manager(self):
        return self._mgr

    def reset(self) -> None:
        self._mgr.reset()
        self._next_slot = [[0] * self.num_heads for _ in range(self.num_layers)]

    def update(self, layer_idx: int, new_k: torch.Tensor, new_v: torch.Tensor) -> None:
        """Append new_k/new_v [frames, H, frame_seqlen, D] to the recent ring of one layer."""
        assert new_k.dim() == 4 and new_v.dim() == 4, "new_k/new_v must be [frames, H, F, D]"
        frames, H, F, D = new_k.shape
        assert H == self.num_heads, f"head count mismatch: {H} vs {self.num_heads}"
        assert F == self.frame_seqlen, f"frame_seqlen mismatch: {F} vs {self.frame_seqlen}"
        assert D == self.head_dim, f"head_dim mismatch: {D} vs {self.head_dim}"
        slots, src_frame, src_head = [], [], []
        for f in range(frames):
            for h in range(H):
                s = self._next_slot[layer_idx][h]
                slots.append((layer_idx * H + h) * self.max_recent + s)
                src_frame.append(f)
                src_head.append(h)
                self._next_slot[layer_idx][h] = (s + 1) % self.max_recent
        dev = new_k.device
        as_i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=dev)
        _ops.ops().pyramidkv_update(self._mgr, new_k, new_v, _ops._empty(torch.int64, dev),
                                    as_i32([2] * len(slots)), as_i32(slots), as_i32(src_frame), as_i32(src_head))
        vc = self._mgr.valid_count()
        vc[layer_idx, :, 2] = torch.clamp(vc[layer_idx, :, 2] + frames, max=self.max_recent)

    def readout(self, current_t: int = 0, pass_kind: int = 0) -> _PackedReadout:
        """Legacy plan + pack over all (layer, head); views into the manager's workspace."""
        cu, sk, sg, sl, dst = _ops.ops().pyramidkv_plan(self._mgr, int(current_t), int(pass_kind))
        _ops.pyramidkv_pack(self._mgr, sk, sg, sl, dst)
        total = int(cu[-1].item())
        return _PackedReadout(k_flat=self._mgr.k_flat_out()[:total], v_flat=self._mgr.v_flat_out()[:total],
                              cu_seqlens_k=cu, total_tokens=total)
