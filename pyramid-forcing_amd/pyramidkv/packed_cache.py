"""PyramidKVPackedCache: the legacy recent-only cache over the manager
(interface of the reference's pyramidkv/packed_cache.py:28-160; same
constructor, ``manager``, ``reset``, ``update(layer_idx, new_k, new_v)`` and
``readout(current_t, pass_kind)``).

Each (layer, head) keeps its last ``max_recent_frames`` frames in a ring of
recent-pool slots: frame number n of a head (counting from the last reset)
lives in slot n % max_recent.  The ring cursor is the manager's
``write_idx[layer, head, 2]`` and the fill level its ``valid_count[layer,
head, 2]``, both device tensors, so ``update`` builds its copy descriptors on
the device and never synchronises with the host.  A call of more frames than
the ring holds writes only the frames that survive it, so no two copies of
one call target the same slot.  ``readout`` runs the legacy planner (slots
0..valid_count-1 of every pool, layer-major) and the pack; its token total is
the one host read.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from . import _ops


class PackedReadout(NamedTuple):
    k_flat: torch.Tensor        # packed K rows [total_tokens, 1, head_dim], a view of the workspace
    v_flat: torch.Tensor
    cu_seqlens_k: torch.Tensor  # int32 offsets of the L*H sequences
    total_tokens: int


_PackedReadout = PackedReadout  # the reference's name for the result type

_RECENT = 2  # pool kind and valid_count column of the recent ring


class PyramidKVPackedCache:
    def __init__(self, num_layers: int, num_heads: int, head_dim: int, frame_seqlen: int,
                 max_recent_frames: int = 4, max_sink_frames: int = 1, max_middle_frames: int = 1,
                 device: str = "cuda:0", kv_dtype: str = "bfloat16"):
        if not _ops.available():
            raise RuntimeError("CUDA scatter extension not available")
        self.num_layers, self.num_heads, self.head_dim = int(num_layers), int(num_heads), int(head_dim)
        self.frame_seqlen = int(frame_seqlen)
        self.max_recent, self.max_sink, self.max_middle = (int(max_recent_frames), int(max_sink_frames),
                                                           int(max_middle_frames))
        # one pack covers every (layer, head) sequence: size the plan for L chunks of H heads
        self._mgr = torch.classes.adahead.PyramidKVCacheManager(
            self.num_layers, self.num_heads, self.head_dim, self.frame_seqlen, self.max_sink, self.max_middle,
            self.max_recent, device, kv_dtype, self.num_layers)
        self._no_pos = None

    @property
    def manager(self):
        return self._mgr

    def reset(self) -> None:
        self._mgr.reset()  # clears write_idx (the ring cursors) and valid_count

    def update(self, layer_idx: int, new_k: torch.Tensor, new_v: torch.Tensor) -> None:
        """Append new_k / new_v [frames, heads, frame_seqlen, head_dim] to
        every head's recent ring of layer ``layer_idx``."""
        if not 0 <= layer_idx < self.num_layers:
            raise IndexError(f"PyramidKVPackedCache.update: layer {layer_idx} outside [0, {self.num_layers})")
        want = (self.num_heads, self.frame_seqlen, self.head_dim)
        if new_k.dim() != 4 or new_k.shape != new_v.shape or tuple(new_k.shape[1:]) != want:
            raise ValueError(f"PyramidKVPackedCache.update: K {tuple(new_k.shape)} / V {tuple(new_v.shape)}; "
                             f"expected equal shapes [frames, {want[0]}, {want[1]}, {want[2]}]")
        frames, H, R = new_k.shape[0], self.num_heads, self.max_recent
        if frames == 0:
            return
        dev = new_k.device
        cursor = self._mgr.write_idx()[layer_idx, :, _RECENT]       # [H] int64, next slot to write
        kept = min(frames, R)                                         # older frames of this call are overwritten
        first = frames - kept
        f = torch.arange(first, frames, device=dev, dtype=torch.int64).view(kept, 1)
        h = torch.arange(H, device=dev, dtype=torch.int64).view(1, H)
        slot = torch.remainder(cursor.view(1, H) + f, R)             # [kept, H] ring slot of frame f
        i32 = lambda t: t.to(torch.int32).reshape(-1).contiguous()
        if self._no_pos is None or self._no_pos.device != dev:
            self._no_pos = torch.empty(0, dtype=torch.int64, device=dev)
        _ops.ops().pyramidkv_update(self._mgr, new_k, new_v, self._no_pos,
                                    torch.full((kept * H,), _RECENT, dtype=torch.int32, device=dev),
                                    i32((layer_idx * H + h) * R + slot), i32(f.expand(kept, H)), i32(h.expand(kept, H)))
        cursor.copy_(torch.remainder(cursor + frames, R))
        vc = self._mgr.valid_count()[layer_idx, :, _RECENT]
        vc.copy_(torch.clamp(vc + frames, max=R))

    def readout(self, current_t: int = 0, pass_kind: int = 0) -> PackedReadout:
        """Legacy plan + pack over all (layer, head) sequences; the tensors
        are views of the manager's workspace, valid until the next readout."""
        cu, kind, slot, length, dst = _ops.ops().pyramidkv_plan(self._mgr, int(current_t), int(pass_kind))
        _ops.pyramidkv_pack(self._mgr, kind, slot, length, dst)
        total = int(cu[-1])
        return PackedReadout(self._mgr.k_flat_out()[:total], self._mgr.v_flat_out()[:total], cu, total)
