"""torch.ops.adahead access (reference: pyramidkv/_ops.py:16-167).

Loads the in-tree torch binding (_lib/libpyramidkv_torch.so, which links
the HIP library _lib/libpyramidkv_hip.so) and exposes the registered ops.
If the binding is missing, ``ops()`` raises the reference's RuntimeError;
there is no CPU fallback.
"""
from __future__ import annotations

import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
TORCH_LIB = os.path.join(_HERE, "_lib", "libpyramidkv_torch.so")
_loaded = None


def _ensure_loaded() -> bool:
    global _loaded
    if _loaded is None:
        try:
            torch.ops.load_library(TORCH_LIB)
            _loaded = True
        except (OSError, RuntimeError):
            _loaded = False
    return _loaded


def available() -> bool:
    return _ensure_loaded() and hasattr(torch.ops, "adahead")


def ops():
    if not _ensure_loaded():
        raise RuntimeError("CUDA scatter extension not available")
    return torch.ops.adahead


_EMPTY = {}


def _empty(dtype, device):
    key = (dtype, str(device))
    t = _EMPTY.get(key)
    if t is None:
        t = _EMPTY[key] = torch.empty(0, dtype=dtype, device=device)
    return t


def pyramidkv_pack(mgr, src_kind, src_slot_global, seg_lengths, dst_token_offsets, *, anchor_t_remap=None,
                   freqs_ft_flat=None, freqs_fy_flat=None, freqs_fx_flat=None) -> None:
    """Empty tensors stand in for omitted RoPE arguments (pure gather)."""
    d = src_kind.device
    e64, ef = _empty(torch.int64, d), _empty(torch.float32, d)
    ops().pyramidkv_pack(mgr, src_kind, src_slot_global, seg_lengths, dst_token_offsets,
                         anchor_t_remap if anchor_t_remap is not None else e64,
                         freqs_ft_flat if freqs_ft_flat is not None else ef,
                         freqs_fy_flat if freqs_fy_flat is not None else ef,
                         freqs_fx_flat if freqs_fx_flat is not None else ef)


_attn_workspaces: dict = {}


def attention_workspace(device) -> torch.Tensor:
    """The device's workspace for ragged_attention's key-split launches
    (allocated on first use and kept; it needs no initialisation).  Calls
    sharing it must be ordered on one stream."""
    device = torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    ws = _attn_workspaces.get(device)
    if ws is None:
        with torch.cuda.device(device):
            n = int(ops().ragged_attention_workspace_size())
        ws = _attn_workspaces[device] = torch.empty(max(n, 1), dtype=torch.uint8, device=device)
    return ws


def ragged_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, softmax_scale=None, kv_per_head=True,
                     causal=False, workspace=None):
    """flash_attn_varlen_func's arithmetic (non-causal) on the ragged layout;
    with a workspace (attention_workspace), launches of a few sequences with
    per-head keys split their keys over every compute unit."""
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    return ops().ragged_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), float(softmax_scale),
                                  bool(kv_per_head), bool(causal), workspace)


def scatter_copy(src_ptrs, lengths, offsets, dst, col_dim: int) -> None:
    """Gather rows from the device addresses in ``src_ptrs`` into ``dst``."""
    ops().scatter_copy(src_ptrs, lengths, offsets, dst, int(col_dim))


def apply_pos_override(pos, starts, ends, vals) -> None:
    """pos[i, 0] = vals[r] for starts[r] <= i < ends[r]."""
    ops().apply_pos_override(pos, starts, ends, vals)


def anchor_store_write_frames(k_seq, v_seq, pos_seq, frame_desc, store_k, store_v, store_pos) -> None:
    """Copy frames (frame_desc rows: source frame, store slot) into store slots."""
    ops().anchor_store_write_frames(k_seq, v_seq, pos_seq, frame_desc, store_k, store_v, store_pos)


def refresh_readout_layout(src_k, src_v, src_pos, src_ptrs_k, src_ptrs_v, src_ptrs_pos, offsets, lengths, flags,
                           dynamic_rope_t, dst_k_raw, dst_v, dst_rope_pos, dst_frame_ids, head_dim: int,
                           current_t: int, history_time_mapping_mode: str, history_relative_t_max: int,
                           history_time_soft_factor: float) -> None:
    """K/V gather with the history time map and frame ids (see the op)."""
    ops().refresh_readout_layout(src_k, src_v, src_pos, src_ptrs_k, src_ptrs_v, src_ptrs_pos, offsets, lengths,
                                 flags, dynamic_rope_t, dst_k_raw, dst_v, dst_rope_pos, dst_frame_ids,
                                 int(head_dim), int(current_t), str(history_time_mapping_mode),
                                 int(history_relative_t_max), float(history_time_soft_factor))
