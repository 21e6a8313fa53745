"""Python side of the per-head state record and its ops (reference:
pyramidkv/_mega_state_ops.py:36-411).

The numpy structured dtype is the byte layout of the 600-byte record the
kernels mutate (field order of anchor_store.cuh:62-132 with natural
alignment); ``pack_states`` / ``unpack_states`` convert the dataclass
mirror, and the ``*_cuda`` wrappers call the registered ops with the
reference's signatures.
"""
from __future__ import annotations

from typing import Iterable, Sequence

import numpy as np
import torch

from . import _mega_state_ref as _ref
from . import _ops

PER_HEAD_STATE_DTYPE = np.dtype(
    [
        ("kind", np.int8), ("sink_capacity", np.int8), ("_pad0", np.int8, (2,)),
        ("period", np.int32), ("bucket_cap", np.int32), ("interval", np.int32), ("capacity", np.int32),
        ("patch_size", np.int32), ("block_frames", np.int32),
        ("lag_offsets", np.int32, (_ref.MAX_LAG_OFFSETS,)), ("lag_offset_count", np.int32),
        ("cyclic_slot", np.int32, (_ref.MAX_PHASE * _ref.MAX_BUCKET,)),
        ("cyclic_t", np.int32, (_ref.MAX_PHASE * _ref.MAX_BUCKET,)),
        ("cyclic_cursor", np.int8, (_ref.MAX_PHASE,)),
        ("tkey_slot", np.int32, (_ref.MAX_T_KEYED,)), ("tkey_t", np.int32, (_ref.MAX_T_KEYED,)),
        ("tkey_count", np.int8), ("tkey_head", np.int8), ("_pad1", np.int8, (2,)),
        ("merge_completed_slot", np.int32, (_ref.MAX_MERGE_BLOCKS,)),
        ("merge_completed_block_id", np.int32, (_ref.MAX_MERGE_BLOCKS,)),
        ("merge_completed_start_t", np.int32, (_ref.MAX_MERGE_BLOCKS,)),
        ("merge_completed_end_t", np.int32, (_ref.MAX_MERGE_BLOCKS,)),
        ("merge_completed_median_t", np.int32, (_ref.MAX_MERGE_BLOCKS,)),
        ("merge_completed_count", np.int8), ("_pad2", np.int8, (3,)),
        ("merge_active_block_id", np.int32, (_ref.MAX_MERGE_ACTIVE,)),
        ("merge_active_slot", np.int32, (_ref.MAX_MERGE_ACTIVE,)),
        ("merge_active_seen", np.int8, (_ref.MAX_MERGE_ACTIVE, _ref.MAX_MERGE_BLOCK_FRAMES)),
        ("merge_active_complete_count", np.int8, (_ref.MAX_MERGE_ACTIVE,)),
        ("_pad3", np.int8, (2,)), ("cached_num_groups", np.int32),
    ],
    align=True,
)

_ABI_CHECKED = False


def _check_abi() -> None:
    """The numpy itemsize must equal sizeof(PerHeadState) of the library."""
    global _ABI_CHECKED
    if _ABI_CHECKED:
        return
    cpp = int(_ops.ops().mega_state_perhead_size())
    py = PER_HEAD_STATE_DTYPE.itemsize
    if cpp != py:
        raise RuntimeError(f"PerHeadState ABI mismatch: numpy dtype itemsize={py}, sizeof(PerHeadState)={cpp}.")
    _ABI_CHECKED = True


_SCALARS = ("kind", "sink_capacity", "period", "bucket_cap", "interval", "capacity", "patch_size", "block_frames",
            "lag_offset_count", "tkey_count", "tkey_head", "merge_completed_count", "cached_num_groups")
_ARRAYS = ("lag_offsets", "cyclic_slot", "cyclic_t", "cyclic_cursor", "tkey_slot", "tkey_t", "merge_completed_slot",
           "merge_completed_block_id", "merge_completed_start_t", "merge_completed_end_t",
           "merge_completed_median_t", "merge_active_block_id", "merge_active_complete_count")


def pack_states(states: Sequence[_ref.PerHeadState]) -> np.ndarray:
    arr = np.zeros(len(states), dtype=PER_HEAD_STATE_DTYPE)
    for i, s in enumerate(states):
        rec = arr[i]
        for n in _SCALARS:
            rec[n] = getattr(s, n)
        for n in _ARRAYS:
            rec[n][:] = getattr(s, n)
        for a in range(_ref.MAX_MERGE_ACTIVE):
            rec["merge_active_seen"][a][:] = [int(b) for b in s.merge_active_seen[a]]
    return arr


def unpack_states(arr: np.ndarray) -> list[_ref.PerHeadState]:
    out = []
    for i in range(arr.shape[0]):
        rec = arr[i]
        kw = {n: int(rec[n]) for n in _SCALARS}
        kw.update({n: [int(x) for x in rec[n]] for n in _ARRAYS})
        kw["merge_active_seen"] = [[bool(b) for b in rec["merge_active_seen"][a]]
                                   for a in range(_ref.MAX_MERGE_ACTIVE)]
        out.append(_ref.PerHeadState(**kw))
    return out


def _to_bytes_tensor(arr: np.ndarray, device) -> torch.Tensor:
    flat = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    return torch.from_numpy(flat).clone().to(device=device, non_blocking=False)


_SINK_MODE = {"lag": 0, "window_clamp": 1}
_HIST_MODE = {"none": 0, "relative_clamp": 1, "relative_softcap": 2}


def mega_plan_cuda(mgr, states_bytes, layer_idx, current_t, pass_kind=1, sink_time_mapping_mode="lag",
                   sink_time_clamp_min=0, sink_time_clamp_max=21, decoupled_sink_time_lag=0,
                   history_time_mapping_mode="none", history_relative_t_max=21, history_time_soft_factor=1.0):
    """Single-chunk plan: (cu_seqlens_k, src_kind, src_slot_global,
    seg_lengths, dst_token_offsets, anchor_t_raw, anchor_t_remap)."""
    return _ops.ops().mega_plan(
        mgr, states_bytes, int(layer_idx), int(current_t), int(pass_kind),
        int(_SINK_MODE.get(sink_time_mapping_mode, 0)), int(sink_time_clamp_min), int(sink_time_clamp_max),
        int(decoupled_sink_time_lag), int(_HIST_MODE.get(history_time_mapping_mode, 0)),
        int(history_relative_t_max), float(history_time_soft_factor))


def mega_plan_multi_cuda(mgr, states_bytes, layer_idx, current_t_list, pass_kind=1, sink_time_mapping_mode="lag",
                         sink_time_clamp_min=0, sink_time_clamp_max=21, decoupled_sink_time_lag=0,
                         history_time_mapping_mode="none", history_relative_t_max=21,
                         history_time_soft_factor=1.0):
    """Multi-chunk plan; dst_token_offsets accumulate across chunks."""
    if not isinstance(current_t_list, torch.Tensor):
        current_t_list = torch.tensor(list(current_t_list), dtype=torch.int64)
    elif current_t_list.dtype != torch.int64:
        current_t_list = current_t_list.to(torch.int64)
    if current_t_list.dim() == 0:
        current_t_list = current_t_list.view(1)
    if current_t_list.device.type != "cpu":
        current_t_list = current_t_list.cpu()
    return _ops.ops().mega_plan_multi(
        mgr, states_bytes, int(layer_idx), current_t_list, int(pass_kind),
        int(_SINK_MODE.get(sink_time_mapping_mode, 0)), int(sink_time_clamp_min), int(sink_time_clamp_max),
        int(decoupled_sink_time_lag), int(_HIST_MODE.get(history_time_mapping_mode, 0)),
        int(history_relative_t_max), float(history_time_soft_factor))


def mega_merge_accum_cuda(mgr, layer_idx, states_bytes, new_k, new_v, new_pos, descriptors, frame_weights=None):
    """Veil merge for one layer; ``frame_weights`` ([F] fp32) selects the
    weighted mean (None = the reference operation)."""
    dk, ds, df, dn = descriptors
    l = layer_idx
    common = (mgr.merge_accum_sum_k()[l], mgr.merge_accum_sum_v()[l], mgr.merge_accum_pos()[l],
              mgr.merge_accum_group_ids()[l], mgr.merge_accum_tokens_per_group()[l],
              mgr.merge_accum_num_groups()[l])
    pools = (mgr.merge_k_pool()[l], mgr.merge_v_pool()[l], mgr.merge_pos_pool()[l], mgr.merge_token_count()[l])
    if frame_weights is None:
        _ops.ops().mega_merge_accum(states_bytes, new_k, new_v, new_pos, dk, ds, df, dn, *common, *pools)
    else:
        _ops.ops().mega_merge_accum_weighted(states_bytes, new_k, new_v, new_pos, dk, ds, df, dn, frame_weights,
                                             *common, mgr.merge_accum_weight_sum()[l], *pools)


def mega_state_update_cuda(states: Sequence[_ref.PerHeadState], new_t_vals: Iterable[int], pass_kind: int,
                           device="cuda"):
    """pack -> kernel -> unpack: (8 descriptor lists..., mutated states)."""
    _check_abi()
    dev = torch.device(device)
    H = len(states)
    t = list(new_t_vals)
    N = H * len(t)
    buf = _to_bytes_tensor(pack_states(states), dev)
    tt = torch.tensor(t, dtype=torch.int64, device=dev)
    desc = [torch.full((N,), -1, dtype=torch.int32, device=dev) for _ in range(8)]
    _ops.ops().mega_state_update(buf, tt, *desc, int(H), int(len(t)), int(pass_kind))
    back = buf.cpu().numpy().view(PER_HEAD_STATE_DTYPE).reshape(H).copy()
    return (*[d.cpu().tolist() for d in desc], unpack_states(back))
