"""ctypes binding of the C ABI in include/pyramidkv_hip.h.

Loads ``_lib/libpyramidkv_hip.so`` (built by csrc/Makefile) and exposes each
entry point with torch-tensor convenience wrappers: tensors are passed as
raw device pointers and the current HIP stream of their device.  Every call
raises ``RuntimeError`` carrying ``pkv_last_error()`` when the library
returns a non-zero status.  There is no fallback: if the library is missing
the first call raises.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libpyramidkv_hip.so")
HEADER_PATH = os.path.normpath(os.path.join(HERE, "..", "..", "include", "pyramidkv_hip.h"))

PKV_OK, PKV_ERR_INVALID, PKV_ERR_HIP, PKV_ERR_CAPACITY, PKV_ERR_UNSUPPORTED = 0, -1, -2, -3, -4

_c_i32, _c_i64, _c_p, _c_f, _c_d = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_double


class Geometry(ctypes.Structure):
    _fields_ = [("num_layers", _c_i32), ("num_heads", _c_i32), ("head_dim", _c_i32), ("frame_seqlen", _c_i32),
                ("max_sink", _c_i32), ("max_middle", _c_i32), ("max_recent", _c_i32),
                ("max_merge_blocks", _c_i32), ("max_merge_active", _c_i32), ("max_merge_tokens", _c_i32),
                ("max_pack_tokens", _c_i64)]


class Pools(ctypes.Structure):
    _fields_ = [(n, _c_p) for n in (
        "sink_k", "sink_v", "middle_k", "middle_v", "recent_k", "recent_v",
        "sink_pos", "middle_pos", "recent_pos", "merge_k", "merge_v", "merge_pos", "merge_token_count",
        "merge_accum_sum_k", "merge_accum_sum_v", "merge_accum_pos", "merge_accum_group_ids",
        "merge_accum_tokens_per_group", "merge_accum_num_groups", "merge_accum_weight_sum", "valid_count",
        "k_flat_out", "v_flat_out", "pos_flat_out")]


class StateDesc(ctypes.Structure):
    _fields_ = [(n, _c_p) for n in ("dst_kind", "dst_slot", "src_frame", "src_head", "merge_accum_slot",
                                    "merge_local_idx", "merge_finalize_completed_idx", "merge_is_new_block")]


class MergeLayer(ctypes.Structure):
    _fields_ = [(n, _c_p) for n in ("accum_sum_k", "accum_sum_v", "accum_pos", "accum_group_ids",
                                    "accum_tokens_per_group", "accum_num_groups", "accum_weight_sum",
                                    "merge_k", "merge_v", "merge_pos", "merge_token_count")]


class Remap(ctypes.Structure):
    _fields_ = [("sink_mode_code", _c_i32), ("sink_clamp_min", _c_i32), ("sink_clamp_max", _c_i32),
                ("decoupled_sink_lag", _c_i32), ("hist_mode_code", _c_i32), ("hist_relative_t_max", _c_i32),
                ("hist_soft_factor", _c_d)]


class PlanOut(ctypes.Structure):
    _fields_ = [(n, _c_p) for n in ("cu_seqlens_k", "src_kind", "src_slot_global", "seg_lengths",
                                    "dst_token_offsets", "anchor_t_raw", "anchor_t_remap")]


class RopeTables(ctypes.Structure):
    _fields_ = [("ft", _c_p), ("fy", _c_p), ("fx", _c_p), ("ft_rows", _c_i32), ("ft_cols", _c_i32),
                ("fy_rows", _c_i32), ("fy_cols", _c_i32), ("fx_rows", _c_i32), ("fx_cols", _c_i32)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", _c_p), ("k", _c_p), ("v", _c_p), ("o", _c_p), ("cu_seqlens_q", _c_p),
                ("cu_seqlens_k", _c_p), ("num_batches", _c_i32), ("num_heads_q", _c_i32), ("head_dim", _c_i32),
                ("kv_per_head", _c_i32), ("q_tok_stride", _c_i64), ("q_head_stride", _c_i64),
                ("kv_tok_stride", _c_i64), ("kv_head_stride", _c_i64), ("o_tok_stride", _c_i64),
                ("o_head_stride", _c_i64), ("max_seqlen_q", _c_i32), ("softmax_scale", _c_f), ("causal", _c_i32)]


class UpdateArgs(ctypes.Structure):
    _fields_ = [("layer", _c_i32), ("frames", _c_i32), ("t0", _c_i64), ("pass_kind", _c_i32),
                ("shift_pending", _c_i32), ("spatial_width", _c_i32), ("reserved", _c_i32),
                ("new_k", _c_p), ("new_v", _c_p), ("tok_stride", _c_i64), ("head_stride", _c_i64),
                ("states_layer", _c_p), ("sink_caps_layer", _c_p), ("committed_vc_layer", _c_p),
                ("workspace", _c_p), ("merge_heads", ctypes.c_uint64)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"pyramidkv HIP library not built: {LIB_PATH} is missing "
                "(run `make -C pyramid-forcing_amd/csrc` or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        L.pkv_last_error.restype = ctypes.c_char_p
        L.pkv_perhead_state_size.restype = _c_i64
        L.pkv_cache_update_workspace_size.restype = _c_i64
        L.pkv_cache_update_workspace_size.argtypes = [ctypes.POINTER(Geometry), _c_i32]
        L.pkv_merge_workspace_size.restype = _c_i64
        L.pkv_merge_workspace_size.argtypes = [_c_i32] * 4
        L.pkv_merge_accum_static.argtypes = [_c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32] + \
            [_c_p] * 10
        L.pkv_evict_merge.argtypes = [_c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_p,
                                      _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p]
        L.pkv_evict_merge_workspace_size.restype = _c_i64
        L.pkv_evict_merge_workspace_size.argtypes = [_c_i32]
        L.pkv_ragged_attn_workspace_size.restype = _c_i64
        L.pkv_ragged_attn_workspace_size.argtypes = []
        L.pkv_ragged_attn_fwd_ws.argtypes = [_c_p, _c_p, _c_i64, _c_p]
        _lib = L
    return _lib


def declared_symbols() -> list[str]:
    """Entry points declared in include/pyramidkv_hip.h."""
    with open(HEADER_PATH) as f:
        txt = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char \*)\s*(pkv_\w+)\s*\(", txt, re.M)))


def check(rc: int, what: str) -> None:
    if rc != PKV_OK:
        msg = lib().pkv_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


# ---------------------------------------------------------------------------
# torch helpers
# ---------------------------------------------------------------------------
def ptr(t):
    """Device pointer of a tensor, None for None or empty."""
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def stream_of(t):
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream


def make_geometry(L, H, D, FSEQ, max_sink, max_middle, max_recent, max_pack_tokens, MMB=6, MMA=2, MTPA=420):
    return Geometry(L, H, D, FSEQ, max_sink, max_middle, max_recent, MMB, MMA, MTPA, max_pack_tokens)


def rope_struct(tables):
    if tables is None:
        return None
    ft, fy, fx = tables
    return RopeTables(ft.data_ptr(), fy.data_ptr(), fx.data_ptr(), ft.shape[0], ft.shape[1] // 2, fy.shape[0],
                      fy.shape[1] // 2, fx.shape[0], fx.shape[1] // 2)


def ragged_attn_workspace_size() -> int:
    """Bytes of the workspace pkv_ragged_attn_fwd_ws splits small launches with."""
    return int(lib().pkv_ragged_attn_workspace_size())


def ragged_attn_fwd(q, k, v, out, cu_q, cu_k, num_batches, heads_q, kv_per_head, max_seqlen_q, scale,
                    q_strides=None, kv_strides=None, o_strides=None, workspace=None):
    """q/out [tokens, H, D] (or strided views), k/v [tokens, (H,) D]; with a
    workspace tensor, pkv_ragged_attn_fwd_ws (key-split small launches)."""
    D = q.shape[-1]
    qs = q_strides or (q.stride(0), q.stride(1) if q.dim() == 3 else 0)
    ks = kv_strides or (k.stride(0), k.stride(1) if (k.dim() == 3 and k.shape[1] > 1) else 0)
    os_ = o_strides or (out.stride(0), out.stride(1) if out.dim() == 3 else 0)
    a = AttnArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), cu_q.data_ptr(), cu_k.data_ptr(),
                 num_batches, heads_q, D, 1 if kv_per_head else 0, qs[0], qs[1], ks[0], ks[1], os_[0], os_[1],
                 max_seqlen_q, float(scale), 0)
    if workspace is not None:
        check(lib().pkv_ragged_attn_fwd_ws(ctypes.byref(a), _c_p(workspace.data_ptr()),
                                           ctypes.c_int64(workspace.numel() * workspace.element_size()),
                                           _c_p(stream_of(q))), "pkv_ragged_attn_fwd_ws")
    else:
        check(lib().pkv_ragged_attn_fwd(ctypes.byref(a), _c_p(stream_of(q))), "pkv_ragged_attn_fwd")
