"""MegaCache: the per-layer cache object the causal DiT calls
(reference: pyramidkv/_mega_cache.py:42-756).

``update`` runs the fused device update (torch.ops.adahead.cache_update:
sink/recent routing against the committed counters, the recent FIFO, the
per-head state machine and the middle / Veil writes) with no host sync.
The reference restores a snapshot of the recent pool at every call so that
the noisy passes of a block and its clean pass all start from the committed
state; because every pass of a block shifts the FIFO by the same amount and
rewrites the same tail slots, the shift is applied once per block here and
later passes of that block only rewrite the tail (identical pool contents,
no snapshot copies).  A host-side marker per layer records the block whose
shift is in the pool; an update for a different block while a noisy pass
is uncommitted is rejected.

The layers' Veil (merge) heads are read from the state records once, when
``build_mega_caches`` builds the caches, and passed to every update as a
bit mask: a record's strategy kind must not change afterwards (a record
rewritten to Veil would advance its state machine without merging).

``attend`` builds the multi-chunk plan on the device, packs K/V (+3D RoPE)
into the flat workspace and runs the ragged attention directly on q's
[L_q, H, D] layout (no permutes).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch

from . import _mega_state_ops, _mega_state_ref as ref, _ops
from .base import HeadComposition
from .cyclic import CyclicStrategy
from .lag import LagStrategy
from .merge import MergeStrategy
from .stride import StrideStrategy

_STRATEGY_TYPES = {c.__name__: c for c in (CyclicStrategy, StrideStrategy, LagStrategy, MergeStrategy)}

_STRATEGY_NAME_TO_KIND = {"RecentStrategy": ref.SK_RECENT, "CyclicStrategy": ref.SK_CYCLIC,
                          "StrideStrategy": ref.SK_STRIDE, "LagStrategy": ref.SK_LAG, "MergeStrategy": ref.SK_MERGE}


@dataclass
class MegaCacheCtx:
    mgr: object
    states_bytes: torch.Tensor
    num_layers: int
    num_heads: int
    head_dim: int
    frame_seqlen: int
    sink_time_mapping_mode: str = "lag"
    sink_time_clamp_min: int = 0
    sink_time_clamp_max: int = 21
    decoupled_sink_time_lag: int = 0
    history_time_mapping_mode: str = "none"
    history_relative_t_max: int = 21
    history_time_soft_factor: float = 1.0
    spatial_width: int = 52
    spatial_height: int = 30
    has_merge_head: bool = False
    # per layer: any Veil (merge) head; layers without one skip the merge launches
    layer_has_merge: list = field(default_factory=list)
    layer_merge_heads: list = field(default_factory=list)  # per layer: bit h set for each Veil head h
    sink_caps_per_head: torch.Tensor = None
    committed_vc: torch.Tensor = None
    freqs: torch.Tensor = None
    freq_parts: tuple = None
    freq_parts_flat: tuple = None
    # per layer: (t0, frames) of the block whose recent shift is in the pool but not committed
    pending_block: list = field(default_factory=list)
    # per layer: the committed recent FIFO (K, V, positions), copied at a block's first noisy pass
    # (allocated on first use); restored when a pass for another block comes before the commit
    recent_backup: dict = field(default_factory=dict)
    cu_q: dict = field(default_factory=dict)
    # key-split attention for attend (off by default: on a rollout's per-layer
    # launches it measured no faster than the unsplit kernels) and the
    # device's workspace for it (_ops.attention_workspace)
    split_attention: bool = False
    attn_workspace: torch.Tensor = None


class MegaCache:
    def __init__(self, ctx: MegaCacheCtx, layer_idx: int):
        self.ctx = ctx
        self.layer_idx = layer_idx
        self._frame_seqlen = ctx.frame_seqlen
        self.frame_seq_length = ctx.frame_seqlen
        self.num_heads = ctx.num_heads
        self.head_dim = ctx.head_dim
        self.batch_size = 1

    @property
    def states_bytes_for_layer(self) -> torch.Tensor:
        return self.ctx.states_bytes[self.layer_idx]

    # ------------------------------------------------------------------
    def update(self, new_k: torch.Tensor, new_v: torch.Tensor, current_start: int, *,
               cache_update_mode: str = "clean", freqs=None) -> None:
        """Insert new raw-K/V frames; new_k/new_v [1, L_in, H, D] bf16."""
        if cache_update_mode == "default":
            cache_update_mode = "clean"
        if cache_update_mode not in ("noisy", "clean"):
            return
        ctx = self.ctx
        FSEQ, H, D = ctx.frame_seqlen, ctx.num_heads, ctx.head_dim
        assert new_k.shape == new_v.shape, "K/V shapes must match"
        B, L_in, Hk, Dk = new_k.shape
        assert B == 1, "MegaCache.update: B>1 not yet supported"
        assert Hk == H and Dk == D
        assert L_in % FSEQ == 0, f"L_in ({L_in}) not multiple of FSEQ ({FSEQ})"
        t0 = current_start // FSEQ
        l = self.layer_idx
        if ctx.committed_vc is None:
            ctx.committed_vc = ctx.mgr.valid_count().clone()
        block = (t0, L_in // FSEQ)
        pending = ctx.pending_block[l]
        clean = cache_update_mode == "clean"
        if pending is not None and pending != block:
            # another block's noisy pass is in the recent FIFO, uncommitted: back to the committed FIFO, as
            # the reference's restore of its snapshot (_mega_cache.py:226-245); this pass then shifts afresh
            self._recent_fifo(restore=True)  # (the backup still holds the committed FIFO)
        elif pending is None and not clean:
            self._recent_fifo(restore=False)  # a block's first noisy pass: keep the committed FIFO
        if pending != block:
            pending = None
        nk = new_k if new_k.dtype == torch.bfloat16 else new_k.to(torch.bfloat16)
        nv = new_v if new_v.dtype == torch.bfloat16 else new_v.to(torch.bfloat16)
        if nk.stride(-1) != 1 or nk.stride(-2) != D:
            nk = nk.contiguous()
        if nv.stride() != nk.stride():
            nv = nv.contiguous()
            nk = nk.contiguous()
        _ops.ops().cache_update(ctx.mgr, ctx.states_bytes[l], ctx.sink_caps_per_head[l], ctx.committed_vc[l], nk, nv,
                                l, t0, 1 if clean else 0, 1 if pending == block else 0, ctx.spatial_width,
                                ctx.layer_merge_heads[l])
        ctx.pending_block[l] = None if clean else block

    def _recent_fifo(self, restore: bool) -> None:
        """Copy this layer's recent K / V / positions into the layer's backup
        (restore=False), or back from it (restore=True)."""
        ctx, l = self.ctx, self.layer_idx
        mgr = ctx.mgr
        pools = (mgr.recent_k_pool()[l], mgr.recent_v_pool()[l], mgr.recent_pos_pool()[l])
        backup = ctx.recent_backup.get(l)
        if restore:
            for dst, src in zip(pools, backup):
                dst.copy_(src)
            return
        if backup is None:
            backup = tuple(torch.empty_like(t) for t in pools)
            ctx.recent_backup[l] = backup
        for dst, src in zip(backup, pools):
            dst.copy_(src)

    def last_update_descriptors(self, frames: int):
        """The 8 state-machine descriptor arrays of the last update call."""
        return _ops.ops().update_descriptors(self.ctx.mgr, int(frames))

    # ------------------------------------------------------------------
    def plan(self, current_start: int, num_chunks: int):
        ctx = self.ctx
        FSEQ = ctx.frame_seqlen
        t_list = [(current_start + c * FSEQ) // FSEQ for c in range(num_chunks)]
        return _mega_state_ops.mega_plan_multi_cuda(
            ctx.mgr, self.states_bytes_for_layer, layer_idx=self.layer_idx, current_t_list=t_list,
            sink_time_mapping_mode=ctx.sink_time_mapping_mode, sink_time_clamp_min=ctx.sink_time_clamp_min,
            sink_time_clamp_max=ctx.sink_time_clamp_max, decoupled_sink_time_lag=ctx.decoupled_sink_time_lag,
            history_time_mapping_mode=ctx.history_time_mapping_mode,
            history_relative_t_max=ctx.history_relative_t_max,
            history_time_soft_factor=ctx.history_time_soft_factor)

    def pack(self, plan, freqs=None):
        """Layer-offset the plan and gather K/V/pos into the flat workspace."""
        from ._mega_attention import _layer_offset_slot_global
        ctx = self.ctx
        cu, sk, sg, sl, dst, _traw, tremap = plan
        mgr = ctx.mgr
        sga = _layer_offset_slot_global(sg, sk, self.layer_idx, int(mgr.max_sink()), int(mgr.max_middle()),
                                        int(mgr.max_recent()), ctx.num_heads, int(mgr.max_merge_blocks()))
        eff = ctx.freqs if ctx.freqs is not None else freqs
        if eff is not None:
            parts = ctx.freq_parts_flat
            if parts is None:
                from .rope import flat_freq_parts
                parts = flat_freq_parts(eff, sk.device)
            _ops.pyramidkv_pack(mgr, sk, sga, sl, dst, anchor_t_remap=tremap, freqs_ft_flat=parts[0],
                                freqs_fy_flat=parts[1], freqs_fx_flat=parts[2])
        else:
            _ops.pyramidkv_pack(mgr, sk, sga, sl, dst)
        return cu

    def attend_kv(self, current_start: int, num_chunks: int, freqs=None) -> torch.Tensor:
        """Plan + layer offset + pack (+RoPE) in one op; returns cu_seqlens_k
        [C*H+1] (a view of the manager's buffer, valid until the next call)."""
        ctx = self.ctx
        FSEQ = ctx.frame_seqlen
        t_list = torch.arange(current_start // FSEQ, current_start // FSEQ + num_chunks, dtype=torch.int64)
        eff = ctx.freqs if ctx.freqs is not None else freqs
        if eff is not None:
            parts = ctx.freq_parts_flat
            if parts is None:
                from .rope import flat_freq_parts
                parts = ctx.freq_parts_flat = flat_freq_parts(eff, ctx.states_bytes.device)
        else:
            parts = (_ops._empty(torch.float32, ctx.states_bytes.device),) * 3
        return _ops.ops().mega_attend_kv(ctx.mgr, self.states_bytes_for_layer, self.layer_idx, t_list,
                                         _mega_state_ops._SINK_MODE.get(ctx.sink_time_mapping_mode, 0),
                                         int(ctx.sink_time_clamp_min), int(ctx.sink_time_clamp_max),
                                         int(ctx.decoupled_sink_time_lag), *parts)

    def attend(self, q: torch.Tensor, current_start: int, *, freqs=None, softmax_scale=None, causal=False,
               max_seqlen_k=None) -> torch.Tensor:
        """Attention of q [1, L_q, H, D] (RoPE applied) over the cache."""
        ctx = self.ctx
        FSEQ = ctx.frame_seqlen
        B, L_q, H, D = q.shape
        assert B == 1, "MegaCache.attend: B>1 not yet supported"
        assert L_q % FSEQ == 0, f"L_q ({L_q}) must be a multiple of FSEQ ({FSEQ})"
        C = L_q // FSEQ
        if C <= int(ctx.mgr.max_attend_chunks()):
            cu_k = self.attend_kv(current_start, C, freqs)
        else:  # more chunks than the fused plan buffers hold: the reference op sequence (raises on overflow)
            cu_k = self.pack(self.plan(current_start, C), freqs)
        cu_q = ctx.cu_q.get(L_q)
        if cu_q is None or cu_q.device != q.device:
            cu_q = ctx.cu_q[L_q] = torch.arange(0, L_q + 1, FSEQ, dtype=torch.int32, device=q.device)
        qb = q[0] if q.dtype == torch.bfloat16 else q[0].to(torch.bfloat16)
        out = _ops.ragged_attention(qb, ctx.mgr.k_flat_out().view(-1, D), ctx.mgr.v_flat_out().view(-1, D), cu_q,
                                    cu_k, FSEQ, softmax_scale, kv_per_head=True, causal=causal,
                                    workspace=self._split_workspace(q.device))
        return out.view(1, L_q, H, D).to(q.dtype)


    def _split_workspace(self, device):
        """The key-split attention workspace when ctx.split_attention is set."""
        ctx = self.ctx
        if not ctx.split_attention:
            return None
        if ctx.attn_workspace is None:
            ctx.attn_workspace = _ops.attention_workspace(device)
        return ctx.attn_workspace


def _composition_to_perhead_state(composition: HeadComposition) -> ref.PerHeadState:
    """HeadComposition -> state record (reference _mega_cache.py:572-628): the
    first middle strategy's record (one strategy kind per head), chosen by
    the strategy's class name as the reference does, so any object with those
    attributes and one of those names encodes the same way; no or an unknown
    strategy: sink + recent only.  The composition's sink frames become the
    record's sink capacity."""
    sink_cap = int(getattr(composition, "sink_frames", 0))
    s = ref.make_recent()
    if composition.middle_strategies:
        mid = composition.middle_strategies[0]
        cls = _STRATEGY_TYPES.get(type(mid).__name__)
        if cls is not None:
            s = cls.state_record(mid)
    s.sink_capacity = sink_cap
    return s


def merge_head_mask(is_merge) -> int:
    """Bit mask of the Veil heads of one layer, as the cache update takes it:
    bit h for head h < 63, bit 63 for any head >= 63 (a signed int64)."""
    m = 0
    for h, v in enumerate(is_merge):
        if v:
            m |= 1 << min(h, 63)
    return m - (1 << 64) if m >= 1 << 63 else m


def build_mega_caches(num_layers: int, num_heads: int, head_dim: int, frame_seqlen: int, max_sink_frames: int,
                      max_middle_frames: int, max_recent_frames: int,
                      compositions: Sequence[Sequence[HeadComposition]], *, max_attend_chunks: int = 8,
                      device: str = "cuda:0", kv_dtype: str = "bfloat16", sink_time_mapping_mode: str = "lag",
                      sink_time_clamp_min: int = 0, sink_time_clamp_max: int = 21, decoupled_sink_time_lag: int = 0,
                      history_time_mapping_mode: str = "none", history_relative_t_max: int = 21,
                      history_time_soft_factor: float = 1.0, spatial_width: int = 52, spatial_height: int = 30,
                      freqs: torch.Tensor | None = None) -> list[MegaCache]:
    """One manager + one [L, H*600] state tensor shared by L MegaCache views."""
    if len(compositions) != num_layers:
        raise ValueError(f"compositions has {len(compositions)} layers, expected {num_layers}")
    _ops.ops()
    mgr = torch.classes.adahead.PyramidKVCacheManager(num_layers, num_heads, head_dim, frame_seqlen, max_sink_frames,
                                                      max_middle_frames, max_recent_frames, device, kv_dtype,
                                                      int(max_attend_chunks))
    size = _mega_state_ops.PER_HEAD_STATE_DTYPE.itemsize
    states_np = np.zeros((num_layers, num_heads), dtype=_mega_state_ops.PER_HEAD_STATE_DTYPE)
    sink_caps = np.zeros((num_layers, num_heads), dtype=np.int64)
    any_merge = False
    layer_merge = []
    layer_heads = []
    for l in range(num_layers):
        if len(compositions[l]) != num_heads:
            raise ValueError(f"compositions[{l}] has {len(compositions[l])} heads, expected {num_heads}")
        per_head = [_composition_to_perhead_state(c) for c in compositions[l]]
        layer_merge.append(any(s.kind == ref.SK_MERGE for s in per_head))
        any_merge = any_merge or layer_merge[-1]
        layer_heads.append(merge_head_mask([s.kind == ref.SK_MERGE for s in per_head]))
        for h, s in enumerate(per_head):
            sink_caps[l, h] = int(s.sink_capacity)
        states_np[l] = _mega_state_ops.pack_states(per_head)
    flat = np.ascontiguousarray(states_np).view(np.uint8).reshape(num_layers, num_heads * size)
    states_bytes = torch.from_numpy(flat).clone().to(device=device).contiguous()
    freq_parts = freq_parts_flat = None
    if freqs is not None:
        from .rope import flat_freq_parts, split_freqs
        freqs = freqs.to(device=device)
        freq_parts = split_freqs(freqs)
        freq_parts_flat = flat_freq_parts(freqs, device)
    ctx = MegaCacheCtx(mgr=mgr, states_bytes=states_bytes, num_layers=num_layers, num_heads=num_heads,
                       head_dim=head_dim, frame_seqlen=frame_seqlen, sink_time_mapping_mode=sink_time_mapping_mode,
                       sink_time_clamp_min=sink_time_clamp_min, sink_time_clamp_max=sink_time_clamp_max,
                       decoupled_sink_time_lag=decoupled_sink_time_lag,
                       history_time_mapping_mode=history_time_mapping_mode,
                       history_relative_t_max=history_relative_t_max,
                       history_time_soft_factor=history_time_soft_factor, spatial_width=spatial_width,
                       spatial_height=spatial_height, has_merge_head=any_merge, layer_has_merge=layer_merge,
                       layer_merge_heads=layer_heads,
                       sink_caps_per_head=torch.from_numpy(sink_caps).to(device=device).contiguous(), freqs=freqs,
                       freq_parts=freq_parts, freq_parts_flat=freq_parts_flat,
                       pending_block=[None] * num_layers)
    return [MegaCache(ctx, l) for l in range(num_layers)]
