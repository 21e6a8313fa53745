"""Per-layer readout / step helpers (reference: pyramidkv/_mega_attention.py).

``_flash_attn_varlen()`` is the swap point the reference fills with
flash-attn 2.8.3's ``flash_attn_varlen_func``; here it returns a function
with the same keyword signature backed by the gfx950 ragged-attention
kernel (torch.ops.adahead.ragged_attention).
"""
from __future__ import annotations

import torch

from . import _mega_state_ops, _ops


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p=0.0,
                           softmax_scale=None, causal=False, **unused):
    """flash_attn_varlen_func semantics for q [total_q, H, D], k/v
    [total_k, H, D] (H equal for q and k/v), non-causal, no dropout."""
    if dropout_p:
        raise NotImplementedError("dropout is not supported by the ragged-attention kernel")
    if q.shape[1] != k.shape[1]:
        raise NotImplementedError("grouped-query attention (different q / kv head counts) is not supported")
    qb = q if q.dtype == torch.bfloat16 else q.to(torch.bfloat16)
    out = _ops.ragged_attention(qb, k, v, cu_seqlens_q.to(torch.int32), cu_seqlens_k.to(torch.int32),
                                int(max_seqlen_q), softmax_scale, kv_per_head=False, causal=causal)
    return out if out.dtype == q.dtype else out.to(q.dtype)


def _flash_attn_varlen():
    return flash_attn_varlen_func


def _layer_offset_slot_global(src_slot_global, src_kind, layer_idx, max_sink, max_middle, max_recent, num_heads,
                              max_merge_blocks=0):
    """Shift per-layer slot ids into the [L, H, slots] pools
    (_mega_attention.py:516-552)."""
    if layer_idx == 0:
        return src_slot_global
    off = torch.tensor([layer_idx * num_heads * max_sink, layer_idx * num_heads * max_middle,
                        layer_idx * num_heads * max_recent, layer_idx * num_heads * max_merge_blocks],
                       dtype=torch.int32, device=src_slot_global.device)
    return src_slot_global + off[src_kind.clamp(min=0).long()] * (src_kind >= 0).to(torch.int32)


def _remap_kwargs(kw):
    keys = ("sink_time_mapping_mode", "sink_time_clamp_min", "sink_time_clamp_max", "decoupled_sink_time_lag",
            "history_time_mapping_mode", "history_relative_t_max", "history_time_soft_factor")
    return {k: kw[k] for k in keys if k in kw}


def mega_readout_kv_only(mgr, per_head_states_bytes, layer_idx, current_t, H, D, *, freqs=None, freq_parts=None,
                         pass_kind=1, **remap):
    """Plan + pack (+RoPE) for one query chunk; returns cloned (k, v, cu_seqlens_k)."""
    cu, sk, sg, sl, dst, _traw, tremap = _mega_state_ops.mega_plan_cuda(
        mgr, per_head_states_bytes, layer_idx=layer_idx, current_t=current_t, pass_kind=pass_kind,
        **_remap_kwargs(remap))
    sga = _layer_offset_slot_global(sg, sk, layer_idx, int(mgr.max_sink()), int(mgr.max_middle()),
                                    int(mgr.max_recent()), H, int(mgr.max_merge_blocks()))
    if freqs is not None:
        from .rope import flat_freq_parts
        ft, fy, fx = flat_freq_parts(freqs, sk.device)
        _ops.pyramidkv_pack(mgr, sk, sga, sl, dst, anchor_t_remap=tremap, freqs_ft_flat=ft, freqs_fy_flat=fy,
                            freqs_fx_flat=fx)
    else:
        _ops.pyramidkv_pack(mgr, sk, sga, sl, dst)
    n = int(cu[-1].item())
    return mgr.k_flat_out()[:n].clone(), mgr.v_flat_out()[:n].clone(), cu.clone()


def _attend_one_chunk(q, k_flat, v_flat, cu_seqlens_k, *, softmax_scale, causal, max_seqlen_k):
    """q [1, L_q, H, D] against per-head ragged K/V -> [1, L_q, H, D]."""
    B, L_q, H, D = q.shape
    cu_q = torch.tensor([0, L_q], dtype=torch.int32, device=q.device)
    qb = q[0] if q.dtype == torch.bfloat16 else q[0].to(torch.bfloat16)
    out = _ops.ragged_attention(qb, k_flat.view(-1, D), v_flat.view(-1, D), cu_q, cu_seqlens_k.to(torch.int32),
                                L_q, softmax_scale, kv_per_head=True, causal=causal)
    return out.view(1, L_q, H, D).to(q.dtype)


def mega_readout(mgr, per_head_states_bytes, q, layer_idx, current_t, *, freqs=None, freq_parts=None, pass_kind=1,
                 softmax_scale=None, causal=False, max_seqlen_k=None, **remap):
    assert q.dim() == 4 and q.shape[0] == 1, "mega_readout: q must be [1, L_q, H, D]"
    _, L_q, H, D = q.shape
    k, v, cu = mega_readout_kv_only(mgr, per_head_states_bytes, layer_idx, current_t, H, D, freqs=freqs,
                                    freq_parts=freq_parts, pass_kind=pass_kind, **remap)
    return _attend_one_chunk(q, k, v, cu, softmax_scale=softmax_scale, causal=causal, max_seqlen_k=max_seqlen_k)


def mega_attention_step(mgr, per_head_states_bytes, q, k_new, v_new, new_t_vals, layer_idx, current_t, *,
                        pass_kind=1, softmax_scale=None, causal=False, max_seqlen_k=None, **remap):
    """State update + middle insertion + readout (_mega_attention.py:394-513)."""
    assert q.shape == k_new.shape == v_new.shape
    B, L_q, H, D = q.shape
    F = int(new_t_vals.shape[0])
    FSEQ = int(mgr.frame_seqlen())
    assert B == 1 and L_q == F * FSEQ
    dev = q.device
    N = H * F
    desc = [torch.full((N,), -1, dtype=torch.int32, device=dev) for _ in range(8)]
    _ops.ops().mega_state_update(per_head_states_bytes, new_t_vals, *desc, int(H), int(F), int(pass_kind))
    max_middle = int(mgr.max_middle())
    slot_global = (desc[1].long() + (layer_idx * H + desc[3].long()) * max_middle).to(torch.int32)
    nk = k_new.view(F, FSEQ, H, D).permute(0, 2, 1, 3).contiguous()
    nv = v_new.view(F, FSEQ, H, D).permute(0, 2, 1, 3).contiguous()
    empty = torch.empty(0, dtype=torch.int64, device=dev)
    _ops.ops().pyramidkv_update(mgr, nk, nv, empty, desc[0], slot_global, desc[2], desc[3])
    return mega_readout(mgr, per_head_states_bytes, q, layer_idx, current_t, pass_kind=pass_kind,
                        softmax_scale=softmax_scale, causal=causal, max_seqlen_k=max_seqlen_k, **remap)
