"""3D RoPE tables and dynamic time remaps.

* ``rope_params`` / ``wan_freqs``: the Wan table definition
  (wan/modules/model.py:29-36; t/h/w concat causal_model.py:585-590):
  row p, pair j = exp(i * p * theta^(-2j/dim)) in float64.
* ``split_freqs`` / ``flat_freq_parts``: the 22/21/21 split and the fp32
  (re, im) interleaved tables the pack kernel reads
  (pyramidkv/_mega_cache.py:713-731).
* ``apply_rope_to_flat_k``: rotates packed K on the GPU
  (torch.ops.adahead.rope_apply); replaces rope.py:18-68 and the Triton
  kernel of triton_rope.py.
* ``map_sink_time`` / ``map_dynamic_pos_time``: rope.py:86-134.
"""
from __future__ import annotations

import torch

from . import _ops


def rope_params(max_seq_len: int, dim: int, theta: float = 10000) -> torch.Tensor:
    assert dim % 2 == 0
    ang = torch.outer(torch.arange(max_seq_len, dtype=torch.float64),
                      1.0 / torch.pow(theta, torch.arange(0, dim, 2, dtype=torch.float64).div(dim)))
    return torch.polar(torch.ones_like(ang), ang)


def wan_freqs(head_dim: int = 128, max_seq_len: int = 1024, theta: float = 10000) -> torch.Tensor:
    d = head_dim
    return torch.cat([rope_params(max_seq_len, d - 4 * (d // 6), theta),
                      rope_params(max_seq_len, 2 * (d // 6), theta),
                      rope_params(max_seq_len, 2 * (d // 6), theta)], dim=1)


def split_freqs(freqs: torch.Tensor):
    c = freqs.shape[1]
    return tuple(p.contiguous() for p in freqs.split([c - 2 * (c // 3), c // 3, c // 3], dim=1))


def flat_freq_parts(freqs: torch.Tensor, device=None):
    """(ft, fy, fx) fp32 [rows, cols*2] with (re, im) interleaved."""
    out = []
    for z in split_freqs(freqs):
        z = z.to(device=device) if device is not None else z
        out.append(torch.view_as_real(z.to(torch.complex64)).contiguous().view(z.shape[0], -1))
    return tuple(out)


def apply_rope_to_flat_k(k_flat: torch.Tensor, pos_3d: torch.Tensor, freqs: torch.Tensor,
                         freq_parts=None, out: torch.Tensor | None = None, freq_parts_flat=None) -> torch.Tensor:
    """Rotate k_flat [n, D] (bf16, on the GPU) at positions pos_3d [n, 3]."""
    if k_flat.numel() == 0:
        return out if out is not None else k_flat
    if k_flat.shape[1] % 2 != 0:
        raise ValueError(f"Head dim must be even, got {k_flat.shape[1]}")
    if freq_parts_flat is None:
        if freq_parts is not None:
            freq_parts_flat = tuple(torch.view_as_real(p.to(torch.complex64)).contiguous().view(p.shape[0], -1)
                                    .to(k_flat.device) for p in freq_parts)
        else:
            freq_parts_flat = flat_freq_parts(freqs, k_flat.device)
    res = _ops.ops().rope_apply(k_flat.contiguous(), pos_3d.to(device=k_flat.device, dtype=torch.long),
                                *freq_parts_flat)
    if out is not None:
        out.copy_(res)
        return out
    return res


def map_sink_time(sync_t_raw: int, sink_time_mapping_mode: str, sink_time_clamp_min: int,
                  sink_time_clamp_max: int, decoupled_sink_time_lag: int) -> int:
    if sink_time_mapping_mode == "window_clamp":
        delta = min(max(sync_t_raw, sink_time_clamp_min), sink_time_clamp_max)
        return max(0, sync_t_raw - delta)
    return max(0, sync_t_raw - decoupled_sink_time_lag)


def map_dynamic_pos_time(dyn_pos: torch.Tensor, current_t: int, history_time_mapping_mode: str,
                         history_relative_t_max: int, history_time_soft_factor: float,
                         inplace: bool = False) -> torch.Tensor:
    mode = history_time_mapping_mode
    if mode == "none" or history_relative_t_max <= 0:
        return dyn_pos
    if mode == "relative_softcap":
        mapped = dyn_pos if inplace else dyn_pos.clone()
        rel = (current_t - mapped[:, 0].long()).clamp(min=0)
        over = (rel - history_relative_t_max).clamp(min=0)
        comp = torch.round(over.to(torch.float32) * history_time_soft_factor).to(torch.long)
        rel_mapped = torch.where(rel <= history_relative_t_max, rel, history_relative_t_max + comp)
        mapped[:, 0] = (current_t - rel_mapped).clamp(min=0)
        return mapped
    if mode != "relative_clamp":
        return dyn_pos
    mapped = dyn_pos if inplace else dyn_pos.clone()
    rel = (current_t - mapped[:, 0].long()).clamp(min=0, max=history_relative_t_max)
    mapped[:, 0] = current_t - rel
    return mapped
