"""Helpers for the GPU parity tests: device pool sets, numpy <-> device
transfers of bf16 bit patterns, and calls through the C ABI (ctypes)."""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from oracle import oracle as O
from pyramidkv import _abi as A

DEV = "cuda:0"


def to_dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)
    return torch.from_numpy(a).to(DEV)


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class DevicePools:
    """All manager tensors of a geometry on the device (zero-filled)."""

    def __init__(self, g: O.Geometry):
        self.g = g
        L, H, D, FS = g.num_layers, g.num_heads, g.head_dim, g.frame_seqlen
        MMB, MMA, MT = g.max_merge_blocks, g.max_merge_active, g.max_merge_tokens
        bf, i64, i32, f32 = torch.bfloat16, torch.int64, torch.int32, torch.float32
        z = lambda *s, dt=bf: torch.zeros(s, dtype=dt, device=DEV)
        self.t = dict(
            sink_k=z(L, H, g.max_sink, FS, D), sink_v=z(L, H, g.max_sink, FS, D),
            middle_k=z(L, H, g.max_middle, FS, D), middle_v=z(L, H, g.max_middle, FS, D),
            recent_k=z(L, H, g.max_recent, FS, D), recent_v=z(L, H, g.max_recent, FS, D),
            sink_pos=z(L, H, g.max_sink, FS, 3, dt=i64), middle_pos=z(L, H, g.max_middle, FS, 3, dt=i64),
            recent_pos=z(L, H, g.max_recent, FS, 3, dt=i64),
            merge_k=z(L, H, MMB, MT, D), merge_v=z(L, H, MMB, MT, D), merge_pos=z(L, H, MMB, MT, 3, dt=i64),
            merge_token_count=z(L, H, MMB, dt=i32),
            merge_accum_sum_k=z(L, H, MMA, MT, D, dt=f32), merge_accum_sum_v=z(L, H, MMA, MT, D, dt=f32),
            merge_accum_pos=z(L, H, MMA, MT, 3, dt=i64), merge_accum_group_ids=z(L, H, MMA, FS, dt=i32),
            merge_accum_tokens_per_group=z(L, H, MMA, MT, dt=f32), merge_accum_num_groups=z(L, H, MMA, dt=i32),
            merge_accum_weight_sum=z(L, H, MMA, dt=f32), valid_count=z(L, H, 3, dt=i64),
            k_flat_out=z(g.max_pack_tokens, D), v_flat_out=z(g.max_pack_tokens, D),
            pos_flat_out=z(g.max_pack_tokens, 3, dt=i64))
        self.geo = A.make_geometry(L, H, D, FS, g.max_sink, g.max_middle, g.max_recent, g.max_pack_tokens, MMB, MMA,
                                   MT)
        self.pools = A.Pools(**{n: self.t[n].data_ptr() for n, _ in A.Pools._fields_})

    def load(self, arrays: dict):
        for n, a in arrays.items():
            self.t[n].copy_(to_dev(a).view(self.t[n].shape))

    def np(self, name):
        return to_np(self.t[name])


def plan_out(C, H, S):
    n = C * H * S
    i32 = dict(dtype=torch.int32, device=DEV)
    i64 = dict(dtype=torch.int64, device=DEV)
    o = dict(cu=torch.full((C * H + 1,), -7, **i32), sk=torch.full((n,), -7, **i32), sg=torch.full((n,), -7, **i32),
             sl=torch.full((n,), -7, **i32), dst=torch.full((n,), -7, **i32), traw=torch.full((n,), -7, **i64),
             tremap=torch.full((n,), -7, **i64))
    s = A.PlanOut(o["cu"].data_ptr(), o["sk"].data_ptr(), o["sg"].data_ptr(), o["sl"].data_ptr(),
                  o["dst"].data_ptr(), o["traw"].data_ptr(), o["tremap"].data_ptr())
    return o, s


def run_plan(dp: DevicePools, states_layer_dev, layer, t_list, remap=(0, 0, 21, 0)):
    g = dp.g
    C, H, S = len(t_list), g.num_heads, g.segs
    o, s = plan_out(C, H, S)
    tl = (ctypes.c_int64 * C)(*t_list)
    rm = A.Remap(remap[0], remap[1], remap[2], remap[3], 0, 21, 1.0)
    total = torch.zeros(1, dtype=torch.int32, device=DEV)
    vc = dp.t["valid_count"][layer]
    mtc = dp.t["merge_token_count"][layer]
    A.check(A.lib().pkv_plan_multi(ctypes.byref(dp.geo), ctypes.c_void_p(states_layer_dev.data_ptr()),
                                   ctypes.c_void_p(vc.data_ptr()), ctypes.c_void_p(mtc.data_ptr()), tl, C,
                                   ctypes.byref(rm), ctypes.byref(s), ctypes.c_void_p(total.data_ptr()), stream()),
            "pkv_plan_multi")
    return o, total


def run_pack(dp: DevicePools, sk, sg, sl, dst, tremap=None, tables_dev=None):
    n = sk.numel()
    rope = A.rope_struct(tables_dev) if tables_dev is not None else None
    A.check(A.lib().pkv_pack(ctypes.byref(dp.geo), ctypes.byref(dp.pools), ctypes.c_void_p(sk.data_ptr()),
                             ctypes.c_void_p(sg.data_ptr()), ctypes.c_void_p(sl.data_ptr()),
                             ctypes.c_void_p(dst.data_ptr()), n,
                             ctypes.c_void_p(tremap.data_ptr()) if tremap is not None else None,
                             ctypes.byref(rope) if rope is not None else None, stream()), "pkv_pack")


def state_desc(n):
    ts = [torch.full((n,), -9, dtype=torch.int32, device=DEV) for _ in range(8)]
    return ts, A.StateDesc(*[t.data_ptr() for t in ts])
