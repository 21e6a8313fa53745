"""Argument checks of the ops whose kernels write through caller tensors:
mega_evict_merge, mega_merge_accum(_weighted), mega_state_update and
cache_update refuse a tensor on the host (or another device), a descriptor
array that is too short and any merge accumulator or pool whose extents
differ from the layout the kernels index, with a RuntimeError raised before
any launch (the state records and accumulators are left as they were).
The reference checks its own arguments the same way (TORCH_CHECK in
scatter_copy_bind.cpp:451-683, mega_merge_accum.cu:268-340)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

if torch.cuda.is_available():
    from gpu_util import DEV, to_dev, to_np
    from pyramidkv import _ops

pytestmark = pytest.mark.gpu

H, F, FSEQ, W, D, MMA, MMB, MT = 2, 1, 16, 4, 128, 2, 6, 420


def _args():
    """Valid mega_evict_merge arguments for H heads and one frame."""
    recs = [O.make_merge(2, 6) for _ in range(H)]
    states = to_dev(O.states_to_bytes(recs))
    f32, i32, i64 = torch.float32, torch.int32, torch.int64
    z = lambda *s, dt=f32: torch.zeros(s, dtype=dt, device=DEV)
    a = dict(states=states, t_vals=torch.tensor([4], dtype=i64, device=DEV),
             nk=torch.randn(F, H, FSEQ, D, device=DEV).to(torch.bfloat16),
             nv=torch.randn(F, H, FSEQ, D, device=DEV).to(torch.bfloat16), w=torch.ones(F, device=DEV),
             desc=[torch.full((H * F,), -7, dtype=i32, device=DEV) for _ in range(8)],
             sum_k=z(H, MMA, MT, D), sum_v=z(H, MMA, MT, D), pos=z(H, MMA, MT, 3, dt=i64),
             gid=z(H, MMA, FSEQ, dt=i32), tpg=z(H, MMA, MT), ng=z(H, MMA, dt=i32), wsum=z(H, MMA),
             mk=z(H, MMB, MT, D, dt=torch.bfloat16), mv=z(H, MMB, MT, D, dt=torch.bfloat16),
             mpos=z(H, MMB, MT, 3, dt=i64), mtc=z(H, MMB, dt=i32))
    a["ws"] = torch.zeros(_ops.ops().mega_evict_merge_workspace_size(H), dtype=torch.uint8, device=DEV)
    return a


def _evict(a):
    _ops.ops().mega_evict_merge(a["states"], a["t_vals"], a["nk"], a["nv"], W, a["w"], *a["desc"], a["sum_k"],
                                a["sum_v"], a["pos"], a["gid"], a["tpg"], a["ng"], a["wsum"], a["mk"], a["mv"],
                                a["mpos"], a["mtc"], a["ws"])


BREAKS = {
    "host descriptor": lambda a: a["desc"].__setitem__(4, a["desc"][4].cpu()),
    "short descriptor": lambda a: a["desc"].__setitem__(6, a["desc"][6][:H * F - 1]),
    "int64 descriptor": lambda a: a["desc"].__setitem__(0, a["desc"][0].long()),
    "host states": lambda a: a.__setitem__("states", a["states"].cpu()),
    "host t_vals": lambda a: a.__setitem__("t_vals", a["t_vals"].cpu()),
    "host workspace": lambda a: a.__setitem__("ws", a["ws"].cpu()),
    "host accumulator": lambda a: a.__setitem__("sum_v", a["sum_v"].cpu()),
    "acc_v other MTPA": lambda a: a.__setitem__("sum_v", a["sum_v"][:, :, :MT - 1].contiguous()),
    "acc_pos two columns": lambda a: a.__setitem__("pos", a["pos"][..., :2].contiguous()),
    "acc_tpg short": lambda a: a.__setitem__("tpg", a["tpg"][:, :, :MT - 2].contiguous()),
    "acc_ng three slots": lambda a: a.__setitem__("ng", torch.zeros(H, MMA + 1, dtype=torch.int32, device=DEV)),
    "acc_wsum one slot": lambda a: a.__setitem__("wsum", a["wsum"][:, :1].contiguous()),
    "group ids short": lambda a: a.__setitem__("gid", a["gid"][:, :, :FSEQ - 1].contiguous()),
    "merge_v other blocks": lambda a: a.__setitem__("mv", a["mv"][:, :MMB - 1].contiguous()),
    "merge_pos int32": lambda a: a.__setitem__("mpos", a["mpos"].int()),
    "token count short": lambda a: a.__setitem__("mtc", a["mtc"][:, :MMB - 1].contiguous()),
    "non-contiguous sums": lambda a: a.__setitem__("sum_k", a["sum_k"].transpose(2, 3).contiguous().transpose(2, 3)),
}


def test_evict_merge_accepts_the_valid_layout():
    a = _args()
    _evict(a)
    torch.cuda.synchronize()
    assert int(to_np(a["desc"][0])[0]) == O.DST_MERGE


@pytest.mark.parametrize("how", sorted(BREAKS))
def test_evict_merge_refuses_before_launch(how):
    print(f"mega_evict_merge with {how}", flush=True)
    a = _args()
    before = {k: to_np(a[k]) for k in ("states", "sum_k", "gid", "ng")}
    BREAKS[how](a)
    with pytest.raises(RuntimeError, match="mega_evict_merge|descriptor"):
        _evict(a)
    torch.cuda.synchronize()
    for k, v in before.items():
        t = a[k]
        if t.device.type == "cuda" and t.shape == v.shape:
            assert np.array_equal(to_np(t), v), f"{k} changed by a refused call"


@pytest.mark.parametrize("how", ["host descriptor", "short descriptor", "acc_pos two columns", "token count short",
                                 "acc_wsum one slot", "host states"])
@pytest.mark.parametrize("weighted", [False, True])
def test_merge_accum_refuses_before_launch(how, weighted):
    a = _args()
    pos = torch.zeros(F, H, FSEQ, 3, dtype=torch.int64, device=DEV)
    if weighted or how != "acc_wsum one slot":
        BREAKS[how](a)
    d = a["desc"]
    ops = _ops.ops()
    with pytest.raises(RuntimeError, match="mega_merge_accum|descriptor"):
        if weighted:
            ops.mega_merge_accum_weighted(a["states"], a["nk"], a["nv"], pos, d[0], d[4], d[6], d[7], a["w"],
                                          a["sum_k"], a["sum_v"], a["pos"], a["gid"], a["tpg"], a["ng"], a["wsum"],
                                          a["mk"], a["mv"], a["mpos"], a["mtc"])
        else:
            if how == "acc_wsum one slot":  # no weight sums in the unweighted op: break its pools instead
                a["mk"] = a["mk"][:, :, :MT - 1].contiguous()
            ops.mega_merge_accum(a["states"], a["nk"], a["nv"], pos, d[0], d[4], d[6], d[7], a["sum_k"], a["sum_v"],
                                 a["pos"], a["gid"], a["tpg"], a["ng"], a["mk"], a["mv"], a["mpos"], a["mtc"])


@pytest.mark.parametrize("how", ["host descriptor", "host t_vals"])
def test_state_update_refuses_other_devices(how):
    a = _args()
    BREAKS[how](a)
    before = to_np(a["states"])
    with pytest.raises(RuntimeError, match="device|CUDA"):
        _ops.ops().mega_state_update(a["states"], a["t_vals"], *a["desc"], H, F, 1)
    assert np.array_equal(to_np(a["states"]), before)


def test_cache_update_refuses_host_counters():
    from pyramidkv import factory
    from pyramidkv._mega_cache import build_mega_caches
    from pyramidkv.base import HeadComposition
    comps = [[HeadComposition(f"h{h}", 0, sink_frames=1, recent_frames=2) for h in range(H)]]
    cache = build_mega_caches(1, H, D, FSEQ, 1, 1, 2, comps, max_attend_chunks=1, device=DEV, spatial_width=W,
                              spatial_height=FSEQ // W, **factory.PYRAMID_FORCING_REMAP)[0]
    ctx = cache.ctx
    nk = torch.randn(1, FSEQ, H, D, device=DEV).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="manager's device"):
        _ops.ops().cache_update(ctx.mgr, ctx.states_bytes[0], ctx.sink_caps_per_head[0].cpu(),
                                ctx.mgr.valid_count()[0].clone(), nk, nk, 0, 0, 1, 0, W, 0)
    assert int(to_np(ctx.mgr.valid_count()).sum()) == 0
