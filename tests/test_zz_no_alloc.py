"""pkv_merge_accum_static (the allocation-free merge entry point: its scratch
is a static device array) against pkv_merge_accum with a caller workspace,
through the C ABI.  Two lanes with identical state records and
accumulators take the same calls; every output buffer must be bit-identical
after each call, and equal to the CPU oracle.  The second call is smaller
than the first, so the static array still holds the first call's larger
snapshot when the second one runs.  Permuted cell positions force the
member-list path, the part of the scratch that scales with the input."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from gpu_util import DEV, state_desc, stream, to_dev, to_np
    from pyramidkv import _abi as A

D, MT, W = 128, 420, 52


def _lane(states_host, H, FSEQ):
    acc = dict(sum_k=np.zeros((H, 2, MT, D), np.float32), sum_v=np.zeros((H, 2, MT, D), np.float32),
               pos=np.zeros((H, 2, MT, 3), np.int64), gid=np.zeros((H, 2, FSEQ), np.int32),
               tpg=np.zeros((H, 2, MT), np.float32), ng=np.zeros((H, 2), np.int32), wsum=np.zeros((H, 2), np.float32),
               mk=np.zeros((H, 6, MT, D), np.uint16), mv=np.zeros((H, 6, MT, D), np.uint16),
               mpos=np.zeros((H, 6, MT, 3), np.int64), mtc=np.zeros((H, 6), np.int32))
    dev = {k: to_dev(v) for k, v in acc.items()}
    ml = A.MergeLayer(*[dev[k].data_ptr() for k in ("sum_k", "sum_v", "pos", "gid", "tpg", "ng", "wsum", "mk", "mv",
                                                     "mpos", "mtc")])
    return acc, dev, ml, to_dev(states_host.copy())


def _call(fn, states_dev, H, F, FSEQ, dk, dv, dpos, ts, wd, ml, ws=None):
    args = [ctypes.c_void_p(states_dev.data_ptr()), H, F, FSEQ, D, 2, 6, MT, ctypes.c_void_p(dk.data_ptr()),
            ctypes.c_void_p(dv.data_ptr()), ctypes.c_void_p(dpos.data_ptr()),
            *[ctypes.c_void_p(ts[i].data_ptr()) for i in (0, 4, 6, 7)],
            ctypes.c_void_p(wd.data_ptr()) if wd is not None else None, ctypes.byref(ml)]
    if ws is not None:
        args.append(ctypes.c_void_p(ws.data_ptr()))
    return fn(*args, stream())


@pytest.mark.parametrize("weighted", [False, True])
def test_static_merge_matches_workspace_merge(weighted):
    rng = np.random.default_rng(11 + weighted)
    H, FSEQ = 12, 1560
    states_host = O.states_to_bytes([O.make_merge(2, int(c)) for c in rng.integers(2, 7, H)])
    acc, dev_a, ml_a, st_a = _lane(states_host, H, FSEQ)
    _, dev_b, ml_b, st_b = _lane(states_host, H, FSEQ)
    cell = rng.permutation(FSEQ)
    # call 1: 6 frames (a block finalizes, the next one starts); call 2: 1 frame
    for t_vals in ([0, 1, 2, 3, 4, 5], [6]):
        F = len(t_vals)
        print(f"no-alloc merge: weighted={weighted} H={H} F={F} FSEQ={FSEQ}", flush=True)
        nk = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
        nv = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
        pos = np.zeros((F, H, FSEQ, 3), np.int64)
        pos[..., 0] = np.asarray(t_vals).reshape(F, 1, 1)
        pos[..., 1] = cell // W
        pos[..., 2] = cell % W
        w = rng.uniform(0.1, 1.0, F).astype(np.float32) if weighted else None
        desc = O.state_update(states_host, t_vals, 1)
        O.merge_accum(states_host, nk, nv, pos, desc, acc, w)
        dk, dv, dpos = to_dev(nk), to_dev(nv), to_dev(pos)
        wd = to_dev(w) if w is not None else None
        tv = torch.tensor(t_vals, dtype=torch.int64, device=DEV)
        descs = []
        for st in (st_a, st_b):
            ts, sd = state_desc(H * F)
            A.check(A.lib().pkv_state_update(ctypes.c_void_p(st.data_ptr()), H, ctypes.c_void_p(tv.data_ptr()), F, 1,
                                             ctypes.byref(sd), stream()), "state_update")
            descs.append(ts)
        ws = torch.empty(A.lib().pkv_merge_workspace_size(H, F, FSEQ, MT), dtype=torch.uint8, device=DEV)
        A.check(_call(A.lib().pkv_merge_accum, st_a, H, F, FSEQ, dk, dv, dpos, descs[0], wd, ml_a, ws), "merge_accum")
        A.check(_call(A.lib().pkv_merge_accum_static, st_b, H, F, FSEQ, dk, dv, dpos, descs[1], wd, ml_b),
                "merge_accum_static")
        torch.cuda.synchronize()
        for k in acc:
            a, b = to_np(dev_a[k]), to_np(dev_b[k])
            assert (a == b).all(), f"{k} differs between the static and workspace entry points"
            assert (b == acc[k]).all(), f"{k} differs from the oracle"


def test_static_merge_rejects_oversized_calls():
    """A call whose snapshots exceed the static array is refused on the host
    before any launch, with an error naming the limit."""
    H, F, FSEQ = 64, 8, 4096
    need = A.lib().pkv_merge_workspace_size(H, F, FSEQ, MT)
    assert need > (1 << 20)
    rc = A.lib().pkv_merge_accum_static(None, H, F, FSEQ, D, 2, 6, MT, None, None, None, None, None, None, None,
                                        None, None, stream())
    assert rc == A.PKV_ERR_CAPACITY
    assert b"static buffer" in A.lib().pkv_last_error()
