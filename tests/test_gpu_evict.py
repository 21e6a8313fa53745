"""mega_evict_merge (pkv_evict_merge): the state update of a clean pass and
the (optionally weighted) Veil merge accumulate of the same frames in one
launch, at the grid positions (t, tok / W, tok % W) that MegaCache.update
gives its frames.  Driven over consecutive calls against the CPU oracle
(oracle.state_update then oracle.merge_accum on those positions, the
restatement of anchor_store_update.cu:43-269 and mega_merge_accum.cu:52-252):
state records, descriptors, every accumulator (fp32 sums, group ids,
counts, positions, weight sums) and the merge pools bit-exact after every
call."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

if torch.cuda.is_available():
    from gpu_util import DEV, to_dev, to_np
    from pyramidkv import _ops

pytestmark = pytest.mark.gpu

D, MMA, MMB, MT = 128, 2, 6, 420


def _evict_run(H, FSEQ, W, calls, seed, weighted, kinds=None, recs=None, tamper=None, D=D):
    """kinds: per head 'merge' or 'cyclic' (default all 'merge'); recs:
    the records themselves; tamper(ci, acc, dacc): called before call ci
    (may rewrite host and device accumulators alike)."""
    rng = np.random.default_rng(seed)
    kinds = kinds or ["merge"] * H
    if recs is None:
        recs = [O.make_merge(2, int(rng.integers(2, 7))) if k == "merge" else O.make_cyclic(4, 2) for k in kinds]
    states_host = O.states_to_bytes(recs)
    states_dev = to_dev(states_host)
    acc = dict(sum_k=np.zeros((H, MMA, MT, D), np.float32), sum_v=np.zeros((H, MMA, MT, D), np.float32),
               pos=np.zeros((H, MMA, MT, 3), np.int64), gid=np.zeros((H, MMA, FSEQ), np.int32),
               tpg=np.zeros((H, MMA, MT), np.float32), ng=np.zeros((H, MMA), np.int32),
               wsum=np.zeros((H, MMA), np.float32), mk=np.zeros((H, MMB, MT, D), np.uint16),
               mv=np.zeros((H, MMB, MT, D), np.uint16), mpos=np.zeros((H, MMB, MT, 3), np.int64),
               mtc=np.zeros((H, MMB), np.int32))
    dacc = {k: to_dev(v) for k, v in acc.items()}
    ops = _ops.ops()
    ws = torch.zeros(ops.mega_evict_merge_workspace_size(H), dtype=torch.uint8, device=DEV)
    tok = np.arange(FSEQ)
    for ci, t_vals in enumerate(calls):
        F = len(t_vals)
        if tamper is not None:
            tamper(ci, acc, dacc)
        print(f"evict_merge H={H} FSEQ={FSEQ} W={W} call {ci} t={t_vals} weighted={weighted}", flush=True)
        nk = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
        nv = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
        pos = np.zeros((F, H, FSEQ, 3), np.int64)
        pos[..., 0] = np.asarray(t_vals).reshape(F, 1, 1)
        pos[..., 1] = tok // W
        pos[..., 2] = tok % W
        w = rng.uniform(0.1, 1.0, F).astype(np.float32) if weighted else None
        desc = O.state_update(states_host, t_vals, 1)
        dm = desc.copy()
        dm[0] = np.where(desc[0] == O.DST_MERGE, desc[0], -1)
        O.merge_accum(states_host, nk, nv, pos, dm, acc, w)
        dd = [torch.full((H * F,), -7, dtype=torch.int32, device=DEV) for _ in range(8)]
        ops.mega_evict_merge(states_dev, torch.tensor(t_vals, dtype=torch.int64, device=DEV),
                             to_dev(nk).view(F, H, FSEQ, D), to_dev(nv).view(F, H, FSEQ, D), W,
                             to_dev(w) if w is not None else None, *dd, dacc["sum_k"], dacc["sum_v"], dacc["pos"],
                             dacc["gid"], dacc["tpg"], dacc["ng"], dacc["wsum"], dacc["mk"], dacc["mv"],
                             dacc["mpos"], dacc["mtc"], ws)
        torch.cuda.synchronize()
        assert np.array_equal(to_np(states_dev), states_host), f"call {ci}: state records differ"
        for i in range(8):
            assert np.array_equal(to_np(dd[i]), desc[i].astype(np.int32)), f"call {ci}: descriptor array {i} differs"
        for k in acc:
            got = to_np(dacc[k])
            if not np.array_equal(got, acc[k]):
                bad = np.argwhere(got != acc[k])
                raise AssertionError(f"call {ci}: {k} differs at {len(bad)} places, first {bad[:4].tolist()}")


def test_evict_single_frames_weighted_production_grid():
    # the config-4 pattern: one 1,560-token frame per head and call
    _evict_run(H=3, FSEQ=1560, W=52, calls=[[e + 1] for e in range(14)], seed=1, weighted=True)


@pytest.mark.parametrize("F,weighted", [(3, False), (3, True), (4, False), (2, True)])
def test_evict_multi_frame_calls_straddling_blocks(F, weighted):
    calls = [[2 + F * b + f for f in range(F)] for b in range(24 // F)]
    _evict_run(H=2, FSEQ=1560, W=52, calls=calls, seed=10 + F, weighted=weighted)


def test_evict_irregular_grid_and_mixed_heads():
    # 7-wide rows with a ragged last row and patch column (group ids scanned,
    # not the closed form), 5 frames per call (a block finalizes and the next
    # begins in one call), and a Wave head beside the Veil heads (state update
    # only)
    calls = [[5 * b + f for f in range(5)] for b in range(5)]
    _evict_run(H=3, FSEQ=7 * 9 + 3, W=7, calls=calls, seed=2, weighted=True, kinds=["merge", "cyclic", "merge"])


@pytest.mark.parametrize("weighted", [False, True])
def test_evict_one_frame_out_of_order_and_repeated(weighted):
    # one frame per call in random order with repeats: blocks begun while both
    # accumulator slots are busy (slot 0 evicted), repeated frames (skipped),
    # completed-FIFO shifts at capacities 2 and 3
    rng = np.random.default_rng(31 + weighted)
    calls = [[int(t)] for t in rng.integers(0, 28, 48)]
    recs = [O.make_merge(2, 2), O.make_merge(2, 3), O.make_merge(2, 6)]
    _evict_run(H=3, FSEQ=1560, W=52, calls=calls, seed=5, weighted=weighted, recs=recs)


def test_evict_one_frame_mixed_kinds_and_patch_sizes():
    # on the regular grid: a Wave head, a patch-1 Veil head (one-frame blocks)
    # and an Anchor head beside patch-2 Veil heads
    recs = [O.make_merge(2, 4), O.make_cyclic(4, 2), O.make_merge(1, 3), O.make_stride(2, 3), O.make_merge(2, 2)]
    _evict_run(H=5, FSEQ=1560, W=52, calls=[[e] for e in range(20)], seed=6, weighted=True, recs=recs)


@pytest.mark.parametrize("how", ["permuted", "swapped_pair"])
def test_evict_one_frame_continues_block_by_its_stored_group_ids(how):
    # a block's stored group ids rewritten between its frames (host and
    # device alike): its later frames follow the stored ids, not the grid
    def tamper(ci, acc, dacc):
        if ci != 2:
            return
        gid = acc["gid"]
        rng = np.random.default_rng(9)
        for h in range(gid.shape[0]):
            for s in range(gid.shape[1]):
                if how == "permuted":
                    gid[h, s] = gid[h, s][rng.permutation(gid.shape[2])]
                else:  # tokens 0 and 60 (groups 0 and 4 of the grid) trade ids
                    gid[h, s, 0], gid[h, s, 60] = gid[h, s, 60].copy(), gid[h, s, 0].copy()
        dacc["gid"].copy_(to_dev(gid))
    _evict_run(H=2, FSEQ=1560, W=52, calls=[[e] for e in range(10)], seed=7, weighted=True, tamper=tamper)


def test_evict_one_frame_head_dim_64():
    # head_dim 64: 8 chunks per group row, twice the groups per workgroup
    calls = [[int(t)] for t in np.random.default_rng(12).integers(0, 20, 24)]
    _evict_run(H=3, FSEQ=1560, W=52, calls=calls, seed=12, weighted=True, D=64)


# ---- several frames per call (evict_frames_kernel on the regular grid) ------

def _grouped(ts, F):
    return [list(map(int, ts[i:i + F])) for i in range(0, len(ts), F)]


@pytest.mark.parametrize("F,weighted", [(5, False), (7, True), (8, True)])
def test_evict_frames_out_of_order_and_repeated(F, weighted):
    # calls of F frames in random order with repeats: blocks begun while both
    # slots are busy (slot 0 evicted), repeated frames, FIFO shifts at
    # capacities 2 and 3, and calls that open with both slots holding blocks
    rng = np.random.default_rng(41 + F)
    recs = [O.make_merge(2, 2), O.make_merge(2, 3), O.make_merge(2, 6)]
    _evict_run(H=3, FSEQ=1560, W=52, calls=_grouped(rng.integers(0, 28, 6 * F), F), seed=15, weighted=weighted,
               recs=recs)


def test_evict_frames_mixed_kinds_and_patch_sizes():
    # heads the several-frame path does not cover (Wave, patch-1 Veil, Anchor)
    # beside patch-2 Veil heads in every launch
    recs = [O.make_merge(2, 4), O.make_cyclic(4, 2), O.make_merge(1, 3), O.make_stride(2, 3), O.make_merge(2, 2)]
    _evict_run(H=5, FSEQ=1560, W=52, calls=_grouped(np.arange(24), 4), seed=16, weighted=True, recs=recs)


@pytest.mark.parametrize("how", ["permuted", "swapped_pair"])
def test_evict_frames_continue_block_by_its_stored_group_ids(how):
    # stored ids rewritten between calls: a call whose first frames continue
    # such a block runs the general tile for the head
    def tamper(ci, acc, dacc):
        if ci != 1:
            return
        gid = acc["gid"]
        rng = np.random.default_rng(19)
        for h in range(gid.shape[0]):
            for s in range(gid.shape[1]):
                if how == "permuted":
                    gid[h, s] = gid[h, s][rng.permutation(gid.shape[2])]
                else:
                    gid[h, s, 0], gid[h, s, 60] = gid[h, s, 60].copy(), gid[h, s, 0].copy()
        dacc["gid"].copy_(to_dev(gid))
    _evict_run(H=2, FSEQ=1560, W=52, calls=_grouped(np.arange(1, 16), 3), seed=17, weighted=True, tamper=tamper)


def test_evict_frames_head_dim_64():
    calls = _grouped(np.random.default_rng(18).integers(0, 20, 30), 5)
    _evict_run(H=3, FSEQ=1560, W=52, calls=calls, seed=18, weighted=True, D=64)


@pytest.mark.parametrize("F", [40, 64])
def test_evict_frames_long_calls(F):
    # the config-4 step as one call (40 frames), and the most frames a call
    # takes; a second call continues the blocks the first left open
    calls = [list(range(1, F + 1)), list(range(F + 1, F + 7))]
    recs = [O.make_merge(2, 6), O.make_merge(2, 2)]
    _evict_run(H=2, FSEQ=1560, W=52, calls=calls, seed=20 + F, weighted=True, recs=recs)
