"""Pins oracle.MegaCacheRef (the CPU model of MegaCache.update's sink /
recent routing and noisy/clean commit) with the reference's own scenarios
and expectations from tests/test_mega_cache_noisy_clean.py:41-231 and the
closed form "sink fills first up to min(cap, max_sink); recent keeps the
last max_recent frames, oldest in slot 0" (IF-LAB-PKU/Pyramid-Forcing,
pyramidkv/_mega_cache.py:217-323, 406-414)."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O
from pyramidkv import _mega_state_ops as S
from pyramidkv._mega_cache import _composition_to_perhead_state
from pyramidkv import HeadComposition, RecentStrategy, StrideStrategy


def _ref_cache(comps_row, D=16, FS=4, max_sink=3, max_middle=8, max_recent=4, W=2):
    st = S.pack_states([_composition_to_perhead_state(c) for c in comps_row]).view(np.uint8).reshape(1, -1)
    caps = np.array([[c.sink_frames for c in comps_row]], np.int64)
    g = O.Geometry(1, len(comps_row), D, FS, max_sink, max_middle, max_recent, max_attend_chunks=3)
    return O.MegaCacheRef(g, st, caps, spatial_width=W), g


def _rand(rng, F, FS, H, D):
    return O.f32_to_bf16(rng.standard_normal((F * FS, H, D)).astype(np.float32))


def _stride_comp():
    return HeadComposition("stride", 1, 3, 4, [StrideStrategy(interval=1, capacity=8)])


def test_noisy_iterations_dont_advance_committed_then_clean_commits():
    """test_mega_cache_noisy_clean.py:41-108"""
    rng = np.random.default_rng(7)
    ref, g = _ref_cache([_stride_comp()])
    F, FS, D = 3, 4, 16
    for _ in range(4):
        ref.update(0, _rand(rng, F, FS, 1, D), _rand(rng, F, FS, 1, D), 0, "noisy")
        assert ref.valid_count[0, 0, 0] == F
        assert ref.committed_vc[0, 0, 0] == 0
    assert O.bytes_to_states(ref.states[0])["tkey_count"][0] == 0
    ck, cv = _rand(rng, F, FS, 1, D), _rand(rng, F, FS, 1, D)
    ref.update(0, ck, cv, 0, "clean")
    assert ref.valid_count[0, 0, 0] == F and ref.committed_vc[0, 0, 0] == F
    assert np.array_equal(ref.sink_k[0, 0, 0], ck.reshape(F, FS, 1, D)[0, :, 0, :])
    assert O.bytes_to_states(ref.states[0])["tkey_count"][0] == F
    # the middle pool got the clean frames (stride interval 1: every frame)
    for f in range(F):
        assert np.array_equal(ref.middle_k[0, 0, f], ck.reshape(F, FS, 1, D)[f, :, 0, :])


def test_block_2_noisy_uses_block_1_committed_baseline():
    """test_mega_cache_noisy_clean.py:111-159"""
    rng = np.random.default_rng(11)
    ref, g = _ref_cache([_stride_comp()])
    F, FS, D = 3, 4, 16
    ref.update(0, _rand(rng, F, FS, 1, D), _rand(rng, F, FS, 1, D), 0, "clean")
    assert ref.committed_vc[0, 0, 0] == 3 and ref.committed_vc[0, 0, 2] == 0
    ref.update(0, _rand(rng, F, FS, 1, D), _rand(rng, F, FS, 1, D), 3 * FS, "noisy")
    assert ref.valid_count[0, 0, 2] == 3 and ref.committed_vc[0, 0, 2] == 0
    kb = _rand(rng, F, FS, 1, D)
    ref.update(0, kb, _rand(rng, F, FS, 1, D), 3 * FS, "noisy")
    assert ref.valid_count[0, 0, 2] == 3 and ref.committed_vc[0, 0, 2] == 0
    for f in range(F):
        assert np.array_equal(ref.recent_k[0, 0, f], kb.reshape(F, FS, 1, D)[f, :, 0, :])


def test_recent_fifo_no_noisy_contamination_across_blocks():
    """test_mega_cache_noisy_clean.py:162-231: after the FIFO shift, recent
    slot 0 holds the clean last frame of the previous block."""
    rng = np.random.default_rng(101)
    comp = HeadComposition("recent_only", -1, 1, 4, [RecentStrategy()])
    ref, g = _ref_cache([comp], max_sink=1)
    F, FS, D = 3, 4, 16
    clean = [(_rand(rng, F, FS, 1, D), _rand(rng, F, FS, 1, D)) for _ in range(3)]
    for b in range(2):
        ref.update(0, *clean[b], b * F * FS, "clean")
    before = ref.recent_k[0, 0].copy()
    # closed form after two blocks: sink = frame 0, recent = frames 2, 3, 4, 5
    allk = np.concatenate([clean[0][0].reshape(F, FS, 1, D), clean[1][0].reshape(F, FS, 1, D)])[:, :, 0, :]
    assert np.array_equal(ref.sink_k[0, 0, 0], allk[0])
    assert np.array_equal(before, allk[2:6])
    noisy = [(_rand(rng, F, FS, 1, D), _rand(rng, F, FS, 1, D)) for _ in range(3)]
    for k_n, v_n in noisy:
        ref.update(0, k_n, v_n, 2 * F * FS, "noisy")
    ref.update(0, *clean[2], 2 * F * FS, "clean")
    after = ref.recent_k[0, 0]
    assert np.array_equal(after[0], before[3])
    assert np.array_equal(after[1:], clean[2][0].reshape(F, FS, 1, D)[:, :, 0, :])
    for k_n, _ in noisy:
        assert not np.array_equal(after[0], k_n.reshape(F, FS, 1, D)[F - 1, :, 0, :])


def test_positions_are_frame_and_grid_coordinates():
    """_mega_cache.py:210-215: pos = (t0 + f, tok // W, tok % W)."""
    rng = np.random.default_rng(3)
    comp = HeadComposition("recent_only", -1, 1, 4, [RecentStrategy()])
    ref, g = _ref_cache([comp], max_sink=1, FS=6, W=3)
    ref.update(0, _rand(rng, 2, 6, 1, 16), _rand(rng, 2, 6, 1, 16), 5 * 6, "clean")
    tok = np.arange(6)
    assert ref.sink_pos[0, 0, 0].tolist() == [[5, t // 3, t % 3] for t in tok]
    assert ref.recent_pos[0, 0, 0].tolist() == [[6, t // 3, t % 3] for t in tok]


def test_update_frames_closed_form_multi_head():
    """orc_update_frames (pyramidkv_update.cu:21-110) against numpy indexing
    of the [F, H, FSEQ, D] source and the [L, H, slots, FSEQ, D] pools: every
    write lands new_k / new_v / new_pos[src_frame, src_head] in slot
    slot_global of its pool; SKIP (-1), MERGE (5, which the reference's
    caller masks before the op) and out-of-range writes leave every pool as
    it was, and so do all slots no write names.  F != H, so a frame / head
    swap in the source offset, or a pool mix-up, fails."""
    rng = np.random.default_rng(11)
    L, H, F, FS, D = 2, 3, 4, 24, 32
    slots = dict(sink=2, middle=5, recent=3)
    pools = {}
    for n, s in slots.items():
        pools[n + "_k"] = rng.integers(0, 1 << 16, (L, H, s, FS, D)).astype(np.uint16)
        pools[n + "_v"] = rng.integers(0, 1 << 16, (L, H, s, FS, D)).astype(np.uint16)
        pools[n + "_pos"] = rng.integers(-9, 9, (L, H, s, FS, 3)).astype(np.int64)
    before = {k: v.copy() for k, v in pools.items()}
    nk = rng.integers(0, 1 << 16, (F, H, FS, D)).astype(np.uint16)
    nv = rng.integers(0, 1 << 16, (F, H, FS, D)).astype(np.uint16)
    npos = rng.integers(100, 200, (F, H, FS, 3)).astype(np.int64)
    names = ["sink", "middle", "recent"]
    # distinct in-range destinations for kinds 0-2, plus SKIP / MERGE / out-of-range entries
    writes, used = [], set()
    while len(writes) < 14:
        k = int(rng.integers(0, 3))
        sg = int(rng.integers(0, L * H * slots[names[k]]))
        if (k, sg) not in used:
            used.add((k, sg))
            writes.append((k, sg, int(rng.integers(0, F)), int(rng.integers(0, H))))
    noop = [(-1, 0, 0, 0), (5, 1, 1, 1), (5, 0, 3, 2), (0, L * H * slots["sink"], 0, 0), (2, -1, 0, 0),
            (1, 0, F, 0), (1, 1, 0, H)]
    allw = writes + noop
    order = rng.permutation(len(allw))
    kind, sg, fr, hd = (np.array([allw[i][j] for i in order], np.int32) for j in range(4))
    O.update_frames(pools, nk, nv, npos, H, FS, D, kind, sg, fr, hd)
    want = {k: v.copy() for k, v in before.items()}
    for k, s, f, h in writes:
        n = names[k]
        l, hh, slot = np.unravel_index(s, (L, H, slots[n]))
        want[n + "_k"][l, hh, slot] = nk[f, h]
        want[n + "_v"][l, hh, slot] = nv[f, h]
        want[n + "_pos"][l, hh, slot] = npos[f, h]
    for name in pools:
        assert np.array_equal(pools[name], want[name]), name
    # the writes did land (the pools are not merely unchanged)
    assert sum(int((pools[n] != before[n]).any(axis=(-2, -1)).sum()) for n in pools if n.endswith("_k")) == 14
    # without positions only K and V move
    p2 = {k: v.copy() for k, v in before.items()}
    O.update_frames(p2, nk, nv, None, H, FS, D, kind, sg, fr, hd)
    for n in names:
        assert np.array_equal(p2[n + "_pos"], before[n + "_pos"])
        assert np.array_equal(p2[n + "_k"], want[n + "_k"])
