"""Pins the oracle's per-head state machine (oracle/pkv_oracle.c:orc_state_update).

Known-answer vectors are the reference's own expectations from
tests/test_mega_state_update_ref.py:36-365 and
tests/test_mega_state_update_cuda.py:220-254 (IF-LAB-PKU/Pyramid-Forcing),
plus invariants that hold for any input (cursor ranges, FIFO saturation) and
a brute-force model of the Anchor ring checked over long random runs.
"""
import numpy as np
import pytest

from oracle import oracle as O

SKIP, MIDDLE, MERGE = O.DST_SKIP, O.DST_MIDDLE, O.DST_MERGE


def run(states, t_vals, pass_kind=1):
    b = O.states_to_bytes(states)
    desc = O.state_update(b, t_vals, pass_kind)
    return desc, O.bytes_to_states(b)


def test_record_size_matches_reference_struct():
    assert O.lib().orc_state_size() == 600 == O.STATE_DTYPE.itemsize
    off = {n: O.STATE_DTYPE.fields[n][1] for n in O.STATE_DTYPE.names}
    # offsets recomputed from anchor_store.cuh:62-132
    assert off["cyclic_cursor"] == 240 and off["tkey_slot"] == 248 and off["tkey_count"] == 440
    assert off["merge_completed_slot"] == 444 and off["merge_completed_count"] == 564
    assert off["merge_active_block_id"] == 568 and off["cached_num_groups"] == 596


def test_recent_emits_skip():
    d, _ = run([O.make_recent()], [10, 11, 12])
    assert d[0].tolist() == [SKIP] * 3 and d[1].tolist() == [-1] * 3
    assert d[2].tolist() == [0, 1, 2] and d[3].tolist() == [0, 0, 0]


def test_noisy_pass_skips_and_leaves_state():
    d, s = run([O.make_cyclic(6, 3)], [0, 1, 2], pass_kind=0)
    assert d[0].tolist() == [SKIP] * 3 and d[1].tolist() == [-1] * 3
    assert s[0]["cyclic_cursor"].tolist() == [0] * 6 and (s[0]["cyclic_slot"] == -1).all()


def test_cyclic_phase_assignment():
    d, s = run([O.make_cyclic(6, 3)], [0, 1, 2, 3, 4, 5])
    assert d[0].tolist() == [MIDDLE] * 6
    assert d[1].tolist() == [0, 3, 6, 9, 12, 15]
    assert s[0]["cyclic_cursor"].tolist() == [1] * 6


def test_cyclic_ring_wrap_and_overwrite():
    d, s = run([O.make_cyclic(2, 2)], [0, 2, 4, 6])
    assert d[1].tolist() == [0, 1, 0, 1] and s[0]["cyclic_cursor"][0] == 0
    _, s = run([O.make_cyclic(2, 2)], [0, 2, 4])
    assert s[0]["cyclic_t"][0] == 4 and s[0]["cyclic_t"][1] == 2


def test_stride_filter_and_fifo():
    d, s = run([O.make_stride(3, 4)], [0, 1, 2, 3, 4, 5, 6])
    assert d[0].tolist() == [MIDDLE, SKIP, SKIP, MIDDLE, SKIP, SKIP, MIDDLE]
    assert s[0]["tkey_count"] == 3 and s[0]["tkey_t"][:3].tolist() == [0, 3, 6]
    _, s = run([O.make_stride(1, 3)], [10, 11, 12, 13, 14])
    assert s[0]["tkey_count"] == 3 and s[0]["tkey_head"] == 2
    assert s[0]["tkey_t"][:3].tolist() == [13, 14, 12]


def test_lag_history():
    _, s = run([O.make_lag(4)], [5, 6, 7])
    assert s[0]["tkey_count"] == 3 and s[0]["tkey_t"][:3].tolist() == [5, 6, 7]
    _, s = run([O.make_lag(2)], [1, 2, 3, 4])
    assert s[0]["tkey_count"] == 2 and s[0]["tkey_t"][:2].tolist() == [3, 4]


def test_pyramid_forcing_combo_heads():
    states = [O.make_cyclic(6, 3) if h % 3 == 0 else O.make_stride(6, 4) if h % 3 == 1 else O.make_recent()
              for h in range(12)]
    d, _ = run(states, [6, 7, 8])
    assert d[3].tolist() == sum(([h] * 3 for h in range(12)), [])
    assert d[2].tolist() == [0, 1, 2] * 12
    for h in range(12):
        k, sl = d[0][h * 3:h * 3 + 3].tolist(), d[1][h * 3:h * 3 + 3].tolist()
        if h % 3 == 0:
            assert k == [MIDDLE] * 3 and sl == [0, 3, 6]
        elif h % 3 == 1:
            assert k == [MIDDLE, SKIP, SKIP] and sl[0] == 0
        else:
            assert k == [SKIP] * 3


def test_invariants_long_runs():
    _, s = run([O.make_cyclic(3, 2)], list(range(100)))
    assert all(0 <= c < 2 for c in s[0]["cyclic_cursor"].tolist())
    _, s = run([O.make_stride(1, 4)], list(range(20)))
    assert s[0]["tkey_count"] == 4
    _, s = run([O.make_lag(5)], list(range(20)))
    assert s[0]["tkey_count"] == 5


def test_merge_first_frame_and_finalize():
    d, s = run([O.make_merge(2, 6)], [0])
    assert d[0].tolist() == [MERGE] and d[1].tolist() == [-1]
    assert d[4].tolist() == [0] and d[5].tolist() == [0] and d[6].tolist() == [-1] and d[7].tolist() == [1]
    assert s[0]["merge_active_block_id"][0] == 0 and s[0]["merge_active_seen"][0][0] == 1
    assert s[0]["merge_active_complete_count"][0] == 1 and s[0]["merge_completed_count"] == 0
    d, s = run([O.make_merge(2, 6)], [0, 1, 2, 3])
    assert d[4].tolist() == [0] * 4 and d[5].tolist() == [0, 1, 2, 3]
    assert d[7].tolist() == [1, 0, 0, 0] and d[6].tolist() == [-1, -1, -1, 0]
    assert s[0]["merge_active_block_id"][0] == -1 and s[0]["merge_completed_count"] == 1
    assert s[0]["merge_completed_block_id"][0] == 0
    # C++-only fields (anchor_store_update.cu:191-214)
    assert s[0]["merge_completed_start_t"][0] == 0 and s[0]["merge_completed_end_t"][0] == 3
    assert s[0]["merge_completed_median_t"][0] == 1


def test_merge_two_blocks_and_fifo_eviction():
    d, s = run([O.make_merge(2, 6)], list(range(8)))
    assert s[0]["merge_completed_count"] == 2 and s[0]["merge_completed_block_id"][:2].tolist() == [0, 1]
    assert s[0]["merge_active_block_id"].tolist() == [-1, -1]
    assert d[7].tolist() == [1, 0, 0, 0, 1, 0, 0, 0] and d[6].tolist() == [-1, -1, -1, 0, -1, -1, -1, 1]
    _, s = run([O.make_merge(2, 2)], list(range(12)))
    assert s[0]["merge_completed_count"] == 2 and s[0]["merge_completed_block_id"][:2].tolist() == [1, 2]


def test_merge_slot_id_shift_quirk():
    """Completed-FIFO eviction shifts slot ids left and reuses the last index
    (anchor_store_update.cu:196-214): from the (cap+1)-th block on every slot
    id collapses towards cap-1."""
    _, s = run([O.make_merge(2, 4)], list(range(4 * 7)))
    st = s[0]
    assert st["merge_completed_count"] == 4
    assert st["merge_completed_block_id"][:4].tolist() == [3, 4, 5, 6]
    assert st["merge_completed_slot"][:4].tolist() == [3, 3, 3, 3]
    assert st["merge_completed_median_t"][:4].tolist() == [13, 17, 21, 25]


def test_merge_duplicate_skips_and_out_of_order():
    d, s = run([O.make_merge(2, 6)], [0, 0])
    assert d[0].tolist() == [MERGE, SKIP]  # device semantics: duplicate frame is skipped
    d, s = run([O.make_merge(2, 6)], [2, 0, 3, 1])
    assert d[5].tolist() == [2, 0, 3, 1] and d[4].tolist() == [0] * 4
    assert s[0]["merge_completed_count"] == 1


def test_merge_two_active_blocks():
    d, s = run([O.make_merge(2, 6)], [0, 4, 1, 5])
    assert d[4].tolist() == [0, 1, 0, 1]
    assert s[0]["merge_active_block_id"].tolist() == [0, 1]
    assert s[0]["merge_active_complete_count"].tolist() == [2, 2]


def test_stride_ring_matches_brute_force():
    """Anchor ring vs a direct list model: the slot of the k-th kept frame is
    k % capacity and the ring holds the last `capacity` kept frames."""
    rng = np.random.default_rng(3)
    for interval, cap in [(6, 4), (2, 5), (1, 24), (3, 1)]:
        t_vals = np.cumsum(rng.integers(1, 3, size=60))
        d, s = run([O.make_stride(interval, cap)], t_vals)
        kept = [int(t) for t in t_vals if t % interval == 0]
        assert s[0]["tkey_count"] == min(len(kept), cap)
        ring = {k % cap: t for k, t in enumerate(kept)}
        for slot, t in ring.items():
            assert s[0]["tkey_t"][slot] == t
        want_slots = [k % cap for k in range(len(kept))]
        got_slots = [int(x) for x, kk in zip(d[1], d[0]) if kk == MIDDLE]
        assert got_slots == want_slots
