"""Pins the oracle's data-movement ops and legacy planner with the
reference's own expectations (IF-LAB-PKU/Pyramid-Forcing
tests/test_scatter_copy.py:119-255, pyramidkv/csrc/pyramidkv_plan.cc:46-133
closed form)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O


def test_pos_override_reference_case():
    """test_scatter_copy.py:119-136"""
    pos = np.zeros((4680, 3), np.int64)
    pos[:, 0] = np.arange(4680) // 1560
    O.pos_override(pos, [0], [1560], [5])
    assert (pos[:1560, 0] == 5).all() and (pos[1560:, 0] != 5).any()
    assert pos[1560:3120, 0].tolist() == [1] * 1560


def test_write_frames_reference_case():
    """test_scatter_copy.py:138-166"""
    fs, d = 4, 8
    k = np.arange(3 * fs * d, dtype=np.float32).reshape(3 * fs, d)
    v = k + 1000
    pos = np.zeros((3 * fs, 3), np.int64)
    pos[:, 0] = np.arange(3 * fs) // fs
    pos[:, 1] = np.arange(3 * fs) % fs
    sk = np.full((4, fs, d), -1, np.float32)
    sv = np.full_like(sk, -2)
    sp = np.full((4, fs, 3), -3, np.int64)
    O.write_frames(k, v, pos, [[2, 0], [0, 3]], sk, sv, sp)
    assert np.array_equal(sk[0], k[8:12]) and np.array_equal(sv[0], v[8:12]) and np.array_equal(sp[0], pos[8:12])
    assert np.array_equal(sk[3], k[:4]) and np.array_equal(sp[3], pos[:4])
    assert (sk[1] == -1).all() and (sp[2] == -3).all()


# Expected (t, frame id) rows of the reference scenario (test_scatter_copy.py:169-255):
# current_t 10, rel_max 3, soft 0.5; segment 0 has t [1, 6, 8] with flag 1 (map),
# segment 1 has t [2, 9] with flag 4 (override to 7).  relative_softcap on t=6:
# rel 4 -> 3 + round(0.5) = 3 (half to even) -> t 7; on t=1: rel 9 -> 3 + round(3.0) = 6 -> t 4.
EXPECT_T = {"none": [1, 6, 8], "relative_clamp": [7, 7, 8], "relative_softcap": [4, 7, 8]}


@pytest.mark.parametrize("frame_mode", ["physical", "mapped"])
@pytest.mark.parametrize("mode", ["none", "relative_clamp", "relative_softcap"])
def test_refresh_readout_reference_case(frame_mode, mode):
    rng = np.random.default_rng(0)
    src_k = [rng.standard_normal((3, 8)).astype(np.float32), rng.standard_normal((2, 8)).astype(np.float32)]
    src_v = [rng.standard_normal((3, 8)).astype(np.float32), rng.standard_normal((2, 8)).astype(np.float32)]
    src_pos = [np.array([[1, 0, 0], [6, 0, 1], [8, 1, 0]], np.int64), np.array([[2, 2, 0], [9, 2, 1]], np.int64)]
    flags = [1, 4]
    if frame_mode == "physical":
        flags = [f | 2 for f in flags]
    dk = np.full((7, 8), -9, np.float32)
    dv = np.full((7, 8), -8, np.float32)
    dp = np.full((7, 3), -7, np.int64)
    df = np.full(7, -6, np.int64)
    O.refresh_readout(src_k, src_v, src_pos, [1, 5], [3, 2], flags, [0, 7], dk, dv, dp, df, 10, mode, 3, 0.5)
    assert np.array_equal(dk[1:4], src_k[0]) and np.array_equal(dv[5:7], src_v[1])
    assert (dk[0] == -9).all() and (dk[4] == -9).all()
    assert dp[1:4, 0].tolist() == EXPECT_T[mode] and dp[5:7, 0].tolist() == [7, 7]
    assert dp[1:4, 1:].tolist() == [[0, 0], [0, 1], [1, 0]]
    if frame_mode == "physical":
        assert df[1:4].tolist() == [1, 6, 8] and df[5:7].tolist() == [2, 9]
    else:
        assert df[1:4].tolist() == EXPECT_T[mode] and df[5:7].tolist() == [7, 7]
    assert df[0] == -6


def test_map_history_t_edges():
    assert O.map_history_t(10, 10, 2, 3, 0.5) == 10          # rel 0
    assert O.map_history_t(0, 10, 1, 3, 0.5) == 7
    assert O.map_history_t(0, 2, 1, 3, 0.5) == 0             # rel 2 within the limit
    assert O.map_history_t(0, 10, 2, 3, 0.25) == 10 - (3 + 2)  # 7 * 0.25 = 1.75 -> 2
    assert O.map_history_t(0, 9, 2, 3, 0.25) == 9 - (3 + 2)    # 6 * 0.25 = 1.5 -> 2 (half to even)
    assert O.map_history_t(0, 13, 2, 3, 0.25) == 13 - (3 + 2)  # 10 * 0.25 = 2.5 -> 2 (half to even)


def test_plan_legacy_closed_form():
    vc = np.zeros((2, 2, 3), np.int64)
    vc[0, 0] = (1, 2, 3)   # sink 1, middle 2, recent 3
    vc[0, 1] = (0, 0, 1)
    vc[1, 1] = (2, 0, 0)
    cu, sk, sg, sl, dst = O.plan_legacy(vc, fseq=10, max_sink=3, max_middle=5, max_recent=4)
    # head (0,0): sink 10, recent 30, middle 20 tokens, in that order
    assert sk[:3].tolist() == [0, 2, 1] and sl[:3].tolist() == [10, 30, 20] and dst[:3].tolist() == [0, 10, 40]
    assert sg[:3].tolist() == [0, 0, 0]
    assert sk[3:6].tolist() == [-1, 2, -1] and sg[4] == 1 * 4 and dst[4] == 60
    assert sk[6:9].tolist() == [-1, -1, -1]
    assert sk[9:12].tolist() == [0, -1, -1] and sg[9] == 3 * 3 and sl[9] == 20 and dst[9] == 70
    assert cu.tolist() == [0, 60, 70, 70, 90]
