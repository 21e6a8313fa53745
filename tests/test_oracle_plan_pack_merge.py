"""Pins the oracle's planner, pack (+RoPE), frame copy and Veil merge.

* Planner: known answers from the reference's tests/test_mega_plan_cuda.py
  (55-103, 129-187, 230-251; the recent-t expectations there are stale per
  the current mega_plan.cc:179-191 and are re-derived: recent segments carry
  t = -1), plus structural invariants of cu_seqlens / offsets.
* Pack: memcpy result equals the concatenation of the named pool slots
  (closed form, the reference's tests/test_pyramidkv_pack.py:40-160), the
  RoPE result is within one bf16 ulp of a complex128 rotation with the same
  tables, and inactive / zero-length segments write nothing.
* RoPE tables: rope_params closed form at t = 0 (identity) and the per-axis
  split sizes 22/21/21 for head_dim 128.
* Merge: the reference's vectors from tests/test_mega_merge_accum_cuda.py
  (55-288: per-token means, 2x2 patch means, counts, group positions) and a
  bit-exact sequential-float32 restatement for the accumulation order.
"""
import numpy as np
import pytest

from oracle import oracle as O


def geo(H=2, D=16, FSEQ=4, max_sink=2, max_middle=4, max_recent=2, L=1, chunks=4):
    return O.Geometry(L, H, D, FSEQ, max_sink, max_middle, max_recent, max_attend_chunks=chunks)


def plan(g, states, vc, t_list, mtc=None, **kw):
    sb = O.states_to_bytes(states)
    if mtc is None:
        mtc = np.zeros((g.num_heads, g.max_merge_blocks), np.int32)
    return O.plan_multi(g, sb, np.asarray(vc, np.int64).reshape(g.num_heads, 3), mtc, t_list, **kw)


def test_plan_empty():
    g = geo(H=2)
    cu, sk, sg, sl, dst, traw, tremap, total = plan(g, [O.make_recent()] * 2, np.zeros((2, 3)), [0])
    assert cu.tolist() == [0, 0, 0] and (sk == -1).all() and (sl == 0).all() and total == 0


def test_plan_sink_only():
    g = geo(H=2, FSEQ=4, max_sink=3)
    vc = np.zeros((2, 3)); vc[:, 0] = 3
    cu, sk, sg, sl, dst, traw, tremap, _ = plan(g, [O.make_recent()] * 2, vc, [10])
    assert cu.tolist() == [0, 12, 24]
    S = g.segs
    for h in range(2):
        b = h * S
        assert sk[b:b + 3].tolist() == [0, 0, 0] and sk[b + 3] == -1
        assert sg[b:b + 3].tolist() == [h * 3 + i for i in range(3)]
        assert sl[b:b + 3].tolist() == [4, 4, 4] and traw[b:b + 3].tolist() == [0, 1, 2]


def test_plan_stride_middle():
    g = geo(H=1, FSEQ=4, max_middle=4)
    s = [O.make_stride(6, 4)]
    b = O.states_to_bytes(s)
    O.state_update(b, [0, 6, 12], 1)
    cu, sk, sg, sl, dst, traw, tremap, _ = O.plan_multi(g, b, np.zeros((1, 3), np.int64),
                                                        np.zeros((1, 6), np.int32), [12])
    assert sk[:3].tolist() == [1, 1, 1] and sg[:3].tolist() == [0, 1, 2] and traw[:3].tolist() == [0, 6, 12]
    assert sk[3] == -1 and cu.tolist() == [0, 12]


def test_plan_cyclic_current_phase_only():
    g = geo(H=1, FSEQ=4, max_middle=4)
    b = O.states_to_bytes([O.make_cyclic(6, 3)])
    O.state_update(b, [0, 6, 7], 1)
    z, m = np.zeros((1, 3), np.int64), np.zeros((1, 6), np.int32)
    cu, sk, sg, sl, dst, traw, *_ = O.plan_multi(g, b, z, m, [6])
    assert sk[:2].tolist() == [1, 1] and sg[:2].tolist() == [0, 1] and traw[:2].tolist() == [0, 6]
    assert sk[2] == -1 and cu.tolist() == [0, 8]
    cu, sk, sg, sl, dst, traw, *_ = O.plan_multi(g, b, z, m, [7])
    # bucket stride is 4 in the plan (mega_plan.cc:199) while the update wrote
    # at phase * bucket_cap = 3: phase 1 reads slots 4..6, which are empty
    assert sk[0] == -1 and cu.tolist() == [0, 0]
    cu, sk, *_ = O.plan_multi(g, b, z, m, [8])
    assert sk[0] == -1 and cu.tolist() == [0, 0]


def test_plan_cyclic_bucket_cap_4_consistent():
    g = geo(H=1, FSEQ=4, max_middle=24)
    b = O.states_to_bytes([O.make_cyclic(6, 4)])
    O.state_update(b, [1, 7, 13], 1)
    cu, sk, sg, sl, dst, traw, *_ = O.plan_multi(g, b, np.zeros((1, 3), np.int64), np.zeros((1, 6), np.int32),
                                                 [19])
    assert sk[:3].tolist() == [1, 1, 1] and sg[:3].tolist() == [4, 5, 6] and traw[:3].tolist() == [1, 7, 13]


def test_plan_tremap_sink_sync_recent_raw():
    g = geo(H=1)
    vc = np.array([[2, 0, 1]])
    cu, sk, sg, sl, dst, traw, tremap, _ = plan(g, [O.make_recent()], vc, [10])
    assert traw[:3].tolist() == [0, 1, -1] and tremap[:3].tolist() == [10, 10, -1]


def test_plan_window_clamp():
    g = geo(H=1, max_sink=4)
    vc = np.array([[4, 0, 0]])
    *_, tremap, _ = plan(g, [O.make_recent()], vc, [100], sink_mode=1, cmin=2, cmax=3)
    assert tremap[:4].tolist() == [97] * 4
    # production remap window_clamp(18, 21) (configs/pyramid-forcing.yaml:73-75)
    assert [O.map_sink_time(t, 1, 18, 21, 0) for t in (0, 18, 20, 21, 40, 117)] == [0, 0, 0, 0, 19, 96]


def test_plan_merge_anchor_and_sink_dedup():
    g = geo(H=1, FSEQ=8, max_sink=3, max_middle=24, max_recent=4)
    st = O.make_merge(2, 4, sink_capacity=3)
    b = O.states_to_bytes([st])
    O.state_update(b, list(range(12)), 1)
    mtc = np.array([[5, 6, 7, 0, 0, 0]], np.int32)
    vc = np.array([[3, 0, 4]])
    cu, sk, sg, sl, dst, traw, tremap, total = O.plan_multi(g, b, vc, mtc, [12])
    # sink 3 + recent 4 + merged blocks 1, 2 (block 0 has start_t 0 and is dropped)
    assert sk[:10].tolist() == [0, 0, 0, 2, 2, 2, 2, 3, 3, -1]
    assert sl[7:9].tolist() == [6, 7] and tremap[7:9].tolist() == [5, 9] and traw[7:9].tolist() == [0, 0]
    assert total == 7 * 8 + 13


@pytest.mark.parametrize("seed", range(4))
def test_plan_offsets_invariants(seed):
    rng = np.random.default_rng(seed)
    g = geo(H=5, FSEQ=7, max_sink=3, max_middle=24, max_recent=4, chunks=3)
    states = []
    for h in range(5):
        kind = rng.integers(0, 4)
        s = [O.make_recent(1), O.make_cyclic(6, 4, 1), O.make_stride(6, 4, 3), O.make_lag(5, 2)][kind]
        states.append(s)
    b = O.states_to_bytes(states)
    for blk in range(8):
        O.state_update(b, [3 * blk, 3 * blk + 1, 3 * blk + 2], 1)
    vc = np.stack([rng.integers(0, 4, 5), np.zeros(5), rng.integers(0, 5, 5)], 1)
    cu, sk, sg, sl, dst, traw, tremap, total = O.plan_multi(g, b, vc, np.zeros((5, 6), np.int32), [24, 25, 26])
    S = g.segs
    assert cu[0] == 0 and (np.diff(cu) >= 0).all() and total == cu[-1] == sl.sum()
    for pair in range(15):
        seg = slice(pair * S, (pair + 1) * S)
        act = sk[seg] >= 0
        n = act.sum()
        assert act[:n].all() and not act[n:].any()  # active entries are a prefix
        assert (dst[seg][:n] == cu[pair] + np.concatenate([[0], np.cumsum(sl[seg][:n])[:-1]])).all()
        assert cu[pair + 1] - cu[pair] == sl[seg][:n].sum()


def _rand_pools(g, rng):
    L, H, D, FS = g.num_layers, g.num_heads, g.head_dim, g.frame_seqlen
    mk = lambda *s: rng.integers(0, 1 << 16, size=s, dtype=np.uint16) & 0xBFFF  # finite bf16
    return dict(
        sink_k=mk(L, H, g.max_sink, FS, D), sink_v=mk(L, H, g.max_sink, FS, D),
        middle_k=mk(L, H, g.max_middle, FS, D), middle_v=mk(L, H, g.max_middle, FS, D),
        recent_k=mk(L, H, g.max_recent, FS, D), recent_v=mk(L, H, g.max_recent, FS, D),
        merge_k=mk(L, H, 6, g.max_merge_tokens, D), merge_v=mk(L, H, 6, g.max_merge_tokens, D),
        sink_pos=rng.integers(0, 40, (L, H, g.max_sink, FS, 3)).astype(np.int64),
        middle_pos=rng.integers(0, 40, (L, H, g.max_middle, FS, 3)).astype(np.int64),
        recent_pos=rng.integers(0, 40, (L, H, g.max_recent, FS, 3)).astype(np.int64),
        merge_pos=rng.integers(0, 40, (L, H, 6, g.max_merge_tokens, 3)).astype(np.int64))


def _rand_segments(g, rng, n):
    kinds = rng.integers(-1, 4, n).astype(np.int32)
    slots = {0: g.max_sink, 1: g.max_middle, 2: g.max_recent, 3: 6}
    sg = np.array([rng.integers(0, g.num_layers * g.num_heads * slots[max(k, 0)]) for k in kinds], np.int32)
    sl = np.array([rng.integers(0, (g.max_merge_tokens if k == 3 else g.frame_seqlen) + 1) for k in kinds],
                  np.int32)
    sl[kinds < 0] = rng.integers(0, 5, (kinds < 0).sum())
    dst = np.concatenate([[0], np.cumsum(np.where(kinds >= 0, sl, 0))[:-1]]).astype(np.int32)
    return kinds, sg, sl, dst


def test_pack_memcpy_is_concatenation():
    rng = np.random.default_rng(0)
    g = geo(L=2, H=3, D=16, FSEQ=8, max_sink=2, max_middle=4, max_recent=2)
    g.max_merge_tokens = 8
    pools = _rand_pools(g, rng)
    sk, sg, sl, dst = _rand_segments(g, rng, 40)
    k, v, p = O.pack(pools, g, sk, sg, sl, dst)
    names = ["sink", "middle", "recent", "merge"]
    for j in range(len(sk)):
        if sk[j] < 0 or sl[j] <= 0:
            continue
        n = names[sk[j]]
        stride = 8
        fk = pools[n + "_k"].reshape(-1, 16)[sg[j] * stride:sg[j] * stride + sl[j]]
        fv = pools[n + "_v"].reshape(-1, 16)[sg[j] * stride:sg[j] * stride + sl[j]]
        fp = pools[n + "_pos"].reshape(-1, 3)[sg[j] * stride:sg[j] * stride + sl[j]]
        assert (k[dst[j]:dst[j] + sl[j]] == fk).all() and (v[dst[j]:dst[j] + sl[j]] == fv).all()
        assert (p[dst[j]:dst[j] + sl[j]] == fp).all()
    used = int(np.where(sk >= 0, sl, 0).sum())
    assert (k[used:] == 0).all()


def test_pack_inactive_and_zero_length_write_nothing():
    rng = np.random.default_rng(1)
    g = geo(L=1, H=1, D=16, FSEQ=8)
    pools = _rand_pools(g, rng)
    k, v, p = O.pack(pools, g, [-1, 0], [0, 0], [8, 0], [0, 0])
    assert (k == 0).all() and (v == 0).all() and (p == 0).all()


def test_rope_tables_closed_form():
    ft, fy, fx = O.rope_tables(128)
    assert ft.shape == (1024, 44) and fy.shape == (1024, 42) and fx.shape == (1024, 42)
    assert (ft[0, 0::2] == 1).all() and (ft[0, 1::2] == 0).all()  # row 0 is the identity rotation
    # row t, pair j of the t-axis table is exp(i t theta^{-2j/44})
    t, j = 17, 5
    ang = t * 10000.0 ** (-2 * j / 44)
    assert ft[t, 2 * j] == np.float32(np.cos(ang)) and ft[t, 2 * j + 1] == np.float32(np.sin(ang))
    # magnitudes are 1 to fp32 precision
    mag = ft[:, 0::2].astype(np.float64) ** 2 + ft[:, 1::2].astype(np.float64) ** 2
    assert np.abs(mag - 1).max() < 1e-6


def test_rope_matches_complex128_within_one_ulp():
    rng = np.random.default_rng(2)
    tables = O.rope_tables(128)
    n = 300
    kf = rng.standard_normal((n, 128)).astype(np.float32)
    k = O.f32_to_bf16(kf)
    pos = np.stack([rng.integers(-3, 1100, n), rng.integers(0, 30, n), rng.integers(0, 52, n)], 1).astype(np.int64)
    got = O.bf16_to_f32(O.rope_apply(k, pos, tables))
    ft, fy, fx = tables
    z = O.bf16_to_f32(k).astype(np.float64).reshape(n, 64, 2)
    zc = z[..., 0] + 1j * z[..., 1]
    rows = [np.clip(pos[:, 0], 0, 1023), np.clip(pos[:, 1], 0, 1023), np.clip(pos[:, 2], 0, 1023)]
    f = np.concatenate([ft[rows[0]].reshape(n, 22, 2), fy[rows[1]].reshape(n, 21, 2),
                        fx[rows[2]].reshape(n, 21, 2)], 1).astype(np.float64)
    want = zc * (f[..., 0] + 1j * f[..., 1])
    want = np.stack([want.real, want.imag], -1).reshape(n, 128)
    ulp = np.abs(O.bf16_to_f32(O.f32_to_bf16(want.astype(np.float32))) - want)
    err = np.abs(got - want)
    # bf16 rounding of the exact value plus one bf16 ulp of slack
    tol = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
    assert (err <= ulp + tol).all()


def _merge_layer_arrays(H, FSEQ, D, MTPA=420):
    return dict(sum_k=np.zeros((H, 2, MTPA, D), np.float32), sum_v=np.zeros((H, 2, MTPA, D), np.float32),
                pos=np.zeros((H, 2, MTPA, 3), np.int64), gid=np.zeros((H, 2, FSEQ), np.int32),
                tpg=np.zeros((H, 2, MTPA), np.float32), ng=np.zeros((H, 2), np.int32),
                wsum=np.zeros((H, 2), np.float32), mk=np.zeros((H, 6, MTPA, D), np.uint16),
                mv=np.zeros((H, 6, MTPA, D), np.uint16), mpos=np.zeros((H, 6, MTPA, 3), np.int64),
                mtc=np.zeros((H, 6), np.int32))


def _drive_merge(H, FSEQ, D, t_vals, pos, seed, weights=None):
    states = O.states_to_bytes([O.make_merge(2, 6) for _ in range(H)])
    desc = O.state_update(states, t_vals, 1)
    F = len(t_vals)
    rng = np.random.default_rng(seed)
    nk = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
    nv = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
    acc = _merge_layer_arrays(H, FSEQ, D)
    O.merge_accum(states, nk, nv, np.ascontiguousarray(pos), desc, acc, weights)
    return nk, nv, acc


def test_merge_identity_grouping_means():
    H, D, FSEQ, F = 2, 16, 8, 4
    pos = np.zeros((F, H, FSEQ, 3), np.int64)
    pos[..., 0] = np.arange(F).reshape(F, 1, 1)
    pos[..., 1] = 2 * np.arange(FSEQ)
    nk, nv, acc = _drive_merge(H, FSEQ, D, [0, 1, 2, 3], pos, 42)
    want = O.bf16_to_f32(nk).astype(np.float64).mean(0)
    got = O.bf16_to_f32(acc["mk"][:, 0, :FSEQ])
    assert np.abs(got - want).max() < 2e-2
    assert acc["mtc"][:, 0].tolist() == [FSEQ] * H
    assert acc["mpos"][0, 0, :FSEQ].tolist() == [[0, 2 * g, 0] for g in range(FSEQ)]


def test_merge_2x2_patches():
    H, D, FSEQ, F = 1, 16, 8, 4
    coords = [(0, 0), (0, 1), (1, 0), (1, 1), (2, 0), (2, 1), (3, 0), (3, 1)]
    pos = np.zeros((F, H, FSEQ, 3), np.int64)
    pos[..., 0] = np.arange(F).reshape(F, 1, 1)
    pos[..., 1:] = np.array(coords)
    nk, nv, acc = _drive_merge(H, FSEQ, D, [0, 1, 2, 3], pos, 11)
    kf = O.bf16_to_f32(nk)
    for g, toks in enumerate([slice(0, 4), slice(4, 8)]):
        want = kf[:, 0, toks].reshape(-1, D).astype(np.float64).mean(0)
        assert np.abs(O.bf16_to_f32(acc["mk"][0, 0, g]) - want).max() < 2e-2
    assert acc["mtc"][0, 0] == 2 and acc["mpos"][0, 0, :2].tolist() == [[0, 0, 0], [0, 2, 0]]


def test_merge_two_blocks_positions():
    H, D, FSEQ, F = 1, 16, 8, 8
    pos = np.zeros((F, H, FSEQ, 3), np.int64)
    pos[..., 0] = np.arange(F).reshape(F, 1, 1)
    pos[..., 1] = 2 * np.arange(FSEQ)
    nk, nv, acc = _drive_merge(H, FSEQ, D, list(range(8)), pos, 7)
    kf = O.bf16_to_f32(nk).astype(np.float64)
    assert np.abs(O.bf16_to_f32(acc["mk"][0, 1, :FSEQ]) - kf[4:8, 0].mean(0)).max() < 2e-2
    assert acc["mtc"][0, :2].tolist() == [FSEQ, FSEQ]
    assert acc["mpos"][0, 0, 0, 0] == 0 and acc["mpos"][0, 1, 0, 0] == 4


def test_merge_sequential_fp32_bit_exact():
    """Production grid (30x52, patch 2): each anchor element is the float32
    sequence ((((0 + x_a) + x_b) + x_c) + x_d) over frames in order and
    tokens ascending, times 1/16."""
    H, D, FSEQ, W = 1, 8, 1560, 52
    pos = np.zeros((4, H, FSEQ, 3), np.int64)
    pos[..., 0] = 4 + np.arange(4).reshape(4, 1, 1)
    pos[..., 1] = np.arange(FSEQ) // W
    pos[..., 2] = np.arange(FSEQ) % W
    nk, nv, acc = _drive_merge(H, FSEQ, D, [4, 5, 6, 7], pos, 5)
    kf = O.bf16_to_f32(nk)
    assert acc["mtc"][0, 0] == 390
    for g in (0, 25, 26, 200, 389):
        gy, gx = divmod(g, 26)
        toks = sorted([(2 * gy + dy) * W + 2 * gx + dx for dy in (0, 1) for dx in (0, 1)])
        s = np.zeros(D, np.float32)
        for f in range(4):
            for t in toks:
                s = (s + kf[f, 0, t]).astype(np.float32)
        want = O.f32_to_bf16((s * np.float32(1.0 / 16.0)).astype(np.float32))
        assert (acc["mk"][0, 0, g] == want).all()
        assert acc["mpos"][0, 0, g].tolist() == [4, 2 * gy, 2 * gx]


def test_merge_weighted_unit_weights_equal_reference():
    H, D, FSEQ = 2, 16, 12
    pos = np.zeros((4, H, FSEQ, 3), np.int64)
    pos[..., 0] = np.arange(4).reshape(4, 1, 1)
    pos[..., 1] = np.arange(FSEQ) // 4
    pos[..., 2] = np.arange(FSEQ) % 4
    _, _, a = _drive_merge(H, FSEQ, D, [0, 1, 2, 3], pos, 9)
    _, _, b = _drive_merge(H, FSEQ, D, [0, 1, 2, 3], pos, 9, weights=np.ones(4, np.float32))
    assert (a["mk"] == b["mk"]).all() and (a["mv"] == b["mv"]).all()
    _, _, c = _drive_merge(H, FSEQ, D, [0, 1, 2, 3], pos, 9, weights=np.array([0.5, 1, 0.25, 1], np.float32))
    assert not (a["mk"] == c["mk"]).all()
