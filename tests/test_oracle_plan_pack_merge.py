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
* Weighted merge (config 4): the float64 closed form sum(w x) / (count *
  sum(w)) per patch group, for blocks spanning several calls; the planted
  mistakes (w applied twice, count * frames divisor) fail the same bar.
* attention_ref: closed forms (uniform keys, one dominant key, two-key
  logistic weights, the scale) and the sequence selection of the ragged
  layouts.
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


def _weighted_rollout(H, D, W, rows, calls, weights, seed):
    """Drive the oracle's state machine + merge accumulate over consecutive
    clean calls (frame lists in `calls`, per-frame weights in `weights`) on
    a regular rows x W grid; returns the frames, the per-call finalize
    descriptors and the accumulator dict."""
    FSEQ = rows * W
    states = O.states_to_bytes([O.make_merge(2, 6) for _ in range(H)])
    acc = _merge_layer_arrays(H, FSEQ, D)
    rng = np.random.default_rng(seed)
    frames, fins = {}, []
    for ts in calls:
        F = len(ts)
        desc = O.state_update(states, ts, 1)
        pos = np.zeros((F, H, FSEQ, 3), np.int64)
        pos[..., 0] = np.array(ts).reshape(F, 1, 1)
        pos[..., 1] = np.arange(FSEQ) // W
        pos[..., 2] = np.arange(FSEQ) % W
        nk = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
        nv = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
        w = np.array([weights[t] for t in ts], np.float32)
        O.merge_accum(states, nk, nv, np.ascontiguousarray(pos), desc, acc, w)
        for i, t in enumerate(ts):
            frames[t] = (O.bf16_to_f32(nk[i]).astype(np.float64), O.bf16_to_f32(nv[i]).astype(np.float64))
        fins.append((ts, desc[6].reshape(H, F)))
    return frames, fins, acc


def _closed_form_block(frames, weights, block, W, rows, p=2, wpow=1, divisor="sum_w"):
    """float64 sum_f w_f * sum_{tok in g} x / (|g| * sum_f w_f) per 2x2 patch
    group g of `block` (4 frames).  wpow / divisor plant the mistakes the
    test must reject (w applied twice; count * frames as the divisor)."""
    ts = list(range(4 * block, 4 * block + 4))
    ws = np.array([weights[t] for t in ts], np.float64)
    cols, grows = W // p, rows // p
    H, FSEQ, D = frames[ts[0]][0].shape
    out_k = np.zeros((H, grows * cols, D))
    out_v = np.zeros((H, grows * cols, D))
    for g in range(grows * cols):
        gy, gx = divmod(g, cols)
        toks = [(p * gy + dy) * W + p * gx + dx for dy in range(p) for dx in range(p)]
        sk = sum(ws[i] ** wpow * frames[t][0][:, toks].sum(1) for i, t in enumerate(ts))
        sv = sum(ws[i] ** wpow * frames[t][1][:, toks].sum(1) for i, t in enumerate(ts))
        div = len(toks) * (ws.sum() if divisor == "sum_w" else len(ts))
        out_k[:, g], out_v[:, g] = sk / div, sv / div
    return out_k, out_v


def test_merge_weighted_closed_form_across_calls():
    """config-4's running weighted average: every finalized anchor equals
    sum(w x) / (count * sum(w)) of its block in float64 within the north
    star's 2e-2 / 2e-3, with blocks that span several calls (weights and
    their running sum carried between calls).  The reference operation is
    the w == 1 case (mega_merge_accum.cu:193-249)."""
    H, D, W, rows = 3, 16, 8, 6
    rng = np.random.default_rng(123)
    weights = {t: float(np.float32(rng.uniform(0.1, 1.0))) for t in range(8)}
    calls = [[0], [1, 2], [3, 4], [5, 6, 7]]
    frames, fins, acc = _weighted_rollout(H, D, W, rows, calls, weights, seed=4)
    done = {}
    for ts, fin in fins:
        for i, t in enumerate(ts):
            for h in range(H):
                if fin[h, i] >= 0:
                    done.setdefault(t // 4, {})[h] = int(fin[h, i])
    assert sorted(done) == [0, 1]
    ng = (rows // 2) * (W // 2)
    for block in (0, 1):
        want_k, want_v = _closed_form_block(frames, weights, block, W, rows)
        wrong = [_closed_form_block(frames, weights, block, W, rows, wpow=2),
                 _closed_form_block(frames, weights, block, W, rows, divisor="frames")]
        for h in range(H):
            slot = done[block][h]
            assert acc["mtc"][h, slot] == ng
            got_k = O.bf16_to_f32(acc["mk"][h, slot, :ng]).astype(np.float64)
            got_v = O.bf16_to_f32(acc["mv"][h, slot, :ng]).astype(np.float64)
            for got, want in ((got_k, want_k[h]), (got_v, want_v[h])):
                err = np.abs(got - want)
                assert err.max() < 2e-2 and err.mean() < 2e-3, (block, h, err.max(), err.mean())
            # the planted mistakes fail the same bar
            for wk, wv in wrong:
                e = np.abs(got_k - wk[h])
                assert e.max() >= 2e-2 or e.mean() >= 2e-3
            assert acc["mpos"][h, slot, 0].tolist() == [4 * block, 0, 0]


def test_merge_weighted_single_frame_calls_and_unit_weight_block():
    """40 single-frame calls (the config-4 eviction pattern, 10 blocks):
    each anchor against the float64 weighted mean; a block whose weights
    are all 1 reduces to the plain mean."""
    H, D, W, rows = 2, 8, 4, 4
    rng = np.random.default_rng(77)
    weights = {t: float(np.float32(rng.uniform(0.1, 1.0))) for t in range(40)}
    for t in range(8, 12):
        weights[t] = 1.0
    frames, fins, acc = _weighted_rollout(H, D, W, rows, [[t] for t in range(40)], weights, seed=8)
    ng = (rows // 2) * (W // 2)
    # which block each anchor slot holds last, from the finalize descriptors
    # (the completed FIFO's slot-id shift keeps rewriting its last slot)
    held = {}
    for ts, fin in fins:
        for h in range(H):
            if fin[h, 0] >= 0:
                held[(h, int(fin[h, 0]))] = ts[0] // 4
    assert len(held) == 6 * H and sorted(set(held.values())) == [0, 1, 2, 3, 4, 9]
    for (h, slot), block in held.items():
        want_k, _ = _closed_form_block(frames, weights, block, W, rows)
        got = O.bf16_to_f32(acc["mk"][h, slot, :ng]).astype(np.float64)
        err = np.abs(got - want_k[h])
        assert err.max() < 2e-2 and err.mean() < 2e-3
        assert acc["mpos"][h, slot, 0, 0] == 4 * block
    # the unit-weight block (t = 8..11) was evicted from the FIFO; rerun it alone
    frames1, _, acc1 = _weighted_rollout(H, D, W, rows, [[8], [9], [10], [11]],
                                         {t: 1.0 for t in range(8, 12)}, seed=8)
    k = np.stack([frames1[t][0] for t in range(8, 12)])  # [4, H, FSEQ, D]
    plain = k.reshape(4, H, rows // 2, 2, W // 2, 2, D).transpose(1, 2, 4, 0, 3, 5, 6)
    plain = plain.reshape(H, ng, 16, D).mean(2)
    got = O.bf16_to_f32(acc1["mk"][:, 0, :ng]).astype(np.float64)
    assert np.abs(got - plain).max() < 2e-2


def test_attention_ref_closed_forms():
    """attention_ref against what the mathematics fixes: identical keys give
    the mean of V; one key that outscores the rest by a wide margin gives its
    V row; two keys give the logistic weights; the scale multiplies the
    logits; an empty key set gives zeros."""
    rng = np.random.default_rng(3)
    D, Lq, Lk = 16, 5, 9
    q = rng.standard_normal((Lq, D))
    v = rng.standard_normal((Lk, D))
    k_same = np.tile(rng.standard_normal((1, D)), (Lk, 1))
    out = O.attention_ref(q, k_same, v)
    assert np.abs(out - v.mean(0)).max() < 1e-12
    # a dominant key: logits 60 units above every other key -> weight 1 - O(e^-60)
    k = rng.standard_normal((Lk, D)) * 0.01
    qd = np.zeros((Lq, D))
    qd[:, 0] = 1.0
    k[4, 0] = 60.0 * np.sqrt(D)
    assert np.abs(O.attention_ref(qd, k, v) - v[4]).max() < 1e-12
    # two keys: p1 = 1 / (1 + exp(s2 - s1)) with s = q.k / sqrt(D)
    k2, v2 = rng.standard_normal((2, D)), rng.standard_normal((2, D))
    s = q @ k2.T / np.sqrt(D)
    p1 = 1.0 / (1.0 + np.exp(s[:, 1] - s[:, 0]))
    want = p1[:, None] * v2[0] + (1 - p1)[:, None] * v2[1]
    assert np.abs(O.attention_ref(q, k2, v2) - want).max() < 1e-12
    # the scale multiplies q.k: scale c with q equals the default scale with q * c * sqrt(D)
    kk = rng.standard_normal((Lk, D))
    c = 0.37
    a = O.attention_ref(q, kk, v, scale=c)
    b = O.attention_ref(q * c * np.sqrt(D), kk, v)
    assert np.abs(a - b).max() < 1e-12
    assert not np.allclose(a, O.attention_ref(q, kk, v))
    assert (O.attention_ref(q, np.zeros((0, D)), np.zeros((0, D))) == 0).all()


def test_ragged_attention_ref_sequence_indexing():
    """Each (batch, head) sequence's V is a constant vector c(b, h), so its
    output is exactly c(b, h) whatever the weights: this pins which key rows
    the per-head (cu_k[b*Hq + h]) and shared (cu_k[b]) layouts select."""
    rng = np.random.default_rng(5)
    D, Hq = 8, 3
    cu_q = np.array([0, 4, 7, 12])
    lens = rng.integers(1, 6, len(cu_q) - 1)
    q = rng.standard_normal((cu_q[-1], Hq, D))
    # per-head ragged KV
    seq_lens = rng.integers(1, 7, (len(cu_q) - 1) * Hq)
    cu_k = np.concatenate([[0], np.cumsum(seq_lens)])
    k = rng.standard_normal((cu_k[-1], D))
    v = np.zeros((cu_k[-1], D))
    for s in range(len(seq_lens)):
        v[cu_k[s]:cu_k[s + 1]] = s + 1.0
    out = O.ragged_attention_ref(q, k, v, cu_q, cu_k, heads_q=Hq, kv_per_head=True)
    for b in range(len(cu_q) - 1):
        for h in range(Hq):
            assert np.abs(out[cu_q[b]:cu_q[b + 1], h] - (b * Hq + h + 1.0)).max() < 1e-12
    # shared KV per batch, [total_k, Hq, D] (flash-attn varlen layout)
    cu_kb = np.concatenate([[0], np.cumsum(lens)])
    kb = rng.standard_normal((cu_kb[-1], Hq, D))
    vb = np.zeros((cu_kb[-1], Hq, D))
    for b in range(len(lens)):
        for h in range(Hq):
            vb[cu_kb[b]:cu_kb[b + 1], h] = 10.0 * b + h
    out = O.ragged_attention_ref(q, kb, vb, cu_q, cu_kb, heads_q=Hq, kv_per_head=False)
    for b in range(len(cu_q) - 1):
        for h in range(Hq):
            assert np.abs(out[cu_q[b]:cu_q[b + 1], h] - (10.0 * b + h)).max() < 1e-12
