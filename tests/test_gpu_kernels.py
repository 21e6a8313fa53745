"""GPU parity of the HIP kernels against the CPU oracle, called through the
C ABI (ctypes).  Integer / index / byte outputs must be bit-exact; the
attention is checked against float64 softmax attention at max-abs 2e-2 and
mean-abs 2e-3 (the north-star bf16 tolerance)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from gpu_util import DEV, DevicePools, run_pack, run_plan, state_desc, stream, to_dev, to_np
    from pyramidkv import _abi as A


def _rand_states(rng, H):
    out = []
    for h in range(H):
        k = int(rng.integers(0, 5))
        sink = int(rng.integers(0, 4))
        out.append([O.make_recent(sink), O.make_cyclic(6, 4, sink), O.make_stride(6, 4, sink),
                    O.make_lag(int(rng.integers(1, 24)), sink), O.make_merge(2, int(rng.integers(1, 7)), sink)][k])
    return out


@pytest.mark.parametrize("seed", [0, 1])
def test_state_update_bit_exact(seed):
    rng = np.random.default_rng(seed)
    H, F = 12, 3
    host = O.states_to_bytes(_rand_states(rng, H))
    dev = to_dev(host)
    ts, desc = state_desc(H * F)
    for blk in range(40):
        t_vals = [3 * blk + f for f in range(F)]
        if rng.random() < 0.1:
            t_vals = [int(x) for x in rng.integers(0, 200, F)]  # out-of-order / duplicate frames too
        pass_kind = int(rng.random() < 0.8)
        want = O.state_update(host, t_vals, pass_kind)
        tv = torch.tensor(t_vals, dtype=torch.int64, device=DEV)
        A.check(A.lib().pkv_state_update(ctypes.c_void_p(dev.data_ptr()), H, ctypes.c_void_p(tv.data_ptr()), F,
                                         pass_kind, ctypes.byref(desc), stream()), "state_update")
        got = np.stack([to_np(t) for t in ts])
        assert (got == want).all(), f"descriptors differ at block {blk}"
        assert (to_np(dev) == host).all(), f"state bytes differ at block {blk}"


def _geom(**kw):
    d = dict(num_layers=2, num_heads=4, head_dim=128, frame_seqlen=96, max_sink=3, max_middle=24, max_recent=4,
             max_attend_chunks=3)
    d.update(kw)
    return O.Geometry(**d)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_plan_bit_exact(seed):
    rng = np.random.default_rng(seed)
    g = _geom(num_heads=12)
    dp = DevicePools(g)
    H = g.num_heads
    host = O.states_to_bytes(_rand_states(rng, H))
    for blk in range(30):
        O.state_update(host, [3 * blk, 3 * blk + 1, 3 * blk + 2], 1)
    vc = np.stack([rng.integers(0, 5, H), np.zeros(H, np.int64), rng.integers(0, 6, H)], 1).astype(np.int64)
    mtc = rng.integers(0, 420, (H, 6)).astype(np.int32)
    layer = 1
    vc_all = np.zeros((g.num_layers, H, 3), np.int64); vc_all[layer] = vc
    mtc_all = np.zeros((g.num_layers, H, 6), np.int32); mtc_all[layer] = mtc
    dp.load(dict(valid_count=vc_all, merge_token_count=mtc_all))
    for t_list, remap in [([90, 91, 92], (1, 18, 21, 0)), ([7], (0, 0, 21, 2)), ([117, 118, 119], (1, 18, 21, 0))]:
        o, total = run_plan(dp, to_dev(host), layer, t_list, remap)
        want = O.plan_multi(g, host, vc, mtc, t_list, *remap)
        for name, w in zip(["cu", "sk", "sg", "sl", "dst", "traw", "tremap"], want[:7]):
            assert (to_np(o[name]) == w).all(), name
        assert int(total.item()) == want[7]


@pytest.mark.parametrize("H,t_list", [(12, [60, 61, 62, 63, 64, 65]), (48, [90, 91])])
def test_plan_bit_exact_beyond_64_pairs(H, t_list):
    """More than 64 (chunk, head) pairs take the plan's two-pass form (count,
    block-wide scan, emit) instead of the one-pass register form."""
    rng = np.random.default_rng(H + len(t_list))
    g = _geom(num_heads=H, max_attend_chunks=len(t_list))
    dp = DevicePools(g)
    host = O.states_to_bytes(_rand_states(rng, H))
    for blk in range(30):
        O.state_update(host, [3 * blk, 3 * blk + 1, 3 * blk + 2], 1)
    vc = np.stack([rng.integers(0, 5, H), np.zeros(H, np.int64), rng.integers(0, 6, H)], 1).astype(np.int64)
    mtc = rng.integers(0, 420, (H, 6)).astype(np.int32)
    layer = 0
    vc_all = np.zeros((g.num_layers, H, 3), np.int64); vc_all[layer] = vc
    mtc_all = np.zeros((g.num_layers, H, 6), np.int32); mtc_all[layer] = mtc
    dp.load(dict(valid_count=vc_all, merge_token_count=mtc_all))
    assert len(t_list) * H > 64
    remap = (1, 18, 21, 0)
    o, total = run_plan(dp, to_dev(host), layer, t_list, remap)
    want = O.plan_multi(g, host, vc, mtc, t_list, *remap)
    for name, w in zip(["cu", "sk", "sg", "sl", "dst", "traw", "tremap"], want[:7]):
        assert (to_np(o[name]) == w).all(), name
    assert int(total.item()) == want[7]


def _tables_dev(tables):
    return tuple(torch.from_numpy(t).to(DEV) for t in tables)


@pytest.mark.parametrize("seed", [0, 1])
def test_pack_with_rope_bit_exact(seed):
    rng = np.random.default_rng(seed)
    g = _geom()
    dp = DevicePools(g)
    L, H = g.num_layers, g.num_heads
    arrays = {}
    for n, slots in [("sink", g.max_sink), ("middle", g.max_middle), ("recent", g.max_recent)]:
        for kv in ("k", "v"):
            arrays[f"{n}_{kv}"] = O.f32_to_bf16(rng.standard_normal((L, H, slots, g.frame_seqlen, 128)).astype(np.float32))
        p = np.zeros((L, H, slots, g.frame_seqlen, 3), np.int64)
        p[..., 0] = rng.integers(0, 1100, (L, H, slots, 1))
        p[..., 1] = np.arange(g.frame_seqlen) // 12
        p[..., 2] = np.arange(g.frame_seqlen) % 12
        arrays[f"{n}_pos"] = p
    for kv in ("k", "v"):
        arrays[f"merge_{kv}"] = O.f32_to_bf16(rng.standard_normal((L, H, 6, 420, 128)).astype(np.float32))
    arrays["merge_pos"] = rng.integers(0, 60, (L, H, 6, 420, 3)).astype(np.int64)
    # special bf16 values in K: signed zeros, subnormals, the largest finite,
    # infinities and NaNs (the rotated products then round through the same
    # cases: overflow, subnormal results, NaN canonicalised to 0x7fc0)
    special = np.array([0x0000, 0x8000, 0x0001, 0x807F, 0x0080, 0x7F7F, 0xFF7F, 0x7F80, 0xFF80, 0x7FC1, 0xFFC0,
                        0x7F81], np.uint16)
    for n in ("sink", "middle", "recent", "merge"):
        flat = arrays[f"{n}_k"].reshape(-1)
        at = rng.choice(flat.size, 4096, replace=False)
        flat[at] = special[rng.integers(0, special.size, at.size)]
    dp.load(arrays)
    # random plan-shaped segment list over both layers
    n = 200
    sk = rng.integers(-1, 4, n).astype(np.int32)
    lim = {0: L * H * g.max_sink, 1: L * H * g.max_middle, 2: L * H * g.max_recent, 3: L * H * 6}
    sg = np.array([rng.integers(0, lim[max(k, 0)]) for k in sk], np.int32)
    sl = np.array([rng.integers(0, (420 if k == 3 else g.frame_seqlen) + 1) for k in sk], np.int32)
    dst = np.concatenate([[0], np.cumsum(np.where(sk >= 0, sl, 0))[:-1]]).astype(np.int32)
    tremap = np.where(rng.random(n) < 0.5, rng.integers(0, 1030, n), -1).astype(np.int64)
    tables = O.rope_tables(128)
    for use_rope in (False, True):
        for name in ("k_flat_out", "v_flat_out", "pos_flat_out"):
            dp.t[name].zero_()
        run_pack(dp, *(to_dev(a) for a in (sk, sg, sl, dst)), to_dev(tremap) if use_rope else None,
                 _tables_dev(tables) if use_rope else None)
        wk, wv, wp = O.pack(arrays, g, sk, sg, sl, dst, tremap if use_rope else None, tables if use_rope else None)
        used = int(np.where(sk >= 0, sl, 0).sum())
        assert (dp.np("k_flat_out")[:used] == wk[:used]).all()
        assert (dp.np("v_flat_out")[:used] == wv[:used]).all()
        assert (dp.np("pos_flat_out")[:used] == wp[:used]).all()
        assert (dp.np("k_flat_out")[used:] == 0).all()


def test_pack_skips_inactive_zero_length_and_out_of_range():
    g = _geom(num_layers=1, num_heads=1, frame_seqlen=64)
    dp = DevicePools(g)
    dp.t["sink_k"].fill_(1.0)
    dp.t["k_flat_out"].fill_(7.5)
    sk = torch.tensor([-1, 0, 0, 1], dtype=torch.int32, device=DEV)
    sg = torch.tensor([0, 0, 99, 0], dtype=torch.int32, device=DEV)  # slot 99 is out of range: skipped
    sl = torch.tensor([64, 0, 64, 64], dtype=torch.int32, device=DEV)
    dst = torch.tensor([0, 0, 0, g.max_pack_tokens - 10], dtype=torch.int32, device=DEV)  # would overflow: skipped
    run_pack(dp, sk, sg, sl, dst)
    torch.cuda.synchronize()
    assert (dp.t["k_flat_out"] == 7.5).all()


def test_rope_apply_bit_exact():
    rng = np.random.default_rng(5)
    n = 5000
    k = O.f32_to_bf16(rng.standard_normal((n, 128)).astype(np.float32))
    pos = np.stack([rng.integers(-5, 1200, n), rng.integers(-2, 40, n), rng.integers(0, 60, n)], 1).astype(np.int64)
    tables = O.rope_tables(128)
    kd, pd = to_dev(k), to_dev(pos)
    out = torch.empty_like(kd)
    td = _tables_dev(tables)
    rs = A.rope_struct(td)
    A.check(A.lib().pkv_rope_apply(ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(pd.data_ptr()),
                                   ctypes.c_int64(n), 128, ctypes.byref(rs), ctypes.c_void_p(out.data_ptr()),
                                   stream()), "rope_apply")
    assert (to_np(out) == O.rope_apply(k, pos, tables)).all()


def test_update_frames_bit_exact():
    rng = np.random.default_rng(6)
    g = _geom(num_layers=2, num_heads=3, frame_seqlen=80)
    dp = DevicePools(g)
    F, H, FS, D = 3, g.num_heads, g.frame_seqlen, 128
    nk = O.f32_to_bf16(rng.standard_normal((F, H, FS, D)).astype(np.float32))
    nv = O.f32_to_bf16(rng.standard_normal((F, H, FS, D)).astype(np.float32))
    npos = rng.integers(0, 100, (F, H, FS, 3)).astype(np.int64)
    n = 9
    kind = rng.integers(-1, 3, n).astype(np.int32)
    slots = {0: g.max_sink, 1: g.max_middle, 2: g.max_recent}
    sgl = np.array([rng.integers(0, g.num_layers * H * slots[max(k, 0)]) for k in kind], np.int32)
    fr = rng.integers(0, F, n).astype(np.int32)
    hd = rng.integers(0, H, n).astype(np.int32)
    # distinct destinations so the result does not depend on write order
    seen = set()
    for i in range(n):
        if (kind[i], sgl[i]) in seen:
            kind[i] = -1
        seen.add((kind[i], sgl[i]))
    # entries that write nothing: MERGE (5; the reference's caller masks it to
    # -1 before this op), a slot past the sink pool, a negative slot, a frame
    # and a head outside the source
    extra = np.array([[5, 0, 0, 0], [0, g.num_layers * H * g.max_sink, 1, 1], [2, -1, 0, 0], [1, 0, F, 0],
                      [1, 1, 0, H]], np.int32)
    kind, sgl, fr, hd = (np.concatenate([a, extra[:, j]]).astype(np.int32) for j, a in enumerate((kind, sgl, fr, hd)))
    n = kind.size
    host = {k: dp.np(k).copy() for k in ["sink_k", "sink_v", "sink_pos", "middle_k", "middle_v", "middle_pos",
                                          "recent_k", "recent_v", "recent_pos"]}
    O.update_frames(host, nk, nv, npos, H, FS, D, kind, sgl, fr, hd)
    dk, dv, dpos = to_dev(nk), to_dev(nv), to_dev(npos)
    args = [to_dev(a) for a in (kind, sgl, fr, hd)]
    A.check(A.lib().pkv_update_frames(ctypes.byref(dp.geo), ctypes.byref(dp.pools), ctypes.c_void_p(dk.data_ptr()),
                                      ctypes.c_void_p(dv.data_ptr()), ctypes.c_void_p(dpos.data_ptr()), F,
                                      *[ctypes.c_void_p(a.data_ptr()) for a in args], n, stream()), "update_frames")
    for k, w in host.items():
        assert (dp.np(k) == w).all(), k


def _merge_run(H, FSEQ, W, blocks_t, seed, weights=None, permute=False):
    """Drive consecutive calls through the state machine + merge on both sides.
    permute: token t sits at a shuffled grid cell instead of cell t (same cells, so the
    same groups, but member lists that are not the row-major closed form)."""
    rng = np.random.default_rng(seed)
    cell = rng.permutation(FSEQ) if permute else np.arange(FSEQ)
    D, MT = 128, 420
    states_host = O.states_to_bytes([O.make_merge(2, int(c)) for c in rng.integers(2, 7, H)])
    states_dev = to_dev(states_host)
    acc = dict(sum_k=np.zeros((H, 2, MT, D), np.float32), sum_v=np.zeros((H, 2, MT, D), np.float32),
               pos=np.zeros((H, 2, MT, 3), np.int64), gid=np.zeros((H, 2, FSEQ), np.int32),
               tpg=np.zeros((H, 2, MT), np.float32), ng=np.zeros((H, 2), np.int32), wsum=np.zeros((H, 2), np.float32),
               mk=np.zeros((H, 6, MT, D), np.uint16), mv=np.zeros((H, 6, MT, D), np.uint16),
               mpos=np.zeros((H, 6, MT, 3), np.int64), mtc=np.zeros((H, 6), np.int32))
    dacc = {k: to_dev(v) for k, v in acc.items()}
    ml = A.MergeLayer(*[dacc[k].data_ptr() for k in ("sum_k", "sum_v", "pos", "gid", "tpg", "ng", "wsum", "mk", "mv",
                                                      "mpos", "mtc")])
    for t_vals in blocks_t:
        F = len(t_vals)
        nk = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
        nv = O.f32_to_bf16(rng.standard_normal((F, H, FSEQ, D)).astype(np.float32))
        pos = np.zeros((F, H, FSEQ, 3), np.int64)
        pos[..., 0] = np.asarray(t_vals).reshape(F, 1, 1)
        pos[..., 1] = cell // W
        pos[..., 2] = cell % W
        w = None if weights is None else rng.uniform(0.1, 1.0, F).astype(np.float32)
        desc = O.state_update(states_host, t_vals, 1)
        O.merge_accum(states_host, nk, nv, pos, desc, acc, w)
        ts, sd = state_desc(H * F)
        tv = torch.tensor(t_vals, dtype=torch.int64, device=DEV)
        A.check(A.lib().pkv_state_update(ctypes.c_void_p(states_dev.data_ptr()), H, ctypes.c_void_p(tv.data_ptr()),
                                         F, 1, ctypes.byref(sd), stream()), "state_update")
        ws = torch.empty(A.lib().pkv_merge_workspace_size(H, F, FSEQ, MT), dtype=torch.uint8, device=DEV)
        dk, dv, dpos = to_dev(nk), to_dev(nv), to_dev(pos)
        wd = to_dev(w) if w is not None else None
        A.check(A.lib().pkv_merge_accum(ctypes.c_void_p(states_dev.data_ptr()), H, F, FSEQ, D, 2, 6, MT,
                                        ctypes.c_void_p(dk.data_ptr()), ctypes.c_void_p(dv.data_ptr()),
                                        ctypes.c_void_p(dpos.data_ptr()),
                                        *[ctypes.c_void_p(ts[i].data_ptr()) for i in (0, 4, 6, 7)],
                                        ctypes.c_void_p(wd.data_ptr()) if wd is not None else None,
                                        ctypes.byref(ml), ctypes.c_void_p(ws.data_ptr()), stream()), "merge_accum")
        for k in ("mk", "mv", "mpos", "mtc", "ng", "gid", "tpg", "pos"):
            assert (to_np(dacc[k]) == acc[k]).all(), k
        assert (to_np(dacc["sum_k"]) == acc["sum_k"]).all() and (to_np(dacc["sum_v"]) == acc["sum_v"]).all()


def test_merge_production_grid_bit_exact():
    blocks = [[3 * b + f for f in range(3)] for b in range(10)]
    _merge_run(H=3, FSEQ=1560, W=52, blocks_t=blocks, seed=1)


def test_merge_irregular_grid_and_reuse_in_call():
    # 7-wide rows: ragged last patch row/col; 5 frames per call so one call
    # finalizes a block and starts the next block in the freed slot
    blocks = [[5 * b + f for f in range(5)] for b in range(6)]
    _merge_run(H=2, FSEQ=7 * 9 + 3, W=7, blocks_t=blocks, seed=2)


def test_merge_one_group_wide_and_permuted_grids():
    # a grid one patch wide has no row wrap in its group ids (member lists
    # from the CSR build); permuted cells keep the group sets but not the
    # closed-form member order, in new blocks and in blocks continued across
    # calls
    blocks = [[3 * b + f for f in range(3)] for b in range(4)]
    _merge_run(H=2, FSEQ=2 * 12, W=2, blocks_t=blocks, seed=4)
    _merge_run(H=2, FSEQ=1560, W=52, blocks_t=blocks, seed=5, permute=True)


def test_merge_weighted_bit_exact():
    blocks = [[3 * b + f for f in range(3)] for b in range(8)]
    _merge_run(H=2, FSEQ=1560, W=52, blocks_t=blocks, seed=3, weights=True)


def _attn_case(rng, Lq_list, Lk_list, H=1, D=128):
    B = len(Lq_list)
    cu_q = np.concatenate([[0], np.cumsum(Lq_list)]).astype(np.int32)
    lk = np.array(Lk_list).reshape(B, H)
    cu_k = np.concatenate([[0], np.cumsum(lk.reshape(-1))]).astype(np.int32)
    q = (rng.standard_normal((cu_q[-1], H, D)) * 0.5).astype(np.float32)
    k = (rng.standard_normal((cu_k[-1], D)) * 0.5).astype(np.float32)
    v = (rng.standard_normal((cu_k[-1], D)) * 0.5).astype(np.float32)
    return O.f32_to_bf16(q), O.f32_to_bf16(k), O.f32_to_bf16(v), cu_q, cu_k


@pytest.mark.parametrize("case", [
    dict(Lq=[1560], Lk=[[6240]]),
    dict(Lq=[300, 257, 1], Lk=[[1], [64], [65]]),
    dict(Lq=[256, 100], Lk=[[0], [4000]]),
    dict(Lq=[1560, 1560], Lk=[[12480, 14040, 17160], [9000, 3, 31]], H=3),
])
def test_attention_vs_float64(case):
    rng = np.random.default_rng(11)
    H = case.get("H", 1)
    q, k, v, cu_q, cu_k = _attn_case(rng, case["Lq"], case["Lk"], H)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    out = torch.full_like(qd, float("nan"))
    A.ragged_attn_fwd(qd, kd, vd, out, to_dev(cu_q), to_dev(cu_k), len(case["Lq"]), H, True, max(case["Lq"]),
                      128 ** -0.5)
    got = O.bf16_to_f32(to_np(out)).astype(np.float64)
    want = O.ragged_attention_ref(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), cu_q, cu_k, H, True)
    err = np.abs(got - want)
    assert np.isfinite(got).all()
    assert err.max() < 2e-2 and err.mean() < 2e-3, (err.max(), err.mean())


def test_attention_keys_outscoring_the_first_tile_vs_float64():
    """The fast pass fixes each row's softmax reference at its first key tile.
    Spiked keys later in the sequence score ~130 log2 units above it (past the
    2^64 headroom: those workgroups recompute with a moving maximum) or ~33
    (inside the headroom: the fast pass keeps them, with P up to 2^33); a spike
    on the last key of a partial tile checks the masking on that path too."""
    rng = np.random.default_rng(5)
    H = 2
    Lq, Lk = [300, 700], [[5000, 130], [2000, 64]]
    q, k, v, cu_q, cu_k = _attn_case(rng, Lq, Lk, H)
    q[:] = O.f32_to_bf16(np.ones(1, np.float32))[0]  # every score = 128 * mean(k row) * scale
    for seq, pos, val in [(0, 4000, 8.0), (1, 100, 2.0), (2, 1999, 8.0)]:
        k[cu_k[seq] + pos] = O.f32_to_bf16(np.full(128, val, np.float32))
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    out = torch.full_like(qd, float("nan"))
    A.ragged_attn_fwd(qd, kd, vd, out, to_dev(cu_q), to_dev(cu_k), len(Lq), H, True, max(Lq), 128 ** -0.5)
    got = O.bf16_to_f32(to_np(out)).astype(np.float64)
    want = O.ragged_attention_ref(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), cu_q, cu_k, H, True)
    err = np.abs(got - want)
    assert np.isfinite(got).all()
    assert err.max() < 2e-2 and err.mean() < 2e-3, (err.max(), err.mean())


def _attn_check(q, k, v, cu_q, cu_k, B, H, kv_per_head=True):
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    out = torch.full_like(qd, float("nan"))
    max_q = int(np.diff(cu_q).max())
    A.ragged_attn_fwd(qd, kd, vd, out, to_dev(cu_q), to_dev(cu_k), B, H, kv_per_head, max_q, 128 ** -0.5)
    got = O.bf16_to_f32(to_np(out)).astype(np.float64)
    want = O.ragged_attention_ref(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), cu_q, cu_k, H, kv_per_head)
    err = np.abs(got - want)
    assert np.isfinite(got).all()
    assert err.max() < 2e-2 and err.mean() < 2e-3, (err.max(), err.mean())


def _large_launch_case(rng, kv_per_head, B=86, H=12, D=128):
    """B x H (sequence, head) pairs.  Query lengths 1-384 with one sequence
    of 800 (three query tiles of 384 rows; the other sequences' extra tiles
    exit), so the launch has at least 1,024 workgroups and runs the 12-wave
    kernel (smaller launches run the 8-wave one); key lengths 0-200 with the
    tile edges (0, 1, 31, 32, 33, 64) among them."""
    Lq = rng.integers(1, 385, size=B)
    Lq[:6] = [384, 1, 800, 33, 383, 257]
    n_kv = B * H if kv_per_head else B
    Lk = rng.integers(0, 201, size=n_kv)
    Lk[:8] = [0, 1, 31, 32, 33, 64, 200, 97]
    cu_q = np.concatenate([[0], np.cumsum(Lq)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(Lk)]).astype(np.int32)
    q = (rng.standard_normal((cu_q[-1], H, D)) * 0.5).astype(np.float32)
    kv_shape = (cu_k[-1], D) if kv_per_head else (cu_k[-1], H, D)
    k = (rng.standard_normal(kv_shape) * 0.5).astype(np.float32)
    v = (rng.standard_normal(kv_shape) * 0.5).astype(np.float32)
    return O.f32_to_bf16(q), O.f32_to_bf16(k), O.f32_to_bf16(v), cu_q, cu_k


@pytest.mark.parametrize("kv_per_head,H", [(True, 12), (False, 12), (True, 11)])
def test_attention_large_launch_vs_float64(kv_per_head, H):
    # 86 x 12 = 1,032 pairs exceed the 1,024 that the XCD-balanced work list
    # ranks (plain work order); 86 x 11 = 946 take the balanced order
    rng = np.random.default_rng(21 + kv_per_head + H)
    q, k, v, cu_q, cu_k = _large_launch_case(rng, kv_per_head, H=H)
    _attn_check(q, k, v, cu_q, cu_k, 86, H, kv_per_head)


@pytest.mark.parametrize("B", [86, 20])
def test_attention_empty_query_sequences_vs_float64(B):
    """Batches without query rows (Lq = 0) between others, in a launch of the
    12-wave kernel (86 x 12 pairs) and of the 8-wave one (20 x 12): their
    sequences have no work items and the other rows are unaffected."""
    rng = np.random.default_rng(41)
    q, k, v, cu_q, cu_k = _large_launch_case(rng, True, B=B)
    Lq = np.diff(cu_q)
    Lq[[1, 7, B - 1]] = 0
    cu_q = np.concatenate([[0], np.cumsum(Lq)]).astype(np.int32)
    q = q[:cu_q[-1]]
    _attn_check(q, k, v, cu_q, cu_k, B, 12)


@pytest.mark.parametrize("B", [86, 20])
def test_attention_longest_key_sequences_vs_float64(B):
    """Sequences at the cache's largest key count (31 frames x 1,560 =
    48,360 keys, the reference's max_seqlen_k) and beyond it (60,001) among
    short ones, in both head_dim-128 kernels; their query rows against
    float64."""
    rng = np.random.default_rng(43)
    q, k, v, cu_q, cu_k = _large_launch_case(rng, True, B=B)
    Lk = np.diff(cu_k)
    Lk[[3, 50 % len(Lk), len(Lk) - 2]] = [48360, 60001, 48360]
    cu_k = np.concatenate([[0], np.cumsum(Lk)]).astype(np.int32)
    k = O.f32_to_bf16((rng.standard_normal((cu_k[-1], 128)) * 0.5).astype(np.float32))
    v = O.f32_to_bf16((rng.standard_normal((cu_k[-1], 128)) * 0.5).astype(np.float32))
    _attn_check(q, k, v, cu_q, cu_k, B, 12)


def test_attention_large_launch_strided_views_vs_float64():
    """Q, K, V and O as the first 128 columns of 256-wide rows (token and head
    strides of the views, K/V rows 512 bytes apart): the 12-wave kernel reads
    and writes through the strides and leaves the other columns untouched."""
    rng = np.random.default_rng(31)
    B, H = 86, 12
    q, k, v, cu_q, cu_k = _large_launch_case(rng, True, B=B, H=H)
    wide = lambda a: np.concatenate([a, np.zeros(a.shape, np.uint16)], axis=-1)
    qw, kw, vw = to_dev(wide(q)), to_dev(wide(k)), to_dev(wide(v))
    qd, kd, vd = qw[..., :128], kw[..., :128], vw[..., :128]
    ow = torch.full_like(qw, float("nan"))
    out = ow[..., :128]
    A.ragged_attn_fwd(qd, kd, vd, out, to_dev(cu_q), to_dev(cu_k), B, H, True, int(np.diff(cu_q).max()), 128 ** -0.5)
    got = O.bf16_to_f32(to_np(out)).astype(np.float64)
    want = O.ragged_attention_ref(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), cu_q, cu_k, H, True)
    err = np.abs(got - want)
    assert np.isfinite(got).all()
    assert err.max() < 2e-2 and err.mean() < 2e-3, (err.max(), err.mean())
    assert torch.isnan(ow[..., 128:]).all()


def test_attention_large_launch_keys_outscoring_the_first_tile_vs_float64():
    """The 12-wave kernel's slow pass: spiked keys past the first tile score
    ~130 log2 units above it (past the headroom) in some sequences, ~33
    (inside it) in others; one spike sits on the last key of a partial tile."""
    rng = np.random.default_rng(8)
    q, k, v, cu_q, cu_k = _large_launch_case(rng, True)
    q[:] = O.f32_to_bf16(np.ones(1, np.float32))[0]
    lk = np.diff(cu_k)
    spiked = [s for s in range(len(lk)) if lk[s] > 40][:40]
    for i, s in enumerate(spiked):
        pos = lk[s] - 1 if i % 3 == 0 else 35
        k[cu_k[s] + pos] = O.f32_to_bf16(np.full(128, 8.0 if i % 2 == 0 else 2.0, np.float32))
    _attn_check(q, k, v, cu_q, cu_k, 86, 12)


@pytest.mark.parametrize("B", [86, 20])
def test_attention_reference_modes_vs_float64(B):
    """Both head_dim-128 kernels (86 x 12 pairs: the 12-wave kernel; 20 x 12:
    the 8-wave one) fix each row's reference at its first key tile's maximum.
    Query rows are scaled by 1, 2 or 4 and each sequence's first tile set to
    a constant, so that the references lie near 0, far above (up to ~196 log2
    units) and far below it (to ~-65, where the later keys then lie past the
    headroom), differing between the rows of one wave; spiked later keys
    reach ~98 units above the reference."""
    rng = np.random.default_rng(17)
    q, k, v, cu_q, cu_k = _large_launch_case(rng, True, B=B)
    alpha = np.array([1.0, 2.0, 4.0], np.float32)[np.arange(q.shape[0]) % 3]
    q[:] = O.f32_to_bf16(np.broadcast_to(alpha[:, None, None], q.shape).astype(np.float32))
    lk = np.diff(cu_k)
    betas = [0.0, 0.8, -1.0, 3.0, -0.5]
    for s_ in range(len(lk)):
        n = min(32, int(lk[s_]))
        k[cu_k[s_]:cu_k[s_] + n] = O.f32_to_bf16(np.full((n, 128), betas[s_ % len(betas)], np.float32))
        if s_ % 7 == 3 and lk[s_] > 40:
            k[cu_k[s_] + lk[s_] - 1] = O.f32_to_bf16(np.full(128, 1.5, np.float32))
    _attn_check(q, k, v, cu_q, cu_k, B, 12)


@pytest.mark.parametrize("B", [86, 20])
def test_attention_row_rebase_vs_float64(B):
    """Keys aligned with single query rows, past the first key tile, scoring
    ~70 or ~85 log2 units above the rest (those rows rescale O and their sum
    in place after the tile and raise their reference) or ~110 (past the
    rebase bound: the workgroup's slow pass), in sequences whose first tile
    scores ~0 and ~40 for their first row.  Other rows meet the spiked keys
    as distractors of large norm.  Both head_dim-128 kernels."""
    rng = np.random.default_rng(29)
    q, k, v, cu_q, cu_k = _large_launch_case(rng, True, B=B)
    H = 12
    c = 128 ** -0.5 * 1.4426950408889634
    qf = O.bf16_to_f32(q)
    lk = np.diff(cu_k)
    # rows of the first batches: a third get a first tile of constant keys scoring ~40 (shift mode)
    for s_ in range(len(lk)):
        b, h = divmod(s_, H)
        if lk[s_] < 40 or np.diff(cu_q)[b] == 0:
            continue
        rows = np.arange(cu_q[b], cu_q[b + 1])
        if s_ % 3 == 1:
            qr = qf[rows[0], h]
            k[cu_k[s_]:cu_k[s_] + 32] = O.f32_to_bf16(np.tile(qr * (40.0 / (c * float(qr @ qr))), (32, 1)))
        units = [70.0, 85.0, 110.0][s_ % 3]
        for j, r in enumerate(rows[:: max(1, len(rows) // 3)][:3]):
            pos = 33 + (7 * j + s_) % max(1, lk[s_] - 33)
            qr = qf[r, h]
            k[cu_k[s_] + pos] = O.f32_to_bf16(qr * (units / (c * float(qr @ qr))))
    _attn_check(q, k, v, cu_q, cu_k, B, H)


def test_attention_tail_tiles_vs_float64():
    """The 12-wave kernel's last query tiles of at most 96 rows (a rollout's
    72 of 4,680) split their keys in four quarters within the workgroup and
    merge them: tails of 1, 8, 32, 33, 64, 72 and 96 rows behind full tiles
    and alone, against key counts with quarters of unequal length, a last
    tile of one key and tile edges; 43 x 12 pairs of up to two query tiles
    make a launch of at least 1,024 workgroups."""
    rng = np.random.default_rng(61)
    B, H = 43, 12
    tails = [1, 8, 32, 33, 64, 72, 96]
    Lq = np.array([(384 if b % 3 else 0) + tails[b % len(tails)] for b in range(B)])
    Lq[0] = 768  # two full tiles, no tail
    Lk = rng.integers(256, 2000, size=B * H)
    Lk[:6] = [256, 257, 288, 1000, 1025, 1999]
    cu_q = np.concatenate([[0], np.cumsum(Lq)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(Lk)]).astype(np.int32)
    q = O.f32_to_bf16((rng.standard_normal((cu_q[-1], H, 128)) * 0.5).astype(np.float32))
    k = O.f32_to_bf16((rng.standard_normal((cu_k[-1], 128)) * 0.5).astype(np.float32))
    v = O.f32_to_bf16((rng.standard_normal((cu_k[-1], 128)) * 0.5).astype(np.float32))
    # a late key far above the rest in a few tails: the moving maximum rescales
    for s_ in range(0, B * H, 17):
        k[cu_k[s_] + Lk[s_] - 1] = O.f32_to_bf16(np.full(128, 3.0, np.float32))
    _attn_check(q, k, v, cu_q, cu_k, B, H)


def test_attention_partial_query_tiles_vs_float64():
    """The 12-wave kernel's last query tiles of every length class: sequences
    of 512 + t or t rows (t = 1 ... 511) leave last tiles of 1-96 rows (the
    key-split tail items), 97-383 rows (the full-tile path with the waves past
    the rows only copying) and full tiles; tails with fewer than 8 key tiles
    (40 and 200 keys) take the full-tile path too; 43 x 12 pairs."""
    rng = np.random.default_rng(67)
    B, H = 43, 12
    tails = [1, 8, 32, 33, 64, 72, 96, 100, 128, 129, 200, 448, 480, 511]
    Lq = np.array([(512 if b % 3 else 0) + tails[b % len(tails)] for b in range(B)])
    Lq[0] = 1024  # two full tiles, no tail
    Lk = rng.integers(256, 2000, size=B * H)
    Lk[:8] = [256, 257, 288, 1000, 1025, 1999, 40, 200]
    cu_q = np.concatenate([[0], np.cumsum(Lq)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(Lk)]).astype(np.int32)
    q = O.f32_to_bf16((rng.standard_normal((cu_q[-1], H, 128)) * 0.5).astype(np.float32))
    k = O.f32_to_bf16((rng.standard_normal((cu_k[-1], 128)) * 0.5).astype(np.float32))
    v = O.f32_to_bf16((rng.standard_normal((cu_k[-1], 128)) * 0.5).astype(np.float32))
    for s_ in range(0, B * H, 17):
        k[cu_k[s_] + Lk[s_] - 1] = O.f32_to_bf16(np.full(128, 3.0, np.float32))
    _attn_check(q, k, v, cu_q, cu_k, B, H)


def test_attention_rejects_causal_and_bad_head_dim():
    q = torch.zeros(4, 1, 128, dtype=torch.bfloat16, device=DEV)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=DEV)
    a = A.AttnArgs(q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), cu.data_ptr(), cu.data_ptr(), 1, 1, 128, 1,
                   128, 0, 128, 0, 128, 0, 4, 0.1, 1)
    assert A.lib().pkv_ragged_attn_fwd(ctypes.byref(a), stream()) == A.PKV_ERR_UNSUPPORTED
    a.causal, a.head_dim = 0, 96
    assert A.lib().pkv_ragged_attn_fwd(ctypes.byref(a), stream()) == A.PKV_ERR_UNSUPPORTED


@pytest.mark.parametrize("F,weighted", [(2, False), (4, False), (4, True)])
def test_merge_multi_frame_calls_bit_exact(F, weighted):
    # calls of 2 and 4 frames on the production grid, offset so that calls
    # straddle block boundaries: one call finalizes a block and starts the
    # next, in the same or the other slot
    blocks = [[2 + F * b + f for f in range(F)] for b in range(24 // F)]
    _merge_run(H=2, FSEQ=1560, W=52, blocks_t=blocks, seed=10 + F, weights=True if weighted else None)
