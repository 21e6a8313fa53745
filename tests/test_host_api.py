"""CPU checks of the pyramidkv host API: the state record layout and
builders against the oracle, the policy compiler on the shipped labels,
the RoPE tables the pack reads, the time remaps, and the registration of
the torch.ops.adahead surface (schemas, custom class, meta dispatch).
No kernel runs here."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pyramidkv import _mega_state_ops as S
from pyramidkv import _mega_state_ref as R
from pyramidkv import _ops, factory
from pyramidkv._mega_cache import _composition_to_perhead_state
from pyramidkv import CyclicStrategy, HeadComposition, LagStrategy, MergeStrategy, RecentStrategy, StrideStrategy
from pyramidkv.rope import flat_freq_parts, map_dynamic_pos_time, map_sink_time, wan_freqs


def test_state_dtype_matches_oracle_layout():
    assert S.PER_HEAD_STATE_DTYPE.itemsize == O.STATE_SIZE == 600
    for name in O.STATE_DTYPE.names:
        assert S.PER_HEAD_STATE_DTYPE.fields[name][1] == O.STATE_DTYPE.fields[name][1], name
    # offsets fixed by the reference struct (anchor_store.cuh:62-132, natural alignment)
    off = {n: S.PER_HEAD_STATE_DTYPE.fields[n][1] for n in S.PER_HEAD_STATE_DTYPE.names}
    assert off["cyclic_cursor"] == 240 and off["tkey_slot"] == 248 and off["tkey_count"] == 440
    assert off["merge_completed_slot"] == 444 and off["merge_completed_count"] == 564
    assert off["merge_active_block_id"] == 568 and off["cached_num_groups"] == 596


@pytest.mark.parametrize("mk", [
    (lambda: R.make_cyclic(6, 4), lambda: O.make_cyclic(6, 4)),
    (lambda: R.make_cyclic(3, 2), lambda: O.make_cyclic(3, 2)),
    (lambda: R.make_stride(6, 4), lambda: O.make_stride(6, 4)),
    (lambda: R.make_lag(21), lambda: O.make_lag(21)),
    (lambda: R.make_merge(2, 4), lambda: O.make_merge(2, 4)),
    (lambda: R.make_recent(), lambda: O.make_recent()),
])
def test_state_builders_bytes_equal_oracle(mk):
    ours, theirs = mk
    a = S.pack_states([ours()]).view(np.uint8)
    b = O.states_to_bytes([theirs()]).view(np.uint8)
    assert np.array_equal(a, b)
    back = S.unpack_states(S.pack_states([ours()]))[0]
    assert S.pack_states([back]).tobytes() == S.pack_states([ours()]).tobytes()


def test_state_builders_validate_ranges():
    with pytest.raises(ValueError):
        R.make_cyclic(7, 1)
    with pytest.raises(ValueError):
        R.make_cyclic(6, 5)
    with pytest.raises(ValueError):
        R.make_stride(6, 25)
    with pytest.raises(ValueError):
        R.make_merge(3, 4)


def test_shipped_policy_compositions():
    comps = factory.shipped_compositions()
    flat = [c for row in comps for c in row]
    kinds = [type(c.middle_strategies[0]).__name__ for c in flat]
    assert len(flat) == 360
    assert kinds.count("CyclicStrategy") == 156
    assert kinds.count("StrideStrategy") == 172
    assert kinds.count("MergeStrategy") == 32
    for c in flat:
        st = _composition_to_perhead_state(c)
        if c.label == -1:
            assert (st.kind, st.period, st.bucket_cap, st.sink_capacity) == (R.SK_CYCLIC, 6, 4, 1)
        elif c.label == 1:
            assert (st.kind, st.interval, st.capacity, st.sink_capacity) == (R.SK_STRIDE, 6, 4, 3)
        else:
            assert (st.kind, st.patch_size, st.capacity, st.sink_capacity) == (R.SK_MERGE, 2, 4, 3)
        assert c.recent_frames == 4


def test_composition_to_state_edge_cases():
    rec = HeadComposition("x", 1, 2, 4, [])
    st = _composition_to_perhead_state(rec)
    assert st.kind == R.SK_RECENT and st.sink_capacity == 2
    unbounded = HeadComposition("s", 1, 3, 4, [StrideStrategy(6, -1)])
    assert _composition_to_perhead_state(unbounded).capacity == R.MAX_T_KEYED
    lag = HeadComposition("l", -1, 1, 4, [LagStrategy([6, 12], history_frames=40)])
    st = _composition_to_perhead_state(lag)
    assert st.kind == R.SK_LAG and st.capacity == R.MAX_T_KEYED
    first = HeadComposition("c", -1, 1, 4, [CyclicStrategy(6, 2), MergeStrategy(2, 4)])
    assert _composition_to_perhead_state(first).kind == R.SK_CYCLIC


def test_strategy_state_records():
    """Each strategy encodes its own record; bounds as the reference's
    make_* helpers check them (_mega_state_ref.py)."""
    st = CyclicStrategy(3, 4).state_record()
    assert (st.kind, st.period, st.bucket_cap) == (R.SK_CYCLIC, 3, 4)
    with pytest.raises(ValueError, match="cyclic period"):
        CyclicStrategy(6, 5).state_record()  # 30 slots > the 6 x 4 ring
    assert StrideStrategy(6, 30).state_record().capacity == R.MAX_T_KEYED
    assert (StrideStrategy(4, 5).state_record().interval, StrideStrategy(4, 5).state_record().capacity) == (4, 5)
    st = LagStrategy([12, 6, 6, 3], history_frames=10).state_record()
    assert (st.kind, st.capacity, st.lag_offset_count, list(st.lag_offsets[:3])) == (R.SK_LAG, 10, 3, [3, 6, 12])
    st = MergeStrategy(2, 4).state_record()
    assert (st.kind, st.patch_size, st.block_frames, st.capacity) == (R.SK_MERGE, 2, 4, 4)
    with pytest.raises(ValueError, match="merge needs"):
        MergeStrategy(3, 4).state_record()  # 9-frame blocks > 4
    with pytest.raises(ValueError, match="merge needs"):
        MergeStrategy(2, -1).state_record()
    assert RecentStrategy().state_record().kind == R.SK_RECENT


def test_composition_dispatches_on_the_strategy_class_name():
    """The reference picks the encoding by the strategy's class name, so an
    object of another class with that name and those attributes encodes the
    same way; an unknown middle strategy means sink + recent only."""
    Foreign = type("StrideStrategy", (), {"interval": 3, "capacity": 7})
    st = _composition_to_perhead_state(HeadComposition("f", 1, 2, 4, [Foreign()]))
    assert (st.kind, st.interval, st.capacity, st.sink_capacity) == (R.SK_STRIDE, 3, 7, 2)
    Other = type("Unknown", (), {})
    assert _composition_to_perhead_state(HeadComposition("u", 1, 2, 4, [Other()])).kind == R.SK_RECENT


def test_policy_compiler_rejects_ambiguous_maps():
    with pytest.raises(ValueError, match="cyclic resolution"):
        factory.build_compositions(1, 1, labels=[[-1]], cyclic_enabled=True, cyclic_osc_only=True)
    with pytest.raises(ValueError, match="mutually exclusive"):
        factory.build_compositions(1, 1, labels=[[2]], label_stride_enabled_map={"2": True},
                                   label_merge_enabled_map={"2": True}, label_merge_patch_size_map={"2": 2},
                                   label_merge_capacity_map={"2": 4})


@pytest.mark.parametrize("D", [64, 128])
def test_rope_tables_equal_oracle(D):
    ours = flat_freq_parts(wan_freqs(D))
    theirs = O.rope_tables(D)
    for a, b in zip(ours, theirs):
        assert a.dtype == torch.float32 and a.shape == b.shape
        assert np.array_equal(a.numpy(), b)


def test_map_sink_time_matches_oracle():
    for t in range(0, 80):
        for mode, code in (("lag", 0), ("window_clamp", 1)):
            for lag in (0, 3):
                assert map_sink_time(t, mode, 18, 21, lag) == O.map_sink_time(t, code, 18, 21, lag)


def test_map_dynamic_pos_time_modes():
    pos = torch.tensor([[0, 1, 2], [10, 0, 0], [30, 5, 5]])
    assert map_dynamic_pos_time(pos, 40, "none", 21, 1.0) is pos
    clamp = map_dynamic_pos_time(pos, 40, "relative_clamp", 21, 1.0)
    assert clamp[:, 0].tolist() == [19, 19, 30]
    soft = map_dynamic_pos_time(pos, 40, "relative_softcap", 21, 0.5)
    # rel 40 -> 21 + round(19*0.5)=31 -> t 9; rel 30 -> 21 + round(4.5)=25 (round half to even: 4) -> 15
    assert soft[:, 0].tolist() == [40 - (21 + 10), 40 - (21 + 4), 30]
    assert pos[:, 0].tolist() == [0, 10, 30]


REQUIRED_OPS = ["pyramidkv_pack", "pyramidkv_update", "mega_state_update", "mega_plan", "mega_plan_multi",
                "mega_state_perhead_size", "mega_merge_accum", "mega_merge_accum_weighted", "mega_evict_merge", "mega_evict_merge_workspace_size",
                "ragged_attention",
                "rope_apply", "cache_update", "update_descriptors", "mega_attend_kv", "dit_layer_norm", "dit_rms_norm",
                "dit_residual_", "dit_gelu_tanh", "dit_residual_layer_norm_"]


def test_dit_row_ops_meta_shapes():
    """The DiT row ops' Meta registrations give the output shapes and dtypes
    (shape inference without a device)."""
    ops = _ops.ops()
    x = torch.empty(7, 256, device="meta")
    y = torch.empty(7, 256, dtype=torch.bfloat16, device="meta")
    out = ops.dit_residual_layer_norm_(x, y, None, None, None, True, 1e-6)
    assert out.shape == (7, 256) and out.dtype == torch.bfloat16 and out.device.type == "meta"
    out = ops.dit_layer_norm(x, None, None, True, 1e-6)
    assert out.shape == (7, 256) and out.dtype == torch.bfloat16
    assert ops.dit_gelu_tanh(y).shape == (7, 256)


def test_torch_ops_surface_registered():
    ops = _ops.ops()
    for name in REQUIRED_OPS:
        assert hasattr(ops, name), name
    assert int(ops.mega_state_perhead_size()) == 600
    mgr = torch.classes.adahead.PyramidKVCacheManager(2, 3, 64, 16, 3, 24, 4, "cpu", "bfloat16", 2)
    assert mgr.max_pack_tokens() == 2 * 3 * (3 + 24 + 4 + 6) * 16
    assert tuple(mgr.sink_k_pool().shape) == (2, 3, 3, 16, 64)
    assert tuple(mgr.valid_count().shape) == (2, 3, 3)
    assert tuple(mgr.k_flat_out().shape) == (mgr.max_pack_tokens(), 1, 64)
    mgr.reset()
    with pytest.raises(RuntimeError):
        torch.classes.adahead.PyramidKVCacheManager(1, 1, 64, 16, 1, 1, 1, "cpu", "int8", 1)


def test_reference_op_schemas():
    """The reference's schemas (adahead_ops.cpp registrations) are unchanged."""
    sch = {s.name: s for s in torch._C._jit_get_all_schemas() if s.name.startswith("adahead::")}
    args = lambda n: [a.name for a in sch["adahead::" + n].arguments]
    assert args("pyramidkv_pack") == ["mgr", "src_kind", "src_slot_global", "seg_lengths", "dst_token_offsets",
                                      "anchor_t_remap", "freqs_ft_flat", "freqs_fy_flat", "freqs_fx_flat"]
    assert args("pyramidkv_update") == ["mgr", "new_k", "new_v", "new_pos", "dst_kind", "dst_slot_global",
                                        "src_frame_in_block", "src_head"]
    assert args("mega_state_update")[-3:] == ["num_heads", "frames_in_block", "pass_kind"]
    assert len(args("mega_plan_multi")) == 12 and len(args("mega_merge_accum")) == 18


def test_meta_dispatch_shapes():
    _ops.ops()
    q = torch.empty(192, 4, 128, dtype=torch.bfloat16, device="meta")
    k = torch.empty(1000, 128, dtype=torch.bfloat16, device="meta")
    cu = torch.empty(4, dtype=torch.int32, device="meta")
    out = torch.ops.adahead.ragged_attention(q, k, k, cu, cu, 64, 0.1, True, False)
    assert out.device.type == "meta" and tuple(out.shape) == (192, 4, 128)
    kr = torch.ops.adahead.rope_apply(k, torch.empty(1000, 3, dtype=torch.long, device="meta"), k, k, k)
    assert tuple(kr.shape) == (1000, 128)


def test_megacache_keeps_and_restores_the_committed_recent_fifo():
    """A block's first noisy pass copies the layer's recent FIFO (the
    committed one: the last pass was clean) into the layer's backup; a pass
    for another block while a noisy pass is pending -- another t0, or the
    same t0 with another frame count (whose shift differs) -- first copies
    it back, as the reference restores its snapshot (_mega_cache.py:226-245).
    Both happen before the launch, which a CPU manager then refuses."""
    from pyramidkv import _ops
    if not _ops.available():
        pytest.skip("torch binding not built")
    from pyramidkv import factory
    from pyramidkv._mega_cache import build_mega_caches
    from pyramidkv.base import HeadComposition
    H, D, FS = 2, 16, 8
    comps = [[HeadComposition(f"h{h}", 0, sink_frames=1, recent_frames=3) for h in range(H)]]
    cache = build_mega_caches(1, H, D, FS, 1, 1, 3, comps, max_attend_chunks=1, device="cpu", spatial_width=4,
                              spatial_height=2, **factory.PYRAMID_FORCING_REMAP)[0]
    mgr = cache.ctx.mgr
    pools = lambda: (mgr.recent_k_pool()[0], mgr.recent_v_pool()[0], mgr.recent_pos_pool()[0])
    kv = lambda F: torch.zeros(1, F * FS, H, D, dtype=torch.bfloat16)
    for i, t in enumerate(pools()):
        t.fill_(i + 1)
    with pytest.raises(Exception):  # the launch: no CPU kernel
        cache.update(kv(3), kv(3), 5 * FS, cache_update_mode="noisy")
    backup = cache.ctx.recent_backup[0]
    assert all(torch.equal(b, t) for b, t in zip(backup, pools()))
    for t in pools():
        t.fill_(9)  # as if the pending pass had shifted and written the FIFO
    cache.ctx.pending_block[0] = (5, 3)
    for start, F in ((8 * FS, 3), (5 * FS, 2)):
        with pytest.raises(Exception):
            cache.update(kv(F), kv(F), start, cache_update_mode="noisy" if F == 3 else "clean")
        assert all(int(t.min()) == int(t.max()) == i + 1 for i, t in enumerate(pools())), (start, F)
        for t in pools():
            t.fill_(9)
