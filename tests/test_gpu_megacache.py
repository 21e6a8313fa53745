"""End-to-end parity of the pyramidkv host API on the GPU: MegaCache
update (fused route + scatter + state machine + Veil merge), the device
plan, pack with fused RoPE and the ragged attention, driven through
torch.ops.adahead exactly as the causal DiT drives the reference's
MegaCache (pyramidkv/_mega_cache.py:136-523), against the CPU model
oracle.MegaCacheRef over multi-block rollouts with noisy and clean
passes.  Pools, counters, state records, plans and packed K/V/pos are
compared bit-exactly; attention within bf16 tolerance of float64."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
if torch.cuda.is_available():
    from gpu_util import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN = 2e-2, 2e-3


def _build(L, H, D, FS, W, labels, max_sink=3, max_middle=24, max_recent=4, chunks=3):
    from pyramidkv import factory
    from pyramidkv._mega_cache import build_mega_caches
    from pyramidkv.rope import wan_freqs
    comps = factory.shipped_compositions(L, H, labels=labels)
    caches = build_mega_caches(L, H, D, FS, max_sink, max_middle, max_recent, comps, max_attend_chunks=chunks,
                               device=DEV, freqs=wan_freqs(D), spatial_width=W, spatial_height=FS // W,
                               **factory.PYRAMID_FORCING_REMAP)
    ctx = caches[0].ctx
    tables = O.rope_tables(D)
    # the pack reads exactly the oracle's tables (their construction is pinned on the CPU)
    ctx.freq_parts_flat = tuple(to_dev(t) for t in tables)
    g = O.Geometry(L, H, D, FS, max_sink, max_middle, max_recent, max_attend_chunks=chunks)
    states = to_np(ctx.states_bytes).reshape(L, -1)
    ref = O.MegaCacheRef(g, states, to_np(ctx.sink_caps_per_head), spatial_width=W, sink_mode=1, cmin=18, cmax=21,
                         lag=0, tables=tables)
    return caches, ref, g


def _compare_pools(caches, ref: O.MegaCacheRef, where: str):
    mgr = caches[0].ctx.mgr
    pairs = [("sink_k", mgr.sink_k_pool()), ("sink_v", mgr.sink_v_pool()), ("sink_pos", mgr.sink_pos_pool()),
             ("middle_k", mgr.middle_k_pool()), ("middle_v", mgr.middle_v_pool()),
             ("middle_pos", mgr.middle_pos_pool()), ("recent_k", mgr.recent_k_pool()),
             ("recent_v", mgr.recent_v_pool()), ("recent_pos", mgr.recent_pos_pool()),
             ("merge_k", mgr.merge_k_pool()), ("merge_v", mgr.merge_v_pool()), ("merge_pos", mgr.merge_pos_pool()),
             ("merge_token_count", mgr.merge_token_count()), ("valid_count", mgr.valid_count())]
    for name, t in pairs:
        want = getattr(ref, name)
        got = to_np(t).reshape(want.shape)
        if not np.array_equal(got, want):
            bad = np.argwhere(got != want)
            raise AssertionError(f"{where}: {name} differs at {len(bad)} places, first {bad[:4].tolist()}")
    got_states = to_np(caches[0].ctx.states_bytes).reshape(ref.states.shape)
    assert np.array_equal(got_states, ref.states), f"{where}: state records differ"
    # Veil accumulators: fp32 group sums, group ids / counts / positions, weight sums
    accs = [("sum_k", mgr.merge_accum_sum_k()), ("sum_v", mgr.merge_accum_sum_v()), ("pos", mgr.merge_accum_pos()),
            ("gid", mgr.merge_accum_group_ids()), ("tpg", mgr.merge_accum_tokens_per_group()),
            ("ng", mgr.merge_accum_num_groups()), ("wsum", mgr.merge_accum_weight_sum())]
    for name, t in accs:
        got = to_np(t)
        for layer, acc in enumerate(ref.acc):
            want = acc[name]
            g = got[layer].reshape(want.shape)
            if not np.array_equal(g, want):
                bad = np.argwhere(g != want)
                raise AssertionError(f"{where}: merge accumulator {name} of layer {layer} differs at {len(bad)} "
                                     f"places, first {bad[:4].tolist()}")


def _compare_attend(cache, ref: O.MegaCacheRef, layer, start, chunks, q_u16, where):
    """Plan + pack bit-exact, attention output vs float64 on the oracle's packed K/V."""
    FS, H, D = ref.g.frame_seqlen, ref.g.num_heads, ref.g.head_dim
    plan = cache.plan(start, chunks)
    want = ref.plan_pack(layer, start, chunks)
    names = ["cu", "sk", "sg", "sl", "dst", "traw", "tremap"]
    n_pairs = chunks * H
    for name, t in zip(names, plan):
        got = to_np(t)
        w = want[name]
        if name == "cu":
            got, w = got[:n_pairs + 1], w[:n_pairs + 1]
        assert np.array_equal(got, w), f"{where}: plan {name} differs"
    cu_k = cache.pack(plan)
    total = want["total"]
    mgr = cache.ctx.mgr
    assert np.array_equal(to_np(mgr.k_flat_out()).reshape(-1, D)[:total], want["k"]), f"{where}: packed K differs"
    assert np.array_equal(to_np(mgr.v_flat_out()).reshape(-1, D)[:total], want["v"]), f"{where}: packed V differs"
    assert np.array_equal(to_np(mgr.pos_flat_out())[:total], want["pos"]), f"{where}: packed pos differs"
    # the fused op MegaCache.attend uses (plan + layer offset + pack in one call) gives the same bytes
    mgr.k_flat_out().zero_()
    cu_fused = cache.attend_kv(start, chunks)
    assert np.array_equal(to_np(cu_fused), want["cu"][:n_pairs + 1]), f"{where}: fused cu_seqlens_k differs"
    assert np.array_equal(to_np(mgr.k_flat_out()).reshape(-1, D)[:total], want["k"]), f"{where}: fused K differs"
    assert np.array_equal(to_np(mgr.v_flat_out()).reshape(-1, D)[:total], want["v"]), f"{where}: fused V differs"
    assert np.array_equal(to_np(mgr.pos_flat_out())[:total], want["pos"]), f"{where}: fused pos differs"
    q = to_dev(q_u16).view(torch.bfloat16).view(1, chunks * FS, H, D)
    out = cache.attend(q, start)
    cu_q = np.arange(0, chunks * FS + 1, FS)
    exp = O.ragged_attention_ref(O.bf16_to_f32(q_u16).astype(np.float64), O.bf16_to_f32(want["k"]),
                                 O.bf16_to_f32(want["v"]), cu_q, want["cu"][:n_pairs + 1], heads_q=H,
                                 kv_per_head=True)
    err = np.abs(out[0].float().cpu().numpy().astype(np.float64) - exp)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, f"{where}: attention max {err.max()} mean {err.mean()}"
    del cu_k


def _rand_bf16(rng, *shape):
    return O.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))


# (FS, W): 64 / 8 tiles into the Veil heads' 2 x 2 patches (member lists in
# closed form); 63 / 9 does not (odd width: lists built from the group ids).
# split: attend runs the key-split attention (ctx.split_attention).
@pytest.mark.parametrize("seed,block_sizes,noisy_passes,FS,W,split", [
    (0, [3] * 9, 2, 64, 8, False),
    (1, [1] + [3] * 8, 1, 64, 8, False),
    (2, [2, 2, 3, 1, 3, 3, 2, 3, 4], 3, 64, 8, False),
    (3, [3] * 6, 1, 63, 9, False),
    (4, [2, 3, 1, 4, 3, 2], 2, 63, 9, False),
    (5, [3] * 9, 1, 64, 8, True),
])
def test_megacache_rollout_bit_exact(seed, block_sizes, noisy_passes, FS, W, split):
    rng = np.random.default_rng(seed)
    L, H, D = 2, 6, 128
    labels = [[-1, 1, 2, -1, 1, 2], [2, -1, 1, 1, 2, -1]]
    print(f"megacache rollout seed={seed} blocks={block_sizes} noisy={noisy_passes} FS={FS} W={W} split={split}",
          flush=True)
    caches, ref, g = _build(L, H, D, FS, W, labels, chunks=4)
    caches[0].ctx.split_attention = split
    t0 = 0
    for bi, F in enumerate(block_sizes):
        start = t0 * FS
        for p in range(noisy_passes + 1):
            mode = "clean" if p == noisy_passes else "noisy"
            for layer in range(L):
                k = _rand_bf16(rng, F * FS, H, D)
                v = _rand_bf16(rng, F * FS, H, D)
                kd = to_dev(k).view(torch.bfloat16).view(1, F * FS, H, D)
                vd = to_dev(v).view(torch.bfloat16).view(1, F * FS, H, D)
                caches[layer].update(kd, vd, start, cache_update_mode=mode)
                ref.update(layer, k, v, start, mode)
                where = f"block {bi} (t0={t0}, F={F}) pass {p} {mode} layer {layer}"
                if mode == "noisy" or bi % 3 == 2 or bi == len(block_sizes) - 1:
                    q = _rand_bf16(rng, F * FS, H, D)
                    _compare_attend(caches[layer], ref, layer, start, F, q, where)
            torch.cuda.synchronize()
            _compare_pools(caches, ref, f"block {bi} pass {p} {mode}")
        t0 += F


@pytest.mark.parametrize("how", ["permuted", "other_width"])
def test_megacache_continues_block_by_its_stored_group_ids(how):
    """A Veil block whose stored group ids are not the ids of the update's
    grid -- as when the block began through mega_merge_accum with explicit
    positions -- continues through MegaCache.update by the stored ids, as
    the reference's accumulate does (mega_merge_accum.cu:193-209).  The ids
    are replaced in the device pools and in the oracle alike between two
    updates: a token permutation of the grid ids, or the ids of a grid of
    another width with the same group count."""
    rng = np.random.default_rng(11)
    L, H, D, FS, W, F = 1, 2, 128, 64, 8, 3
    print(f"stored group ids ({how})", flush=True)
    caches, ref, g = _build(L, H, D, FS, W, [[2, 2]], chunks=F)
    mgr = caches[0].ctx.mgr

    def step(t0):
        k, v = _rand_bf16(rng, F * FS, H, D), _rand_bf16(rng, F * FS, H, D)
        caches[0].update(to_dev(k).view(torch.bfloat16).view(1, F * FS, H, D),
                         to_dev(v).view(torch.bfloat16).view(1, F * FS, H, D), t0 * FS, cache_update_mode="clean")
        ref.update(0, k, v, t0 * FS, "clean")

    step(0)  # frames 0-2 begin block 0 (4 frames) of every head
    torch.cuda.synchronize()
    slot = int(to_np(caches[0].last_update_descriptors(F)[4])[0])
    gid = ref.acc[0]["gid"]
    if how == "permuted":
        new_ids = gid[:, slot, ::-1].copy()
    else:  # the 2 x 2 patches of a 16-wide grid: 2 x 8 groups, as many as 4 x 4
        t = np.arange(FS)
        new_ids = np.broadcast_to(((t // 16) // 2) * 8 + (t % 16) // 2, (H, FS)).astype(np.int32).copy()
    assert not np.array_equal(new_ids, gid[:, slot])
    gid[:, slot] = new_ids
    mgr.merge_accum_group_ids()[0, :, slot].copy_(to_dev(new_ids))
    step(3)  # frame 3 completes block 0 through the stored ids; frames 4-5 begin block 1
    torch.cuda.synchronize()
    _compare_pools(caches, ref, f"after the continued block ({how})")
    assert int(to_np(mgr.merge_token_count())[0, 0].max()) > 0, "block 0 was finalized"


@pytest.mark.parametrize("FS,W", [(64, 8), (63, 9)])
def test_megacache_pass_for_another_block_before_the_commit(FS, W):
    """Noisy passes for a block, then a pass for another block before the
    first block's clean pass -- another t0, or the same t0 with another frame
    count -- as the reference allows (it restores its committed snapshot
    first, _mega_cache.py:226-245): pools, counters, records, accumulators,
    plan and packed K/V/pos bit-exact against the oracle after every pass,
    which restores the committed recent FIFO on every update."""
    rng = np.random.default_rng(11)
    L, H, D = 2, 6, 128
    labels = [[-1, 1, 2, -1, 1, 2], [2, -1, 1, 1, 2, -1]]
    caches, ref, g = _build(L, H, D, FS, W, labels, chunks=4)
    # (t0, frames, mode): blocks of 3 frames committed until the recent window
    # shifts, then abandoned noisy passes of other blocks between the passes
    passes = [(0, 3, "clean"), (3, 3, "clean"),
              (6, 3, "noisy"), (6, 3, "noisy"), (9, 3, "noisy"), (9, 3, "clean"),
              (12, 3, "noisy"), (12, 2, "noisy"), (12, 2, "clean"),
              (14, 3, "noisy"), (17, 1, "clean"), (18, 3, "noisy"), (18, 3, "noisy"), (18, 3, "clean")]
    for pi, (t0, F, mode) in enumerate(passes):
        print(f"pass {pi}: t0={t0} F={F} {mode} FS={FS}", flush=True)
        for layer in range(L):
            k = _rand_bf16(rng, F * FS, H, D)
            v = _rand_bf16(rng, F * FS, H, D)
            kd = to_dev(k).view(torch.bfloat16).view(1, F * FS, H, D)
            vd = to_dev(v).view(torch.bfloat16).view(1, F * FS, H, D)
            caches[layer].update(kd, vd, t0 * FS, cache_update_mode=mode)
            ref.update(layer, k, v, t0 * FS, mode)
            q = _rand_bf16(rng, F * FS, H, D)
            _compare_attend(caches[layer], ref, layer, t0 * FS, F, q, f"pass {pi} layer {layer}")
        torch.cuda.synchronize()
        _compare_pools(caches, ref, f"pass {pi} (t0={t0}, F={F}, {mode})")


def test_megacache_modes_other_than_noisy_clean_are_noops():
    L, H, D, FS, W = 1, 2, 64, 16, 4
    caches, _ref, _g = _build(L, H, D, FS, W, [[1, 2]], chunks=2)
    k = torch.ones(1, FS, H, D, dtype=torch.bfloat16, device=DEV)
    caches[0].update(k, k, 0, cache_update_mode="readonly")
    assert int(caches[0].ctx.mgr.valid_count().abs().sum()) == 0
    caches[0].update(k, k, 0, cache_update_mode="default")  # default == clean
    assert int(caches[0].ctx.mgr.valid_count()[0, :, 0].sum()) == 2


def test_megacache_plan_overflow_raises():
    """More planned tokens than the pack workspace holds is an error with the
    reference's message, not a silent truncation."""
    L, H, D, FS, W = 1, 2, 64, 16, 4
    caches, _ref, _g = _build(L, H, D, FS, W, [[1, 1]], max_middle=8, chunks=1)
    k = torch.ones(1, 3 * FS, H, D, dtype=torch.bfloat16, device=DEV)
    for b in range(8):
        caches[0].update(k, k, 3 * b * FS, cache_update_mode="clean")
    q = torch.ones(1, 3 * FS, H, D, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="exceed pack-workspace capacity"):
        caches[0].attend(q, 24 * FS)


def test_flash_attn_varlen_swap_point_matches_float64():
    from pyramidkv._mega_attention import _flash_attn_varlen
    rng = np.random.default_rng(7)
    H, D = 3, 128
    cu_q = np.array([0, 100, 164, 300], np.int32)
    cu_k = np.array([0, 500, 501, 900], np.int32)
    q = _rand_bf16(rng, int(cu_q[-1]), H, D)
    k = _rand_bf16(rng, int(cu_k[-1]), H, D)
    v = _rand_bf16(rng, int(cu_k[-1]), H, D)
    f = _flash_attn_varlen()
    out = f(to_dev(q).view(torch.bfloat16), to_dev(k).view(torch.bfloat16), to_dev(v).view(torch.bfloat16),
            to_dev(cu_q), to_dev(cu_k), 136, 400, softmax_scale=None, causal=False)
    qf, kf, vf = (O.bf16_to_f32(a).astype(np.float64) for a in (q, k, v))
    exp = np.zeros_like(qf)
    for b in range(3):
        for h in range(H):
            exp[cu_q[b]:cu_q[b + 1], h] = O.attention_ref(qf[cu_q[b]:cu_q[b + 1], h], kf[cu_k[b]:cu_k[b + 1], h],
                                                          vf[cu_k[b]:cu_k[b + 1], h])
    err = np.abs(out.float().cpu().numpy() - exp)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN


# ---------------------------------------------------------------------------
# the reference's own MegaCache scenarios (tests/test_mega_cache_noisy_clean.py:41-231)
# ---------------------------------------------------------------------------
def _single_head_caches(comp, max_sink=3, max_middle=8, max_recent=4, D=16, FSEQ=4):
    from pyramidkv._mega_cache import build_mega_caches
    return build_mega_caches(1, 1, D, FSEQ, max_sink, max_middle, max_recent, [[comp]], device=DEV,
                             kv_dtype="bfloat16")


def _states(cache, H):
    from pyramidkv import _mega_state_ops as S
    return S.unpack_states(cache.states_bytes_for_layer.cpu().numpy().view(S.PER_HEAD_STATE_DTYPE).reshape(H).copy())


def test_reference_noisy_iterations_then_clean_commits():
    from pyramidkv import HeadComposition, StrideStrategy
    H, D, FSEQ, F = 1, 16, 4, 3
    cache = _single_head_caches(HeadComposition("stride", 1, 3, 4, [StrideStrategy(interval=1, capacity=8)]))[0]
    torch.manual_seed(7)
    mk = lambda: torch.randn(1, F * FSEQ, H, D, dtype=torch.bfloat16, device=DEV)
    vc = cache.ctx.mgr.valid_count()
    for i in range(4):
        cache.update(mk(), mk(), current_start=0, cache_update_mode="noisy")
        assert int(vc[0, 0, 0].item()) == F
        assert int(cache.ctx.committed_vc[0, 0, 0].item()) == 0
    assert _states(cache, H)[0].tkey_count == 0
    ck, cv = mk(), mk()
    cache.update(ck, cv, current_start=0, cache_update_mode="clean")
    assert int(vc[0, 0, 0].item()) == F and int(cache.ctx.committed_vc[0, 0, 0].item()) == F
    assert torch.equal(cache.ctx.mgr.sink_k_pool()[0, 0, 0], ck.view(1, F, FSEQ, H, D)[0, 0, :, 0, :])
    assert _states(cache, H)[0].tkey_count == F


def test_reference_block_2_noisy_uses_block_1_committed_baseline():
    from pyramidkv import HeadComposition, StrideStrategy
    H, D, FSEQ, F = 1, 16, 4, 3
    cache = _single_head_caches(HeadComposition("stride", 1, 3, 4, [StrideStrategy(interval=1, capacity=8)]))[0]
    torch.manual_seed(11)
    mk = lambda: torch.randn(1, F * FSEQ, H, D, dtype=torch.bfloat16, device=DEV)
    cache.update(mk(), mk(), current_start=0, cache_update_mode="clean")
    assert int(cache.ctx.committed_vc[0, 0, 0].item()) == 3 and int(cache.ctx.committed_vc[0, 0, 2].item()) == 0
    cache.update(mk(), mk(), current_start=3 * FSEQ, cache_update_mode="noisy")
    vc = cache.ctx.mgr.valid_count()
    assert int(vc[0, 0, 2].item()) == 3 and int(cache.ctx.committed_vc[0, 0, 2].item()) == 0
    kb = mk()
    cache.update(kb, mk(), current_start=3 * FSEQ, cache_update_mode="noisy")
    assert int(vc[0, 0, 2].item()) == 3 and int(cache.ctx.committed_vc[0, 0, 2].item()) == 0
    assert torch.equal(cache.ctx.mgr.recent_k_pool()[0, 0, :3], kb.view(F, FSEQ, H, D)[:, :, 0, :])


def test_reference_recent_fifo_no_noisy_contamination():
    from pyramidkv import HeadComposition, RecentStrategy
    H, D, FSEQ, F = 1, 16, 4, 3
    cache = _single_head_caches(HeadComposition("recent_only", -1, 1, 4, [RecentStrategy()]), max_sink=1)[0]
    torch.manual_seed(101)
    mk = lambda: torch.randn(1, F * FSEQ, H, D, dtype=torch.bfloat16, device=DEV)
    clean = [(mk(), mk()) for _ in range(3)]
    for b in range(2):
        cache.update(*clean[b], current_start=b * F * FSEQ, cache_update_mode="clean")
    before = cache.ctx.mgr.recent_k_pool()[0].clone()
    noisy = [(mk(), mk()) for _ in range(3)]
    for k_n, v_n in noisy:
        cache.update(k_n, v_n, current_start=2 * F * FSEQ, cache_update_mode="noisy")
    cache.update(*clean[2], current_start=2 * F * FSEQ, cache_update_mode="clean")
    after = cache.ctx.mgr.recent_k_pool()[0]
    assert torch.equal(after[0, 0], before[0, 3])
    for k_n, _ in noisy:
        assert not torch.equal(after[0, 0], k_n.view(1, F, FSEQ, H, D)[0, F - 1, :, 0, :])
