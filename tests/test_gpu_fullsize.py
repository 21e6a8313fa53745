"""The BASELINE configurations 2-5 at their full sizes on the GPU.

* Config 2: the 360-sequence ragged attention launch (30 layers x 12 heads,
  4,680 queries per head, 6,240-32,760 keys from the seeded label matrix).
  Sampled whole sequences (the longest, the shortest, one of each label
  kind and evenly spread ones) against float64 at max-abs 2e-2 / mean-abs
  2e-3; every output row of every sequence finite and, column by column,
  inside [min V, max V] of its sequence (a softmax output is a convex
  combination of the value rows).
* Config 3: the 30-layer step at generation step 40 of a 120-frame rollout
  under the shipped policy.  For every layer: the state records, the
  state-machine descriptors of the step's update, the valid counts and the
  device plan (cu_seqlens_k and every segment array) bit-exact against the
  oracle's state machine and planner.  For three layers chosen to cover the
  label mixes, the oracle MegaCache model runs the whole rollout on the same
  data: pools and the packed K / V / positions bit-exact.
  Then the production pass pattern at full size on those three layers:
  chunks of 4 noisy passes and a clean pass, checked after every pass.
* Config 4: 40 single-frame weighted Veil evictions of 12 heads, through the
  reference's two ops, through the one-launch mega_evict_merge and as one
  call of 40 frames, all bit-exact against the oracle (anchors, positions,
  counts and the fp32 accumulators).
* Config 5: the causal DiT rollout in the Wan2.1-T2V-1.3B shape for 8
  chunks: finite outputs, and the caches advanced as the policy dictates
  (state records against the oracle state machine, valid counts and merge
  anchor counts against their closed forms).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from gpu_util import DEV, to_dev, to_np
    from pyramidkv import _abi as A

L, H, D, FSEQ, QTOK = 30, 12, 128, 1560, 4680
REMAP = (1, 18, 21, 0)  # window_clamp(18, 21), the shipped dynamic-RoPE remap


def _config2_lengths(seed: int = 0):
    """The seeded 30 x 12 label matrix over {-1, 1, 2} and the per-(layer,
    head) KV lengths: sink 1 + middle + recent 3 frames of 1,560 tokens,
    Wave middle 10 frames, Anchor 0-12, Veil 6, capped at 21 frames."""
    rng = np.random.default_rng(seed)
    labels = rng.choice([-1, 1, 2], size=(L, H))
    anchor_frames = rng.integers(0, 13, size=(L, H))
    middle = np.where(labels == -1, 10, np.where(labels == 1, anchor_frames, 6))
    return labels, (np.minimum(1 + middle + 3, 21) * FSEQ).astype(np.int64)


def test_config2_full_launch():
    labels, lk = _config2_lengths(0)
    print(f"config 2: {L * H} sequences, Q={QTOK}, keys {lk.min()}-{lk.max()}", flush=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(0)
    total_k = int(lk.sum())
    q = (torch.randn(L * QTOK, H, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    k = (torch.randn(total_k, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    v = (torch.randn(total_k, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    out = torch.full_like(q, float("nan"))
    cu_q = torch.arange(0, L * QTOK + 1, QTOK, dtype=torch.int32, device=DEV)
    cu_k_np = np.concatenate([[0], np.cumsum(lk.reshape(-1))]).astype(np.int32)
    cu_k = torch.from_numpy(cu_k_np).to(DEV)
    A.ragged_attn_fwd(q, k, v, out, cu_q, cu_k, L, H, True, QTOK, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    # every row inside its sequence's per-column value range (bf16 rounding slack)
    flat = lk.reshape(-1)
    for s in range(L * H):
        layer, head = divmod(s, H)
        vs = v[int(cu_k_np[s]):int(cu_k_np[s + 1])].float()
        lo, hi = vs.amin(0), vs.amax(0)
        o = out[layer * QTOK:(layer + 1) * QTOK, head].float()
        slack = 2e-2 * torch.maximum(lo.abs(), hi.abs()) + 1e-3
        assert bool(((o >= lo - slack) & (o <= hi + slack)).all()), f"sequence {s} leaves its value range"
    # sampled sequences against float64
    lab = labels.reshape(-1)
    picks = [int(np.argmax(flat)), int(np.argmin(flat))]
    picks += [int(np.flatnonzero(lab == kind)[0]) for kind in (-1, 1, 2)]
    picks += [int(i) for i in np.linspace(0, L * H - 1, 5).round()]
    for s in dict.fromkeys(picks):
        layer, head = divmod(s, H)
        qs = q[layer * QTOK:(layer + 1) * QTOK, head].float().cpu().numpy().astype(np.float64)
        ks = k[int(cu_k_np[s]):int(cu_k_np[s + 1])].float().cpu().numpy()
        vs = v[int(cu_k_np[s]):int(cu_k_np[s + 1])].float().cpu().numpy()
        want = O.attention_ref(qs, ks, vs, D ** -0.5)
        got = out[layer * QTOK:(layer + 1) * QTOK, head].float().cpu().numpy().astype(np.float64)
        err = np.abs(got - want)
        assert err.max() < 2e-2 and err.mean() < 2e-3, (s, int(flat[s]), err.max(), err.mean())


def _oracle_layers(labels) -> list[int]:
    """Layer 0, the layer with the most Veil heads and the one with the most
    Wave heads (distinct)."""
    lab = np.asarray(labels)
    out = [0, int(np.argmax((lab == 2).sum(1))), int(np.argmax((lab == -1).sum(1)))]
    return list(dict.fromkeys(out))


def test_config3_full_step40():
    from pyramidkv import factory
    from pyramidkv._mega_cache import build_mega_caches
    from pyramidkv.rope import wan_freqs
    F, steps = 3, 40
    labels = factory.load_head_labels(factory.SHIPPED_LABELS_CSV, L, H)
    comps = factory.shipped_compositions(L, H)
    caches = build_mega_caches(L, H, D, FSEQ, 3, 24, 4, comps, max_attend_chunks=8, device=DEV,
                               freqs=wan_freqs(D), spatial_width=52, spatial_height=30,
                               **factory.PYRAMID_FORCING_REMAP)
    ctx = caches[0].ctx
    mgr = ctx.mgr
    tables = O.rope_tables(D)
    ctx.freq_parts_flat = tuple(to_dev(t) for t in tables)
    geo = O.Geometry(L, H, D, FSEQ, 3, 24, 4, max_attend_chunks=8)
    states0 = to_np(ctx.states_bytes).reshape(L, -1)
    sink_caps = to_np(ctx.sink_caps_per_head).reshape(L, H)
    ref = O.MegaCacheRef(geo, states0, sink_caps, spatial_width=52, sink_mode=1, cmin=18, cmax=21, lag=0,
                         tables=tables)
    watch = _oracle_layers(labels)
    print(f"config 3: 30 layers x 12 heads, step {steps}, oracle data path on layers {watch}", flush=True)
    # the index-only model of every layer: state machine, merge anchor counts
    st = [states0[l].copy() for l in range(L)]
    mtc = np.zeros((L, H, 6), np.int32)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(3)
    for step in range(steps):
        start = step * F * FSEQ
        t_vals = [step * F + f for f in range(F)]
        for l in range(L):
            kd = torch.randn(1, F * FSEQ, H, D, generator=gen, device=DEV).to(torch.bfloat16)
            vd = torch.randn(1, F * FSEQ, H, D, generator=gen, device=DEV).to(torch.bfloat16)
            caches[l].update(kd, vd, start, cache_update_mode="clean")
            desc = O.state_update(st[l], t_vals, 1)
            fin = desc[6].reshape(H, F)
            for h, f in zip(*np.nonzero(fin >= 0)):
                mtc[l, h, fin[h, f]] = 390  # a 30 x 52 grid in 2 x 2 patches
            if l in watch:
                ref.update(l, to_np(kd).reshape(F * FSEQ, H, D), to_np(vd).reshape(F * FSEQ, H, D), start, "clean")
            if step == steps - 1:
                got = np.stack([to_np(t) for t in caches[l].last_update_descriptors(F)])
                assert np.array_equal(got, desc), f"layer {l}: step-{steps} descriptors differ"
    torch.cuda.synchronize()
    # every layer: state records, valid counts, anchor counts, the plan
    got_states = to_np(ctx.states_bytes).reshape(L, -1)
    vc = np.zeros((L, H, 3), np.int64)
    vc[..., 0] = np.minimum(sink_caps, 3)
    vc[..., 2] = 4
    assert np.array_equal(to_np(mgr.valid_count()), vc)
    assert np.array_equal(to_np(mgr.merge_token_count()), mtc)
    start = (steps - 1) * F * FSEQ
    t_list = [start // FSEQ + c for c in range(F)]
    names = ["cu", "sk", "sg", "sl", "dst", "traw", "tremap"]
    for l in range(L):
        assert np.array_equal(got_states[l], st[l]), f"layer {l}: state records differ"
        want = O.plan_multi(geo, st[l], vc[l], mtc[l], t_list, *REMAP)
        plan = caches[l].plan(start, F)
        for name, t, w in zip(names, plan, want):
            got = to_np(t)
            if name == "cu":
                got, w = got[:F * H + 1], w[:F * H + 1]
            assert np.array_equal(got, w), f"layer {l}: plan {name} differs"
        cu = caches[l].attend_kv(start, F)
        assert np.array_equal(to_np(cu), want[0][:F * H + 1]), f"layer {l}: fused plan cu_seqlens_k differs"
        if l in watch:
            w = ref.plan_pack(l, start, F)
            n = w["total"]
            assert np.array_equal(to_np(mgr.k_flat_out()).reshape(-1, D)[:n], w["k"]), f"layer {l}: packed K"
            assert np.array_equal(to_np(mgr.v_flat_out()).reshape(-1, D)[:n], w["v"]), f"layer {l}: packed V"
            assert np.array_equal(to_np(mgr.pos_flat_out())[:n], w["pos"]), f"layer {l}: packed pos"
    for name, t in [("sink_k", mgr.sink_k_pool()), ("sink_v", mgr.sink_v_pool()), ("sink_pos", mgr.sink_pos_pool()),
                    ("middle_k", mgr.middle_k_pool()), ("middle_v", mgr.middle_v_pool()),
                    ("middle_pos", mgr.middle_pos_pool()), ("recent_k", mgr.recent_k_pool()),
                    ("recent_v", mgr.recent_v_pool()), ("recent_pos", mgr.recent_pos_pool()),
                    ("merge_k", mgr.merge_k_pool()), ("merge_v", mgr.merge_v_pool()),
                    ("merge_pos", mgr.merge_pos_pool())]:
        for l in watch:
            assert np.array_equal(to_np(t[l]), getattr(ref, name)[l]), f"layer {l}: pool {name} differs"


def test_config3_noisy_clean_chunks():
    """Full size, shipped policy, on the three layers config 3 watches (as a
    cache of three layers): 6 chunks of 3 frames, each run as the pipeline
    runs it -- 4 noisy passes, then the clean pass (causal_inference.py:
    445-502) -- so that the recent FIFO shifts once per block, evicted frames
    reach the middle and merge pools, and noisy passes read the committed
    baseline.  After every pass: pools, valid and merge counts, state
    records and the Veil accumulators bit-exact against MegaCacheRef; for
    every noisy pass the plan and the packed K / V / positions bit-exact,
    and for each chunk's first noisy pass the attention on 64 sampled query
    rows of every (frame, head) within the north star's tolerance of
    float64."""
    from pyramidkv import factory
    from pyramidkv._mega_cache import build_mega_caches
    from pyramidkv.rope import wan_freqs
    F, chunks, noisy = 3, 6, 4
    labels_all = factory.load_head_labels(factory.SHIPPED_LABELS_CSV, L, H)
    watch = _oracle_layers(labels_all)
    Lw = len(watch)
    comps = factory.shipped_compositions(Lw, H, labels=[list(labels_all[l]) for l in watch])
    caches = build_mega_caches(Lw, H, D, FSEQ, 3, 24, 4, comps, max_attend_chunks=8, device=DEV,
                               freqs=wan_freqs(D), spatial_width=52, spatial_height=30,
                               **factory.PYRAMID_FORCING_REMAP)
    ctx = caches[0].ctx
    mgr = ctx.mgr
    tables = O.rope_tables(D)
    ctx.freq_parts_flat = tuple(to_dev(t) for t in tables)
    geo = O.Geometry(Lw, H, D, FSEQ, 3, 24, 4, max_attend_chunks=8)
    ref = O.MegaCacheRef(geo, to_np(ctx.states_bytes).reshape(Lw, -1), to_np(ctx.sink_caps_per_head).reshape(Lw, H),
                         spatial_width=52, sink_mode=1, cmin=18, cmax=21, lag=0, tables=tables)
    print(f"config 3 noisy/clean: layers {watch} of the shipped policy, {chunks} chunks x ({noisy} noisy + 1 clean)",
          flush=True)
    pools = [("sink_k", mgr.sink_k_pool), ("sink_v", mgr.sink_v_pool), ("sink_pos", mgr.sink_pos_pool),
             ("middle_k", mgr.middle_k_pool), ("middle_v", mgr.middle_v_pool), ("middle_pos", mgr.middle_pos_pool),
             ("recent_k", mgr.recent_k_pool), ("recent_v", mgr.recent_v_pool), ("recent_pos", mgr.recent_pos_pool),
             ("merge_k", mgr.merge_k_pool), ("merge_v", mgr.merge_v_pool), ("merge_pos", mgr.merge_pos_pool),
             ("merge_token_count", mgr.merge_token_count), ("valid_count", mgr.valid_count)]
    accs = [("sum_k", mgr.merge_accum_sum_k), ("sum_v", mgr.merge_accum_sum_v), ("pos", mgr.merge_accum_pos),
            ("gid", mgr.merge_accum_group_ids), ("tpg", mgr.merge_accum_tokens_per_group),
            ("ng", mgr.merge_accum_num_groups), ("wsum", mgr.merge_accum_weight_sum)]
    rng = np.random.default_rng(33)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(33)
    for c in range(chunks):
        start = c * F * FSEQ
        for p in range(noisy + 1):
            mode = "clean" if p == noisy else "noisy"
            where = f"chunk {c} pass {p} ({mode})"
            for l in range(Lw):
                kd = torch.randn(1, F * FSEQ, H, D, generator=gen, device=DEV).to(torch.bfloat16)
                vd = torch.randn(1, F * FSEQ, H, D, generator=gen, device=DEV).to(torch.bfloat16)
                caches[l].update(kd, vd, start, cache_update_mode=mode)
                ref.update(l, to_np(kd).reshape(F * FSEQ, H, D), to_np(vd).reshape(F * FSEQ, H, D), start, mode)
                if mode != "noisy":
                    continue
                want = ref.plan_pack(l, start, F)
                cu = caches[l].attend_kv(start, F)
                n_pairs, total = F * H, want["total"]
                assert np.array_equal(to_np(cu), want["cu"][:n_pairs + 1]), f"{where} layer {l}: cu_seqlens_k"
                assert np.array_equal(to_np(mgr.k_flat_out()).reshape(-1, D)[:total], want["k"]), f"{where}: K"
                assert np.array_equal(to_np(mgr.v_flat_out()).reshape(-1, D)[:total], want["v"]), f"{where}: V"
                assert np.array_equal(to_np(mgr.pos_flat_out())[:total], want["pos"]), f"{where}: pos"
                if p != 0:
                    continue
                q = torch.randn(1, F * FSEQ, H, D, generator=gen, device=DEV).to(torch.bfloat16)
                out = caches[l].attend(q, start)[0].float().cpu().numpy().astype(np.float64)
                qf = q[0].float().cpu().numpy().astype(np.float64)
                kf = O.bf16_to_f32(want["k"]).astype(np.float64)
                vf = O.bf16_to_f32(want["v"]).astype(np.float64)
                errs = []
                for f in range(F):
                    rows = f * FSEQ + rng.choice(FSEQ, 64, replace=False)
                    for h in range(H):
                        lo, hi = want["cu"][f * H + h], want["cu"][f * H + h + 1]
                        sc = qf[rows, h] @ kf[lo:hi].T * D ** -0.5
                        pr = np.exp(sc - sc.max(axis=1, keepdims=True))
                        pr /= pr.sum(axis=1, keepdims=True)
                        errs.append(np.abs(out[rows, h] - pr @ vf[lo:hi]))
                err = np.concatenate(errs)
                assert err.max() < 2e-2 and err.mean() < 2e-3, f"{where} layer {l}: attention {err.max()} {err.mean()}"
            torch.cuda.synchronize()
            for name, fn in pools:
                want = getattr(ref, name)
                got = to_np(fn()).reshape(want.shape)
                if not np.array_equal(got, want):
                    bad = np.argwhere(got != want)
                    raise AssertionError(f"{where}: {name} differs at {len(bad)} places, first {bad[:4].tolist()}")
            assert np.array_equal(to_np(ctx.states_bytes).reshape(ref.states.shape), ref.states), f"{where}: records"
            for name, fn in accs:
                got = to_np(fn())
                for l in range(Lw):
                    w = ref.acc[l][name]
                    assert np.array_equal(got[l].reshape(w.shape), w), f"{where}: accumulator {name} of layer {l}"


def test_config4_weighted_evictions():
    from pyramidkv import _ops
    ops = _ops.ops()
    E, MMA, MMB, MT = 40, 2, 6, 420
    rng = np.random.default_rng(4)
    print(f"config 4: {E} single-frame weighted evictions, {H} heads, FSEQ {FSEQ}", flush=True)
    states = O.states_to_bytes([O.make_merge(2, 6) for _ in range(H)]).view(np.uint8).reshape(-1)
    sd = to_dev(states.copy())
    acc = dict(sum_k=np.zeros((H, MMA, MT, D), np.float32), sum_v=np.zeros((H, MMA, MT, D), np.float32),
               pos=np.zeros((H, MMA, MT, 3), np.int64), gid=np.zeros((H, MMA, FSEQ), np.int32),
               tpg=np.zeros((H, MMA, MT), np.float32), ng=np.zeros((H, MMA), np.int32),
               wsum=np.zeros((H, MMA), np.float32), mk=np.zeros((H, MMB, MT, D), np.uint16),
               mv=np.zeros((H, MMB, MT, D), np.uint16), mpos=np.zeros((H, MMB, MT, 3), np.int64),
               mtc=np.zeros((H, MMB), np.int32))
    dacc = {n: to_dev(a) for n, a in acc.items()}
    desc = [torch.full((H,), -1, dtype=torch.int32, device=DEV) for _ in range(8)]
    # the same evictions through the one-launch op (the bench's config-4 path)
    sd1 = to_dev(states.copy())
    dacc1 = {n: to_dev(a) for n, a in acc.items()}
    desc1 = [torch.full((H,), -1, dtype=torch.int32, device=DEV) for _ in range(8)]
    tok = np.arange(FSEQ)
    ws = torch.zeros(ops.mega_evict_merge_workspace_size(H), dtype=torch.uint8, device=DEV)
    frames_k, frames_v, weights, want_desc = [], [], [], []
    for e in range(E):
        k = O.f32_to_bf16(rng.standard_normal((1, H, FSEQ, D)).astype(np.float32))
        v = O.f32_to_bf16(rng.standard_normal((1, H, FSEQ, D)).astype(np.float32))
        pos = np.zeros((1, H, FSEQ, 3), np.int64)
        pos[..., 0] = e + 1
        pos[..., 1] = tok // 52
        pos[..., 2] = tok % 52
        w = rng.uniform(0.1, 1.0, 1).astype(np.float32)
        d_ = O.state_update(states, [e + 1], 1)
        O.merge_accum(states, k, v, pos, d_, acc, weights=w)
        frames_k.append(k)
        frames_v.append(v)
        weights.append(w)
        want_desc.append(d_.copy())
        ops.mega_state_update(sd, torch.tensor([e + 1], dtype=torch.int64, device=DEV), *desc, H, 1, 1)
        ops.mega_merge_accum_weighted(sd, to_dev(k).view(torch.bfloat16), to_dev(v).view(torch.bfloat16), to_dev(pos),
                                      desc[0], desc[4], desc[6], desc[7], to_dev(w), dacc["sum_k"], dacc["sum_v"],
                                      dacc["pos"], dacc["gid"], dacc["tpg"], dacc["ng"], dacc["wsum"], dacc["mk"],
                                      dacc["mv"], dacc["mpos"], dacc["mtc"])
        ops.mega_evict_merge(sd1, torch.tensor([e + 1], dtype=torch.int64, device=DEV), to_dev(k).view(torch.bfloat16),
                             to_dev(v).view(torch.bfloat16), 52, to_dev(w), *desc1, dacc1["sum_k"], dacc1["sum_v"],
                             dacc1["pos"], dacc1["gid"], dacc1["tpg"], dacc1["ng"], dacc1["wsum"], dacc1["mk"],
                             dacc1["mv"], dacc1["mpos"], dacc1["mtc"], ws)
    # all 40 evictions as one call of 40 frames (the several-frame kernel)
    sd40 = to_dev(O.states_to_bytes([O.make_merge(2, 6) for _ in range(H)]).view(np.uint8).reshape(-1).copy())
    dacc40 = {n: to_dev(np.zeros_like(a)) for n, a in acc.items()}
    desc40 = [torch.full((H * E,), -7, dtype=torch.int32, device=DEV) for _ in range(8)]
    ops.mega_evict_merge(sd40, torch.arange(1, E + 1, dtype=torch.int64, device=DEV),
                         to_dev(np.concatenate(frames_k)).view(torch.bfloat16),
                         to_dev(np.concatenate(frames_v)).view(torch.bfloat16), 52, to_dev(np.concatenate(weights)),
                         *desc40, dacc40["sum_k"], dacc40["sum_v"], dacc40["pos"], dacc40["gid"], dacc40["tpg"],
                         dacc40["ng"], dacc40["wsum"], dacc40["mk"], dacc40["mv"], dacc40["mpos"], dacc40["mtc"], ws)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(sd), states)
    assert np.array_equal(to_np(sd1), states), "mega_evict_merge: state records differ"
    assert np.array_equal(to_np(sd40), states), "mega_evict_merge, 40 frames: state records differ"
    for i in range(8):
        want = np.stack([want_desc[e][i] for e in range(E)], axis=1).reshape(-1)  # index h * E + e
        if i == 2:  # src_frame: the frame's index within the call
            want = np.tile(np.arange(E), H)
        assert np.array_equal(to_np(desc40[i]), want.astype(np.int32)), f"40 frames: descriptor array {i} differs"
    for i in range(8):
        assert torch.equal(desc[i], desc1[i]), f"mega_evict_merge: descriptor array {i} differs"
    for n, a in acc.items():
        for tag, dd in (("two ops", dacc), ("mega_evict_merge", dacc1), ("mega_evict_merge, 40 frames", dacc40)):
            got = to_np(dd[n])
            assert np.array_equal(got.view(a.dtype) if got.dtype != a.dtype else got, a), f"{tag}: {n} differs"


def test_config5_full_shape_rollout():
    from pyramidkv import factory
    from pyramidkv._mega_cache import build_mega_caches
    from pyramidkv.causal_dit import CausalDiT, WanShape, rollout
    from pyramidkv.rope import wan_freqs
    shape = WanShape()
    chunks = 8
    print(f"config 5: Wan2.1-1.3B shape ({shape.num_blocks} blocks, dim {shape.dim}), {chunks} chunks", flush=True)
    model = CausalDiT(shape, DEV, seed=0)
    labels = np.random.default_rng(0).choice([-1, 1, 2], size=(shape.num_blocks, shape.heads)).tolist()
    comps = factory.shipped_compositions(shape.num_blocks, shape.heads, labels=labels)
    caches = build_mega_caches(shape.num_blocks, shape.heads, shape.head_dim, shape.frame_seqlen, 3, 24, 4, comps,
                               max_attend_chunks=3, device=DEV, freqs=wan_freqs(shape.head_dim),
                               spatial_width=shape.grid_w, spatial_height=shape.grid_h,
                               **factory.PYRAMID_FORCING_REMAP)
    ctx = caches[0].ctx
    states0 = to_np(ctx.states_bytes).reshape(shape.num_blocks, -1)
    g = torch.Generator(device=DEV)
    g.manual_seed(1)
    model.set_context(torch.randn(shape.text_len, shape.text_dim, generator=g, device=DEV).to(torch.bfloat16))
    r = rollout(model, caches, chunks, timed_from=1, seed=0)
    assert r["chunks"] == chunks - 1 and 0.0 < r["cache_ms"] < r["ms"]
    x = torch.randn(shape.in_channels, 3, shape.grid_h * 2, shape.grid_w * 2, generator=g, device=DEV)
    vel = model.forward(x.to(torch.bfloat16), 500.0, chunks * 3 * shape.frame_seqlen, caches, "noisy")
    assert torch.isfinite(vel.float()).all()
    # the clean passes committed 3 * chunks frames: the index state follows the policy
    frames = 3 * chunks
    caps = to_np(ctx.sink_caps_per_head).reshape(shape.num_blocks, shape.heads)
    vc = to_np(ctx.mgr.valid_count())
    assert np.array_equal(vc[..., 0], np.minimum(caps, 3))
    assert np.array_equal(vc[..., 2], np.minimum(frames - np.minimum(caps, 3), 4))
    mtc = np.zeros((shape.num_blocks, shape.heads, 6), np.int32)
    ng = (shape.grid_h // 2) * (shape.grid_w // 2)
    got_states = to_np(ctx.states_bytes).reshape(shape.num_blocks, -1)
    for l in range(shape.num_blocks):
        st = states0[l].copy()
        for c in range(chunks):
            desc = O.state_update(st, [3 * c + f for f in range(3)], 1)
            fin = desc[6].reshape(shape.heads, 3)
            for h, f in zip(*np.nonzero(fin >= 0)):
                mtc[l, h, fin[h, f]] = ng
        assert np.array_equal(got_states[l], st), f"block {l}: state records differ from the policy's state machine"
    assert np.array_equal(to_np(ctx.mgr.merge_token_count()), mtc)
    # attention over the rollout's own packed pyramid (after the noisy pass of chunk `chunks`), for the first
    # and the last block: MegaCache.attend against float64 on 40 query rows of every (frame, head) sequence
    start = chunks * 3 * shape.frame_seqlen
    H, D, FS = shape.heads, shape.head_dim, shape.frame_seqlen
    rows = np.random.default_rng(3).choice(FS, size=40, replace=False)
    for l in (0, shape.num_blocks - 1):
        q = (torch.randn(1, 3 * FS, H, D, generator=g, device=DEV) * 2.0).to(torch.bfloat16)
        out = caches[l].attend(q, start)
        cu_k = to_np(caches[l].attend_kv(start, 3)).astype(np.int64)
        kf = O.bf16_to_f32(to_np(ctx.mgr.k_flat_out().view(-1, D))).astype(np.float64)
        vf = O.bf16_to_f32(to_np(ctx.mgr.v_flat_out().view(-1, D))).astype(np.float64)
        qf = O.bf16_to_f32(to_np(q[0])).astype(np.float64)
        got = O.bf16_to_f32(to_np(out[0])).astype(np.float64)
        errs = []
        for f in range(3):
            for h in range(H):
                s_ = f * H + h
                k_, v_ = kf[cu_k[s_]:cu_k[s_ + 1]], vf[cu_k[s_]:cu_k[s_ + 1]]
                assert len(k_) > 0
                want = O.attention_ref(qf[f * FS + rows, h], k_, v_)
                errs.append(np.abs(got[f * FS + rows, h] - want))
        err = np.concatenate(errs)
        assert np.isfinite(got).all()
        assert err.max() < 2e-2 and err.mean() < 2e-3, (l, err.max(), err.mean())
