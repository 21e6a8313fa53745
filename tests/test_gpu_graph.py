"""HIP-graph capture of the per-step cache path.

One step of the causal DiT's cache traffic -- for every layer a noisy pass
(MegaCache.update, then MegaCache.attend: device plan, layer offset, pack
with fused RoPE, ragged attention) followed by the clean pass of the same
block -- is captured once with torch.cuda.graph and replayed.  Each replay
starts from the same full cache state (pools, merge accumulators, state
records, counters) and must reproduce the bytes of an eager run of the same
step: pools, state records and counters bit-exact, every attention output
equal to the eager kernel's.  The replayed state is also checked against
the CPU oracle (oracle.MegaCacheRef driven with the same data): pools,
counters and state records bit-exact, every replayed attention output within
max-abs 2e-2 / mean-abs 2e-3 of float64 attention over the oracle's packed
K / V.  Capture itself fails if any op synchronises
with the host, so a passing capture shows the step is sync-free (the plan
never leaves the device).  The replays are interleaved with eager work and
synchronisations, and every replay is checked, not only the first.
Reference counterpart: pipeline/graph_runner.py and tests/test_no_host_syncs.py
of the reference, which capture the same step on CUDA."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
if torch.cuda.is_available():
    from gpu_util import DEV, to_dev
    from test_gpu_megacache import _build, _compare_pools

pytestmark = pytest.mark.gpu


def _mutable(caches):
    """Every device buffer a step reads and writes, by name."""
    ctx = caches[0].ctx
    mgr = ctx.mgr
    names = ["sink_k_pool", "sink_v_pool", "sink_pos_pool", "middle_k_pool", "middle_v_pool", "middle_pos_pool",
             "recent_k_pool", "recent_v_pool", "recent_pos_pool", "merge_k_pool", "merge_v_pool", "merge_pos_pool",
             "merge_token_count", "merge_accum_sum_k", "merge_accum_sum_v", "merge_accum_pos",
             "merge_accum_group_ids", "merge_accum_tokens_per_group", "merge_accum_num_groups",
             "merge_accum_weight_sum", "valid_count"]
    out = {n: getattr(mgr, n)() for n in names}
    out["states_bytes"] = ctx.states_bytes
    out["committed_vc"] = ctx.committed_vc
    return out


def _restore(live, snap):
    for n, t in live.items():
        t.copy_(snap[n])


def _rand(rng, *shape):
    """(host bf16 bits, device tensor) of the same N(0, 1) draw."""
    host = O.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))
    return host, to_dev(host).view(torch.bfloat16)


def test_cache_step_graph_replays_match_eager():
    rng = np.random.default_rng(7)
    # frame_seqlen >= the merge anchors' token cap (420), as at the production
    # shape, so the plan's static token bound fits the pack workspace and no
    # host check of the packed total is needed
    L, H, D, FS, W, F = 2, 6, 128, 448, 16, 3
    labels = [[-1, 1, 2, -1, 1, 2], [2, -1, 1, 1, 2, -1]]
    print("graph capture: L=2 H=6 D=128 FSEQ=448, noisy + clean step of 3 frames", flush=True)
    caches, ref, _ = _build(L, H, D, FS, W, labels, chunks=F)
    # prefill 8 clean blocks so that every strategy has middle / merge content
    for b in range(8):
        for layer in range(L):
            (kh, kd), (vh, vd) = _rand(rng, F * FS, H, D), _rand(rng, F * FS, H, D)
            caches[layer].update(kd.view(1, F * FS, H, D), vd.view(1, F * FS, H, D), b * F * FS,
                                 cache_update_mode="clean")
            ref.update(layer, kh, vh, b * F * FS, "clean")
    start = 8 * F * FS
    host = {(p, layer): (_rand(rng, F * FS, H, D), _rand(rng, F * FS, H, D), _rand(rng, F * FS, H, D))
            for p in ("noisy", "clean") for layer in range(L)}
    ins = {key: tuple(d.view(1, F * FS, H, D) for _, d in val) for key, val in host.items()}

    # the oracle's state after the step, and float64 attention on its packed K / V at each call
    want_attn = []
    cu_q = np.arange(0, F * FS + 1, FS)
    for mode in ("noisy", "clean"):
        for layer in range(L):
            (kh, _), (vh, _), (qh, _) = host[(mode, layer)]
            ref.update(layer, kh, vh, start, mode)
            w = ref.plan_pack(layer, start, F)
            want_attn.append(O.ragged_attention_ref(O.bf16_to_f32(qh).astype(np.float64), O.bf16_to_f32(w["k"]),
                                                    O.bf16_to_f32(w["v"]), cu_q, w["cu"][:F * H + 1], heads_q=H,
                                                    kv_per_head=True))

    def step():
        outs = []
        for mode in ("noisy", "clean"):
            for layer in range(L):
                k, v, q = ins[(mode, layer)]
                caches[layer].update(k, v, start, cache_update_mode=mode)
                outs.append(caches[layer].attend(q, start))
        return outs

    live = _mutable(caches)
    snap = {n: t.clone() for n, t in live.items()}

    # eager reference run
    outs = step()
    torch.cuda.synchronize()
    want = {n: t.clone() for n, t in live.items()}
    want_out = [o.clone() for o in outs]

    # warm-up on a side stream (first-call allocations), then capture
    _restore(live, snap)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _restore(live, snap)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_outs = step()
    torch.cuda.synchronize()

    for r in range(3):
        # eager work between replays: a full eager step, then a synchronisation
        if r > 0:
            _restore(live, snap)
            step()
            torch.cuda.synchronize()
        _restore(live, snap)
        graph.replay()
        torch.cuda.synchronize()
        for n, t in live.items():
            assert torch.equal(t, want[n]), f"replay {r}: {n} differs from the eager step"
        for i, (g, w) in enumerate(zip(g_outs, want_out)):
            assert torch.equal(g, w), f"replay {r}: attention output {i} differs from the eager step"
        # against the oracle
        _compare_pools(caches, ref, f"replay {r}")
        for i, (g, w) in enumerate(zip(g_outs, want_attn)):
            err = np.abs(g[0].float().cpu().numpy().astype(np.float64) - w)
            assert err.max() < 2e-2 and err.mean() < 2e-3, f"replay {r}: attention {i} vs float64 {err.max()}"
