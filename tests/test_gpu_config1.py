"""BASELINE config 1 on the GPU: the single-layer pyramid cache step at full
size.

12 heads x head_dim 128, 1,560-token frames (a 30 x 52 grid); every head
keeps a sink of 1 frame and a recent window of 3 frames with no middle;
Q/K/V ~ N(0, 1) from a seed.  The cache already holds frame 0 in its sink;
the step scatters the new 3-frame chunk (t = 18, 19, 20) into the recent
window, packs sink + recent with the Wan 3D RoPE (22/21/21 complex pairs,
theta 10^4) at remapped temporal positions -- the sink's t becomes
window_clamp(18, 21) of the chunk, 0, and the recent frames keep t = 18..20,
all inside [0, 21) -- rotates the queries at their own positions and runs
the non-causal chunk attention: 12 x 4,680 queries over 6,240 keys
(179.4 GFLOP).

The reference runs this step as fp32 PyTorch on the CPU.  Here the oracle's
restatement of the same step (pools, plan, pack, RoPE; float64 attention) is
the checker: the packed K/V/pos and the rotated queries are bit-exact, the
bf16 attention output is within the north-star tolerance (max-abs 2e-2,
mean-abs 2e-3)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
if torch.cuda.is_available():
    from gpu_util import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu

H, D, FS, W, F, T0 = 12, 128, 1560, 52, 3, 18


def test_config1_single_layer_step():
    from pyramidkv import factory
    from pyramidkv._mega_cache import build_mega_caches
    from pyramidkv.base import HeadComposition
    from pyramidkv.rope import wan_freqs
    print("config 1: 12 heads, sink 1 + recent 3 frames, chunk t=18..20, 4680 x 6240 attention", flush=True)
    rng = np.random.default_rng(0)
    comps = [[HeadComposition(f"h{h}", 0, sink_frames=1, recent_frames=3) for h in range(H)]]
    caches = build_mega_caches(1, H, D, FS, 1, 1, 3, comps, max_attend_chunks=F, device=DEV, freqs=wan_freqs(D),
                               spatial_width=W, spatial_height=FS // W, **factory.PYRAMID_FORCING_REMAP)
    cache = caches[0]
    ctx = cache.ctx
    tables = O.rope_tables(D)
    ctx.freq_parts_flat = tuple(to_dev(t) for t in tables)
    g = O.Geometry(1, H, D, FS, 1, 1, 3, max_attend_chunks=F)
    ref = O.MegaCacheRef(g, to_np(ctx.states_bytes).reshape(1, -1), to_np(ctx.sink_caps_per_head), spatial_width=W,
                         sink_mode=1, cmin=18, cmax=21, lag=0, tables=tables)
    draw = lambda n: O.f32_to_bf16(rng.standard_normal((n, H, D)).astype(np.float32))
    bf = lambda a, n: to_dev(a).view(torch.bfloat16).view(1, n, H, D)

    # frame 0 -> the sink
    k0, v0 = draw(FS), draw(FS)
    cache.update(bf(k0, FS), bf(v0, FS), 0, cache_update_mode="clean")
    ref.update(0, k0, v0, 0, "clean")
    # the step: scatter the chunk t = 18..20, plan + pack with RoPE, attention
    start = T0 * FS
    k, v, q = draw(F * FS), draw(F * FS), draw(F * FS)
    cache.update(bf(k, F * FS), bf(v, F * FS), start, cache_update_mode="clean")
    ref.update(0, k, v, start, "clean")
    want = ref.plan_pack(0, start, F)
    cu = to_np(cache.attend_kv(start, F))
    total = want["total"]
    # each of the 3 query frames (one chunk each) attends to sink + recent = 6,240 tokens per head
    assert total == F * H * (FS + F * FS) and np.array_equal(cu, want["cu"][:F * H + 1])
    mgr = ctx.mgr
    assert np.array_equal(to_np(mgr.k_flat_out()).reshape(-1, D)[:total], want["k"]), "packed K (roped) differs"
    assert np.array_equal(to_np(mgr.v_flat_out()).reshape(-1, D)[:total], want["v"]), "packed V differs"
    assert np.array_equal(to_np(mgr.pos_flat_out())[:total], want["pos"]), "packed positions differ"
    # the sink's temporal position is remapped to 0, the recent frames keep theirs
    t_packed = want["pos"][:, 0]
    assert t_packed.max() < 21

    # queries rotated at (t, y, x) of their own tokens, on the GPU and by the oracle
    tok = np.arange(F * FS)
    qpos = np.stack([T0 + tok // FS, (tok % FS) // W, tok % W], axis=1).astype(np.int64)
    qpos_rows = np.repeat(qpos, H, axis=0)
    q_rot_ref = O.rope_apply(q.reshape(-1, D), qpos_rows, tables)
    from pyramidkv import _ops
    q_rot = _ops.ops().rope_apply(to_dev(q).view(torch.bfloat16).view(-1, D), to_dev(qpos_rows), *ctx.freq_parts_flat)
    assert np.array_equal(to_np(q_rot.view(torch.uint16)), q_rot_ref), "rotated queries differ"

    out = cache.attend(q_rot.view(1, F * FS, H, D), start)
    cu_q = np.arange(0, F * FS + 1, FS)
    exp = O.ragged_attention_ref(O.bf16_to_f32(q_rot_ref.reshape(F * FS, H, D)).astype(np.float64),
                                 O.bf16_to_f32(want["k"]).astype(np.float64),
                                 O.bf16_to_f32(want["v"]).astype(np.float64), cu_q, want["cu"][:F * H + 1],
                                 heads_q=H, kv_per_head=True)
    got = out[0].float().cpu().numpy().astype(np.float64)
    err = np.abs(got - exp)
    assert np.isfinite(got).all()
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
