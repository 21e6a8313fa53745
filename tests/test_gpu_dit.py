"""The config-5 rollout harness on the GPU.

* The cross-attention path (ragged attention with one K/V sequence per
  batch in flash_attn_varlen_func's [total_k, H, D] layout, kv_per_head=False)
  against float64 softmax attention, head_dim 128 and 64, at the tolerance
  of the attention tests (max-abs 2e-2, mean-abs 2e-3).
* A small causal DiT rollout through the pyramid cache (4 noisy forwards and
  one clean forward per chunk, the reference pipeline's block loop): the
  caches advance every chunk, the outputs stay finite, and the pyramid-path
  time is a proper share of the step time."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
if torch.cuda.is_available():
    from gpu_util import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D,Nq,T,H", [(128, 4680, 512, 12), (128, 300, 77, 3), (64, 129, 512, 2)])
def test_cross_attention_shared_kv_vs_float64(D, Nq, T, H):
    from pyramidkv import _ops
    rng = np.random.default_rng(D + Nq)
    q = O.f32_to_bf16((rng.standard_normal((Nq, H, D)) * 0.5).astype(np.float32))
    k = O.f32_to_bf16((rng.standard_normal((T, H, D)) * 0.5).astype(np.float32))
    v = O.f32_to_bf16((rng.standard_normal((T, H, D)) * 0.5).astype(np.float32))
    cu_q = np.array([0, Nq], np.int32)
    cu_k = np.array([0, T], np.int32)
    bf = lambda a: to_dev(a).view(torch.bfloat16)
    out = _ops.ragged_attention(bf(q), bf(k), bf(v), to_dev(cu_q), to_dev(cu_k), Nq, None, kv_per_head=False)
    got = O.bf16_to_f32(to_np(out.view(torch.uint16))).astype(np.float64)
    want = O.ragged_attention_ref(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), cu_q, cu_k, H,
                                  kv_per_head=False)
    err = np.abs(got - want)
    assert np.isfinite(got).all()
    assert err.max() < 2e-2 and err.mean() < 2e-3, (err.max(), err.mean())


def test_causal_dit_rollout_small():
    from pyramidkv import factory
    from pyramidkv._mega_cache import build_mega_caches
    from pyramidkv.causal_dit import CausalDiT, WanShape, rollout
    from pyramidkv.rope import wan_freqs
    s = WanShape(num_blocks=2, dim=256, heads=2, ffn=512, in_channels=4, text_dim=32, text_len=16, freq_dim=64,
                 grid_h=6, grid_w=8)
    print("causal DiT rollout: 2 blocks, dim 256, 2 heads of 128, 48 tokens per frame, 4 chunks", flush=True)
    model = CausalDiT(s, DEV, seed=3)
    labels = [[-1, 2], [1, 2]]
    comps = factory.shipped_compositions(s.num_blocks, s.heads, labels=labels)
    caches = build_mega_caches(s.num_blocks, s.heads, s.head_dim, s.frame_seqlen, 3, 24, 4, comps,
                               max_attend_chunks=3, device=DEV, freqs=wan_freqs(s.head_dim), spatial_width=s.grid_w,
                               spatial_height=s.grid_h, **factory.PYRAMID_FORCING_REMAP)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    model.set_context(torch.randn(s.text_len, s.text_dim, generator=g, device=DEV).to(torch.bfloat16))
    r = rollout(model, caches, 4, timed_from=1, seed=1)
    assert r["chunks"] == 3 and r["chunks_per_s"] > 0
    assert 0.0 < r["cache_ms"] < r["ms"]
    # the clean passes committed 12 frames: every head's recent FIFO is full (max_recent = 4)
    vc = to_np(caches[0].ctx.mgr.valid_count())
    assert (vc[..., 2] == 4).all(), vc
    x = torch.randn(s.in_channels, 3, s.grid_h * 2, s.grid_w * 2, generator=g, device=DEV).to(torch.bfloat16)
    vel = model.forward(x, 500.0, 4 * 3 * s.frame_seqlen, caches, "noisy")
    assert vel.shape == x.shape and torch.isfinite(vel.float()).all()
