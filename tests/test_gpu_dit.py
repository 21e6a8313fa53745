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


def _bf16_close(got: torch.Tensor, want: torch.Tensor, ulps: float = 1.0) -> None:
    """got (bf16 result) within `ulps` bf16 units of the float64 value want
    (a unit is 2^-7 of the value's binade; a small floor covers near-zeros)."""
    g, w = got.double(), want.double()
    tol = ulps * 2.0 ** -7 * w.abs() + 1e-6
    bad = (g - w).abs() > tol
    assert not bad.any(), (g[bad][:5], w[bad][:5])


@pytest.mark.parametrize("rows,C", [(4680, 1536), (37, 256), (5, 4096)])
def test_dit_row_ops_vs_float64(rows, C):
    """The DiT block's row operations (LayerNorm with modulation or affine
    weights, RMSNorm of a column slice, gated residual, tanh GELU) against
    float64 torch formulas; bf16 results within one bf16 unit, the fp32
    residual within fp32 rounding."""
    import torch.nn.functional as F
    from pyramidkv import _ops
    ops = _ops.ops()
    g = torch.Generator(device=DEV)
    g.manual_seed(rows + C)
    eps = 1e-6
    x = torch.randn(rows, C, generator=g, device=DEV) * 3.0 + 1.5  # a mean well away from 0
    scale = torch.randn(C, generator=g, device=DEV) * 0.1
    shift = torch.randn(C, generator=g, device=DEV) * 0.1
    ln = F.layer_norm(x.double(), (C,), eps=eps)
    _bf16_close(ops.dit_layer_norm(x, scale, shift, True, eps), ln * (1 + scale.double()) + shift.double())
    _bf16_close(ops.dit_layer_norm(x, scale, shift, False, eps), ln * scale.double() + shift.double(), ulps=1.0)
    _bf16_close(ops.dit_layer_norm(x, None, None, True, eps), ln)
    wide = (torch.randn(rows, 3 * C, generator=g, device=DEV) * 2.0).to(torch.bfloat16)
    col = wide[:, C:2 * C]
    w = torch.rand(C, generator=g, device=DEV) + 0.5
    cd = col.double()
    _bf16_close(ops.dit_rms_norm(col, w, eps), cd * torch.rsqrt(cd.pow(2).mean(-1, keepdim=True) + eps) * w.double())
    x0 = torch.randn(rows, C, generator=g, device=DEV)
    gate = torch.randn(C, generator=g, device=DEV)
    xr = x0.clone()
    ops.dit_residual_(xr, wide[:, :C], gate)
    want = x0.double() + wide[:, :C].double() * gate.double()
    assert ((xr.double() - want).abs() <= 2.0 ** -22 * (want.abs() + (wide[:, :C].double() * gate.double()).abs())).all()
    xr = x0.clone()
    ops.dit_residual_(xr, wide[:, :C], None)
    assert torch.equal(xr, x0 + wide[:, :C].float())
    hb = (torch.randn(rows, C, generator=g, device=DEV) * 3.0).to(torch.bfloat16)
    _bf16_close(ops.dit_gelu_tanh(hb), F.gelu(hb.double(), approximate="tanh"), ulps=1.0)


@pytest.mark.parametrize("rows,C", [(4680, 1536), (37, 256), (5, 4096)])
@pytest.mark.parametrize("gated,one_plus", [(True, True), (False, True), (True, False)])
def test_dit_residual_layer_norm_equals_the_two_ops(rows, C, gated, one_plus):
    """The fused residual update + LayerNorm leaves the same fp32 stream and
    the same bf16 output as dit_residual_ followed by dit_layer_norm (bit
    for bit), for gated and ungated updates and both scale forms."""
    from pyramidkv import _ops
    ops = _ops.ops()
    g = torch.Generator(device=DEV)
    g.manual_seed(7 * rows + C)
    eps = 1e-6
    x0 = torch.randn(rows, C, generator=g, device=DEV) * 2.0 + 0.5
    wide = (torch.randn(rows, 2 * C, generator=g, device=DEV) * 2.0).to(torch.bfloat16)
    y = wide[:, C:]  # a column slice: rows with a stride
    gate = torch.randn(C, generator=g, device=DEV) if gated else None
    mul = torch.randn(C, generator=g, device=DEV) * 0.1
    add = torch.randn(C, generator=g, device=DEV) * 0.1
    xa = x0.clone()
    ops.dit_residual_(xa, y, gate)
    want = ops.dit_layer_norm(xa, mul, add, one_plus, eps)
    xb = x0.clone()
    got = ops.dit_residual_layer_norm_(xb, y, gate, mul, add, one_plus, eps)
    assert torch.equal(xb, xa)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
