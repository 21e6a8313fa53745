"""A random-init causal DiT in the Wan2.1-T2V-1.3B shape that drives the
pyramid cache the way the reference's CausalWanModel does at inference, for
the end-to-end rollout measurement: latent chunks per second, and the share
of the step time spent in the pyramid path (cache update, plan, pack and the
ragged self-attention).

Structure followed (IF-LAB-PKU/Pyramid-Forcing file:line):

* attention block, wan/modules/causal_model.py:320-440: norm1 + modulation
  -> self-attention through the pyramid cache -> gated residual; norm3 ->
  cross-attention to the text context -> residual; norm2 + modulation ->
  GELU(tanh) FFN -> gated residual;
* self-attention projections and the q/k RMSNorm, causal_model.py:66-93;
  raw K and V go to MegaCache.update and the roped query to MegaCache.attend,
  causal_model.py:205-217;
* query RoPE at absolute frame positions, causal_model.py:30-63 (here in
  fp32 by the rope_apply kernel rather than float64);
* embeddings, head and the inference forward, causal_model.py:442-470 and
  800-920; the text context is embedded once and every block's
  cross-attention K/V are computed once per rollout (the crossattn_cache);
* per chunk, 4 noisy denoising forwards and one clean forward that commits
  the cache, pipeline/causal_inference.py:445-502, with flow matching:
  sigma = t / 1000, x0 = x_t - sigma * v, re-noised as
  (1 - sigma') x0 + sigma' noise.

Weights are drawn at random (no checkpoint exists here); the measurement is
of throughput, not of sample quality.
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _ops
from .rope import flat_freq_parts, wan_freqs

# The rollout's GEMM solutions (hipBLASLt / rocBLAS), as torch's TunableOp
# chose them on an MI355X for every GEMM shape of the rollout (written by
# `python bench.py --tune-gemms`).  Its first lines pin the torch, HIP,
# hipBLASLt and rocBLAS versions and the GPU architecture.
GEMM_TUNING_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_tuning_gfx950.csv")


def use_tuned_gemms(path: str = GEMM_TUNING_FILE) -> bool:
    """Select GEMM solutions from a TunableOp results file (process-wide,
    torch.cuda.tunable, tuning off).  Shapes the file does not list, and
    every shape when its validator lines do not match this process's
    libraries, keep torch's default choice.  Returns whether the file was
    read."""
    import torch.cuda.tunable as tunable
    if not os.path.exists(path):
        return False
    tunable.enable(True)
    tunable.tuning_enable(False)
    return bool(tunable.read_file(path))


@dataclass
class WanShape:
    num_blocks: int = 30
    dim: int = 1536
    heads: int = 12
    ffn: int = 8960
    in_channels: int = 16
    patch: tuple = (1, 2, 2)
    text_dim: int = 4096
    text_len: int = 512
    freq_dim: int = 256
    grid_h: int = 30  # latent tokens per frame = grid_h * grid_w after the patch
    grid_w: int = 52
    eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.dim // self.heads

    @property
    def frame_seqlen(self) -> int:
        return self.grid_h * self.grid_w


def _linear(i: int, o: int, gen, device, std: float = 0.02):
    w = (torch.randn(o, i, generator=gen, device=device) * std).to(torch.bfloat16)
    b = torch.zeros(o, device=device, dtype=torch.bfloat16)
    return w, b


def _sinusoid(freq_dim: int, t: float, device) -> torch.Tensor:
    """sinusoidal_embedding_1d of causal_model.py (cos then sin halves)."""
    half = freq_dim // 2
    pos = torch.tensor([float(t)], dtype=torch.float64, device=device)
    sin = torch.outer(pos, torch.pow(10000, -torch.arange(half, dtype=torch.float64, device=device).div(half)))
    return torch.cat([torch.cos(sin), torch.sin(sin)], dim=1).float()


class CausalDiT:
    """Inference-only forward with per-block pyramid caches."""

    def __init__(self, shape: WanShape = WanShape(), device: str = "cuda:0", seed: int = 0):
        self.s = s = shape
        self.device = device
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        pt, ph, pw = s.patch
        self.patch_in = s.in_channels * pt * ph * pw
        self.w_patch = _linear(self.patch_in, s.dim, g, device)
        self.w_time = (_linear(s.freq_dim, s.dim, g, device), _linear(s.dim, s.dim, g, device))
        self.w_tproj = _linear(s.dim, 6 * s.dim, g, device)
        self.w_text = (_linear(s.text_dim, s.dim, g, device), _linear(s.dim, s.dim, g, device))
        self.blocks = []
        for _ in range(s.num_blocks):
            blk = {
                "mod": torch.randn(6, s.dim, generator=g, device=device) / s.dim ** 0.5,
                "q": _linear(s.dim, s.dim, g, device), "k": _linear(s.dim, s.dim, g, device),
                "v": _linear(s.dim, s.dim, g, device), "o": _linear(s.dim, s.dim, g, device),
                "norm_q": torch.ones(s.dim, device=device), "norm_k": torch.ones(s.dim, device=device),
                "norm3_w": torch.ones(s.dim, device=device), "norm3_b": torch.zeros(s.dim, device=device),
                "cq": _linear(s.dim, s.dim, g, device), "ck": _linear(s.dim, s.dim, g, device),
                "cv": _linear(s.dim, s.dim, g, device), "co": _linear(s.dim, s.dim, g, device),
                "cnorm_q": torch.ones(s.dim, device=device), "cnorm_k": torch.ones(s.dim, device=device),
                "ffn1": _linear(s.dim, s.ffn, g, device), "ffn2": _linear(s.ffn, s.dim, g, device),
            }
            # q, k and v as one [3*dim, dim] GEMM
            blk["qkv"] = (torch.cat([blk["q"][0], blk["k"][0], blk["v"][0]]).contiguous(),
                          torch.cat([blk["q"][1], blk["k"][1], blk["v"][1]]).contiguous())
            self.blocks.append(blk)
        self.head_mod = torch.randn(2, s.dim, generator=g, device=device) / s.dim ** 0.5
        self.w_head = _linear(s.dim, self.patch_in, g, device)
        self.freq_parts_flat = flat_freq_parts(wan_freqs(s.head_dim), device)
        self.cross_kv = None
        self._pos_cache = {}

    # -- helpers ---------------------------------------------------------
    @staticmethod
    def _mm(x: torch.Tensor, wb) -> torch.Tensor:
        w, b = wb
        return F.linear(x.to(torch.bfloat16), w, b)

    def _rms(self, x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        """WanRMSNorm on bf16 rows (a column slice of a wider GEMM output is
        fine): bf16(x * rsqrt(mean(x^2) + eps) * weight), one HIP launch."""
        return _ops.ops().dit_rms_norm(x, weight, self.s.eps)

    def _ln_mod(self, x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor) -> torch.Tensor:
        """bf16(LN(x) * (1 + scale) + shift) of the fp32 residual stream."""
        return _ops.ops().dit_layer_norm(x, scale, shift, True, self.s.eps)

    def _ln_affine(self, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """bf16(LN(x) * w + b), WanLayerNorm with elementwise affine."""
        return _ops.ops().dit_layer_norm(x, w, b, False, self.s.eps)

    def _query_pos(self, t0: int, frames: int) -> torch.Tensor:
        """(t, y, x) of every (token, head) row of the roped query, t absolute."""
        key = (t0, frames)
        pos = self._pos_cache.get(key)
        if pos is None:
            s = self.s
            tok = torch.arange(frames * s.frame_seqlen, device=self.device)
            t = t0 + tok // s.frame_seqlen
            r = tok % s.frame_seqlen
            p = torch.stack([t, r // s.grid_w, r % s.grid_w], dim=1).to(torch.int64)
            pos = p.repeat_interleave(s.heads, dim=0).contiguous()
            self._pos_cache = {key: pos}
        return pos

    def set_context(self, text: torch.Tensor) -> None:
        """Embed the [text_len, text_dim] context and cache every block's
        cross-attention K [text_len, H, D] (RMSNorm applied) and V."""
        s = self.s
        c = self._mm(F.gelu(self._mm(text, self.w_text[0]).float(), approximate="tanh"), self.w_text[1])
        self.cross_kv = []
        for blk in self.blocks:
            k = self._rms(self._mm(c, blk["ck"]), blk["cnorm_k"]).view(s.text_len, s.heads, s.head_dim)
            v = self._mm(c, blk["cv"]).view(s.text_len, s.heads, s.head_dim)
            self.cross_kv.append((k.contiguous(), v.contiguous()))
        self._cu_text = torch.tensor([0, s.text_len], dtype=torch.int32, device=self.device)

    # -- forward ---------------------------------------------------------
    def forward(self, latent: torch.Tensor, t: float, current_start: int, caches, cache_update_mode: str,
                timer=None) -> torch.Tensor:
        """latent [C, F, grid_h*ph, grid_w*pw] -> velocity of the same shape.
        timer(block, phase) is called with phase "begin"/"end" around each
        block's pyramid-cache work when given."""
        s = self.s
        C, Fr, Hl, Wl = latent.shape
        pt, ph, pw = s.patch
        N = Fr * s.frame_seqlen
        # patch embedding (a Conv3d with stride = kernel is a patchify + GEMM)
        x = latent.view(C, Fr, s.grid_h, ph, s.grid_w, pw).permute(1, 2, 4, 0, 3, 5).reshape(N, self.patch_in)
        x = self._mm(x, self.w_patch).float()
        e = _sinusoid(s.freq_dim, t, self.device)
        e = self._mm(F.silu(self._mm(e, self.w_time[0]).float()), self.w_time[1]).float()
        e0 = self._mm(F.silu(e), self.w_tproj).float().view(6, s.dim)
        qpos = self._query_pos(current_start // s.frame_seqlen, Fr)
        if not hasattr(self, "_cu_q") or self._cu_q_n != N:
            self._cu_q = torch.tensor([0, N], dtype=torch.int32, device=self.device)
            self._cu_q_n = N
        ops = _ops.ops()
        D = s.dim
        eps = s.eps
        mods = [blk["mod"] + e0 for blk in self.blocks]
        hm = self.head_mod + e.view(1, s.dim)
        # each residual update is fused with the norm that reads the updated
        # stream next (one pass over x): attention -> cross-attention norm,
        # cross-attention -> feed-forward norm, feed-forward -> the next
        # block's (or the head's) modulated norm
        xn = self._ln_mod(x, mods[0][1], mods[0][0])
        for bi, blk in enumerate(self.blocks):
            mod = mods[bi]
            qkv = self._mm(xn, blk["qkv"])
            q = self._rms(qkv[:, :D], blk["norm_q"])
            k = self._rms(qkv[:, D:2 * D], blk["norm_k"])
            v = qkv[:, 2 * D:]
            q_rot = _ops.ops().rope_apply(q.view(N * s.heads, s.head_dim), qpos, *self.freq_parts_flat)
            if timer is not None:
                timer(bi, "begin")
            cache = caches[bi]
            cache.update(k.view(1, N, s.heads, s.head_dim), v.view(1, N, s.heads, s.head_dim), current_start,
                         cache_update_mode=cache_update_mode)
            y = cache.attend(q_rot.view(1, N, s.heads, s.head_dim), current_start)
            if timer is not None:
                timer(bi, "end")
            # cross-attention to the cached text K/V
            xc = ops.dit_residual_layer_norm_(x, self._mm(y.view(N, s.dim), blk["o"]), mod[2], blk["norm3_w"],
                                              blk["norm3_b"], False, eps)
            qc = self._rms(self._mm(xc, blk["cq"]), blk["cnorm_q"]).view(N, s.heads, s.head_dim)
            kc, vc = self.cross_kv[bi]
            yc = _ops.ragged_attention(qc, kc, vc, self._cu_q, self._cu_text, N, None, kv_per_head=False)
            # feed-forward
            xn2 = ops.dit_residual_layer_norm_(x, self._mm(yc.view(N, s.dim), blk["co"]), None, mod[4], mod[3], True,
                                               eps)
            # FFN up-projection with the bias and tanh-GELU in the GEMM's
            # epilogue (applied to the fp32 product before the bf16 rounding;
            # 147-150 against 158-173 us for the GEMM and dit_gelu_tanh)
            w1, b1 = blk["ffn1"]
            h = torch._addmm_activation(b1, xn2.to(torch.bfloat16), w1.t(), use_gelu=True)
            nxt = mods[bi + 1] if bi + 1 < len(self.blocks) else hm
            xn = ops.dit_residual_layer_norm_(x, self._mm(h, blk["ffn2"]), mod[5], nxt[1], nxt[0], True, eps)
        out = self._mm(xn, self.w_head)
        return out.view(Fr, s.grid_h, s.grid_w, C, ph, pw).permute(3, 0, 1, 4, 2, 5).reshape(C, Fr, Hl, Wl)


def rollout(model: CausalDiT, caches, num_chunks: int, frames_per_chunk: int = 3,
            denoising_steps=(1000, 750, 500, 250), context_noise: float = 0.0, seed: int = 0,
            timed_from: int = 1, measure_cache: bool = True):
    """The pipeline's block loop over num_chunks chunks.  Chunks before
    timed_from run untimed (warm-up); the rest are timed with HIP events.
    Returns the latent chunks per second, the timed milliseconds, and the
    pyramid-path milliseconds (cache update + plan + pack + self-attention,
    from events around each block's cache calls; None when measure_cache is
    off)."""
    s = model.s
    dev = model.device
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    shape = (s.in_channels, frames_per_chunk, s.grid_h * s.patch[1], s.grid_w * s.patch[2])
    events = []

    def timer(bi, phase):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        events.append(ev)

    t_start = t_end = None
    for c in range(num_chunks):
        if c == timed_from:
            torch.cuda.synchronize()
            t_start = torch.cuda.Event(enable_timing=True)
            t_start.record()
        tm = timer if (measure_cache and c >= timed_from) else None
        start = c * frames_per_chunk * s.frame_seqlen
        noisy = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
        x0 = None
        for i, t in enumerate(denoising_steps):
            vel = model.forward(noisy, t, start, caches, "noisy", timer=tm)
            sigma = t / 1000.0
            x0 = (noisy.float() - sigma * vel.float())
            if i + 1 < len(denoising_steps):
                sn = denoising_steps[i + 1] / 1000.0
                noisy = ((1.0 - sn) * x0 + sn * torch.randn(shape, generator=g, device=dev)).to(torch.bfloat16)
        model.forward(x0.to(torch.bfloat16), context_noise, start, caches, "clean", timer=tm)
    t_end = torch.cuda.Event(enable_timing=True)
    t_end.record()
    torch.cuda.synchronize()
    timed = num_chunks - timed_from
    ms = t_start.elapsed_time(t_end) if timed > 0 else 0.0
    cache_ms = None
    if measure_cache:
        cache_ms = sum(events[i].elapsed_time(events[i + 1]) for i in range(0, len(events), 2))
    return dict(chunks=timed, ms=ms, chunks_per_s=(timed / (ms * 1e-3)) if ms > 0 else None, cache_ms=cache_ms,
                forwards_per_chunk=len(denoising_steps) + 1)
