"""Benchmark of the pyramid KV-cache hot path on one MI355X.

Headline (the ``value`` field): ragged-cache attention TFLOP/s on the
BASELINE workload "config 2": 30 layers x 12 heads, head_dim 128, bf16,
4,680 query tokens per head, per-head KV length 1,560 (sink) + middle +
4,680 (recent) with the middle set by a seeded 30x12 label matrix over
{-1, 1, 2} (Wave 10 frames, Anchor 0-12 frames, Veil 6 frames; 1 frame =
1,560 tokens; capped at 21 frames).  One step = one launch of the ragged
attention kernel over all 360 (layer, head) sequences, inputs resident in
HBM.  Secondary lines report the cache update + plan + pack path.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "pyramid-forcing_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "ragged-attn TFLOP/s + cache update/pack GB/s (% roofline); latent chunks/s"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
FSEQ, H, L, D, QTOK = 1560, 12, 30, 128, 4680


def config2_lengths(seed: int = 0):
    """Seeded label matrix and per-(layer, head) KV lengths (tokens)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    labels = rng.choice([-1, 1, 2], size=(L, H))
    anchor_frames = rng.integers(0, 13, size=(L, H))
    middle = np.where(labels == -1, 10, np.where(labels == 1, anchor_frames, 6))
    frames = np.minimum(1 + middle + 3, 21)
    return labels, (frames * FSEQ).astype(np.int64)


def bench_attention(steps: int, warmup: int, seed: int = 0):
    import numpy as np
    import torch

    from pyramidkv import _abi as A

    labels, lk = config2_lengths(seed)
    dev = "cuda:0"
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    total_k = int(lk.sum())
    q = (torch.randn(L * QTOK, H, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    k = (torch.randn(total_k, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    v = (torch.randn(total_k, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    out = torch.empty_like(q)
    cu_q = torch.arange(0, L * QTOK + 1, QTOK, dtype=torch.int32, device=dev)
    cu_k = torch.from_numpy(np.concatenate([[0], np.cumsum(lk.reshape(-1))]).astype(np.int32)).to(dev)
    flops = float((4.0 * QTOK * D * lk).sum())

    def step():
        A.ragged_attn_fwd(q, k, v, out, cu_q, cu_k, L, H, True, QTOK, D ** -0.5)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for s, e in ev:
        s.record()
        step()
        e.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = sum(s.elapsed_time(e) for s, e in ev) / steps
    return dict(flops=flops, kernel_ms=kern_ms, wall_s=wall, mean_lk=float(lk.mean()), labels=labels, lk=lk,
                q=q, k=k, v=v, cu_k=cu_k)


def cpu_baseline_attention(lk, seed: int = 0, budget_s: float = 15.0):
    """The oracle's attention (numpy float32 BLAS) on a bounded sample of
    the same workload: whole (layer, head) sequences, Q = 4,680 tokens,
    repeated until about budget_s of CPU work; reported in TFLOP/s."""
    import numpy as np

    from oracle import oracle as O
    rng = np.random.default_rng(seed)
    flat = lk.reshape(-1)
    idx = 0
    flops = 0.0
    secs = 0.0
    n = 0
    while secs < budget_s and n < 8:
        Lk = int(flat[idx % flat.size])
        q = (rng.standard_normal((QTOK, D)) * 0.5).astype(np.float32)
        k = (rng.standard_normal((Lk, D)) * 0.5).astype(np.float32)
        v = (rng.standard_normal((Lk, D)) * 0.5).astype(np.float32)
        t0 = time.perf_counter()
        O.attention_ref(q, k, v, D ** -0.5, dtype=np.float32)
        secs += time.perf_counter() - t0
        flops += 4.0 * QTOK * Lk * D
        idx += 1
        n += 1
    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] + [1])
    except Exception:
        cores = os.cpu_count() or 1
    return dict(value=flops / secs / 1e12, unit="TFLOP/s", cores=int(cores), kind="port",
                sample=f"{n} whole (layer, head) sequences of config 2 (Q=4680, mean Lk="
                       f"{np.mean([flat[i % flat.size] for i in range(n)]):.0f}), numpy float32 softmax attention, "
                       f"{secs:.1f} s")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the pyramid-cache path needs no exchange between GPUs and this build "
              f"runs on a single MI355X (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a HIP device"

    r = bench_attention(args.steps, args.warmup)
    tflops = r["flops"] / (r["kernel_ms"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall_s"] * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config2_ragged_attention", "layers": L, "heads": H, "head_dim": D,
                   "q_tokens_per_head": QTOK, "kv_tokens_mean": round(r["mean_lk"], 1),
                   "kv_tokens_total": int(r["lk"].sum()), "labels_seed": 0, "flop_per_step": r["flops"]},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "kernel": "attn_fwd_kernel<128,2>", "avg_launch_ms": round(r["kernel_ms"], 4)},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_attention(r["lk"])
    print(json.dumps(line))


if __name__ == "__main__":
    main()
