"""Queue launches of the 12-wave attention kernel: one workgroup per compute
unit claims (sequence, query tile) items from per-XCD counters that the
last workgroup clears (reference call site of the attention:
pyramidkv/_mega_cache.py:540-559).

Checked against float64 softmax attention at the north star's tolerance
(max-abs 2e-2, mean-abs 2e-3), and for the counters themselves: repeated
launches on one stream repeat bit for bit (a counter left set would skip
items, and their rows would keep the NaN the output starts with), launches
on two streams at once (two counter blocks) give what each gives alone, and
sequences without queries or keys between the others leave no item
unclaimed or claimed twice."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

if torch.cuda.is_available():
    from gpu_util import DEV, to_dev, to_np
    from pyramidkv import _abi as A

pytestmark = pytest.mark.gpu

D = 128


def _case(rng, Lq, Lk, H):
    cu_q = np.concatenate([[0], np.cumsum(Lq)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(np.asarray(Lk).reshape(-1))]).astype(np.int32)
    q = O.f32_to_bf16((rng.standard_normal((cu_q[-1], H, D)) * 0.5).astype(np.float32))
    k = O.f32_to_bf16((rng.standard_normal((cu_k[-1], D)) * 0.5).astype(np.float32))
    v = O.f32_to_bf16((rng.standard_normal((cu_k[-1], D)) * 0.5).astype(np.float32))
    return q, k, v, cu_q, cu_k


def _launch(dev_case, B, H, max_q):
    qd, kd, vd, cqd, ckd = dev_case
    out = torch.full_like(qd, float("nan"))
    A.ragged_attn_fwd(qd, kd, vd, out, cqd, ckd, B, H, True, max_q, D ** -0.5)
    return out


def _check(got_u16, q, k, v, cu_q, cu_k, H):
    got = O.bf16_to_f32(got_u16).astype(np.float64)
    want = O.ragged_attention_ref(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), cu_q, cu_k, H, True)
    assert np.isfinite(got).all(), "rows left unwritten"
    err = np.abs(got - want)
    assert err.max() < 2e-2 and err.mean() < 2e-3, (err.max(), err.mean())


def _mixed(rng, B=40, H=12):
    """Query lengths of 1-3 tiles (tails of 1-383 rows, some over the
    tail-mode bound of 96), a few sequences without queries, per-head key
    lengths 0-1500 (some empty): at least 1,024 items."""
    Lq = rng.integers(385, 1153, size=B)
    Lq[:8] = [0, 1152, 769, 0, 384, 400, 1100, 0]
    Lk = rng.integers(0, 1501, size=(B, H))
    Lk[1, :4] = [0, 1, 32, 300]
    Lk[5, :3] = [0, 0, 257]
    return Lq, Lk


def test_queue_launch_vs_float64_and_repeats():
    rng = np.random.default_rng(71)
    H = 12
    Lq, Lk = _mixed(rng, H=H)
    q, k, v, cu_q, cu_k = _case(rng, Lq, Lk, H)
    B, max_q = len(Lq), int(Lq.max())
    print(f"queue launch B={B} H={H} items~{int(np.sum((Lq + 383) // 384)) * H}", flush=True)
    dev_case = (to_dev(q), to_dev(k), to_dev(v), to_dev(cu_q), to_dev(cu_k))
    first = to_np(_launch(dev_case, B, H, max_q))
    _check(first, q, k, v, cu_q, cu_k, H)
    for _ in range(3):
        again = to_np(_launch(dev_case, B, H, max_q))
        assert np.array_equal(first, again), "a repeated launch on the stream differs"


def test_queue_launches_on_two_streams_at_once():
    rng = np.random.default_rng(73)
    H = 12
    cases = []
    for _ in range(2):
        Lq, Lk = _mixed(rng, H=H)
        q, k, v, cu_q, cu_k = _case(rng, Lq, Lk, H)
        cases.append(((to_dev(q), to_dev(k), to_dev(v), to_dev(cu_q), to_dev(cu_k)), len(Lq), int(Lq.max()),
                      (q, k, v, cu_q, cu_k)))
    alone = [to_np(_launch(c[0], c[1], H, c[2])) for c in cases]
    streams = [torch.cuda.Stream(device=DEV) for _ in cases]
    torch.cuda.synchronize()
    outs = []
    for _ in range(2):
        for (dc, B, mq, _), st in zip(cases, streams):
            with torch.cuda.stream(st):
                outs.append(_launch(dc, B, H, mq))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert np.array_equal(to_np(o), alone[i % 2]), f"launch {i} on stream {i % 2} differs from its launch alone"
    c = cases[1][3]
    _check(alone[1], c[0], c[1], c[2], c[3], c[4], H)


def test_queue_launches_beyond_the_counter_blocks():
    """70 streams, one launch each: the first 64 streams of the process on
    this device (fewer, if earlier tests took some) get counter blocks, the
    rest run one tile per workgroup; every launch equals the default
    stream's bit for bit."""
    rng = np.random.default_rng(79)
    H = 12
    Lq, Lk = _mixed(rng, H=H)
    q, k, v, cu_q, cu_k = _case(rng, Lq, Lk, H)
    B, max_q = len(Lq), int(Lq.max())
    dev_case = (to_dev(q), to_dev(k), to_dev(v), to_dev(cu_q), to_dev(cu_k))
    want = to_np(_launch(dev_case, B, H, max_q))
    streams = [torch.cuda.Stream(device=DEV) for _ in range(70)]
    outs = []
    torch.cuda.synchronize()
    for st in streams:
        with torch.cuda.stream(st):
            outs.append(_launch(dev_case, B, H, max_q))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert np.array_equal(to_np(o), want), f"stream {i} differs"
