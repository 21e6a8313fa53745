"""Key-split attention (pkv_ragged_attn_fwd_ws): launches of a few sequences
with per-head keys -- one layer's heads, as MegaCache.attend issues them
(reference call site pyramidkv/_mega_cache.py:540-559) -- split each
sequence's keys into chunks that spread over every compute unit, and a
second launch merges each query tile's chunks in chunk order.

Checked against float64 softmax attention at the north star's tolerance
(max-abs 2e-2, mean-abs 2e-3): mixed key lengths (empty, one key, tile
edges, and long sequences that split), partial query tiles, every reference
mode of the fast pass and the slow pass inside a chunk, and strided
layouts through the torch op.  The split output also agrees with the unsplit kernels',
repeats bit for bit, and a workspace below the required size runs the
unsplit kernels."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

if torch.cuda.is_available():
    from gpu_util import DEV, to_dev, to_np
    from pyramidkv import _abi as A
    from pyramidkv import _ops

pytestmark = pytest.mark.gpu

D = 128


def _case(rng, Lq, Lk, H, scale=0.5):
    B = len(Lq)
    cu_q = np.concatenate([[0], np.cumsum(Lq)]).astype(np.int32)
    lk = np.asarray(Lk).reshape(B * H)
    cu_k = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = (rng.standard_normal((cu_q[-1], H, D)) * scale).astype(np.float32)
    k = (rng.standard_normal((cu_k[-1], D)) * scale).astype(np.float32)
    v = (rng.standard_normal((cu_k[-1], D)) * scale).astype(np.float32)
    return O.f32_to_bf16(q), O.f32_to_bf16(k), O.f32_to_bf16(v), cu_q, cu_k


def _run(q, k, v, cu_q, cu_k, B, H, workspace):
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    out = torch.full_like(qd, float("nan"))
    A.ragged_attn_fwd(qd, kd, vd, out, to_dev(cu_q), to_dev(cu_k), B, H, True, int(np.diff(cu_q).max()),
                      D ** -0.5, workspace=workspace)
    torch.cuda.synchronize()
    return to_np(out)


def _check(got_u16, q, k, v, cu_q, cu_k, H):
    got = O.bf16_to_f32(got_u16).astype(np.float64)
    want = O.ragged_attention_ref(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), cu_q, cu_k, H, True)
    err = np.abs(got - want)
    assert np.isfinite(got).all()
    assert err.max() < 2e-2 and err.mean() < 2e-3, (err.max(), err.mean())
    return got


def _ws():
    return _ops.attention_workspace(DEV)


def test_workspace_size_reported():
    n = A.ragged_attn_workspace_size()
    assert n > 0 and n == int(_ops.ops().ragged_attention_workspace_size())
    assert _ws().numel() >= n


@pytest.mark.parametrize("case", [
    # one layer's heads at a rollout's shape, scaled down: long per-head keys over few query tiles
    dict(Lq=[1000], Lk=[[8000, 5000, 3100, 7777]], H=4),
    # tile edges and empty / one-key heads beside long ones; a partial query tile of 8 rows
    dict(Lq=[392, 1], Lk=[[0, 1, 31, 33, 9000, 64], [6000, 32, 4097, 0, 1, 12000]], H=6),
    # a batch without queries between two with
    dict(Lq=[500, 0, 300], Lk=[[7000, 100], [5000, 5000], [2, 9999]], H=2),
])
def test_split_launch_vs_float64_and_unsplit(case):
    rng = np.random.default_rng(41)
    H = case["H"]
    q, k, v, cu_q, cu_k = _case(rng, case["Lq"], case["Lk"], H)
    print(f"split attention Lq={case['Lq']} Lk={case['Lk']}", flush=True)
    B = len(case["Lq"])
    got = _run(q, k, v, cu_q, cu_k, B, H, _ws())
    split = _check(got, q, k, v, cu_q, cu_k, H)
    plain = O.bf16_to_f32(_run(q, k, v, cu_q, cu_k, B, H, None)).astype(np.float64)
    assert np.abs(split - plain).max() < 2e-2
    again = _run(q, k, v, cu_q, cu_k, B, H, _ws())
    assert np.array_equal(got, again), "split launch is not deterministic"


def test_split_reference_modes_and_slow_pass_in_chunks():
    """Query rows scaled by 1, 2 and 4 and per-head constant key blocks at the
    start of different chunks, so that a row's chunks take different
    references (P = 2^S, P = 2^(S - m), and the moving-maximum pass after a
    spike ~98 or ~130 log2 units above a chunk's first tile) before they are
    merged."""
    rng = np.random.default_rng(43)
    H = 4
    Lq, Lk = [1000], [[9000, 8000, 6000, 7500]]
    q, k, v, cu_q, cu_k = _case(rng, Lq, Lk, H)
    alpha = np.array([1.0, 2.0, 4.0], np.float32)[np.arange(q.shape[0]) % 3]
    q[:] = O.f32_to_bf16(np.broadcast_to(alpha[:, None, None], q.shape).astype(np.float32))
    lk = np.diff(cu_k)
    for h in range(H):
        for j, (pos, val) in enumerate([(0, 0.8), (2500, -1.0), (4000, 3.0), (lk[h] - 1, 1.5), (5500, 8.0)]):
            if pos < lk[h] and (h + j) % 2 == 0:
                n = min(32, int(lk[h] - pos)) if val not in (1.5, 8.0) else 1
                k[cu_k[h] + pos:cu_k[h] + pos + n] = O.f32_to_bf16(np.full((n, D), val, np.float32))
    got = _run(q, k, v, cu_q, cu_k, 1, H, _ws())
    _check(got, q, k, v, cu_q, cu_k, H)


def test_split_needs_the_whole_workspace():
    """A workspace below pkv_ragged_attn_workspace_size runs the unsplit
    kernels: the output equals the launch without a workspace bit for bit."""
    rng = np.random.default_rng(47)
    q, k, v, cu_q, cu_k = _case(rng, [800], [[7000, 3000]], 2)
    small = torch.empty(A.ragged_attn_workspace_size() - 1, dtype=torch.uint8, device=DEV)
    got = _run(q, k, v, cu_q, cu_k, 1, 2, small)
    plain = _run(q, k, v, cu_q, cu_k, 1, 2, None)
    assert np.array_equal(got, plain)
    _check(got, q, k, v, cu_q, cu_k, 2)


def test_split_through_the_torch_op_on_strided_views():
    """ragged_attention with the device workspace on Q / K / V / O that are
    the first 128 columns of 256-wide rows."""
    rng = np.random.default_rng(53)
    H = 3
    q, k, v, cu_q, cu_k = _case(rng, [700], [[6500, 2000, 9100]], H)
    wide = lambda a: np.concatenate([a, np.zeros(a.shape, np.uint16)], axis=-1)
    qw, kw, vw = to_dev(wide(q)), to_dev(wide(k)), to_dev(wide(v))
    out = _ops.ragged_attention(qw[..., :D], kw[..., :D], vw[..., :D], to_dev(cu_q), to_dev(cu_k), 700,
                                workspace=_ws())
    torch.cuda.synchronize()
    _check(to_np(out), q, k, v, cu_q, cu_k, H)
