"""GPU parity of the data-movement ops (scatter_copy, apply_pos_override,
refresh_readout_layout, anchor_store_write_frames), the legacy
pyramidkv_plan and PyramidKVPackedCache against the oracle, through
torch.ops.adahead as the reference's _ops.py wrappers call them.
Everything here is byte / integer work: bit-exact."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ops():
    from pyramidkv import _ops
    return _ops


def _i64(xs):
    return torch.tensor(list(xs), dtype=torch.int64, device=DEV)


@pytest.mark.parametrize("dtype,cols", [(torch.bfloat16, 128), (torch.float32, 8), (torch.int64, 3),
                                        (torch.bfloat16, 3), (torch.uint8, 5)])
def test_scatter_copy_matches_concat(dtype, cols):
    """Segments of mixed lengths and alignments land at their offsets; rows
    between segments and out-of-range segments stay untouched."""
    rng = np.random.default_rng(cols)
    lens = [0, 1, 37, 1560, 5, 64]
    srcs = []
    for n in lens:
        if dtype == torch.uint8:
            srcs.append(torch.randint(0, 255, (n, cols), dtype=torch.uint8, device=DEV))
        elif dtype == torch.int64:
            srcs.append(torch.randint(-9, 9, (n, cols), dtype=torch.int64, device=DEV))
        else:
            srcs.append(torch.randn(n, cols, device=DEV).to(dtype))
    offs, o = [], 3
    for n in lens:
        offs.append(o)
        o += n + int(rng.integers(0, 3))
    total = o + 2
    fill = 7 if dtype in (torch.int64, torch.uint8) else -5.0
    dst = torch.full((total, cols), fill, device=DEV).to(dtype)
    ptrs = [s.data_ptr() for s in srcs]
    # an extra segment that would run past the end is skipped
    extra = torch.ones(10, cols, device=DEV).to(dtype)
    _ops().scatter_copy(_i64(ptrs + [extra.data_ptr()]), _i64(lens + [10]), _i64(offs + [total - 4]), dst, cols)
    want = torch.full((total, cols), fill, device=DEV).to(dtype)
    for s, n, of in zip(srcs, lens, offs):
        want[of:of + n] = s
    torch.cuda.synchronize()
    assert torch.equal(dst, want)


def test_apply_pos_override_reference_case_and_clipping():
    pos = torch.zeros(4680, 3, dtype=torch.int64, device=DEV)
    pos[:, 0] = torch.arange(4680, device=DEV) // 1560
    pos[:, 1] = 4
    _ops().apply_pos_override(pos, _i64([0, 4000]), _i64([1560, 9999]), _i64([5, 9]))
    want = np.zeros((4680, 3), np.int64)
    want[:, 0] = np.arange(4680) // 1560
    want[:, 1] = 4
    O.pos_override(want, [0, 4000], [1560, 4680], [5, 9])  # the end 9999 is clipped to the 4680 rows
    assert np.array_equal(pos.cpu().numpy(), want)


def test_anchor_store_write_frames_reference_case():
    fs, d = 4, 8
    k = torch.arange(3 * fs * d, device=DEV, dtype=torch.float32).reshape(3 * fs, d)
    v = k + 1000
    pos = torch.zeros(3 * fs, 3, device=DEV, dtype=torch.long)
    pos[:, 0] = torch.arange(3 * fs, device=DEV) // fs
    pos[:, 1] = torch.arange(3 * fs, device=DEV) % fs
    desc = torch.tensor([[2, 0], [0, 3], [7, 1], [1, 9], [-1, 2]], device=DEV, dtype=torch.long)
    sk = torch.full((4, fs, d), -1.0, device=DEV)
    sv = torch.full_like(sk, -2)
    sp = torch.full((4, fs, 3), -3, device=DEV, dtype=torch.long)
    _ops().anchor_store_write_frames(k, v, pos, desc, sk, sv, sp)
    wk, wv, wp = np.full((4, fs, d), -1, np.float32), np.full((4, fs, d), -2, np.float32), np.full((4, fs, 3), -3)
    O.write_frames(k.cpu().numpy(), v.cpu().numpy(), pos.cpu().numpy(), [[2, 0], [0, 3]], wk, wv, wp)
    assert np.array_equal(sk.cpu().numpy(), wk) and np.array_equal(sv.cpu().numpy(), wv)
    assert np.array_equal(sp.cpu().numpy(), wp)


def test_anchor_store_write_frames_production_frame():
    fs, d = 1560, 128
    k = torch.randn(3 * fs, d, device=DEV).to(torch.bfloat16)
    v = torch.randn(3 * fs, d, device=DEV).to(torch.bfloat16)
    pos = torch.randint(0, 50, (3 * fs, 3), device=DEV, dtype=torch.long)
    sk = torch.zeros(6, fs, d, device=DEV, dtype=torch.bfloat16)
    sv = torch.zeros_like(sk)
    sp = torch.zeros(6, fs, 3, device=DEV, dtype=torch.long)
    _ops().anchor_store_write_frames(k, v, pos, torch.tensor([[1, 5], [2, 0]], device=DEV), sk, sv, sp)
    assert torch.equal(sk[5], k[fs:2 * fs]) and torch.equal(sv[0], v[2 * fs:]) and torch.equal(sp[5], pos[fs:2 * fs])
    assert not sk[1].any()


@pytest.mark.parametrize("frame_mode", ["physical", "mapped"])
@pytest.mark.parametrize("mode", ["none", "relative_clamp", "relative_softcap"])
@pytest.mark.parametrize("seed", [0, 1])
def test_refresh_readout_layout_matches_oracle(frame_mode, mode, seed):
    rng = np.random.default_rng(seed)
    D = 128 if seed else 8
    lens = [3, 2, 0, 1560, 7]
    src_k = [torch.randn(n, D, device=DEV).to(torch.bfloat16) for n in lens]
    src_v = [torch.randn(n, D, device=DEV).to(torch.bfloat16) for n in lens]
    src_pos = [torch.from_numpy(np.stack([rng.integers(0, 40, n), rng.integers(0, 30, n), rng.integers(0, 52, n)],
                                         1).astype(np.int64)).to(DEV) for n in lens]
    flags = [int(x) for x in rng.integers(0, 8, len(lens))]
    flags[0], flags[1] = 1, 4
    if frame_mode == "physical":
        flags = [f | 2 for f in flags]
    else:
        flags = [f & ~2 for f in flags]
    rope_t = [int(x) for x in rng.integers(0, 30, len(lens))]
    offs, o = [], 1
    for n in lens:
        offs.append(o)
        o += n + 1
    total = o
    n_seg = len(lens)
    out_k = torch.full((total, D), -9.0, device=DEV).to(torch.bfloat16)
    out_v = torch.full((total, D), -8.0, device=DEV).to(torch.bfloat16)
    out_p = torch.full((total, 3), -7, device=DEV, dtype=torch.long)
    out_f = torch.full((total,), -6, device=DEV, dtype=torch.long)
    e = lambda: torch.empty(n_seg, device=DEV, dtype=torch.int64)
    _ops().refresh_readout_layout(src_k, src_v, src_pos, e(), e(), e(), _i64(offs), _i64(lens), _i64(flags),
                                  _i64(rope_t), out_k, out_v, out_p, out_f, D, 33, mode, 7, 0.5)
    h16 = lambda t: t.cpu().view(torch.int16).numpy()
    wk, wv = np.full((total, D), h16(torch.tensor(-9.0).to(torch.bfloat16)), np.int16), \
        np.full((total, D), h16(torch.tensor(-8.0).to(torch.bfloat16)), np.int16)
    wp, wf = np.full((total, 3), -7, np.int64), np.full(total, -6, np.int64)
    O.refresh_readout([h16(t) for t in src_k], [h16(t) for t in src_v], [t.cpu().numpy() for t in src_pos], offs,
                      lens, flags, rope_t, wk, wv, wp, wf, 33, mode, 7, 0.5)
    assert np.array_equal(h16(out_k), wk) and np.array_equal(h16(out_v), wv)
    assert np.array_equal(out_p.cpu().numpy(), wp) and np.array_equal(out_f.cpu().numpy(), wf)


def test_pyramidkv_plan_legacy_matches_oracle():
    mgr = torch.classes.adahead.PyramidKVCacheManager(3, 5, 64, 16, 3, 6, 4, DEV, "bfloat16", 2)
    rng = np.random.default_rng(3)
    vc = np.stack([rng.integers(0, 4, (3, 5)), rng.integers(0, 7, (3, 5)), rng.integers(0, 5, (3, 5))],
                  -1).astype(np.int64)
    mgr.valid_count().copy_(torch.from_numpy(vc))
    got = _ops().ops().pyramidkv_plan(mgr, 0, 1)
    want = O.plan_legacy(vc, 16, 3, 6, 4)
    for g, w in zip(got, want):
        assert np.array_equal(g.cpu().numpy(), w)


def test_packed_cache_update_and_readout():
    """Legacy FIFO-recent cache: the readout is every head's recent ring in
    slot order (the reference's PyramidKVPackedCache semantics)."""
    from pyramidkv.packed_cache import PyramidKVPackedCache
    L, H, D, FS, R = 2, 3, 64, 16, 4
    cache = PyramidKVPackedCache(L, H, D, FS, max_recent_frames=R, device=DEV)
    frames = []
    for b in range(3):
        k = torch.randn(2, H, FS, D, device=DEV).to(torch.bfloat16)
        v = torch.randn(2, H, FS, D, device=DEV).to(torch.bfloat16)
        for layer in range(L):
            cache.update(layer, k, v)
        frames.append((k, v))
    out = cache.readout()
    # per head: ring slots 0..3 hold frames 4, 5, 2, 3 of the 6 written (slot = frame % 4)
    allk = torch.cat([f[0] for f in frames])  # [6, H, FS, D]
    assert out.total_tokens == L * H * R * FS
    cu = out.cu_seqlens_k.cpu().tolist()
    for layer in range(L):
        for h in range(H):
            q = layer * H + h
            seg = out.k_flat[cu[q]:cu[q + 1]].view(R, FS, D)
            for s in range(R):
                fidx = [4, 5, 2, 3][s]
                assert torch.equal(seg[s], allk[fidx, h])
    cache.reset()
    assert int(cache.manager.valid_count().abs().sum()) == 0


def test_packed_cache_ring_partial_and_oversized_calls():
    """Calls of 1, 3 and 6 frames into a 4-slot ring (the 6-frame call wraps
    the ring one and a half times), a partially filled layer, and a reset
    that restarts the ring at slot 0: every head's readout equals the last
    min(n, 4) frames written to it, in ring-slot order (slot = n % 4)."""
    from pyramidkv.packed_cache import PyramidKVPackedCache
    L, H, D, FS, R = 2, 2, 64, 8, 4
    cache = PyramidKVPackedCache(L, H, D, FS, max_recent_frames=R, device=DEV)
    written = [[], []]

    def put(layer, n):
        k = torch.randn(n, H, FS, D, device=DEV).to(torch.bfloat16)
        v = torch.randn(n, H, FS, D, device=DEV).to(torch.bfloat16)
        cache.update(layer, k, v)
        written[layer].extend((k[i], v[i]) for i in range(n))

    def check():
        out = cache.readout()
        cu = out.cu_seqlens_k.cpu().tolist()
        for layer in range(L):
            n = len(written[layer])
            held = min(n, R)
            slots = {i % R: written[layer][i] for i in range(n - held, n)}
            for h in range(H):
                q = layer * H + h
                assert cu[q + 1] - cu[q] == held * FS
                kk = out.k_flat[cu[q]:cu[q + 1]].view(held, FS, D)
                vv = out.v_flat[cu[q]:cu[q + 1]].view(held, FS, D)
                for s in range(held):
                    assert torch.equal(kk[s], slots[s][0][h]) and torch.equal(vv[s], slots[s][1][h])

    put(0, 1)
    put(1, 3)
    check()
    put(0, 6)
    put(1, 1)
    check()
    assert cache.manager.write_idx()[:, :, 2].cpu().tolist() == [[3, 3], [0, 0]]
    cache.reset()
    written = [[], []]
    put(0, 2)
    check()
