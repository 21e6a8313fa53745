"""CPU oracle for the pyramid KV-cache hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module; the product package
(pyramid-forcing_amd/pyramidkv) never does.  It is the checker the HIP
kernels are compared against, never the thing measured or shipped.

What is restated here (reference = IF-LAB-PKU/Pyramid-Forcing; paths relative
to its root):

* ctypes wrappers over oracle/pkv_oracle.c (state machine, planner, pack +
  RoPE, frame copy, Veil merge accumulate);
* ``rope_tables``: wan/modules/model.py:29-36 (rope_params) and
  wan/modules/causal_model.py:585-590 (t/h/w table concat), split and
  flattened as pyramidkv/_mega_cache.py:713-731 does;
* ``layer_offset_slot_global``: pyramidkv/_mega_attention.py:516-552;
* ``map_sink_time``: pyramidkv/rope.py:86-101;
* ``MegaCacheRef``: pyramidkv/_mega_cache.py:136-569 (MegaCache.update /
  MegaCache.attend), with the reference's committed-snapshot restore and
  FIFO shift-left literally as written (not the build's shift-once scheme);
* ``attention_ref``: textbook softmax(QK^T * scale) V in float64 -- the
  arithmetic the reference delegates to flash-attn 2.8.3.

Parity pinning is documented per function in tests/ (known-answer vectors
from the reference's own tests, closed forms and brute force).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libpkv_oracle.so")

STATE_SIZE = 600
MAX_PHASE, MAX_BUCKET, MAX_T_KEYED = 6, 4, 24
MAX_MERGE_BLOCKS, MAX_MERGE_ACTIVE, MAX_MERGE_BLOCK_FRAMES = 6, 2, 4
MAX_MERGE_TOKENS = 420
SK_RECENT, SK_CYCLIC, SK_STRIDE, SK_LAG, SK_MERGE = 0, 1, 2, 3, 4
DST_SKIP, DST_MIDDLE, DST_MERGE = -1, 1, 5

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.orc_state_size.restype = ctypes.c_int64
        _lib.orc_map_sink_time.restype = ctypes.c_int64
        _lib.orc_map_sink_time.argtypes = [ctypes.c_int64] + [ctypes.c_int] * 4
        _lib.orc_plan_multi.restype = ctypes.c_int32
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle buffers must be contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------
# bf16 bit patterns <-> float32
# ---------------------------------------------------------------------------
def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even; NaN -> 0x7fc0."""
    f = np.ascontiguousarray(f, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = 0x7FC0
    return r


# ---------------------------------------------------------------------------
# per-head state record (anchor_store.cuh:62-132, _mega_state_ops.py:36-77)
# ---------------------------------------------------------------------------
STATE_DTYPE = np.dtype(
    [
        ("kind", np.int8), ("sink_capacity", np.int8), ("_pad0", np.int8, (2,)),
        ("period", np.int32), ("bucket_cap", np.int32), ("interval", np.int32),
        ("capacity", np.int32), ("patch_size", np.int32), ("block_frames", np.int32),
        ("lag_offsets", np.int32, (4,)), ("lag_offset_count", np.int32),
        ("cyclic_slot", np.int32, (24,)), ("cyclic_t", np.int32, (24,)),
        ("cyclic_cursor", np.int8, (6,)),
        ("tkey_slot", np.int32, (24,)), ("tkey_t", np.int32, (24,)),
        ("tkey_count", np.int8), ("tkey_head", np.int8), ("_pad1", np.int8, (2,)),
        ("merge_completed_slot", np.int32, (6,)), ("merge_completed_block_id", np.int32, (6,)),
        ("merge_completed_start_t", np.int32, (6,)), ("merge_completed_end_t", np.int32, (6,)),
        ("merge_completed_median_t", np.int32, (6,)),
        ("merge_completed_count", np.int8), ("_pad2", np.int8, (3,)),
        ("merge_active_block_id", np.int32, (2,)), ("merge_active_slot", np.int32, (2,)),
        ("merge_active_seen", np.int8, (2, 4)), ("merge_active_complete_count", np.int8, (2,)),
        ("_pad3", np.int8, (2,)), ("cached_num_groups", np.int32),
    ],
    align=True,
)
assert STATE_DTYPE.itemsize == STATE_SIZE


def blank_state(kind: int = SK_RECENT, sink_capacity: int = 0, **params) -> np.ndarray:
    """A fresh record with the reference's initial values
    (_mega_state_ref.py:59-113; C++-only merge fields zero, D6)."""
    s = np.zeros((), dtype=STATE_DTYPE)
    s["kind"] = kind
    s["sink_capacity"] = sink_capacity
    s["cyclic_slot"] = -1
    s["tkey_slot"] = -1
    s["merge_completed_slot"] = -1
    s["merge_completed_block_id"] = -1
    s["merge_active_block_id"] = -1
    for k, v in params.items():
        s[k] = v
    return s


def make_cyclic(period, bucket_cap, sink_capacity=0):
    return blank_state(SK_CYCLIC, sink_capacity, period=period, bucket_cap=bucket_cap)


def make_stride(interval, capacity, sink_capacity=0):
    return blank_state(SK_STRIDE, sink_capacity, interval=interval, capacity=capacity)


def make_lag(history_frames, sink_capacity=0):
    return blank_state(SK_LAG, sink_capacity, capacity=history_frames)


def make_merge(patch_size=2, capacity=6, sink_capacity=0):
    return blank_state(SK_MERGE, sink_capacity, patch_size=patch_size, capacity=capacity,
                       block_frames=patch_size * patch_size)


def make_recent(sink_capacity=0):
    return blank_state(SK_RECENT, sink_capacity)


def states_to_bytes(states) -> np.ndarray:
    arr = np.zeros(len(states), dtype=STATE_DTYPE)
    for i, s in enumerate(states):
        arr[i] = s
    return arr.view(np.uint8).reshape(-1).copy()


def bytes_to_states(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint8).view(STATE_DTYPE)


# ---------------------------------------------------------------------------
# C restatement wrappers
# ---------------------------------------------------------------------------
def state_update(states_bytes: np.ndarray, t_vals, pass_kind: int) -> np.ndarray:
    """anchor_store_update.cu:233-313.  Mutates states_bytes (uint8, H*600);
    returns int32 [8, H*F] descriptors."""
    H = states_bytes.size // STATE_SIZE
    t = np.ascontiguousarray(np.asarray(t_vals, dtype=np.int64))
    F = t.size
    desc = np.zeros((8, H * F), dtype=np.int32)
    lib().orc_state_update(_p(states_bytes), ctypes.c_int(H), _p(t), ctypes.c_int(F), ctypes.c_int(pass_kind),
                           _p(desc))
    return desc


def map_sink_time(t, mode_code, cmin, cmax, lag) -> int:
    return int(lib().orc_map_sink_time(int(t), int(mode_code), int(cmin), int(cmax), int(lag)))


@dataclass
class Geometry:
    num_layers: int
    num_heads: int
    head_dim: int
    frame_seqlen: int
    max_sink: int
    max_middle: int
    max_recent: int
    max_attend_chunks: int = 8
    max_merge_blocks: int = MAX_MERGE_BLOCKS
    max_merge_active: int = MAX_MERGE_ACTIVE
    max_merge_tokens: int = MAX_MERGE_TOKENS

    @property
    def segs(self) -> int:
        return self.max_sink + self.max_middle + self.max_recent + self.max_merge_blocks

    @property
    def max_pack_tokens(self) -> int:
        """pyramidkv_manager.cc:341-349"""
        return self.max_attend_chunks * self.num_heads * self.segs * self.frame_seqlen


def plan_multi(g: Geometry, states_layer: np.ndarray, vc_layer: np.ndarray, mtc_layer: np.ndarray, t_list,
               sink_mode=0, cmin=0, cmax=21, lag=0):
    """mega_plan.cc:513-654 for one layer.  Returns (cu, sk, sg, sl, dst,
    traw, tremap, total)."""
    t = np.ascontiguousarray(np.asarray(t_list, dtype=np.int64))
    C = t.size
    H = g.num_heads
    N = C * H * g.segs
    cu = np.zeros(C * H + 1, np.int32)
    sk, sg, sl, dst = (np.zeros(N, np.int32) for _ in range(4))
    traw, tremap = np.zeros(N, np.int64), np.zeros(N, np.int64)
    vc = np.ascontiguousarray(vc_layer, dtype=np.int64)
    mtc = np.ascontiguousarray(mtc_layer, dtype=np.int32)
    total = lib().orc_plan_multi(
        ctypes.c_int(H), ctypes.c_int(g.frame_seqlen), ctypes.c_int(g.max_sink), ctypes.c_int(g.max_middle),
        ctypes.c_int(g.max_recent), ctypes.c_int(g.max_merge_blocks), _p(np.ascontiguousarray(states_layer)),
        _p(vc), _p(mtc), _p(t), ctypes.c_int(C), ctypes.c_int(sink_mode), ctypes.c_int(cmin), ctypes.c_int(cmax),
        ctypes.c_int(lag), _p(cu), _p(sk), _p(sg), _p(sl), _p(dst), _p(traw), _p(tremap))
    return cu, sk, sg, sl, dst, traw, tremap, int(total)


def layer_offset_slot_global(sg, sk, layer, g: Geometry):
    """_mega_attention.py:516-552"""
    sg = np.asarray(sg, np.int32)
    if layer == 0:
        return sg.copy()
    off = np.array([layer * g.num_heads * g.max_sink, layer * g.num_heads * g.max_middle,
                    layer * g.num_heads * g.max_recent, layer * g.num_heads * g.max_merge_blocks], np.int32)
    kind = np.clip(sk, 0, None)
    return (sg + off[kind] * (sk >= 0)).astype(np.int32)


def pack(pools: dict, g: Geometry, sk, sg, sl, dst, tremap=None, tables=None, capacity=None, out=None):
    """pyramidkv_pack.cu:28-185.  pools: dict of numpy arrays with keys
    sink_k/v/pos, middle_k/v/pos, recent_k/v/pos, merge_k/v/pos (bf16 as
    uint16).  Returns (k_out, v_out, pos_out); out: those three arrays to
    write into instead (segments write only their own rows, so disjoint
    segment sets may pack into one output concurrently)."""
    cap = g.max_pack_tokens if capacity is None else capacity
    D = g.head_dim
    if out is not None:
        k_out, v_out, pos_out = out
    else:
        k_out = np.zeros((cap, D), np.uint16)
        v_out = np.zeros((cap, D), np.uint16)
        pos_out = np.zeros((cap, 3), np.int64)
    names = ["sink", "middle", "recent", "merge"]
    pk = (ctypes.c_void_p * 4)(*[_p(pools[n + "_k"]).value for n in names])
    pv = (ctypes.c_void_p * 4)(*[_p(pools[n + "_v"]).value for n in names])
    pp = (ctypes.c_void_p * 4)(*[(_p(pools[n + "_pos"]).value if pools.get(n + "_pos") is not None else None)
                                  for n in names])
    sk, sg, sl, dst = (np.ascontiguousarray(np.asarray(a, np.int32)) for a in (sk, sg, sl, dst))
    if tables is not None and tremap is not None:
        ft, fy, fx = tables
        tr = np.ascontiguousarray(np.asarray(tremap, np.int64))
        rope_args = [_p(tr), _p(ft), ctypes.c_int(ft.shape[0]), ctypes.c_int(ft.shape[1] // 2), _p(fy),
                     ctypes.c_int(fy.shape[0]), ctypes.c_int(fy.shape[1] // 2), _p(fx), ctypes.c_int(fx.shape[0]),
                     ctypes.c_int(fx.shape[1] // 2)]
    else:
        rope_args = [None, None, ctypes.c_int(0), ctypes.c_int(0), None, ctypes.c_int(0), ctypes.c_int(0), None,
                     ctypes.c_int(0), ctypes.c_int(0)]
    lib().orc_pack(pk, pv, pp, ctypes.c_int(g.frame_seqlen), ctypes.c_int(g.max_merge_tokens), ctypes.c_int(D),
                   _p(sk), _p(sg), _p(sl), _p(dst), ctypes.c_int(sk.size), *rope_args, _p(k_out), _p(v_out),
                   _p(pos_out))
    return k_out, v_out, pos_out


def rope_apply(k_u16: np.ndarray, pos: np.ndarray, tables) -> np.ndarray:
    n, D = k_u16.shape
    ft, fy, fx = tables
    out = np.zeros_like(k_u16)
    lib().orc_rope_apply(_p(np.ascontiguousarray(k_u16)), _p(np.ascontiguousarray(pos, np.int64)),
                         ctypes.c_int64(n), ctypes.c_int(D), _p(ft), ctypes.c_int(ft.shape[0]),
                         ctypes.c_int(ft.shape[1] // 2), _p(fy), ctypes.c_int(fy.shape[0]),
                         ctypes.c_int(fy.shape[1] // 2), _p(fx), ctypes.c_int(fx.shape[0]),
                         ctypes.c_int(fx.shape[1] // 2), _p(out))
    return out


def update_frames(pools: dict, new_k, new_v, new_pos, H, FSEQ, D, kind, slot_global, src_frame, src_head):
    """pyramidkv_update.cu:21-110 (pools mutated in place): new_k/new_v
    [F, H, FSEQ, D], new_pos [F, H, FSEQ, 3] or None; write i copies frame
    (src_frame[i], src_head[i]) into slot slot_global[i] of pool kind[i]
    (0 sink, 1 middle, 2 recent).  Other kinds, slots outside the pool and
    sources outside [F, H] write nothing."""
    names = ["sink", "middle", "recent"]
    pk = (ctypes.c_void_p * 3)(*[_p(pools[n + "_k"]).value for n in names])
    pv = (ctypes.c_void_p * 3)(*[_p(pools[n + "_v"]).value for n in names])
    pp = (ctypes.c_void_p * 3)(*[_p(pools[n + "_pos"]).value for n in names])
    nslots = np.array([pools[n + "_k"].size // (FSEQ * D) for n in names], np.int64)
    F = new_k.size // (H * FSEQ * D)
    arrs = [np.ascontiguousarray(np.asarray(a, np.int32)) for a in (kind, slot_global, src_frame, src_head)]
    lib().orc_update_frames(_p(new_k), _p(new_v), _p(new_pos) if new_pos is not None else None, ctypes.c_int(F),
                            ctypes.c_int(H), ctypes.c_int(FSEQ), ctypes.c_int(D), pk, pv, pp, _p(nslots),
                            *[_p(a) for a in arrs], ctypes.c_int(arrs[0].size))


def merge_accum(states_layer, new_k, new_v, new_pos, desc, acc: dict, weights=None):
    """mega_merge_accum.cu:52-252 for one layer.  new_k/new_v uint16
    [F,H,FSEQ,D], new_pos int64 [F,H,FSEQ,3], desc int32 [8,H*F] (state
    update output).  acc: dict of one layer's accumulator / pool arrays
    (sum_k, sum_v, pos, gid, tpg, ng, wsum, mk, mv, mpos, mtc), mutated."""
    F, H, FSEQ, D = new_k.shape
    MMA = acc["sum_k"].shape[1]
    MTPA = acc["sum_k"].shape[2]
    MMB = acc["mk"].shape[1]
    w = None if weights is None else np.ascontiguousarray(np.asarray(weights, np.float32))
    d = [np.ascontiguousarray(desc[i]) for i in (0, 4, 6, 7)]
    lib().orc_merge_accum(
        _p(np.ascontiguousarray(states_layer)), ctypes.c_int(H), ctypes.c_int(F), ctypes.c_int(FSEQ), ctypes.c_int(D),
        ctypes.c_int(MMA), ctypes.c_int(MMB), ctypes.c_int(MTPA), _p(new_k), _p(new_v), _p(new_pos),
        *[_p(x) for x in d], _p(w), _p(acc["sum_k"]), _p(acc["sum_v"]), _p(acc["pos"]), _p(acc["gid"]),
        _p(acc["tpg"]), _p(acc["ng"]), _p(acc["wsum"]), _p(acc["mk"]), _p(acc["mv"]), _p(acc["mpos"]),
        _p(acc["mtc"]))


# ---------------------------------------------------------------------------
# RoPE tables (model.py:29-36, causal_model.py:585-590, _mega_cache.py:713-731)
# ---------------------------------------------------------------------------
def rope_params_np(max_seq_len: int, dim: int, theta: float = 10000.0) -> np.ndarray:
    ang = np.outer(np.arange(max_seq_len, dtype=np.float64),
                   1.0 / np.power(theta, np.arange(0, dim, 2, dtype=np.float64) / dim))
    return np.cos(ang) + 1j * np.sin(ang)


def rope_tables(head_dim: int = 128, max_seq_len: int = 1024, theta: float = 10000.0):
    d = head_dim
    freqs = np.concatenate([rope_params_np(max_seq_len, d - 4 * (d // 6), theta),
                            rope_params_np(max_seq_len, 2 * (d // 6), theta),
                            rope_params_np(max_seq_len, 2 * (d // 6), theta)], axis=1)
    c = d // 2
    split = [c - 2 * (c // 3), c // 3, c // 3]
    parts = np.split(freqs, np.cumsum(split)[:-1], axis=1)

    def flat(z):
        z64 = z.astype(np.complex64)
        return np.ascontiguousarray(np.stack([z64.real, z64.imag], axis=-1).reshape(z.shape[0], -1),
                                    dtype=np.float32)

    return tuple(flat(z) for z in parts)


# ---------------------------------------------------------------------------
# attention (the arithmetic flash_attn_varlen_func computes)
# ---------------------------------------------------------------------------
def attention_ref(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None,
                  dtype=np.float64) -> np.ndarray:
    """softmax(q k^T * scale) v for one sequence; q [Lq, D], k/v [Lk, D]
    (float arrays).  Empty k gives zeros."""
    D = q.shape[-1]
    if scale is None:
        scale = D ** -0.5
    if k.shape[0] == 0:
        return np.zeros_like(q, dtype=dtype)
    s = (q.astype(dtype) @ k.astype(dtype).T) * dtype(scale)
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ v.astype(dtype)


def ragged_attention_ref(q_flat, k_flat, v_flat, cu_q, cu_k, heads_q=1, kv_per_head=True, scale=None):
    """q_flat [total_q, Hq, D]; k/v [total_k, D] per-head ragged (sequence
    b*Hq+h at cu_k[b*Hq+h]), or with kv_per_head=False one K/V sequence per
    batch b at cu_k[b], as [total_k, D] shared by the heads or [total_k, Hq, D]
    (flash_attn_varlen_func's layout) -- float64 output [total_q, Hq, D]."""
    out = np.zeros(q_flat.shape, np.float64)
    B = len(cu_q) - 1
    for b in range(B):
        for h in range(heads_q):
            s = b * heads_q + h if kv_per_head else b
            q = q_flat[cu_q[b]:cu_q[b + 1], h]
            k = k_flat[cu_k[s]:cu_k[s + 1]]
            vv = v_flat[cu_k[s]:cu_k[s + 1]]
            if k.ndim == 3:
                k, vv = k[:, h], vv[:, h]
            out[cu_q[b]:cu_q[b + 1], h] = attention_ref(q, k, vv, scale)
    return out


# ---------------------------------------------------------------------------
# MegaCache model (pyramidkv/_mega_cache.py)
# ---------------------------------------------------------------------------
class MegaCacheRef:
    """CPU model of the reference's MegaCache for all layers: pools as numpy
    arrays (bf16 as uint16), update() / plan_pack() following
    _mega_cache.py:136-523 step by step, including the committed snapshots
    of valid_count and the recent pool that are restored at every update."""

    def __init__(self, g: Geometry, states_bytes: np.ndarray, sink_caps: np.ndarray, spatial_width: int = 52,
                 sink_mode=0, cmin=0, cmax=21, lag=0, tables=None):
        self.g = g
        L, H, D, FS = g.num_layers, g.num_heads, g.head_dim, g.frame_seqlen
        self.states = np.ascontiguousarray(states_bytes.reshape(L, H * STATE_SIZE)).copy()
        self.sink_caps = np.asarray(sink_caps, np.int64).reshape(L, H)
        self.W = spatial_width
        self.remap = (sink_mode, cmin, cmax, lag)
        self.tables = tables
        z = lambda *s: np.zeros(s, np.uint16)
        self.sink_k, self.sink_v = z(L, H, g.max_sink, FS, D), z(L, H, g.max_sink, FS, D)
        self.middle_k, self.middle_v = z(L, H, g.max_middle, FS, D), z(L, H, g.max_middle, FS, D)
        self.recent_k, self.recent_v = z(L, H, g.max_recent, FS, D), z(L, H, g.max_recent, FS, D)
        self.sink_pos = np.zeros((L, H, g.max_sink, FS, 3), np.int64)
        self.middle_pos = np.zeros((L, H, g.max_middle, FS, 3), np.int64)
        self.recent_pos = np.zeros((L, H, g.max_recent, FS, 3), np.int64)
        MMB, MMA, MT = g.max_merge_blocks, g.max_merge_active, g.max_merge_tokens
        self.merge_k, self.merge_v = z(L, H, MMB, MT, D), z(L, H, MMB, MT, D)
        self.merge_pos = np.zeros((L, H, MMB, MT, 3), np.int64)
        self.merge_token_count = np.zeros((L, H, MMB), np.int32)
        self.acc = [dict(sum_k=np.zeros((H, MMA, MT, D), np.float32), sum_v=np.zeros((H, MMA, MT, D), np.float32),
                         pos=np.zeros((H, MMA, MT, 3), np.int64), gid=np.zeros((H, MMA, FS), np.int32),
                         tpg=np.zeros((H, MMA, MT), np.float32), ng=np.zeros((H, MMA), np.int32),
                         wsum=np.zeros((H, MMA), np.float32)) for _ in range(L)]
        self.valid_count = np.zeros((L, H, 3), np.int64)
        self.committed_vc = None
        self.committed_recent = None
        self.has_merge = bool((bytes_to_states(self.states.reshape(-1))["kind"] == SK_MERGE).any())
        self.last_desc = None

    def update(self, layer: int, new_k: np.ndarray, new_v: np.ndarray, current_start: int, mode: str = "clean"):
        """_mega_cache.py:136-414; new_k/new_v uint16 [L_in, H, D]."""
        g = self.g
        if mode == "default":
            mode = "clean"
        if mode not in ("noisy", "clean"):
            return
        FS, H, D = g.frame_seqlen, g.num_heads, g.head_dim
        F = new_k.shape[0] // FS
        t0 = current_start // FS
        nk = np.ascontiguousarray(new_k.reshape(F, FS, H, D).transpose(0, 2, 1, 3))
        nv = np.ascontiguousarray(new_v.reshape(F, FS, H, D).transpose(0, 2, 1, 3))
        idx = np.arange(FS)
        pos = np.zeros((F, H, FS, 3), np.int64)
        pos[..., 0] = (t0 + np.arange(F)).reshape(F, 1, 1)
        pos[..., 1] = idx // self.W
        pos[..., 2] = idx % self.W
        if self.committed_vc is None:
            self.committed_vc = self.valid_count.copy()
        else:
            self.valid_count[layer] = self.committed_vc[layer]
        if self.committed_recent is None:
            self.committed_recent = (self.recent_k.copy(), self.recent_v.copy(), self.recent_pos.copy())
        else:
            self.recent_k[layer] = self.committed_recent[0][layer]
            self.recent_v[layer] = self.committed_recent[1][layer]
            self.recent_pos[layer] = self.committed_recent[2][layer]
        max_sink, max_recent = g.max_sink, g.max_recent
        for h in range(H):
            cap = min(int(self.sink_caps[layer, h]), max_sink)
            sc, rc = int(self.valid_count[layer, h, 0]), int(self.valid_count[layer, h, 2])
            sw = max(0, min(F, cap - sc))
            rw = F - sw
            for i in range(sw):
                self.sink_k[layer, h, sc + i] = nk[i, h]
                self.sink_v[layer, h, sc + i] = nv[i, h]
                self.sink_pos[layer, h, sc + i] = pos[i, h]
            self.valid_count[layer, h, 0] = sc + sw
            if rw == 0:
                continue
            total = rc + rw
            if total <= max_recent:
                for i in range(rw):
                    self.recent_k[layer, h, rc + i] = nk[sw + i, h]
                    self.recent_v[layer, h, rc + i] = nv[sw + i, h]
                    self.recent_pos[layer, h, rc + i] = pos[sw + i, h]
                self.valid_count[layer, h, 2] = total
            else:
                ev = total - max_recent
                for arr in (self.recent_k, self.recent_v, self.recent_pos):
                    arr[layer, h, :max_recent - ev] = arr[layer, h, ev:max_recent].copy()
                for i in range(rw):
                    s = max_recent - rw + i
                    self.recent_k[layer, h, s] = nk[sw + i, h]
                    self.recent_v[layer, h, s] = nv[sw + i, h]
                    self.recent_pos[layer, h, s] = pos[sw + i, h]
                self.valid_count[layer, h, 2] = max_recent
        if mode == "clean":
            st = self.states[layer]
            desc = state_update(st, t0 + np.arange(F), 1)
            self.last_desc = desc
            kind, slot_local = desc[0], desc[1]
            kind_pool = np.where(kind == DST_MERGE, -1, kind)
            slot_global = (slot_local.astype(np.int64) + (layer * H + desc[3].astype(np.int64)) * g.max_middle)
            pools = dict(sink_k=self.sink_k, sink_v=self.sink_v, sink_pos=self.sink_pos,
                         middle_k=self.middle_k, middle_v=self.middle_v, middle_pos=self.middle_pos,
                         recent_k=self.recent_k, recent_v=self.recent_v, recent_pos=self.recent_pos)
            update_frames(pools, nk, nv, pos, H, FS, D, kind_pool, slot_global.astype(np.int32), desc[2], desc[3])
            if self.has_merge:
                dm = desc.copy()
                dm[0] = np.where(kind == DST_MERGE, kind, -1)
                a = self.acc[layer]
                lay = dict(sum_k=a["sum_k"], sum_v=a["sum_v"], pos=a["pos"], gid=a["gid"], tpg=a["tpg"],
                           ng=a["ng"], wsum=a["wsum"], mk=self.merge_k[layer], mv=self.merge_v[layer],
                           mpos=self.merge_pos[layer], mtc=self.merge_token_count[layer])
                merge_accum(st, nk, nv, pos, dm, lay)
            self.committed_vc[layer] = self.valid_count[layer]
            for arr, snap in zip((self.recent_k, self.recent_v, self.recent_pos), self.committed_recent):
                snap[layer] = arr[layer]

    def pools(self, layer: int | None = None) -> dict:
        return dict(sink_k=self.sink_k, sink_v=self.sink_v, sink_pos=self.sink_pos,
                    middle_k=self.middle_k, middle_v=self.middle_v, middle_pos=self.middle_pos,
                    recent_k=self.recent_k, recent_v=self.recent_v, recent_pos=self.recent_pos,
                    merge_k=self.merge_k, merge_v=self.merge_v, merge_pos=self.merge_pos)

    def plan_pack(self, layer: int, current_start: int, num_chunks: int):
        """_mega_cache.py:461-501: multi-chunk plan, layer offset, fused pack."""
        g = self.g
        t_list = [(current_start + c * g.frame_seqlen) // g.frame_seqlen for c in range(num_chunks)]
        cu, sk, sg, sl, dst, traw, tremap, total = plan_multi(
            g, self.states[layer], self.valid_count[layer], self.merge_token_count[layer], t_list, *self.remap)
        sga = layer_offset_slot_global(sg, sk, layer, g)
        k, v, p = pack(self.pools(), g, sk, sga, sl, dst, tremap, self.tables)
        return dict(cu=cu, sk=sk, sg=sg, sl=sl, dst=dst, traw=traw, tremap=tremap, total=total, k=k[:total],
                    v=v[:total], pos=p[:total])


# ---------------------------------------------------------------------------
# data-movement ops (pyramidkv/csrc/scatter_copy.cu) and the legacy planner
# (pyramidkv/csrc/pyramidkv_plan.cc)
# ---------------------------------------------------------------------------
def scatter_copy(srcs, lengths, offsets, dst: np.ndarray) -> None:
    """scatter_copy.cu:13-47: segment i copies lengths[i] rows of srcs[i]
    (row-major, same columns as dst) to dst rows offsets[i]..; dst mutated."""
    for s, n, o in zip(srcs, lengths, offsets):
        n, o = int(n), int(o)
        if n <= 0:
            continue
        dst[o:o + n] = np.asarray(s).reshape(-1, *dst.shape[1:])[:n]


def pos_override(pos: np.ndarray, starts, ends, vals) -> None:
    """scatter_copy.cu:53-71: pos[i, 0] = val for start <= i < end."""
    for s, e, v in zip(starts, ends, vals):
        pos[int(s):int(e), 0] = int(v)


def map_history_t(src_t: int, current_t: int, mode: int, rel_max: int, soft: float) -> int:
    """scatter_copy.cu:142-160: mode 0 keeps t, 1 clamps the relative time
    at rel_max, 2 compresses the excess by `soft` with round-half-to-even on
    the float32 product; the result is clamped at 0."""
    rel = max(0, current_t - src_t)
    mapped = src_t
    if mode == 1:
        mapped = current_t - min(rel, rel_max)
    elif mode == 2:
        if rel > rel_max:
            rel = rel_max + int(np.rint(np.float32(rel - rel_max) * np.float32(soft)))
        mapped = current_t - rel
    return max(0, mapped)


_HIST_CODES = {"none": 0, "relative_clamp": 1, "relative_softcap": 2}


def refresh_readout(src_k, src_v, src_pos, offsets, lengths, flags, rope_t, dst_k, dst_v, dst_pos, dst_frame,
                    current_t: int, mode: str, rel_max: int, soft: float) -> None:
    """scatter_copy.cu:77-168 (all outputs mutated): flags bit 2 overrides
    t with rope_t, else bit 0 applies the history map; bit 1 makes the frame
    id the source t."""
    code = _HIST_CODES.get(mode, 0)
    for i, (o, n) in enumerate(zip(offsets, lengths)):
        o, n, f = int(o), int(n), int(flags[i])
        if n <= 0:
            continue
        dst_k[o:o + n] = src_k[i][:n]
        dst_v[o:o + n] = src_v[i][:n]
        for r in range(n):
            t0 = int(src_pos[i][r, 0])
            t = t0
            if f & 4:
                t = int(rope_t[i])
            elif (f & 1) and rel_max > 0:
                t = map_history_t(t0, current_t, code, rel_max, soft)
            dst_pos[o + r] = (t, src_pos[i][r, 1], src_pos[i][r, 2])
            dst_frame[o + r] = t0 if (f & 2) else t


def write_frames(k_seq, v_seq, pos_seq, frame_desc, store_k, store_v, store_pos) -> None:
    """scatter_copy.cu:170-225: frame (src, slot) -> store slot (stores mutated)."""
    fs = store_k.shape[1]
    for src, slot in np.asarray(frame_desc).reshape(-1, 2):
        src, slot = int(src), int(slot)
        if src < 0 or slot < 0:
            continue
        store_k[slot] = k_seq[src * fs:(src + 1) * fs]
        store_v[slot] = v_seq[src * fs:(src + 1) * fs]
        store_pos[slot] = pos_seq[src * fs:(src + 1) * fs]


def plan_legacy(vc: np.ndarray, fseq: int, max_sink: int, max_middle: int, max_recent: int):
    """pyramidkv_plan.cc:46-133: per (layer, head) the segments sink, recent,
    middle over slots 0..valid_count-1; returns (cu, sk, sg, sl, dst)."""
    L, H, _ = vc.shape
    n = L * H
    slots = {0: max_sink, 1: max_middle, 2: max_recent}
    cu = np.zeros(n + 1, np.int32)
    sk = np.full(3 * n, -1, np.int32)
    sg, sl, dst = (np.zeros(3 * n, np.int32) for _ in range(3))
    run = 0
    for q in range(n):
        l, h = divmod(q, H)
        for kp, kind in enumerate((0, 2, 1)):
            d = q * 3 + kp
            v = int(vc[l, h, kind])
            if v <= 0:
                continue
            sk[d], sg[d], sl[d], dst[d] = kind, q * slots[kind], v * fseq, run
            run += v * fseq
        cu[q + 1] = run
    return cu, sk, sg, sl, dst
