// Cache-update kernels for gfx950: the per-head state machine, the
// descriptor-driven frame copy (pyramidkv_update), the fused MegaCache.update
// (sink/recent routing + recent FIFO shift + middle writes + positions in one
// pass over the new chunk) and the Veil merge accumulator.
//
// All K/V traffic moves in 16-byte (8 x bf16) vector loads/stores; a
// workgroup of 256 threads owns one head and a tile of tokens, so every
// thread touches the same (token, 16-byte chunk) positions in every slot it
// reads or writes and the in-place recent shift needs no inter-thread
// ordering.

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "pkv_common.h"
#include "pkv_state_machine.h"

namespace pkv {

// ---------------------------------------------------------------------------
// error plumbing
// ---------------------------------------------------------------------------
static thread_local char g_err[512];

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return PKV_OK;
}

// ---------------------------------------------------------------------------
// sources of new frames and of their (t, y, x) positions
// ---------------------------------------------------------------------------
struct FrameSrc {
  const uint16_t *k, *v;
  int64_t frame_stride, head_stride, tok_stride;  // elements
  __device__ int64_t off(int f, int h, int tok) const {
    return f * frame_stride + h * head_stride + static_cast<int64_t>(tok) * tok_stride;
  }
};

// Either an explicit [F,H,FSEQ,3] int64 tensor, or the arithmetic grid the
// reference builds in MegaCache.update (_mega_cache.py:203-215):
// (t0 + f, tok / W, tok % W), identical for every head.
struct PosSrc {
  const int64_t *pos;
  int64_t t0;
  int32_t width, H, FSEQ;
  __device__ void get(int f, int h, int tok, int64_t &t, int64_t &y, int64_t &x) const {
    if (pos) {
      const int64_t *p = pos + ((static_cast<int64_t>(f) * H + h) * FSEQ + tok) * 3;
      t = p[0];
      y = p[1];
      x = p[2];
    } else {
      t = t0 + f;
      y = tok / width;
      x = tok % width;
    }
  }
};

__device__ inline uint4 ld16(const uint16_t *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ inline void st16(uint16_t *p, uint4 v) { *reinterpret_cast<uint4 *>(p) = v; }

// ---------------------------------------------------------------------------
// mega_state_update (standalone op)
// ---------------------------------------------------------------------------
__global__ void state_update_kernel(HeadState *states, int H, const int64_t *t_vals, int F,
                                    int pass_kind, pkv_state_desc out) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h < H) run_head(states, h, t_vals, F, pass_kind, out);
}

// ---------------------------------------------------------------------------
// pyramidkv_update: descriptor-driven frame -> pool slot copy
// (pyramidkv_update.cu:21-110).  grid = (token tiles, n_writes).
// ---------------------------------------------------------------------------
constexpr int kTokTile = 32;

struct PoolPtrs {
  uint16_t *k[3], *v[3];
  int64_t *pos[3];
  int64_t slots[3];  // L*H*max_slots of each kind, for bounds checks
};

__global__ void copy_frames_kernel(FrameSrc src, const int64_t *new_pos, PoolPtrs pools,
                                   const int32_t *dst_kind, const int32_t *dst_slot_global,
                                   const int32_t *src_frame, const int32_t *src_head, int H,
                                   int FSEQ, int D, int F) {
  const int op = blockIdx.y;
  const int kind = dst_kind[op];
  if (kind < 0 || kind > 2) return;
  const int64_t sg = dst_slot_global[op];
  const int f = src_frame[op], h = src_head[op];
  if (sg < 0 || sg >= pools.slots[kind] || f < 0 || f >= F || h < 0 || h >= H) return;
  const int tok0 = blockIdx.x * kTokTile;
  const int cpt = D / 8;
  uint16_t *dk = pools.k[kind] + sg * FSEQ * D;
  uint16_t *dv = pools.v[kind] + sg * FSEQ * D;
  for (int i = threadIdx.x; i < kTokTile * cpt; i += blockDim.x) {
    const int tok = tok0 + i / cpt, c = (i % cpt) * 8;
    if (tok >= FSEQ) break;
    const int64_t so = src.off(f, h, tok) + c;
    st16(dk + static_cast<int64_t>(tok) * D + c, ld16(src.k + so));
    st16(dv + static_cast<int64_t>(tok) * D + c, ld16(src.v + so));
  }
  if (new_pos && pools.pos[kind]) {
    int64_t *dp = pools.pos[kind] + sg * FSEQ * 3;
    const int64_t *sp = new_pos + (static_cast<int64_t>(f) * H + h) * FSEQ * 3;
    for (int i = threadIdx.x; i < kTokTile * 3; i += blockDim.x) {
      const int tok = tok0 + i / 3;
      if (tok >= FSEQ) break;
      dp[static_cast<int64_t>(tok0) * 3 + i] = sp[static_cast<int64_t>(tok0) * 3 + i];
    }
  }
}

// ---------------------------------------------------------------------------
// fused MegaCache.update
// ---------------------------------------------------------------------------
// Per-head routing record produced by route_kernel and consumed by
// scatter_kernel.
struct Route {
  int32_t sink_writes;   // frames 0..sink_writes-1 go to sink slots sink_first..
  int32_t sink_first;
  int32_t recent_first;  // frame sink_writes+i goes to recent slot recent_first+i
  int32_t shift;         // move recent slot j+shift -> j for j < keep (0: none)
  int32_t keep;
  int32_t pad[3];
};

struct Workspace {
  int32_t *desc[8];  // [H*F] each: the pkv_state_desc arrays
  Route *route;      // [H]
};

__host__ __device__ inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

__host__ __device__ inline Workspace carve_workspace(void *base, int H, int F) {
  Workspace w;
  char *p = static_cast<char *>(base);
  const int64_t dbytes = align_up(static_cast<int64_t>(H) * F * 4, 256);
  for (int i = 0; i < 8; ++i) w.desc[i] = reinterpret_cast<int32_t *>(p + i * dbytes);
  w.route = reinterpret_cast<Route *>(p + 8 * dbytes);
  return w;
}

// One thread per head: restore the committed counters, route the F new
// frames between sink and recent (_mega_cache.py:226-323), advance the
// state machine on clean passes (_mega_cache.py:329-347) and commit the
// counters (_mega_cache.py:406-414).  The recent FIFO's shift-left is
// applied once per block: noisy passes of a block and its clean pass all
// restore the same committed state, shift by the same amount and overwrite
// the same tail slots, so a pass that finds the shift already applied
// (shift_pending) only rewrites the tail.  That reproduces the reference's
// snapshot-and-restore contents without copying the recent pool.
// A workgroup covers kRouteHeads heads; their state records are copied into
// LDS with coalesced 4-byte accesses, updated there by one thread per head,
// and copied back.
constexpr int kRouteHeads = 64;
constexpr int kRouteThreads = 256;
__device__ void route_head(HeadState &s, int h, int F, int64_t t0, int pass_kind, int shift_pending, int max_sink,
                           int max_recent, const int64_t *sink_caps, int64_t *committed_vc, int64_t *vc,
                           const Workspace &ws);

__global__ void __launch_bounds__(kRouteThreads) route_kernel(HeadState *states, int H, int F, int64_t t0,
                                                              int pass_kind, int shift_pending, int max_sink,
                                                              int max_recent, const int64_t *sink_caps,
                                                              int64_t *committed_vc, int64_t *vc, Workspace ws) {
  __shared__ __attribute__((aligned(16))) HeadState s_st[kRouteHeads];
  const int h0 = blockIdx.x * kRouteHeads;
  const int nh = min(kRouteHeads, H - h0);
  const int words = nh * static_cast<int>(sizeof(HeadState)) / 8;
  uint2 *g = reinterpret_cast<uint2 *>(states + h0);
  uint2 *l = reinterpret_cast<uint2 *>(s_st);
  stage_words(l, g, words);
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < nh)
    route_head(s_st[threadIdx.x], h0 + threadIdx.x, F, t0, pass_kind, shift_pending, max_sink, max_recent, sink_caps,
               committed_vc, vc, ws);
  __syncthreads();
  if (pass_kind == 1)
    for (int i = threadIdx.x; i < words; i += blockDim.x) g[i] = l[i];
}

__device__ void route_head(HeadState &s, int h, int F, int64_t t0, int pass_kind, int shift_pending, int max_sink,
                           int max_recent, const int64_t *sink_caps, int64_t *committed_vc, int64_t *vc,
                           const Workspace &ws) {
  const int64_t sc = committed_vc[h * 3 + 0];
  const int64_t mc = committed_vc[h * 3 + 1];
  const int64_t rc = committed_vc[h * 3 + 2];
  int64_t cap = sink_caps[h];
  if (cap > max_sink) cap = max_sink;
  int64_t sw = cap - sc;
  if (sw > F) sw = F;
  if (sw < 0) sw = 0;
  const int64_t rw = F - sw;
  Route r;
  r.sink_writes = static_cast<int32_t>(sw);
  r.sink_first = static_cast<int32_t>(sc);
  r.shift = 0;
  r.keep = 0;
  int64_t rc_post = rc;
  if (rw > 0) {
    const int64_t total = rc + rw;
    if (total <= max_recent) {
      r.recent_first = static_cast<int32_t>(rc);
      rc_post = total;
    } else {
      const int64_t evict = total - max_recent;
      if (!shift_pending) {
        r.shift = static_cast<int32_t>(evict);
        r.keep = static_cast<int32_t>(max_recent - evict);
      }
      r.recent_first = static_cast<int32_t>(max_recent - rw);
      rc_post = max_recent;
    }
  } else {
    r.recent_first = static_cast<int32_t>(rc);
  }
  ws.route[h] = r;
  vc[h * 3 + 0] = sc + sw;
  vc[h * 3 + 1] = mc;
  vc[h * 3 + 2] = rc_post;

  pkv_state_desc out;
  out.dst_kind = ws.desc[0];
  out.dst_slot = ws.desc[1];
  out.src_frame = ws.desc[2];
  out.src_head = ws.desc[3];
  out.merge_accum_slot = ws.desc[4];
  out.merge_local_idx = ws.desc[5];
  out.merge_finalize_completed_idx = ws.desc[6];
  out.merge_is_new_block = ws.desc[7];
  for (int f = 0; f < F; ++f) {
    FrameDesc d = skip_desc();
    if (pass_kind == 1) d = sm_step(s, static_cast<int32_t>(t0 + f));
    store_desc(out, h * F + f, f, h, d);
  }
  if (pass_kind == 1) {
    committed_vc[h * 3 + 0] = sc + sw;
    committed_vc[h * 3 + 1] = mc;
    committed_vc[h * 3 + 2] = rc_post;
  }
}

// grid = (ceil(FSEQ / kScatTok), H), one thread per (token, 16-byte chunk).
// Each thread first loads everything it will write (the recent slots the
// FIFO shift moves and every new frame), then stores: the shift into
// ascending slots, the new frames into their sink / recent slots and, for
// middle descriptors, into their middle slots.  Loading before storing keeps
// several 16-byte reads in flight per thread and makes the in-place shift
// safe whatever slots the new frames land in.
constexpr int kScatTok = 16;
constexpr int kScatBatch = 4;  // frames (and shifted slots) staged per batch
struct ScatterArgs {
  FrameSrc src;
  PosSrc pos;
  PoolPtrs pools;
  Workspace ws;
  int layer, H, F, FSEQ, D, max_sink, max_middle, max_recent;
};

// tile bx of head h (kScatTok tokens)
__device__ void scatter_body(const ScatterArgs &sa, int bx, int h) {
  const FrameSrc &src = sa.src;
  const PosSrc &pos = sa.pos;
  const PoolPtrs &pools = sa.pools;
  const Workspace &ws = sa.ws;
  const int layer = sa.layer, H = sa.H, F = sa.F, FSEQ = sa.FSEQ, D = sa.D;
  const int max_sink = sa.max_sink, max_middle = sa.max_middle, max_recent = sa.max_recent;
  const Route r = ws.route[h];
  const int tok0 = bx * kScatTok;
  const int cpt = D / 8;
  const int64_t lh = static_cast<int64_t>(layer) * H + h;
  const int64_t slot_elems = static_cast<int64_t>(FSEQ) * D;
  uint16_t *sink_k = pools.k[0] + lh * max_sink * slot_elems;
  uint16_t *sink_v = pools.v[0] + lh * max_sink * slot_elems;
  uint16_t *mid_k = pools.k[1] + lh * max_middle * slot_elems;
  uint16_t *mid_v = pools.v[1] + lh * max_middle * slot_elems;
  uint16_t *rec_k = pools.k[2] + lh * max_recent * slot_elems;
  uint16_t *rec_v = pools.v[2] + lh * max_recent * slot_elems;
  const int32_t *dkind = ws.desc[0];
  const int32_t *dslot = ws.desc[1];

  for (int i = threadIdx.x; i < kScatTok * cpt; i += blockDim.x) {
    const int tok = tok0 + i / cpt, c = (i % cpt) * 8;
    if (tok >= FSEQ) break;
    const int64_t e = static_cast<int64_t>(tok) * D + c;
    uint4 kk[kScatBatch], vv[kScatBatch];
    // recent FIFO shift: slot j <- slot j + shift for j < keep (all sources
    // of a batch read before its stores; batches ascend, and a slot written
    // by one batch is never a source of a later batch since sources are
    // >= shift > destinations of earlier batches)
    for (int j0 = 0; j0 < r.keep; j0 += kScatBatch) {
      const int n = min(kScatBatch, r.keep - j0);
#pragma unroll
      for (int b = 0; b < kScatBatch; ++b)
        if (b < n) {
          kk[b] = ld16(rec_k + (j0 + b + r.shift) * slot_elems + e);
          vv[b] = ld16(rec_v + (j0 + b + r.shift) * slot_elems + e);
        }
#pragma unroll
      for (int b = 0; b < kScatBatch; ++b)
        if (b < n) {
          st16(rec_k + (j0 + b) * slot_elems + e, kk[b]);
          st16(rec_v + (j0 + b) * slot_elems + e, vv[b]);
        }
    }
    for (int f0 = 0; f0 < F; f0 += kScatBatch) {
      const int n = min(kScatBatch, F - f0);
#pragma unroll
      for (int b = 0; b < kScatBatch; ++b)
        if (b < n) {
          const int64_t so = src.off(f0 + b, h, tok) + c;
          kk[b] = ld16(src.k + so);
          vv[b] = ld16(src.v + so);
        }
#pragma unroll
      for (int b = 0; b < kScatBatch; ++b) {
        if (b >= n) continue;
        const int f = f0 + b;
        if (f < r.sink_writes) {
          const int64_t s = r.sink_first + f;
          st16(sink_k + s * slot_elems + e, kk[b]);
          st16(sink_v + s * slot_elems + e, vv[b]);
        } else {
          const int64_t s = r.recent_first + (f - r.sink_writes);
          st16(rec_k + s * slot_elems + e, kk[b]);
          st16(rec_v + s * slot_elems + e, vv[b]);
        }
        if (dkind[h * F + f] == PKV_DST_MIDDLE) {
          const int64_t s = dslot[h * F + f];
          if (s >= 0 && s < max_middle) {
            st16(mid_k + s * slot_elems + e, kk[b]);
            st16(mid_v + s * slot_elems + e, vv[b]);
          }
        }
      }
    }
  }

  // positions: one thread per token of the tile
  const int t = threadIdx.x;
  if (t < kScatTok && tok0 + t < FSEQ) {
    const int tok = tok0 + t;
    const int64_t pe = static_cast<int64_t>(tok) * 3;
    const int64_t pslot = static_cast<int64_t>(FSEQ) * 3;
    int64_t *sink_p = pools.pos[0] + lh * max_sink * pslot;
    int64_t *mid_p = pools.pos[1] + lh * max_middle * pslot;
    int64_t *rec_p = pools.pos[2] + lh * max_recent * pslot;
    for (int j = 0; j < r.keep; ++j) {
      const int64_t *sp = rec_p + (j + r.shift) * pslot + pe;
      const int64_t a = sp[0], b = sp[1], cc = sp[2];
      int64_t *dp = rec_p + j * pslot + pe;
      dp[0] = a;
      dp[1] = b;
      dp[2] = cc;
    }
    for (int f = 0; f < F; ++f) {
      int64_t pt, py, px;
      pos.get(f, h, tok, pt, py, px);
      int64_t *dp;
      if (f < r.sink_writes)
        dp = sink_p + (r.sink_first + f) * pslot + pe;
      else
        dp = rec_p + (r.recent_first + (f - r.sink_writes)) * pslot + pe;
      dp[0] = pt;
      dp[1] = py;
      dp[2] = px;
      if (dkind[h * F + f] == PKV_DST_MIDDLE) {
        const int64_t s = dslot[h * F + f];
        if (s >= 0 && s < max_middle) {
          int64_t *mp = mid_p + s * pslot + pe;
          mp[0] = pt;
          mp[1] = py;
          mp[2] = px;
        }
      }
    }
  }
}

__global__ void __launch_bounds__(256) scatter_kernel(ScatterArgs sa) { scatter_body(sa, blockIdx.x, blockIdx.y); }

// ---------------------------------------------------------------------------
// Veil merge accumulator (mega_merge_accum.cu:52-252)
// ---------------------------------------------------------------------------
// Two launches.  merge_prep_kernel (one workgroup per head, frames in order)
// owns every piece of state shared between frames: on a new block it groups
// the frame's tokens into patch x patch spatial groups, writes the group
// ids, tokens-per-group, group positions and group count, and builds the
// per-group member lists in ascending token order; for each merge frame it
// snapshots the member lists, group count and running weight sum into a
// per-(head, frame) workspace entry, and on finalize writes the anchor
// positions and token count.  merge_accum_kernel (many workgroups per head)
// then only reads those snapshots: each workgroup owns a fixed range of
// groups of its head, zeroes them on a new block, adds the frame's tokens
// in ascending order (one fp32 add per token, the reference's accumulation
// sequence) and writes bf16(sum * (1 / divisor)) on finalize.
constexpr int kGroupsPerWg = 16;
constexpr int kMergeThreads = 256;
constexpr int kMaxMergeFseq = 8192;
constexpr int kMaxMergeGroups = 1024;

struct MergeWs {  // one entry per (head, frame)
  int32_t *members;  // [H*F][FSEQ]
  int32_t *gstart;   // [H*F][MTPA+1]
  int32_t *ng;       // [H*F]
  float *wsum;       // [H*F]
  int32_t *width;    // [H*F]: W > 0 when the groups are the regular patch grid
                     // of a W-wide frame (members in closed form, no CSR
                     // snapshot), 0 when members / gstart hold the lists
};

__host__ __device__ inline int64_t merge_ws_bytes(int H, int F, int FSEQ, int MTPA) {
  const int64_t n = static_cast<int64_t>(H) * F;
  return align_up(n * FSEQ * 4, 256) + align_up(n * (MTPA + 1) * 4, 256) + 3 * align_up(n * 4, 256);
}

__host__ __device__ inline MergeWs carve_merge_ws(void *base, int H, int F, int FSEQ, int MTPA) {
  const int64_t n = static_cast<int64_t>(H) * F;
  char *p = static_cast<char *>(base);
  MergeWs w;
  w.members = reinterpret_cast<int32_t *>(p);
  p += align_up(n * FSEQ * 4, 256);
  w.gstart = reinterpret_cast<int32_t *>(p);
  p += align_up(n * (MTPA + 1) * 4, 256);
  w.ng = reinterpret_cast<int32_t *>(p);
  p += align_up(n * 4, 256);
  w.wsum = reinterpret_cast<float *>(p);
  p += align_up(n * 4, 256);
  w.width = reinterpret_cast<int32_t *>(p);
  return w;
}

struct MergeArgs {
  const HeadState *states;
  FrameSrc src;
  PosSrc pos;
  const int32_t *desc_kind, *desc_slot, *desc_fin, *desc_new;
  const float *weights;  // [F] or null
  pkv_merge_layer ml;
  MergeWs ws;
  int H, F, FSEQ, D, MMA, MMB, MTPA;
};

// Stable CSR of gid[0..FSEQ) over groups [0, ng): gstart (exclusive prefix
// of the counts) and members (tokens of each group in ascending order),
// built by all four waves.  Wave w owns a contiguous quarter of the tokens
// and walks it in 64-token chunks; inside a chunk the tokens sharing a group
// id are found with one ballot per bit of the id (the match mask), so the
// rank of a token among its group's tokens of the chunk is a popcount and
// the highest such lane alone updates the per-(wave, group) counter.
// Pass 1 counts, a block-wide scan turns the counts into per-(wave, group)
// bases (quarters in order), pass 2 places the tokens.
constexpr int kMergeWaves = kMergeThreads / 64;

__device__ inline uint64_t group_match(int g, bool valid, int bits) {
  uint64_t match = __ballot(valid);
  for (int b = 0; b < bits; ++b) {
    const uint64_t ones = __ballot(valid && ((g >> b) & 1));
    match &= ((g >> b) & 1) ? ones : ~ones;
  }
  return match;
}

__device__ void build_csr(const int32_t *gid, int FSEQ, int ng, int32_t *cntw, int32_t *gstart, int32_t *members,
                          int32_t *part) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kMergeWaves * ng; i += blockDim.x) cntw[i] = 0;
  int bits = 1;
  while ((1 << bits) < ng) ++bits;
  const int quarter = ((FSEQ + kMergeWaves * 64 - 1) / (kMergeWaves * 64)) * 64;
  const int t_begin = wave * quarter, t_end = min(FSEQ, t_begin + quarter);
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int32_t *mycnt = cntw + wave * ng;
  __syncthreads();
  // pass 1: counts per (wave, group)
  for (int c0 = t_begin; c0 < t_end; c0 += 64) {
    const int t = c0 + lane;
    const bool valid = t < t_end;
    const int g = valid ? gid[t] : 0;
    const uint64_t match = group_match(g, valid, bits);
    if (valid && (match >> lane) == 1ull) mycnt[g] += __popcll(match);
    // LDS accesses of one wave execute in program order: the next chunk
    // sees these updates without a barrier
  }
  __syncthreads();
  // scan: gstart[g] = sum of all counts of groups < g; cntw[w][g] becomes the
  // base of wave w's tokens of group g
  const int per = (ng + blockDim.x - 1) / blockDim.x;
  const int g0 = tid * per, g1 = min(ng, g0 + per);
  int32_t acc = 0;
  for (int g = g0; g < g1; ++g)
    for (int w = 0; w < kMergeWaves; ++w) acc += cntw[w * ng + g];
  part[tid] = acc;
  __syncthreads();
  for (int off = 1; off < static_cast<int>(blockDim.x); off <<= 1) {
    const int32_t v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int32_t base = part[tid] - acc;
  for (int g = g0; g < g1; ++g) {
    gstart[g] = base;
    for (int w = 0; w < kMergeWaves; ++w) {
      const int32_t c = cntw[w * ng + g];
      cntw[w * ng + g] = base;
      base += c;
    }
  }
  if (tid == static_cast<int>(blockDim.x) - 1) gstart[ng] = part[tid];
  __syncthreads();
  // pass 2: placement
  for (int c0 = t_begin; c0 < t_end; c0 += 64) {
    const int t = c0 + lane;
    const bool valid = t < t_end;
    const int g = valid ? gid[t] : 0;
    const uint64_t match = group_match(g, valid, bits);
    if (valid) {
      const int b = mycnt[g];
      members[b + __popcll(match & below)] = t;
      if ((match >> lane) == 1ull) mycnt[g] = b + __popcll(match);
    }
  }
  __syncthreads();
}

constexpr int kMaxMergeFrames = 64;
constexpr int kMaxMergeSlots = 8;

// One workgroup per head, frames in order.  All descriptors and running
// weight sums are read in one round trip; the group lists built for a block
// stay in LDS for the later frames of that block in the same call.
// Member lists of the arithmetic position grid (y = tok / W, x = tok % W,
// the positions MegaCache.update gives its frames) when it tiles exactly
// into patch x patch groups: group g = (gy, gx) holds the patch's tokens in
// ascending order, so member slot i is token
// (gy*patch + r/patch) * W + gx*patch + r%patch with g = i / patch^2,
// r = i % patch^2, and gstart[g] = g * patch^2.  The same lists as the
// stable CSR build, without its ballots and scans.
__device__ inline bool grid_groups_regular(const PosSrc &pos, int patch, int MTPA) {
  if (pos.pos || patch <= 0 || pos.width <= 0 || pos.FSEQ % pos.width != 0) return false;
  const int rows_tok = pos.FSEQ / pos.width;
  if (rows_tok % patch != 0 || pos.width % patch != 0) return false;
  return (rows_tok / patch) * (pos.width / patch) <= MTPA;
}

__device__ inline void grid_groups_csr(const PosSrc &pos, int patch, int32_t *members, int32_t *gstart) {
  const int W = pos.width, pp = patch * patch, cols = W / patch, ng = pos.FSEQ / pp;
  for (int i = threadIdx.x; i < pos.FSEQ; i += blockDim.x) {
    const int g = i / pp, r = i % pp;
    members[i] = ((g / cols) * patch + r / patch) * W + (g % cols) * patch + r % patch;
  }
  for (int g = threadIdx.x; g <= ng; g += blockDim.x) gstart[g] = g * pp;
  __syncthreads();
}

// LDS words merge_prep_body uses: group ids and member lists [FSEQ] each,
// group starts [MTPA + 1], per-wave counts [kMergeWaves * MTPA] (a group
// count never exceeds MTPA), scan partials [kMergeThreads]
__host__ __device__ inline int64_t merge_prep_lds_words(int FSEQ, int MTPA) {
  return 2 * static_cast<int64_t>(FSEQ) + (1 + kMergeWaves) * static_cast<int64_t>(MTPA) + 1 + kMergeThreads;
}

// Width W of the regular patch grid that the group ids gid[0..FSEQ) form
// (group of token t = ((t / W) / patch) * (W / patch) + (t % W) / patch,
// the ids the grid positions y = t / W, x = t % W give), or 0.  W is where
// the ids first fall back (the end of the first token row); every id is then
// checked.  Grids one group wide have no such fall and report 0 (their
// lists then come from the CSR build, which gives the same lists).
__device__ int regular_grid_width(const int32_t *gid, int FSEQ, int patch, int ng) {
  __shared__ int s_w, s_bad;
  if (threadIdx.x == 0) {
    s_w = FSEQ;
    s_bad = 0;
  }
  __syncthreads();
  if (patch > 0 && ng * patch * patch == FSEQ) {
    int wl = FSEQ;
    for (int t = 1 + threadIdx.x; t < FSEQ; t += blockDim.x)
      if (gid[t] < gid[t - 1]) wl = min(wl, t);
    if (wl < FSEQ) atomicMin(&s_w, wl);
  }
  __syncthreads();
  const int W = s_w;
  if (W >= FSEQ || W % patch != 0 || FSEQ % W != 0) return 0;
  const int cols = W / patch;
  bool bad = false;
  for (int t = threadIdx.x; t < FSEQ; t += blockDim.x) bad |= gid[t] != ((t / W) / patch) * cols + (t % W) / patch;
  if (bad) s_bad = 1;
  __syncthreads();
  return s_bad ? 0 : W;
}

__device__ void merge_prep_body(const MergeArgs &a, int h, int32_t *smem) {
  int32_t *gid = smem;
  int32_t *members = gid + a.FSEQ;
  int32_t *gstart = members + a.FSEQ;
  int32_t *cntw = gstart + a.MTPA + 1;
  int32_t *part = cntw + kMergeWaves * a.MTPA;
  __shared__ int32_t s_desc[kMaxMergeFrames][4];
  __shared__ float s_wsum[kMaxMergeSlots];
  __shared__ int32_t s_ng[kMaxMergeSlots];
  __shared__ int32_t s_maxy, s_maxx, s_irregular;
  const int tid = threadIdx.x;
  const int MTPA = a.MTPA;
  const int32_t bf = a.states[h].block_frames;
  const int32_t patch = a.states[h].patch_size;
  if (tid < a.F) {
    const int di = h * a.F + tid;
    s_desc[tid][0] = a.desc_kind[di];
    s_desc[tid][1] = a.desc_slot[di];
    s_desc[tid][2] = a.desc_new[di];
    s_desc[tid][3] = a.desc_fin[di];
  }
  if (tid < a.MMA) {
    const int64_t hs = static_cast<int64_t>(h) * a.MMA + tid;
    s_wsum[tid] = a.ml.accum_weight_sum ? a.ml.accum_weight_sum[hs] : 0.0f;
    s_ng[tid] = a.ml.accum_num_groups[hs];
  }
  __syncthreads();
  // The group lists of the slot last seen: its regular grid width (members
  // in closed form), or its CSR in LDS (width 0)
  int list_slot = -1, list_w = 0;
  int ng = 0;
  for (int f = 0; f < a.F; ++f) {
    const int di = h * a.F + f;
    const int kind = s_desc[f][0], slot = s_desc[f][1], is_new = s_desc[f][2], fin = s_desc[f][3];
    if (kind != PKV_DST_MERGE_ACCUM || slot < 0 || slot >= a.MMA) continue;
    const int64_t hs = static_cast<int64_t>(h) * a.MMA + slot;
    int32_t *gids_g = a.ml.accum_group_ids + hs * a.FSEQ;
    if (is_new) {
      if (tid == 0) {
        s_maxy = -1;
        s_maxx = -1;
        s_irregular = 0;
      }
      __syncthreads();
      int32_t my = -1, mx = -1;
      for (int t = tid; t < a.FSEQ; t += blockDim.x) {
        int64_t pt, py, px;
        a.pos.get(f, h, t, pt, py, px);
        const int32_t y = static_cast<int32_t>(py), x = static_cast<int32_t>(px);
        my = y > my ? y : my;
        mx = x > mx ? x : mx;
      }
      atomicMax(&s_maxy, my);
      atomicMax(&s_maxx, mx);
      __syncthreads();
      const int32_t cols = (s_maxx >= 0 && patch > 0) ? (s_maxx / patch + 1) : 1;
      const int32_t rows = (s_maxy >= 0 && patch > 0) ? (s_maxy / patch + 1) : 1;
      ng = rows * cols;
      if (ng > MTPA) ng = MTPA;
      // the positions are the regular grid of a W-wide frame (W = max x + 1)
      // when every token t sits at (t / W, t % W) and patch tiles the grid
      const int32_t W = s_maxx + 1;
      const bool grid_ok = patch > 0 && W > 0 && a.FSEQ % W == 0 && W % patch == 0 &&
                           (a.FSEQ / W) % patch == 0 && ng == a.FSEQ / (patch * patch);
      bool irregular = !grid_ok;
      for (int t = tid; t < a.FSEQ; t += blockDim.x) {
        int64_t pt, py, px;
        a.pos.get(f, h, t, pt, py, px);
        const int32_t y = static_cast<int32_t>(py), x = static_cast<int32_t>(px);
        int32_t g = (patch > 0 ? y / patch : 0) * cols + (patch > 0 ? x / patch : 0);
        if (g < 0 || g >= ng) g = 0;
        gid[t] = g;
        gids_g[t] = g;
        irregular |= grid_ok && (py != t / W || px != t % W);
      }
      if (irregular) s_irregular = 1;
      int64_t tpos, ty, tx;
      a.pos.get(f, h, 0, tpos, ty, tx);
      for (int g = tid; g < ng; g += blockDim.x) {
        int64_t *ap = a.ml.accum_pos + (hs * MTPA + g) * 3;
        ap[0] = tpos;
        ap[1] = (g / cols) * patch;
        ap[2] = (g % cols) * patch;
      }
      if (tid == 0) {
        a.ml.accum_num_groups[hs] = ng;
        s_ng[slot] = ng;
        s_wsum[slot] = 0.0f;
        if (a.ml.accum_weight_sum) a.ml.accum_weight_sum[hs] = 0.0f;
      }
      __syncthreads();
      list_slot = slot;
      list_w = s_irregular ? 0 : W;
      if (!list_w) build_csr(gid, a.FSEQ, ng, cntw, gstart, members, part);
      float *tpg = a.ml.accum_tokens_per_group + hs * MTPA;
      for (int g = tid; g < MTPA; g += blockDim.x) {
        const int32_t cnt = list_w ? patch * patch : (g < ng ? gstart[g + 1] - gstart[g] : 0);
        tpg[g] = g < ng ? static_cast<float>(cnt) * static_cast<float>(bf) : 0.0f;
      }
    } else if (list_slot != slot) {
      ng = s_ng[slot];
      if (ng > MTPA) ng = MTPA;
      list_slot = slot;
      if (grid_groups_regular(a.pos, patch, MTPA) && ng == a.FSEQ / (patch * patch)) {
        list_w = a.pos.width;  // the arithmetic positions of MegaCache.update
      } else {
        for (int t = tid; t < a.FSEQ; t += blockDim.x) gid[t] = gids_g[t];
        __syncthreads();
        list_w = regular_grid_width(gid, a.FSEQ, patch, ng);
        if (!list_w) build_csr(gid, a.FSEQ, ng, cntw, gstart, members, part);
      }
    }
    // per-frame snapshot for the accumulation launch: the grid width, or
    // the member lists
    if (!list_w) {
      int32_t *wm = a.ws.members + static_cast<int64_t>(di) * a.FSEQ;
      int32_t *wg = a.ws.gstart + static_cast<int64_t>(di) * (MTPA + 1);
      for (int t = tid; t < a.FSEQ; t += blockDim.x) wm[t] = members[t];
      for (int g = tid; g <= ng; g += blockDim.x) wg[g] = gstart[g];
    }
    if (tid == 0) {
      a.ws.ng[di] = ng;
      a.ws.width[di] = list_w;
      float ws = 1.0f;
      if (a.weights && a.ml.accum_weight_sum) {
        ws = s_wsum[slot] + a.weights[f];
        s_wsum[slot] = ws;
        a.ml.accum_weight_sum[hs] = ws;
      }
      a.ws.wsum[di] = ws;
    }
    if (fin >= 0 && fin < a.MMB) {
      const int64_t hp = static_cast<int64_t>(h) * a.MMB + fin;
      for (int g = tid; g < ng; g += blockDim.x) {
        const int64_t *ap = a.ml.accum_pos + (hs * MTPA + g) * 3;
        int64_t *mp = a.ml.merge_pos + (hp * MTPA + g) * 3;
        mp[0] = ap[0];
        mp[1] = ap[1];
        mp[2] = ap[2];
      }
      if (tid == 0) a.ml.merge_token_count[hp] = ng;
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(kMergeThreads) merge_prep_kernel(MergeArgs a) {
  extern __shared__ int32_t smem[];
  merge_prep_body(a, blockIdx.x, smem);
}

// The scatter of one update (blocks [0, n_scatter), gx tiles per head) and
// its merge preparation (the next H blocks) touch disjoint memory, so they
// share one launch and overlap: the latency-bound per-head merge work runs
// beside the bandwidth-bound scatter.
static_assert(kMergeThreads == 256, "scatter and merge prep share the block size");
__global__ void __launch_bounds__(256) scatter_merge_prep_kernel(ScatterArgs sa, MergeArgs ma, int gx,
                                                                  int n_scatter) {
  extern __shared__ int32_t smem[];
  const int b = blockIdx.x;
  if (b < n_scatter)
    scatter_body(sa, b % gx, b / gx);
  else
    merge_prep_body(ma, b - n_scatter, smem);
}

// Workgroup = (range of kGroupsPerWg groups, head); thread = (group, 8-wide
// dim chunk), so every accumulator element has one owner thread for all
// frames.  The member lists of the workgroup's groups for every merge frame
// are staged in LDS first; each thread keeps its accumulators in registers
// across the frames of a slot, loads a batch of member tokens before adding
// them (ascending token order, frames in descriptor order: the reference's
// fp32 addition sequence) and stores the accumulators when the slot changes
// and at the end.
constexpr int kAccMembersLds = 4096;  // staged member ids per workgroup
constexpr int kAccBatch = 8;          // member tokens loaded per batch
constexpr int kAccPreFrames = 4;      // merge frames whose members one thread loads up front

template <bool kPre>
__global__ void __launch_bounds__(kMergeThreads) merge_accum_kernel(MergeArgs a) {
  __shared__ int32_t s_desc[kMaxMergeFrames][4];
  __shared__ int32_t s_ng[kMaxMergeFrames];
  __shared__ int32_t s_w[kMaxMergeFrames];  // regular grid width, 0: CSR lists
  __shared__ float s_wsum[kMaxMergeFrames];
  __shared__ float s_wt[kMaxMergeFrames];  // frame weights (1 without weights)
  __shared__ int32_t s_gs[kMaxMergeFrames][kGroupsPerWg + 1];  // member-slice offsets (relative to s_off)
  __shared__ int32_t s_off[kMaxMergeFrames];
  __shared__ int32_t s_mem[kAccMembersLds];
  __shared__ int32_t s_nmerge, s_staged;
  const int h = blockIdx.y;
  const int g0 = blockIdx.x * kGroupsPerWg;
  const int tid = threadIdx.x;
  const int D = a.D, MTPA = a.MTPA;
  const int cpt = D / 8;
  const int32_t bf = a.states[h].block_frames;
  const int32_t patch = a.states[h].patch_size;
  if (tid < a.F) {
    const int di = h * a.F + tid;
    const int kind = a.desc_kind[di], slot = a.desc_slot[di];
    const bool merge = kind == PKV_DST_MERGE_ACCUM && slot >= 0 && slot < a.MMA;
    s_desc[tid][0] = merge ? 1 : 0;
    s_desc[tid][1] = slot;
    s_desc[tid][2] = a.desc_new[di];
    s_desc[tid][3] = a.desc_fin[di];
    s_ng[tid] = merge ? a.ws.ng[di] : 0;
    s_w[tid] = merge ? a.ws.width[di] : 0;
    s_wsum[tid] = merge ? a.ws.wsum[di] : 1.0f;
    s_wt[tid] = a.weights ? a.weights[tid] : 1.0f;
  }
  __syncthreads();
  if (tid == 0) {
    int n = 0;
    for (int f = 0; f < a.F; ++f) n += s_desc[f][0];
    s_nmerge = n;
  }
  __syncthreads();
  if (s_nmerge == 0) return;
  // group-range offsets of every merge frame with CSR lists (gstart is read
  // from the frame's snapshot) and the total member count they span; frames
  // on the regular grid stage nothing
  if (tid < a.F && s_desc[tid][0] && s_w[tid]) {
    const int f = tid;
    for (int j = 0; j <= kGroupsPerWg; ++j) s_gs[f][j] = 0;
    s_off[f] = 0;
  } else if (tid < a.F && s_desc[tid][0]) {
    const int f = tid;
    const int32_t *gstart = a.ws.gstart + static_cast<int64_t>(h * a.F + f) * (MTPA + 1);
    const int ng = s_ng[f];
    const int lo = min(g0, ng), hi = min(g0 + kGroupsPerWg, ng);
    const int32_t base = gstart[lo];
    for (int j = 0; j <= kGroupsPerWg; ++j) s_gs[f][j] = gstart[min(lo + j, hi)] - base;
    s_off[f] = base;  // absolute start of the slice in the frame's member list
  }
  __syncthreads();
  if (tid == 0) {
    int total = 0;
    for (int f = 0; f < a.F; ++f)
      if (s_desc[f][0]) total += s_gs[f][kGroupsPerWg];
    s_staged = total <= kAccMembersLds;
  }
  __syncthreads();
  const bool staged = s_staged;
  if (staged) {
    int pos = 0;
    for (int f = 0; f < a.F; ++f) {
      if (!s_desc[f][0]) continue;
      const int n = s_gs[f][kGroupsPerWg];
      const int32_t *mem = a.ws.members + static_cast<int64_t>(h * a.F + f) * a.FSEQ + s_off[f];
      for (int i = tid; i < n; i += blockDim.x) s_mem[pos + i] = mem[i];
      pos += n;
    }
  }
  __syncthreads();
  // kPre (calls of 2 to kAccPreFrames frames), every merge frame on the
  // regular grid of 2 x 2 patches (the production Veil groups): each thread
  // issues the member loads of all its frames at once, so the frames cost one
  // memory round trip instead of one each.  The additions keep their order.
  bool pre = kPre && patch == 2 && a.F <= kAccPreFrames;
  for (int f = 0; f < a.F && pre; ++f) pre = !s_desc[f][0] || s_w[f] > 0;

  for (int it = tid; it < kGroupsPerWg * cpt; it += blockDim.x) {
    const int gl = it / cpt, c = (it % cpt) * 8;
    const int g = g0 + gl;
    if (g >= MTPA) break;
    constexpr int kPreF = kPre ? kAccPreFrames : 1;
    uint4 fk[kPreF][4], fv[kPreF][4];
    if (pre) {
#pragma unroll
      for (int f = 0; f < kPreF; ++f) {
        if (f >= a.F || !s_desc[f][0] || g >= s_ng[f]) continue;
        const int W = s_w[f];
        const int gcols = W / 2;
        const int gbase = (g / gcols) * 2 * W + (g % gcols) * 2;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int64_t so = a.src.off(f, h, gbase + (m >> 1) * W + (m & 1)) + c;
          fk[f][m] = ld16(a.src.k + so);
          fv[f][m] = ld16(a.src.v + so);
        }
      }
    }
    float ak[8], av[8];
    int cur = -1;  // slot whose accumulators are in registers
    int pos = 0;   // start of the current frame's staged members
    // one member token (K and V chunks) added to the accumulators
    auto add_token = [&](const uint4 &k4, const uint4 &v4, float w) {
      const uint32_t kw[4] = {k4.x, k4.y, k4.z, k4.w};
      const uint32_t vw[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float k0 = bf16_to_f32(static_cast<uint16_t>(kw[e] & 0xffff));
        const float k1 = bf16_to_f32(static_cast<uint16_t>(kw[e] >> 16));
        const float v0 = bf16_to_f32(static_cast<uint16_t>(vw[e] & 0xffff));
        const float v1 = bf16_to_f32(static_cast<uint16_t>(vw[e] >> 16));
        if (a.weights) {
          ak[2 * e] = __fadd_rn(ak[2 * e], __fmul_rn(w, k0));
          ak[2 * e + 1] = __fadd_rn(ak[2 * e + 1], __fmul_rn(w, k1));
          av[2 * e] = __fadd_rn(av[2 * e], __fmul_rn(w, v0));
          av[2 * e + 1] = __fadd_rn(av[2 * e + 1], __fmul_rn(w, v1));
        } else {
          ak[2 * e] += k0;
          ak[2 * e + 1] += k1;
          av[2 * e] += v0;
          av[2 * e + 1] += v1;
        }
      }
    };
    // one merge frame: slot switch, new-block reset, member additions and
    // the finalize write (inlined with a constant f in the prefetch loop)
    auto frame = [&](int f) {
      if (!s_desc[f][0]) return;
      const int slot = s_desc[f][1], is_new = s_desc[f][2], fin = s_desc[f][3];
      const int ng = s_ng[f];
      const int fpos = pos;
      pos += s_gs[f][kGroupsPerWg];
      const int64_t hs = static_cast<int64_t>(h) * a.MMA + slot;
      if (slot != cur) {
        if (cur >= 0) {
          const int64_t ho = static_cast<int64_t>(h) * a.MMA + cur;
          float *pk = a.ml.accum_sum_k + (ho * MTPA + g) * D + c;
          float *pv = a.ml.accum_sum_v + (ho * MTPA + g) * D + c;
          for (int e = 0; e < 8; ++e) { pk[e] = ak[e]; pv[e] = av[e]; }
        }
        cur = slot;
        if (!is_new) {
          const float *pk = a.ml.accum_sum_k + (hs * MTPA + g) * D + c;
          const float *pv = a.ml.accum_sum_v + (hs * MTPA + g) * D + c;
          for (int e = 0; e < 8; ++e) { ak[e] = pk[e]; av[e] = pv[e]; }
        }
      }
      if (is_new)
        for (int e = 0; e < 8; ++e) { ak[e] = 0.0f; av[e] = 0.0f; }
      const float w = s_wt[f];
      // members of group g: closed form on the regular grid of width W
      // (ascending: rows of the patch, then columns), else the staged or
      // snapshotted CSR slice
      const int W = s_w[f];
      const int gcols = W > 0 ? W / patch : 1;
      const int gbase = W > 0 ? (g / gcols) * patch * W + (g % gcols) * patch : 0;
      if (g < ng && pre) {
        // the 2 x 2 patch's tokens, loaded above in ascending order
#pragma unroll
        for (int m = 0; m < 4; ++m) add_token(fk[f % kPreF][m], fv[f % kPreF][m], w);
      } else if (g < ng) {
        const int m0 = W > 0 ? 0 : s_gs[f][gl], m1 = W > 0 ? patch * patch : s_gs[f][gl + 1];
        const int32_t *gmem = a.ws.members + static_cast<int64_t>(h * a.F + f) * a.FSEQ + s_off[f];
        for (int mb = m0; mb < m1; mb += kAccBatch) {
          const int n = min(kAccBatch, m1 - mb);
          uint4 kk[kAccBatch], vv[kAccBatch];
#pragma unroll
          for (int b = 0; b < kAccBatch; ++b)
            if (b < n) {
              const int m = mb + b;
              const int tok = W > 0 ? gbase + (m / patch) * W + m % patch : (staged ? s_mem[fpos + m] : gmem[m]);
              const int64_t so = a.src.off(f, h, tok) + c;
              kk[b] = ld16(a.src.k + so);
              vv[b] = ld16(a.src.v + so);
            }
#pragma unroll
          for (int b = 0; b < kAccBatch; ++b)
            if (b < n) add_token(kk[b], vv[b], w);
        }
      }
      if (fin >= 0 && fin < a.MMB && g < ng) {
        const int32_t count = W > 0 ? patch * patch : s_gs[f][gl + 1] - s_gs[f][gl];
        const float div = a.weights ? static_cast<float>(count) * s_wsum[f]
                                    : static_cast<float>(count) * static_cast<float>(bf);
        const float inv = div > 0.0f ? 1.0f / div : 0.0f;
        const int64_t hp = static_cast<int64_t>(h) * a.MMB + fin;
        uint4 ok, ov;
        ok.x = pack_bf16x2(ak[0] * inv, ak[1] * inv);
        ok.y = pack_bf16x2(ak[2] * inv, ak[3] * inv);
        ok.z = pack_bf16x2(ak[4] * inv, ak[5] * inv);
        ok.w = pack_bf16x2(ak[6] * inv, ak[7] * inv);
        ov.x = pack_bf16x2(av[0] * inv, av[1] * inv);
        ov.y = pack_bf16x2(av[2] * inv, av[3] * inv);
        ov.z = pack_bf16x2(av[4] * inv, av[5] * inv);
        ov.w = pack_bf16x2(av[6] * inv, av[7] * inv);
        st16(a.ml.merge_k + (hp * MTPA + g) * D + c, ok);
        st16(a.ml.merge_v + (hp * MTPA + g) * D + c, ov);
      }
    };
    if (pre) {
#pragma unroll
      for (int f = 0; f < kPreF; ++f)
        if (f < a.F) frame(f);
    } else {
      for (int f = 0; f < a.F; ++f) frame(f);
    }
    if (cur >= 0) {
      const int64_t ho = static_cast<int64_t>(h) * a.MMA + cur;
      float *pk = a.ml.accum_sum_k + (ho * MTPA + g) * D + c;
      float *pv = a.ml.accum_sum_v + (ho * MTPA + g) * D + c;
      for (int e = 0; e < 8; ++e) { pk[e] = ak[e]; pv[e] = av[e]; }
    }
  }
}

static int check_merge(const MergeArgs &ma) {
  if (ma.FSEQ > kMaxMergeFseq)
    return fail(PKV_ERR_UNSUPPORTED, "merge_accum: frame_seqlen %d exceeds %d", ma.FSEQ, kMaxMergeFseq);
  if (ma.MTPA > kMaxMergeGroups)
    return fail(PKV_ERR_UNSUPPORTED, "merge_accum: %d tokens per anchor exceed %d", ma.MTPA, kMaxMergeGroups);
  if (ma.D % 8 != 0) return fail(PKV_ERR_INVALID, "merge_accum: head_dim %d not a multiple of 8", ma.D);
  if (ma.F > kMaxMergeFrames)
    return fail(PKV_ERR_UNSUPPORTED, "merge_accum: %d frames per call exceed %d", ma.F, kMaxMergeFrames);
  if (ma.MMA > kMaxMergeSlots)
    return fail(PKV_ERR_UNSUPPORTED, "merge_accum: %d active merge blocks exceed %d", ma.MMA, kMaxMergeSlots);
  return PKV_OK;
}

// dynamic LDS of the merge preparation; above 64 KB the kernel must be
// allowed to use it first
static int merge_prep_smem(const MergeArgs &ma, const void *kernel, size_t &smem) {
  smem = static_cast<size_t>(merge_prep_lds_words(ma.FSEQ, ma.MTPA)) * sizeof(int32_t);
  if (smem > 65536 &&
      hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)) != hipSuccess)
    return fail(PKV_ERR_HIP, "merge_accum: cannot reserve %zu bytes of LDS", smem);
  return PKV_OK;
}

static int launch_merge_accum(const MergeArgs &ma, hipStream_t st) {
  dim3 grid((ma.MTPA + kGroupsPerWg - 1) / kGroupsPerWg, ma.H);
  // the member prefetch pays where several frames would each cost a memory
  // round trip; single-frame calls keep the smaller register footprint
  if (ma.F >= 2 && ma.F <= kAccPreFrames)
    hipLaunchKernelGGL(merge_accum_kernel<true>, grid, dim3(kMergeThreads), 0, st, ma);
  else
    hipLaunchKernelGGL(merge_accum_kernel<false>, grid, dim3(kMergeThreads), 0, st, ma);
  return check_launch("merge_accum_kernel");
}

static int launch_merge(const MergeArgs &ma, hipStream_t st) {
  int rc = check_merge(ma);
  if (rc) return rc;
  size_t smem;
  if ((rc = merge_prep_smem(ma, reinterpret_cast<const void *>(merge_prep_kernel), smem))) return rc;
  hipLaunchKernelGGL(merge_prep_kernel, dim3(ma.H), dim3(kMergeThreads), smem, st, ma);
  if ((rc = check_launch("merge_prep_kernel"))) return rc;
  return launch_merge_accum(ma, st);
}

// Scratch of pkv_merge_accum_static: the per-(head, frame) merge snapshots
// (MergeWs) in a file-scope device array, for callers that cannot allocate.
// Each device holds its own copy at its own address; host code never uses
// the symbol itself, only the address hipGetSymbolAddress returns for the
// current device, looked up once per device.  Every snapshot entry the
// accumulate launch reads is written by the preparation launch of the same
// call, so the array needs no clearing between calls; calls that overlap on
// one device (two streams) race on it.
static __device__ __align__(256) uint8_t scratch[PKV_MERGE_STATIC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;

static int merge_scratch_device_ptr(void **out) {
  static std::mutex mu;
  static void *dev_ptr[kMaxScratchDevices];
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PKV_ERR_HIP, "merge_accum_static: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(PKV_ERR_UNSUPPORTED, "merge_accum_static: device %d beyond %d", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (!dev_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(PKV_ERR_HIP, "merge_accum_static: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    dev_ptr[dev] = p;
  }
  *out = dev_ptr[dev];
  return PKV_OK;
}

static PoolPtrs pool_ptrs(const pkv_geometry *g, const pkv_pools *p) {
  PoolPtrs pp;
  pp.k[0] = p->sink_k; pp.v[0] = p->sink_v; pp.pos[0] = p->sink_pos;
  pp.k[1] = p->middle_k; pp.v[1] = p->middle_v; pp.pos[1] = p->middle_pos;
  pp.k[2] = p->recent_k; pp.v[2] = p->recent_v; pp.pos[2] = p->recent_pos;
  const int64_t lh = static_cast<int64_t>(g->num_layers) * g->num_heads;
  pp.slots[0] = lh * g->max_sink;
  pp.slots[1] = lh * g->max_middle;
  pp.slots[2] = lh * g->max_recent;
  return pp;
}

int check_geometry(const pkv_geometry *g) {
  if (!g) return fail(PKV_ERR_INVALID, "geometry is NULL");
  if (g->num_layers <= 0 || g->num_heads <= 0 || g->head_dim <= 0 || g->frame_seqlen <= 0)
    return fail(PKV_ERR_INVALID, "geometry: num_layers/num_heads/head_dim/frame_seqlen must be > 0");
  if (g->head_dim % 8 != 0) return fail(PKV_ERR_INVALID, "geometry: head_dim %d must be a multiple of 8", g->head_dim);
  if (g->max_sink < 0 || g->max_middle < 0 || g->max_recent < 0)
    return fail(PKV_ERR_INVALID, "geometry: max_*_frames must be >= 0");
  return PKV_OK;
}

}  // namespace pkv

using namespace pkv;

extern "C" {

int pkv_abi_version(void) { return PKV_ABI_VERSION; }
int64_t pkv_perhead_state_size(void) { return static_cast<int64_t>(sizeof(HeadState)); }
const char *pkv_last_error(void) { return g_err; }

int pkv_state_update(uint8_t *states, int32_t num_heads, const int64_t *new_t_vals,
                     int32_t frames_in_block, int32_t pass_kind, const pkv_state_desc *desc,
                     pkv_stream_t stream) {
  if (num_heads == 0 || frames_in_block == 0) return PKV_OK;
  if (!states || !new_t_vals || !desc || num_heads < 0 || frames_in_block < 0)
    return fail(PKV_ERR_INVALID, "mega_state_update: bad arguments");
  const int threads = 64;
  hipLaunchKernelGGL(state_update_kernel, dim3((num_heads + threads - 1) / threads), dim3(threads), 0,
                     as_stream(stream), reinterpret_cast<HeadState *>(states), num_heads, new_t_vals,
                     frames_in_block, pass_kind, *desc);
  return check_launch("state_update_kernel");
}

int pkv_update_frames(const pkv_geometry *geo, const pkv_pools *pools, const uint16_t *new_k,
                      const uint16_t *new_v, const int64_t *new_pos, int32_t frames_in_block,
                      const int32_t *dst_kind, const int32_t *dst_slot_global, const int32_t *src_frame,
                      const int32_t *src_head, int32_t n_writes, pkv_stream_t stream) {
  int rc = check_geometry(geo);
  if (rc) return rc;
  if (n_writes == 0) return PKV_OK;
  if (!new_k || !new_v || !dst_kind || !dst_slot_global || !src_frame || !src_head || n_writes < 0)
    return fail(PKV_ERR_INVALID, "pyramidkv_update: bad arguments");
  const int H = geo->num_heads, FSEQ = geo->frame_seqlen, D = geo->head_dim;
  FrameSrc src{new_k, new_v, static_cast<int64_t>(H) * FSEQ * D, static_cast<int64_t>(FSEQ) * D, D};
  dim3 grid((FSEQ + kTokTile - 1) / kTokTile, n_writes);
  hipLaunchKernelGGL(copy_frames_kernel, grid, dim3(256), 0, as_stream(stream), src, new_pos,
                     pool_ptrs(geo, pools), dst_kind, dst_slot_global, src_frame, src_head, H, FSEQ, D,
                     frames_in_block);
  return check_launch("copy_frames_kernel");
}

int pkv_merge_accum(const uint8_t *states, int32_t H, int32_t F, int32_t FSEQ, int32_t D, int32_t MMA,
                    int32_t MMB, int32_t MTPA, const uint16_t *new_k, const uint16_t *new_v,
                    const int64_t *new_pos, const int32_t *desc_dst_kind,
                    const int32_t *desc_merge_accum_slot,
                    const int32_t *desc_merge_finalize_completed_idx,
                    const int32_t *desc_merge_is_new_block, const float *frame_weights,
                    const pkv_merge_layer *ml, void *workspace, pkv_stream_t stream) {
  if (H == 0 || F == 0) return PKV_OK;
  if (!states || !new_k || !new_v || !new_pos || !ml || !workspace || H < 0 || F < 0 || FSEQ <= 0 ||
      D <= 0 || MMA <= 0 || MMB <= 0 || MTPA <= 0)
    return fail(PKV_ERR_INVALID, "mega_merge_accum: bad arguments");
  if (frame_weights && !ml->accum_weight_sum)
    return fail(PKV_ERR_INVALID, "mega_merge_accum: weighted merge needs accum_weight_sum");
  MergeArgs ma;
  ma.states = reinterpret_cast<const HeadState *>(states);
  ma.src = FrameSrc{new_k, new_v, static_cast<int64_t>(H) * FSEQ * D, static_cast<int64_t>(FSEQ) * D, D};
  ma.pos = PosSrc{new_pos, 0, 1, H, FSEQ};
  ma.desc_kind = desc_dst_kind;
  ma.desc_slot = desc_merge_accum_slot;
  ma.desc_fin = desc_merge_finalize_completed_idx;
  ma.desc_new = desc_merge_is_new_block;
  ma.weights = frame_weights;
  ma.ml = *ml;
  if (!frame_weights) ma.ml.accum_weight_sum = nullptr;
  ma.ws = carve_merge_ws(workspace, H, F, FSEQ, MTPA);
  ma.H = H; ma.F = F; ma.FSEQ = FSEQ; ma.D = D; ma.MMA = MMA; ma.MMB = MMB; ma.MTPA = MTPA;
  return launch_merge(ma, as_stream(stream));
}

int64_t pkv_merge_workspace_size(int32_t H, int32_t F, int32_t FSEQ, int32_t MTPA) {
  return merge_ws_bytes(H, F, FSEQ, MTPA);
}

int pkv_merge_accum_static(const uint8_t *states, int32_t H, int32_t F, int32_t FSEQ, int32_t D, int32_t MMA,
                           int32_t MMB, int32_t MTPA, const uint16_t *new_k, const uint16_t *new_v,
                           const int64_t *new_pos, const int32_t *desc_dst_kind,
                           const int32_t *desc_merge_accum_slot,
                           const int32_t *desc_merge_finalize_completed_idx,
                           const int32_t *desc_merge_is_new_block, const float *frame_weights,
                           const pkv_merge_layer *ml, pkv_stream_t stream) {
  if (H == 0 || F == 0) return PKV_OK;
  if (H < 0 || F < 0 || FSEQ <= 0 || MTPA <= 0) return fail(PKV_ERR_INVALID, "merge_accum_static: bad arguments");
  const int64_t need = merge_ws_bytes(H, F, FSEQ, MTPA);
  if (need > PKV_MERGE_STATIC_SCRATCH_BYTES)
    return fail(PKV_ERR_CAPACITY,
                "merge_accum_static: %lld bytes of scratch needed for %d heads x %d frames x %d tokens; "
                "the static buffer holds %d (use pkv_merge_accum with a workspace)",
                static_cast<long long>(need), H, F, FSEQ, PKV_MERGE_STATIC_SCRATCH_BYTES);
  void *ws = nullptr;
  int rc = merge_scratch_device_ptr(&ws);
  if (rc) return rc;
  return pkv_merge_accum(states, H, F, FSEQ, D, MMA, MMB, MTPA, new_k, new_v, new_pos, desc_dst_kind,
                         desc_merge_accum_slot, desc_merge_finalize_completed_idx, desc_merge_is_new_block,
                         frame_weights, ml, ws, stream);
}

static int64_t update_ws_bytes(int H, int F) {
  return 8 * align_up(static_cast<int64_t>(H) * F * 4, 256) + align_up(static_cast<int64_t>(H) * sizeof(Route), 256);
}

int64_t pkv_cache_update_workspace_size(const pkv_geometry *geo, int32_t frames) {
  if (!geo || frames <= 0) return 0;
  return update_ws_bytes(geo->num_heads, frames) +
         merge_ws_bytes(geo->num_heads, frames, geo->frame_seqlen, geo->max_merge_tokens);
}

int pkv_cache_update(const pkv_geometry *geo, const pkv_pools *pools, const pkv_update_args *a,
                     pkv_stream_t stream) {
  int rc = check_geometry(geo);
  if (rc) return rc;
  if (!pools || !a || !a->new_k || !a->new_v || !a->states_layer || !a->sink_caps_layer ||
      !a->committed_vc_layer || !a->workspace)
    return fail(PKV_ERR_INVALID, "cache_update: NULL argument");
  const int H = geo->num_heads, FSEQ = geo->frame_seqlen, D = geo->head_dim;
  if (a->layer < 0 || a->layer >= geo->num_layers) return fail(PKV_ERR_INVALID, "cache_update: layer out of range");
  if (a->frames <= 0 || a->frames > geo->max_recent)
    return fail(PKV_ERR_UNSUPPORTED, "cache_update: frames per block (%d) must be in [1, max_recent=%d]",
                a->frames, geo->max_recent);
  if (a->spatial_width <= 0) return fail(PKV_ERR_INVALID, "cache_update: spatial_width must be > 0");
  hipStream_t st = as_stream(stream);
  Workspace ws = carve_workspace(a->workspace, H, a->frames);
  int64_t *vc = pools->valid_count + static_cast<int64_t>(a->layer) * H * 3;
  hipLaunchKernelGGL(route_kernel, dim3((H + kRouteHeads - 1) / kRouteHeads), dim3(kRouteThreads), 0, st,
                     reinterpret_cast<HeadState *>(a->states_layer), H, a->frames, a->t0, a->pass_kind,
                     a->shift_pending, geo->max_sink, geo->max_recent, a->sink_caps_layer,
                     a->committed_vc_layer, vc, ws);
  if ((rc = check_launch("route_kernel"))) return rc;
  FrameSrc src{a->new_k, a->new_v, static_cast<int64_t>(FSEQ) * a->tok_stride, a->head_stride, a->tok_stride};
  PosSrc pos{nullptr, a->t0, a->spatial_width, H, FSEQ};
  ScatterArgs sa{src, pos, pool_ptrs(geo, pools), ws, a->layer, H, a->frames, FSEQ, D,
                 geo->max_sink, geo->max_middle, geo->max_recent};
  const int gx = (FSEQ + kScatTok - 1) / kScatTok;
  if (!(a->pass_kind == 1 && a->has_merge_head)) {
    hipLaunchKernelGGL(scatter_kernel, dim3(gx, H), dim3(256), 0, st, sa);
    return check_launch("scatter_kernel");
  }
  const int64_t l = a->layer;
  const int MMA = geo->max_merge_active, MMB = geo->max_merge_blocks, MTPA = geo->max_merge_tokens;
  MergeArgs ma;
  ma.states = reinterpret_cast<const HeadState *>(a->states_layer);
  ma.src = src;
  ma.pos = pos;
  ma.desc_kind = ws.desc[0];
  ma.desc_slot = ws.desc[4];
  ma.desc_fin = ws.desc[6];
  ma.desc_new = ws.desc[7];
  ma.weights = nullptr;
  ma.ml.accum_sum_k = pools->merge_accum_sum_k + l * H * MMA * MTPA * D;
  ma.ml.accum_sum_v = pools->merge_accum_sum_v + l * H * MMA * MTPA * D;
  ma.ml.accum_pos = pools->merge_accum_pos + l * H * MMA * MTPA * 3;
  ma.ml.accum_group_ids = pools->merge_accum_group_ids + l * H * MMA * FSEQ;
  ma.ml.accum_tokens_per_group = pools->merge_accum_tokens_per_group + l * H * MMA * MTPA;
  ma.ml.accum_num_groups = pools->merge_accum_num_groups + l * H * MMA;
  ma.ml.accum_weight_sum = nullptr;
  ma.ml.merge_k = pools->merge_k + l * H * MMB * MTPA * D;
  ma.ml.merge_v = pools->merge_v + l * H * MMB * MTPA * D;
  ma.ml.merge_pos = pools->merge_pos + l * H * MMB * MTPA * 3;
  ma.ml.merge_token_count = pools->merge_token_count + l * H * MMB;
  ma.ws = carve_merge_ws(static_cast<char *>(a->workspace) + update_ws_bytes(H, a->frames), H, a->frames, FSEQ,
                         MTPA);
  ma.H = H; ma.F = a->frames; ma.FSEQ = FSEQ; ma.D = D; ma.MMA = MMA; ma.MMB = MMB; ma.MTPA = MTPA;
  if ((rc = check_merge(ma))) return rc;
  size_t smem;
  if ((rc = merge_prep_smem(ma, reinterpret_cast<const void *>(scatter_merge_prep_kernel), smem))) return rc;
  hipLaunchKernelGGL(scatter_merge_prep_kernel, dim3(gx * H + H), dim3(256), smem, st, sa, ma, gx, gx * H);
  if ((rc = check_launch("scatter_merge_prep_kernel"))) return rc;
  return launch_merge_accum(ma, st);
}

}  // extern "C"
