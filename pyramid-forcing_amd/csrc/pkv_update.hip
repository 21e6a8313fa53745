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

#include <algorithm>
#include <mutex>
#include <type_traits>

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
// non-temporal 16-byte store (written through, not kept dirty in L2)
__device__ inline void st16_nt(void *p, uint4 v) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(p));
}

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

__host__ __device__ inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

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
      if (a.ml.accum_weight_sum) {
        ws = s_wsum[slot] + (a.weights ? a.weights[f] : 1.0f);
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
  for (int it = tid; it < kGroupsPerWg * cpt; it += blockDim.x) {
    const int gl = it / cpt, c = (it % cpt) * 8;
    const int g = g0 + gl;
    if (g >= MTPA) break;
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
    // the finalize write
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
      if (g < ng) {
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
    for (int f = 0; f < a.F; ++f) frame(f);
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
  hipLaunchKernelGGL(merge_accum_kernel, grid, dim3(kMergeThreads), 0, st, ma);
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

// ---------------------------------------------------------------------------
// fused MegaCache.update (_mega_cache.py:136-414): one launch per call
// ---------------------------------------------------------------------------
// The grid holds, for every head, n_merge merge tiles (the Veil accumulate
// of a clean pass in a layer with a Veil head; they come first in the grid
// so that their longer dependency chains start early) and n_scat token
// tiles (the new frames routed to sink / recent slots, the recent FIFO
// shift, the middle-pool writes and the positions).
//
// Every workgroup of head h stages h's state record and committed counters
// and routes the frames itself (_mega_cache.py:226-323).  The workgroups
// that need descriptors -- token tiles of Wave / Anchor / lag heads for the
// middle slots, merge tiles of Veil heads -- also run the state machine over
// the call's frames (_mega_cache.py:329-347) on their LDS copy of the
// record.  The inputs are the same for all of them, so all derive the same
// routing and descriptors.  No workgroup writes what another one reads: the
// workgroup that arrives last at the head's counter arrive[h] (zero between
// calls; that workgroup resets it) writes the advanced record, the counters
// (_mega_cache.py:406-414), the descriptors and the merge bookkeeping that
// every merge tile of the head reads (group ids, group count, weight sum).
// Each workgroup increments the counter only after a barrier that follows
// its last read of that shared data.
//
// The recent FIFO shift-left is applied once per block: noisy passes of a
// block and its clean pass all restore the same committed counters, shift
// by the same amount and overwrite the same tail slots, so a pass that
// finds the shift already applied (shift_pending) only rewrites the tail.
// That reproduces the reference's snapshot-and-restore contents without
// copying the recent pool.
constexpr int kUpdThreads = 256;
constexpr int kUpdMaxFrames = 64;
constexpr int kScatBatch = 4;   // new frames loaded per batch
constexpr int kShiftBatch = 2;  // shifted recent slots loaded per batch
constexpr int kUpdAccBatch = 4; // member tokens loaded per batch by a merge tile
constexpr int kStateWords = static_cast<int>(sizeof(HeadState) / 4);

// A value every lane holds alike (read from LDS after a barrier), made
// visibly uniform so that branches on it stay scalar branches and the code
// on either side shares registers
__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
constexpr int kArriveFan = 8;      // arrival sub-counters per head
constexpr int kArriveStride = 32;  // int32 words between counters (128 bytes)

// 16-byte access at a 32-bit byte offset from a workgroup-uniform base: the
// base stays in scalar registers and the address costs one vector register
__device__ inline uint4 ld16o(const void *base, uint32_t off) {
  return *reinterpret_cast<const uint4 *>(static_cast<const char *>(base) + off);
}
__device__ inline void st16o(void *base, uint32_t off, uint4 v) {
  *reinterpret_cast<uint4 *>(static_cast<char *>(base) + off) = v;
}
// 16-byte raw buffer load at byte offset off with the non-temporal
// (streaming) cache policy, for data read once: the address is a 32-bit
// offset from a buffer resource (word 3: 32-bit format, no swizzle; reads
// past num_records return zero)
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kCpolNt = 2;  // buffer instruction cache policy: non-temporal
__device__ inline __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, int num_records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, num_records, kRsrcWord3);
}
__device__ inline uint4 bld16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, kCpolNt);
  return make_uint4(q[0], q[1], q[2], q[3]);
}
static_assert(kStateWords <= kUpdThreads, "one state word per thread");

// list sources of a merge frame's groups
constexpr int kSrcNone = -2;  // not a merge frame (slot untouched)
constexpr int kSrcGrid = -1;  // the call's arithmetic grid (block began in this call)
                              // s >= 0: the group ids stored for slot s

struct Route {
  int64_t vc_post[3];    // counters after the call
  int32_t sink_writes;   // frames 0..sink_writes-1 go to sink slots sink_first..
  int32_t sink_first;
  int32_t recent_first;  // frame sink_writes+i goes to recent slot recent_first+i
  int32_t shift;         // move recent slot j+shift -> j for j < keep (0: none)
  int32_t keep;
};

// _mega_cache.py:226-323 for one head: frames fill the sink up to the
// head's cap, the rest enter the recent FIFO, evicting from its front when
// it is full
__device__ inline Route route_frames(int64_t sc, int64_t mc, int64_t rc, int64_t cap, int F, int max_sink,
                                     int max_recent, int shift_pending) {
  // counters outside their pools (only a corrupted record holds them) are
  // clamped so that every write stays inside the head's slots
  sc = sc < 0 ? 0 : sc;
  rc = rc < 0 ? 0 : (rc > max_recent ? max_recent : rc);
  if (cap > max_sink) cap = max_sink;
  int64_t sw = cap - sc;
  if (sw > F) sw = F;
  if (sw < 0) sw = 0;
  const int64_t rw = F - sw;
  Route r;
  r.sink_writes = static_cast<int32_t>(sw);
  r.sink_first = static_cast<int32_t>(sc);
  r.recent_first = static_cast<int32_t>(rc);
  r.shift = 0;
  r.keep = 0;
  int64_t rc_post = rc;
  if (rw > 0) {
    const int64_t total = rc + rw;
    if (total <= max_recent) {
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
  }
  r.vc_post[0] = sc + sw;
  r.vc_post[1] = mc;
  r.vc_post[2] = rc_post;
  return r;
}

struct UpdArgs {
  HeadState *states;
  const int64_t *sink_caps;
  int64_t *committed_vc, *vc;
  FrameSrc src;
  PoolPtrs pools;
  pkv_merge_layer ml;  // this layer's merge pools
  pkv_state_desc desc;
  int32_t *arrive;     // [H]
  int32_t *early;      // evict_kernel: per head, arrivals after the record reads (one 128-byte line each)
  // byte strides of the new frames (frame, head, token); every offset into
  // them and into one head's pools is below 2^31
  uint32_t src_fb, src_hb, src_tb;
  int64_t t0;
  const int64_t *t_vals;  // [F] frame times, or null: t0 + f
  const float *weights;   // [F] frame weights, or null: 1 (the reference's unweighted merge)
  int counters;           // 1: route the frames and commit the counters; 0: records and merges only
  int layer, H, F, FSEQ, D, width, max_sink, max_middle, max_recent, MMA, MMB, MTPA;
  int pass_kind, shift_pending;
  int n_merge, n_scat;  // merge tiles per merge head (0: no merges this call), token tiles per head
  int n_mh;             // merge heads
  uint64_t merge_heads; // bit h (bit 63 for every head >= 63): h is a merge head
};

struct UpdShared {
  HeadState st;
  FrameDesc desc[kUpdMaxFrames];
  Route r;
  int32_t staged, machine_done, last;
  int32_t g_ng[kMaxMergeSlots];  // stored group counts and weight sums of the slots
  float g_wsum[kMaxMergeSlots];
  int64_t f_t[kUpdMaxFrames];    // frame times and weights
  float f_w[kUpdMaxFrames];
  float f_wsum[kUpdMaxFrames];   // the block's weight sum after frame f
  // merge bookkeeping: per frame, the list source and group count of its
  // block; per slot, the source, group count and weight sum after the call
  // and the stored-id check (-1 not done, 0 not the regular grid, else its
  // width); the call's grid: group count, columns, regular width (0: none)
  int32_t f_src[kUpdMaxFrames];
  int32_t f_ng[kUpdMaxFrames];
  int64_t f_tpos[kUpdMaxFrames];
  int32_t s_src[kMaxMergeSlots];
  int32_t s_ng[kMaxMergeSlots];
  int64_t s_tpos[kMaxMergeSlots];
  float s_wsum[kMaxMergeSlots];
  int32_t s_grid[kMaxMergeSlots];
  int32_t grid_ng, grid_cols, grid_w;
};

// group of token t on the arithmetic grid (y = t / W, x = t % W) in patches
// of p (mega_merge_accum.cu:100-184, ids past the group count fold into 0)
__device__ inline int32_t grid_gid(int t, int W, int p, int cols, int ng) {
  const int32_t y = t / W, x = t % W;
  const int32_t g = (p > 0 ? y / p : 0) * cols + (p > 0 ? x / p : 0);
  return (g < 0 || g >= ng) ? 0 : g;
}

// thread 0: descriptors of the call's frames on the LDS record
// (anchor_store_update.cu:257-269; noisy passes emit SKIP)
__device__ void upd_machine(const UpdArgs &a, UpdShared &sh) {
  for (int f = 0; f < a.F; ++f)
    sh.desc[f] = a.pass_kind == 1 ? sm_step(sh.st, static_cast<int32_t>(sh.f_t[f])) : skip_desc();
  sh.machine_done = 1;
}

// thread 0, after upd_machine on a Veil head: where each merge frame's
// group lists come from, and every touched slot's group count and running
// weight sum (1 per frame without weights)
__device__ void upd_merge_plan(const UpdArgs &a, int h, UpdShared &sh) {
  const int p = sh.st.patch_size, FSEQ = a.FSEQ, W = a.width, MTPA = a.MTPA;
  const int maxx = min(W, FSEQ) - 1, maxy = (FSEQ - 1) / W;
  const int cols = p > 0 ? maxx / p + 1 : 1, rows = p > 0 ? maxy / p + 1 : 1;
  const int we = maxx + 1;
  sh.grid_cols = cols;
  sh.grid_ng = min(rows * cols, MTPA);
  sh.grid_w = (p > 0 && FSEQ % we == 0 && we % p == 0 && (FSEQ / we) % p == 0 && rows * cols <= MTPA) ? we : 0;
  for (int s = 0; s < a.MMA; ++s) {
    sh.s_src[s] = kSrcNone;
    sh.s_grid[s] = -1;
  }
  for (int f = 0; f < a.F; ++f) {
    const FrameDesc d = sh.desc[f];
    sh.f_src[f] = kSrcNone;
    if (d.kind != PKV_DST_MERGE_ACCUM || d.accum_slot < 0 || d.accum_slot >= a.MMA) continue;
    const int s = d.accum_slot;
    if (d.is_new_block) {
      sh.s_src[s] = kSrcGrid;
      sh.s_ng[s] = sh.grid_ng;
      sh.s_tpos[s] = sh.f_t[f];
      sh.s_wsum[s] = 0.0f;
    } else if (sh.s_src[s] == kSrcNone) {
      sh.s_src[s] = s;
      sh.s_ng[s] = min(sh.g_ng[s], MTPA);
      sh.s_tpos[s] = 0;
      sh.s_wsum[s] = sh.g_wsum[s];
    }
    sh.s_wsum[s] += sh.f_w[f];
    sh.f_wsum[f] = sh.s_wsum[s];
    sh.f_src[f] = sh.s_src[s];
    sh.f_ng[f] = sh.s_ng[s];
    sh.f_tpos[f] = sh.s_tpos[s];
  }
}

// Width W of the regular patch grid when the group ids stored for a block
// are exactly its ids (group of token t = ((t / W) / p) * (W / p) +
// (t % W) / p), else 0; the same in every thread (a block-wide vote).
__device__ int stored_grid_width(const int32_t *gids, int FSEQ, int W, int p, int ng) {
  const bool ok = W > 0 && p > 0 && FSEQ % W == 0 && W % p == 0 && (FSEQ / W) % p == 0 && ng == FSEQ / (p * p);
  bool bad = false;
  if (ok) {
    const int cols = W / p;
    for (int t = threadIdx.x; t < FSEQ; t += blockDim.x) bad |= gids[t] != ((t / W) / p) * cols + (t % W) / p;
  }
  const int any_bad = __syncthreads_or(bad);
  return ok && !any_bad ? W : 0;
}

// Merge tile mt of head h: groups [mt * gpt, (mt + 1) * gpt), thread =
// (group, 8-wide dim chunk), every accumulator element owned by one thread
// for all frames (mega_merge_accum.cu:52-252).  Per frame in order: a slot
// switch stores / loads the accumulators, a new block zeroes them and its
// owner threads write the group's token count and position, the members are
// added in ascending token order (one fp32 add each), and a finalize writes
// bf16(sum * (1 / (count * block_frames))) and the anchor position.
// Groups per merge tile: each wave covers 64 / (D / 8) groups of K (even
// waves) or V (odd waves), the wave pairs side by side
__host__ __device__ inline int merge_tile_groups(int D) { return (kUpdThreads / 128) * (64 / (D / 8)); }

// Dynamic LDS of a merge tile (int32 words): the group ids its scan reads
// [FSEQ] and the stored group ids of every accumulator slot [MMA][FSEQ],
// each region starting on a 16-byte boundary.
__host__ __device__ inline int merge_fseq_words(int FSEQ) { return (FSEQ + 3) & ~3; }
__host__ __device__ inline int64_t merge_lds_words(int FSEQ, int MMA) {
  return static_cast<int64_t>(merge_fseq_words(FSEQ)) * (1 + MMA);
}

// Patch chunks of a merge tile's groups in every frame of a call, loaded
// before the record is staged and the state machine run: the members of a
// group on the regular grid of width W = min(spatial width, FSEQ) depend on
// nothing else.  merge_prefetch returns W, or 0 when the call does not
// qualify (then nothing is loaded); frames whose lists turn out otherwise
// load their members themselves.
constexpr int kPreFrames = 3;
constexpr int kPrePatch = 2;  // the Veil patch of the shipped policy
constexpr int kPreTok = kPrePatch * kPrePatch;
struct MergePre {
  uint4 x[kPreFrames][kPreTok];
};

// thread -> (group, K or V, 8-wide chunk) of merge tile mt, shared by the
// prefetch and the tile
struct MergeLane {
  int g, c, is_v, own;
  __device__ MergeLane(const UpdArgs &a, int mt) {
    const int cpt = a.D / 8, gpw = 64 / cpt;
    const int wave = static_cast<int>(threadIdx.x) >> 6, lane = static_cast<int>(threadIdx.x) & 63;
    is_v = wave & 1;  // wave-uniform: K or V
    g = mt * merge_tile_groups(a.D) + (wave >> 1) * gpw + lane / cpt;
    c = (lane % cpt) * 8;
    own = lane / cpt < gpw && g < a.MTPA;
  }
};

__device__ __forceinline__ int merge_prefetch(const UpdArgs &a, int h, int mt, MergePre &pre) {
  // the patch size is assumed to be kPrePatch, so that the loads depend on
  // nothing the kernel reads; the tile drops them for any other patch
  constexpr int p = kPrePatch;
  const int FSEQ = a.FSEQ, W = min(a.width, FSEQ);
  const MergeLane ln(a, mt);
  if (a.F > kPreFrames || FSEQ % W != 0 || W % p != 0 || (FSEQ / W) % p != 0) return 0;
  if (ln.own && ln.g < FSEQ / (p * p)) {
    const uint16_t *src = ln.is_v ? a.src.v : a.src.k;
    const int gcols = W / p;
    const int gbase = (ln.g / gcols) * p * W + (ln.g % gcols) * p;
#pragma unroll
    for (int f = 0; f < kPreFrames; ++f)
#pragma unroll
      for (int m = 0; m < kPreTok; ++m)
        if (f < a.F && m < p * p)
          pre.x[f][m] = ld16o(src, f * a.src_fb + h * a.src_hb + ln.c * 2 + (gbase + (m / p) * W + m % p) * a.src_tb);
  }
  return W;
}

// Merge tiles stage the stored group ids of every slot into LDS with the
// record (one round trip for what the tile reads before its frames;
// upd_stage's barrier orders the LDS writes)
__device__ __forceinline__ void merge_stage(const UpdArgs &a, int h, int32_t *dyn) {
  const int tid = threadIdx.x, FSEQ = a.FSEQ, fw = merge_fseq_words(FSEQ);
  const int32_t *gids = a.ml.accum_group_ids + static_cast<int64_t>(h) * a.MMA * FSEQ;
  if (FSEQ % 4 == 0) {  // 16-byte pieces (the slots' ids start 16-byte aligned)
    const int per = FSEQ / 4, n = a.MMA * per;
    const int4 *g4 = reinterpret_cast<const int4 *>(gids);
    constexpr int kB = 4;
    for (int i0 = 0; i0 < n; i0 += kB * kUpdThreads) {
      int4 v[kB];
#pragma unroll
      for (int k = 0; k < kB; ++k) v[k] = g4[min(i0 + tid + k * kUpdThreads, n - 1)];
#pragma unroll
      for (int k = 0; k < kB; ++k) {
        const int i = i0 + tid + k * kUpdThreads;
        if (i < n) reinterpret_cast<int4 *>(dyn + fw + (i / per) * fw)[i % per] = v[k];
      }
    }
  } else {
    const int n = a.MMA * FSEQ;
    for (int i = tid; i < n; i += kUpdThreads) dyn[fw + (i / FSEQ) * fw + i % FSEQ] = gids[i];
  }
}

__device__ void upd_merge_tile(const UpdArgs &a, int h, int mt, UpdShared &sh, int32_t *dyn, const MergePre &pre,
                               int spec) {
  const int tid = threadIdx.x, D = a.D, MTPA = a.MTPA, FSEQ = a.FSEQ;
  const MergeLane ln(a, mt);
  const int g = ln.g, c = ln.c;
  const bool own = ln.own;
  const bool meta = own && !ln.is_v && c == 0;  // writes the group's count and positions
  const int32_t p = sh.st.patch_size, bf = sh.st.block_frames;
  const pkv_merge_layer &ml = a.ml;
  const uint16_t *src = ln.is_v ? a.src.v : a.src.k;
  float *acc_sum = ln.is_v ? ml.accum_sum_v : ml.accum_sum_k;
  uint16_t *merge_out = ln.is_v ? ml.merge_v : ml.merge_k;
  float ax[8];
  int cur = -1;
  int ids_src = kSrcNone;  // source of the group ids the scan reads
  auto store_acc = [&](int slot) {
    const int64_t o = ((static_cast<int64_t>(h) * a.MMA + slot) * MTPA + g) * D + c;
    for (int e = 0; e < 8; ++e) acc_sum[o + e] = ax[e];
  };
  // one member chunk added to the accumulators (one fp32 add per element)
  // (w * x in fp32, then one add: the weighted merge; w = 1 without weights
  // leaves x unchanged, so the sums are the reference's)
  float w = 1.0f;
  auto add16 = [&](const uint4 &x) {
    const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ax[2 * e] += w * bf16_to_f32(static_cast<uint16_t>(xw[e] & 0xffff));
      ax[2 * e + 1] += w * bf16_to_f32(static_cast<uint16_t>(xw[e] >> 16));
    }
  };
  // Width of the regular grid whose closed-form lists frame f's block
  // uses, or 0 (all threads: the first use of a stored slot votes on its ids)
  auto frame_width = [&](int f) {
    const int src_kind = sh.f_src[f];
    if (src_kind == kSrcGrid) return sh.grid_w;
    if (sh.s_grid[src_kind] < 0) {
      const int64_t hs = static_cast<int64_t>(h) * a.MMA + src_kind;
      sh.s_grid[src_kind] =
          stored_grid_width(dyn + merge_fseq_words(FSEQ) * (1 + src_kind), FSEQ, min(a.width, FSEQ), p, sh.f_ng[f]);
    }
    return sh.s_grid[src_kind];
  };
  // Merge frame f.  kClosed: the lists are the closed form of width spec
  // and pf holds the patch's chunks, loaded up front.  Otherwise, on a
  // regular grid of width W the members are loaded here, and without one
  // each thread scans the block's group ids (staged in LDS) for its group's
  // tokens in ascending order -- the path of grids that do not tile into
  // patches and of blocks begun with other positions.
  auto frame = [&](int f, const uint4 *pf, auto closed_tag) {
    constexpr bool kClosed = decltype(closed_tag)::value;
    const int src_kind = sh.f_src[f];
    if (src_kind == kSrcNone) return;
    const FrameDesc d = sh.desc[f];
    const int slot = d.accum_slot, is_new = d.is_new_block, fin = d.finalize_idx;
    const int ng = sh.f_ng[f];
    const int64_t hs = static_cast<int64_t>(h) * a.MMA + slot;
    w = sh.f_w[f];
    int W = spec;
    if constexpr (!kClosed) {
      W = frame_width(f);
      if (uni(W == 0 && ids_src != src_kind)) {
        if (src_kind == kSrcGrid) {  // stored ids are staged already
          __syncthreads();  // readers of the previous ids are done
          for (int t = tid; t < FSEQ; t += blockDim.x) dyn[t] = grid_gid(t, a.width, p, sh.grid_cols, sh.grid_ng);
          __syncthreads();
        }
        ids_src = src_kind;
      }
    }
    if (own) {
      if (slot != cur) {
        if (cur >= 0) store_acc(cur);
        cur = slot;
        if (!is_new) {
          const int64_t o = (hs * MTPA + g) * D + c;
          for (int e = 0; e < 8; ++e) ax[e] = acc_sum[o + e];
        }
      }
      if (is_new)
        for (int e = 0; e < 8; ++e) ax[e] = 0.0f;
      int cnt = p * p;  // members of group g
      if (g < ng) {
        if constexpr (kClosed) {
#pragma unroll
          for (int m = 0; m < kPreTok; ++m)
            if (m < p * p) add16(pf[m]);
        } else {
          const uint32_t fo = f * a.src_fb + h * a.src_hb + c * 2;
          if (W) {
            const int gcols = W / p;
            const int gbase = (g / gcols) * p * W + (g % gcols) * p;
            for (int mb = 0; mb < p * p; mb += kUpdAccBatch) {
              const int n = min(kUpdAccBatch, p * p - mb);
              uint4 xx[kUpdAccBatch];
#pragma unroll
              for (int b = 0; b < kUpdAccBatch; ++b)
                if (b < n) xx[b] = ld16o(src, fo + (gbase + ((mb + b) / p) * W + (mb + b) % p) * a.src_tb);
#pragma unroll
              for (int b = 0; b < kUpdAccBatch; ++b)
                if (b < n) add16(xx[b]);
            }
          } else {
            const int32_t *ids = src_kind == kSrcGrid ? dyn : dyn + merge_fseq_words(FSEQ) * (1 + src_kind);
            cnt = 0;
            for (int t = 0; t < FSEQ; ++t)
              if (ids[t] == g) {
                add16(ld16o(src, fo + t * a.src_tb));
                ++cnt;
              }
          }
        }
      }
      if (is_new && meta) {
        ml.accum_tokens_per_group[hs * MTPA + g] = g < ng ? static_cast<float>(cnt) * static_cast<float>(bf) : 0.0f;
        if (g < ng) {
          int64_t *ap = ml.accum_pos + (hs * MTPA + g) * 3;
          ap[0] = sh.f_tpos[f];
          ap[1] = (g / sh.grid_cols) * p;
          ap[2] = (g % sh.grid_cols) * p;
        }
      }
      if (fin >= 0 && fin < a.MMB && g < ng) {
        // count * sum(w) for weighted merges, else the reference's count * block_frames
        const float div = static_cast<float>(cnt) * (a.weights ? sh.f_wsum[f] : static_cast<float>(bf));
        const float inv = div > 0.0f ? 1.0f / div : 0.0f;
        const int64_t hp = static_cast<int64_t>(h) * a.MMB + fin;
        uint4 ox;
        ox.x = pack_bf16x2(ax[0] * inv, ax[1] * inv);
        ox.y = pack_bf16x2(ax[2] * inv, ax[3] * inv);
        ox.z = pack_bf16x2(ax[4] * inv, ax[5] * inv);
        ox.w = pack_bf16x2(ax[6] * inv, ax[7] * inv);
        st16(merge_out + (hp * MTPA + g) * D + c, ox);
        if (meta) {
          int64_t *mp = ml.merge_pos + (hp * MTPA + g) * 3;
          if (src_kind == kSrcGrid) {
            mp[0] = sh.f_tpos[f];
            mp[1] = (g / sh.grid_cols) * p;
            mp[2] = (g % sh.grid_cols) * p;
          } else {
            const int64_t *ap = ml.accum_pos + (hs * MTPA + g) * 3;
            const int64_t p0 = ap[0], p1 = ap[1], p2 = ap[2];
            mp[0] = p0;
            mp[1] = p1;
            mp[2] = p2;
          }
        }
      }
    }
    if (fin >= 0 && fin < a.MMB && mt == 0 && tid == 0) ml.merge_token_count[static_cast<int64_t>(h) * a.MMB + fin] = ng;
  };
  // the prefetched chunks serve when the patch is the prefetch's and every
  // merge frame's lists are the closed form of width spec (uniform)
  bool closed = spec != 0 && p == kPrePatch;
  for (int f = 0; f < a.F && closed; ++f)
    if (sh.f_src[f] != kSrcNone) closed = frame_width(f) == spec;
  if (uni(closed)) {
#pragma unroll
    for (int f = 0; f < kPreFrames; ++f)
      if (f < a.F) frame(f, pre.x[f], std::true_type{});
  } else {
    for (int f = 0; f < a.F; ++f) frame(f, nullptr, std::false_type{});
  }
  if (own && cur >= 0) store_acc(cur);
}

// Arrival of tile idx of head h, in two levels: tile idx counts on
// sub-counter idx % kArriveFan, the last arrival of each sub-counter counts
// on the head counter, and the last of those is the head's last workgroup.
// Each counter sits on its own 128-byte line, so arrivals at one address
// stay few.  arrive_take (thread 0) returns the sub-counter's previous
// value; arrive_last resolves it, resetting every counter it completes.
__device__ inline int32_t *arrive_counters(const UpdArgs &a, int h) {
  return a.arrive + static_cast<int64_t>(h) * (kArriveFan + 1) * kArriveStride;
}

// Whether head h's clean passes accumulate merges, and the i-th such head
__device__ inline bool is_merge_head(const UpdArgs &a, int h) {
  return a.n_merge > 0 && ((a.merge_heads >> (h < 63 ? h : 63)) & 1);
}
__device__ inline int merge_head_at(const UpdArgs &a, int i) {
  uint64_t m = a.merge_heads & ~(uint64_t{1} << 63);
  const int low = __popcll(m);
  if (i >= low) return 63 + (i - low);
  for (int k = 0; k < i; ++k) m &= m - 1;
  return __builtin_ctzll(m);
}

// Token tiles in grid order: the heads without Veil merges first, then the
// Veil heads (whose token tiles stage no record and write no middle copies),
// so that the tiles left for the grid's last dispatch round are the short
// ones.  Position i -> head, ascending within each part.
__device__ inline int token_head_at(const UpdArgs &a, int i) {
  if (a.n_mh == 0) return i;
  const int n0 = a.H - a.n_mh;
  if (i >= n0) return merge_head_at(a, i - n0);
  const int hl = min(a.H, 63);
  uint64_t m = ~a.merge_heads & ((uint64_t{1} << hl) - 1);
  const int low = __popcll(m);
  if (i >= low) return 63 + (i - low);  // heads >= 63 without merges (bit 63 clear)
  for (int k = 0; k < i; ++k) m &= m - 1;
  return __builtin_ctzll(m);
}

__device__ inline int arrive_take(const UpdArgs &a, int h, int idx) {
  return atomicAdd(arrive_counters(a, h) + (idx % kArriveFan) * kArriveStride, 1);
}

__device__ inline int arrive_last(const UpdArgs &a, int h, int idx, int ticket) {
  const int n_tiles = (is_merge_head(a, h) ? a.n_merge : 0) + a.n_scat;
  const int sub = idx % kArriveFan;
  const int sub_n = n_tiles / kArriveFan + (sub < n_tiles % kArriveFan ? 1 : 0);
  if (ticket != sub_n - 1) return 0;
  int32_t *ctr = arrive_counters(a, h);
  atomicExch(ctr + sub * kArriveStride, 0);
  int32_t *hc = ctr + kArriveFan * kArriveStride;
  const int last = atomicAdd(hc, 1) == min(kArriveFan, n_tiles) - 1;
  if (last) atomicExch(hc, 0);
  return last;
}

// Copy h's record into LDS (every thread; ends with a barrier)
__device__ __forceinline__ void upd_stage(const UpdArgs &a, UpdShared &sh, int h) {
  // with the record, on a clean pass of a layer with merges, the stored
  // group counts and weight sums of h's accumulator slots: one round trip
  // and the call's frame times and weights
  const int tid = threadIdx.x;
  const int64_t hs0 = static_cast<int64_t>(h) * a.MMA;
  constexpr int kNg = kStateWords, kWs = kNg + kMaxMergeSlots, kFr = kWs + kMaxMergeSlots;
  static_assert(kFr + kUpdMaxFrames <= kUpdThreads, "one staged value per thread");
  if (tid < kStateWords) {
    reinterpret_cast<uint32_t *>(&sh.st)[tid] = reinterpret_cast<const uint32_t *>(a.states + h)[tid];
  } else if (tid < kWs) {
    if (is_merge_head(a, h) && tid - kNg < a.MMA) sh.g_ng[tid - kNg] = a.ml.accum_num_groups[hs0 + tid - kNg];
  } else if (tid < kFr) {
    const int s = tid - kWs;
    if (is_merge_head(a, h) && s < a.MMA) sh.g_wsum[s] = a.ml.accum_weight_sum ? a.ml.accum_weight_sum[hs0 + s] : 0.0f;
  } else if (tid < kFr + a.F) {
    const int f = tid - kFr;
    sh.f_t[f] = a.t_vals ? a.t_vals[f] : a.t0 + f;
    sh.f_w[f] = a.weights ? a.weights[f] : 1.0f;
  }
  __syncthreads();
}

// Routing of head h from its committed counters, computed by every thread
// from scalar reads (read before the head's last workgroup rewrites them)
__device__ __forceinline__ Route upd_route(const UpdArgs &a, int h) {
  const int64_t *cvc = a.committed_vc + h * 3;
  return route_frames(ld_uniform(cvc), ld_uniform(cvc + 1), ld_uniform(cvc + 2), ld_uniform(a.sink_caps + h), a.F,
                      a.max_sink, a.max_recent, a.shift_pending);
}

// Token tile `tile` of head h: thread = (token, 16-byte chunk), one item
// per thread.  The routing needs only the committed counters, so the new
// frames' chunks and the first recent slots the FIFO shift moves are loaded
// at once; the record is staged and the state machine run only for heads
// whose frames may go to middle slots (Wave, Anchor, lag).
__device__ __forceinline__ void upd_token_tile(const UpdArgs &a, UpdShared &sh, int h, int tile, int &ticket) {
  const int tid = threadIdx.x;
  const int F = a.F, FSEQ = a.FSEQ, D = a.D;
  const int cpt = D / 8, ttok = kUpdThreads / cpt;
  const int tok = tile * ttok + tid / cpt, c = (tid % cpt) * 8;
  const bool item = tid < ttok * cpt && tok < FSEQ;
  const Route r = upd_route(a, h);
  const int kind = ld_uniform(&a.states[h].kind);
  const bool middle = a.pass_kind == 1 && (kind == SK_CYCLIC || kind == SK_STRIDE || kind == SK_LAG);
  const int64_t lh = static_cast<int64_t>(a.layer) * a.H + h;
  const int64_t slot_elems = static_cast<int64_t>(FSEQ) * D;
  const uint32_t slot_b = static_cast<uint32_t>(slot_elems) * 2;
  const PoolPtrs &pools = a.pools;
  uint16_t *rec_k = pools.k[2] + lh * a.max_recent * slot_elems;
  uint16_t *rec_v = pools.v[2] + lh * a.max_recent * slot_elems;
  const uint32_t to = h * a.src_hb + tok * a.src_tb + c * 2;
  const uint32_t e = (tok * D + c) * 2;
  uint4 kk[kScatBatch], vv[kScatBatch], sk[kShiftBatch], sv[kShiftBatch];
  if (item) {
#pragma unroll
    for (int f = 0; f < kScatBatch; ++f)
      if (f < F) {
        kk[f] = ld16o(a.src.k, to + f * a.src_fb);
        vv[f] = ld16o(a.src.v, to + f * a.src_fb);
      }
#pragma unroll
    for (int q = 0; q < kShiftBatch; ++q)
      if (q < r.keep) {
        sk[q] = ld16o(rec_k, (q + r.shift) * slot_b + e);
        sv[q] = ld16o(rec_v, (q + r.shift) * slot_b + e);
      }
  }
  if (middle) {  // uniform
    upd_stage(a, sh, h);
    if (tid == 0) upd_machine(a, sh);
    __syncthreads();
  }
  if (tid == 0) {
    sh.staged = middle;
    sh.machine_done = middle;
    sh.r = r;
  }
  // every read of the head's shared data (its record and committed
  // counters) is done: arrive now, so that the head's write-back overlaps
  // the stores below
  __syncthreads();
  if (tid == 0) ticket = arrive_take(a, h, (is_merge_head(a, h) ? a.n_merge : 0) + tile);
  uint16_t *sink_k = pools.k[0] + lh * a.max_sink * slot_elems;
  uint16_t *sink_v = pools.v[0] + lh * a.max_sink * slot_elems;
  uint16_t *mid_k = pools.k[1] + lh * a.max_middle * slot_elems;
  uint16_t *mid_v = pools.v[1] + lh * a.max_middle * slot_elems;
  const bool desc_ok = middle;
  if (item) {
    // recent FIFO shift: slot j <- slot j + shift for j < keep (all sources
    // of a batch read before its stores; batches ascend, and a slot written
    // by one batch is never a source of a later batch since sources are
    // >= shift > destinations of earlier batches; the new frames are stored
    // after every shift store)
    for (int j0 = 0; j0 < r.keep; j0 += kShiftBatch) {
      const int n = min(kShiftBatch, r.keep - j0);
      if (j0 > 0) {
#pragma unroll
        for (int q = 0; q < kShiftBatch; ++q)
          if (q < n) {
            sk[q] = ld16o(rec_k, (j0 + q + r.shift) * slot_b + e);
            sv[q] = ld16o(rec_v, (j0 + q + r.shift) * slot_b + e);
          }
      }
#pragma unroll
      for (int q = 0; q < kShiftBatch; ++q)
        if (q < n) {
          st16o(rec_k, (j0 + q) * slot_b + e, sk[q]);
          st16o(rec_v, (j0 + q) * slot_b + e, sv[q]);
        }
    }
    for (int f0 = 0; f0 < F; f0 += kScatBatch) {
      const int n = min(kScatBatch, F - f0);
      if (f0 > 0) {
#pragma unroll
        for (int q = 0; q < kScatBatch; ++q)
          if (q < n) {
            kk[q] = ld16o(a.src.k, to + (f0 + q) * a.src_fb);
            vv[q] = ld16o(a.src.v, to + (f0 + q) * a.src_fb);
          }
      }
#pragma unroll
      for (int q = 0; q < kScatBatch; ++q) {
        if (q >= n) continue;
        const int f = f0 + q;
        if (f < r.sink_writes) {
          const uint32_t o = (r.sink_first + f) * slot_b + e;
          st16o(sink_k, o, kk[q]);
          st16o(sink_v, o, vv[q]);
        } else {
          const uint32_t o = (r.recent_first + (f - r.sink_writes)) * slot_b + e;
          st16o(rec_k, o, kk[q]);
          st16o(rec_v, o, vv[q]);
        }
        if (desc_ok && sh.desc[f].kind == PKV_DST_MIDDLE) {
          const int s = sh.desc[f].slot;
          if (s >= 0 && s < a.max_middle) {
            st16o(mid_k, s * slot_b + e, kk[q]);
            st16o(mid_v, s * slot_b + e, vv[q]);
          }
        }
      }
    }
  }
  // positions (t0 + f, tok / W, tok % W): one thread per token of the tile
  const int pt = tile * ttok + tid;
  if (tid < ttok && pt < FSEQ) {
    const int64_t pe = static_cast<int64_t>(pt) * 3;
    const int64_t pslot = static_cast<int64_t>(FSEQ) * 3;
    int64_t *sink_p = pools.pos[0] + lh * a.max_sink * pslot;
    int64_t *mid_p = pools.pos[1] + lh * a.max_middle * pslot;
    int64_t *rec_p = pools.pos[2] + lh * a.max_recent * pslot;
    for (int j = 0; j < r.keep; ++j) {
      const int64_t *sp = rec_p + (j + r.shift) * pslot + pe;
      const int64_t p0 = sp[0], p1 = sp[1], p2 = sp[2];
      int64_t *dp = rec_p + j * pslot + pe;
      dp[0] = p0;
      dp[1] = p1;
      dp[2] = p2;
    }
    const int64_t py = pt / a.width, px = pt % a.width;
    for (int f = 0; f < F; ++f) {
      const int64_t ptt = a.t0 + f;
      int64_t *dp;
      if (f < r.sink_writes)
        dp = sink_p + (r.sink_first + f) * pslot + pe;
      else
        dp = rec_p + (r.recent_first + (f - r.sink_writes)) * pslot + pe;
      dp[0] = ptt;
      dp[1] = py;
      dp[2] = px;
      if (desc_ok && sh.desc[f].kind == PKV_DST_MIDDLE) {
        const int64_t s = sh.desc[f].slot;
        if (s >= 0 && s < a.max_middle) {
          int64_t *mp = mid_p + s * pslot + pe;
          mp[0] = ptt;
          mp[1] = py;
          mp[2] = px;
        }
      }
    }
  }
}

// Merge tile `tile` of head h: record, stored group ids and the frames'
// patch chunks loaded together, the state machine and merge bookkeeping on
// thread 0, the tile's groups accumulated, then the arrival
__device__ __forceinline__ void upd_merge_wg(const UpdArgs &a, UpdShared &sh, int32_t *dyn, int h, int tile,
                                             int &ticket, int tiles = 1) {
  const int tid = threadIdx.x;
  Route r{};
  if (a.counters) r = upd_route(a, h);
  MergePre pre;
  int spec = a.pass_kind == 1 ? merge_prefetch(a, h, tile * tiles, pre) : 0;
  merge_stage(a, h, dyn);
  upd_stage(a, sh, h);
  if (tid == 0) {
    sh.staged = 1;
    sh.machine_done = 0;
    sh.r = r;
    if (a.pass_kind == 1 && sh.st.kind == SK_MERGE) {
      upd_machine(a, sh);
      upd_merge_plan(a, h, sh);
    }
  }
  __syncthreads();
  if (uni(sh.st.kind == SK_MERGE) && a.pass_kind == 1) {
    for (int j = 0; j < tiles; ++j) {  // merge tiles tile * tiles .. (several in an eviction workgroup)
      const int mt = tile * tiles + j;
      if (mt * merge_tile_groups(a.D) >= a.MTPA) break;
      if (j > 0) spec = merge_prefetch(a, h, mt, pre);
      upd_merge_tile(a, h, mt, sh, dyn, pre, spec);
    }
  }
  __syncthreads();  // every read of the head's shared data is done
  if (tid == 0) ticket = arrive_take(a, h, tile);
}

// Arrival index `idx` of head h resolved and, in the head's last
// workgroup, the write-back: record, counters, descriptors and the merge
// slots' group counts, weight sums and group ids
__device__ __forceinline__ void upd_finish(const UpdArgs &a, UpdShared &sh, int h, int idx, int ticket) {
  const int tid = threadIdx.x;
  const int F = a.F, FSEQ = a.FSEQ;
  if (tid == 0) sh.last = arrive_last(a, h, idx, ticket);
  __syncthreads();
  if (!uni(sh.last)) return;
  if (!uni(sh.staged)) upd_stage(a, sh, h);
  const bool merge_head = is_merge_head(a, h) && a.pass_kind == 1 && uni(sh.st.kind == SK_MERGE);
  if (!uni(sh.machine_done)) {
    if (tid == 0) {
      upd_machine(a, sh);
      if (merge_head) upd_merge_plan(a, h, sh);
    }
    __syncthreads();
  }
  if (a.pass_kind == 1 && tid < kStateWords)
    reinterpret_cast<uint32_t *>(a.states + h)[tid] = reinterpret_cast<const uint32_t *>(&sh.st)[tid];
  if (a.counters && tid < 3) {
    a.vc[h * 3 + tid] = sh.r.vc_post[tid];
    if (a.pass_kind == 1) a.committed_vc[h * 3 + tid] = sh.r.vc_post[tid];
  }
  if (tid < F) store_desc(a.desc, h * F + tid, tid, h, sh.desc[tid]);
  if (merge_head) {
    const int p = sh.st.patch_size;
    for (int s = 0; s < a.MMA; ++s) {
      const int src = sh.s_src[s];
      if (src == kSrcNone) continue;
      const int64_t hs = static_cast<int64_t>(h) * a.MMA + s;
      if (tid == 0) {
        if (src == kSrcGrid) a.ml.accum_num_groups[hs] = sh.s_ng[s];
        if (a.ml.accum_weight_sum) a.ml.accum_weight_sum[hs] = sh.s_wsum[s];
      }
      if (src == kSrcGrid)
        for (int t = tid; t < FSEQ; t += blockDim.x)
          a.ml.accum_group_ids[hs * FSEQ + t] = grid_gid(t, a.width, p, sh.grid_cols, sh.grid_ng);
    }
  }
}

__global__ void __launch_bounds__(kUpdThreads) update_kernel(UpdArgs a) {
  extern __shared__ __attribute__((aligned(16))) int32_t dyn[];
  __shared__ __attribute__((aligned(16))) UpdShared sh;
  const int b = blockIdx.x;
  const int n_mt = a.n_mh * a.n_merge;
  const bool merge_tile = b < n_mt;
  const int h = merge_tile ? merge_head_at(a, b / a.n_merge) : token_head_at(a, (b - n_mt) / a.n_scat);
  const int tile = merge_tile ? b % a.n_merge : (b - n_mt) % a.n_scat;
  int ticket = 0;  // thread 0: the arrival sub-counter's previous value
  if (merge_tile)
    upd_merge_wg(a, sh, dyn, h, tile, ticket);
  else
    upd_token_tile(a, sh, h, tile, ticket);
  upd_finish(a, sh, h, merge_tile ? tile : (is_merge_head(a, h) ? a.n_merge : 0) + tile, ticket);
}

// ---- Veil step in registers ------------------------------------------------
//
// A Veil step (anchor_store_update.cu:122-231) changes only the record's
// last 39 words: the completed FIFO, the active blocks' ids, seen flags and
// frame counts.  The step splits into a decision -- scalar arithmetic on
// six of those words, the block frames and the capacity -- and its
// application to the words, one word per lane of a wave (the FIFO shift
// reads the next lane's word).  The eviction kernel uses it in place of the
// state machine on one thread over the LDS record, whose chain of dependent
// LDS accesses was the longest step of an eviction.
constexpr int kVeilWord0 = static_cast<int>(offsetof(HeadState, merge_completed_slot) / 4);
constexpr int kVeilWords = kStateWords - kVeilWord0;
constexpr int kVlCount = static_cast<int>(offsetof(HeadState, merge_completed_count) / 4) - kVeilWord0;
constexpr int kVlId = static_cast<int>(offsetof(HeadState, merge_active_block_id) / 4) - kVeilWord0;
constexpr int kVlSeen = static_cast<int>(offsetof(HeadState, merge_active_seen) / 4) - kVeilWord0;
constexpr int kVlDone = static_cast<int>(offsetof(HeadState, merge_active_complete_count) / 4) - kVeilWord0;
static_assert(kVeilWords <= 64, "one record word per lane");
static_assert(kMaxMergeActive == 2 && kMaxMergeBlockFrames == 4, "one seen word per active block");
static_assert(offsetof(HeadState, merge_completed_slot) % 4 == 0 && offsetof(HeadState, merge_completed_count) % 4 == 0 &&
                  offsetof(HeadState, merge_active_seen) % 4 == 0 &&
                  offsetof(HeadState, merge_active_complete_count) % 4 == 0,
              "word-aligned Veil fields");
static_assert(kVlCount == 5 * kMaxMergeBlocks, "the completed FIFO's five arrays precede its count");

__device__ inline int32_t lane_word(uint32_t w, int l) {
  return __builtin_amdgcn_readlane(static_cast<int>(w), l);
}

// The record words a Veil decision reads
struct VeilWords {
  uint32_t count;         // merge_completed_count (low byte)
  int32_t id0, id1;       // merge_active_block_id
  uint32_t seen0, seen1;  // merge_active_seen rows
  uint32_t done;          // merge_active_complete_count (two low bytes)
};

// A decided Veil step: the frame's descriptor and the record's new values
struct VeilStep {
  FrameDesc d;
  int32_t cap, shift, block_id, start, end, median, cc, id0, id1, done0, done1;
  uint32_t seen0, seen1;
  __device__ bool changes() const { return d.kind == PKV_DST_MERGE_ACCUM; }
};

// sm_merge's decision, with its parameter guards; a skipped frame (guards,
// or a frame already seen) changes nothing
__device__ inline VeilStep veil_decide(const VeilWords &v, int32_t bf, int32_t cap, int32_t t) {
  VeilStep s;
  s.d = skip_desc();
  if (bf <= 0 || bf > kMaxMergeBlockFrames || cap <= 0 || cap > kMaxMergeBlocks || t < 0) return s;
  const int32_t block_id = t / bf, local = t % bf;
  int32_t id0 = v.id0, id1 = v.id1;
  uint32_t seen0 = v.seen0, seen1 = v.seen1;
  int32_t done0 = static_cast<int8_t>(v.done & 0xffu), done1 = static_cast<int8_t>((v.done >> 8) & 0xffu);
  int32_t cc = static_cast<int8_t>(v.count & 0xffu);
  int a = id0 == block_id ? 0 : (id1 == block_id ? 1 : -1);
  int is_new = 0;
  if (a < 0) {  // a free slot, else slot 0 is evicted; the slot taken is cleared
    a = id0 == -1 ? 0 : (id1 == -1 ? 1 : 0);
    is_new = 1;
  }
  int32_t id = a ? id1 : id0, done = a ? done1 : done0;
  uint32_t seen = a ? seen1 : seen0;
  if (is_new) {
    id = block_id;
    seen = 0;
    done = 0;
  }
  if ((seen >> (8 * local)) & 0xffu) return s;  // a repeated frame leaves the record as it is
  seen |= 1u << (8 * local);
  done = static_cast<int8_t>(done + 1);
  int32_t fin = -1;
  s.shift = 0;
  s.start = s.end = s.median = 0;
  if (done >= bf) {  // the block completes into the FIFO
    s.start = block_id * bf;
    s.end = s.start + bf - 1;
    s.median = (s.start + s.end) / 2;
    s.shift = cc >= cap;
    fin = s.shift ? cap - 1 : cc;
    if (!s.shift) cc = static_cast<int8_t>(cc + 1);
    id = -1;
    seen = 0;
    done = 0;
  }
  if (a) {
    id1 = id;
    seen1 = seen;
    done1 = done;
  } else {
    id0 = id;
    seen0 = seen;
    done0 = done;
  }
  s.cap = cap;
  s.block_id = block_id;
  s.cc = cc;
  s.id0 = id0;
  s.id1 = id1;
  s.seen0 = seen0;
  s.seen1 = seen1;
  s.done0 = done0;
  s.done1 = done1;
  s.d.kind = PKV_DST_MERGE_ACCUM;
  s.d.slot = -1;
  s.d.accum_slot = a;
  s.d.local_idx = local;
  s.d.finalize_idx = fin;
  s.d.is_new_block = is_new;
  return s;
}

// Record word kVeilWord0 + lane after the step (w: its value before, next:
// the next lane's value before)
__device__ inline uint32_t veil_apply(const VeilStep &s, uint32_t w, uint32_t next, int lane) {
  if (!s.changes()) return w;
  const int fin = s.d.finalize_idx;
  uint32_t nw = w;
  if (lane < kVlCount) {  // FIFO arrays: slot, block id, start, end, median
    const int arr = lane / kMaxMergeBlocks, e = lane % kMaxMergeBlocks;
    if (fin >= 0 && s.shift && e < s.cap - 1) nw = next;
    if (fin >= 0 && e == fin)
      nw = static_cast<uint32_t>(arr == 0 ? fin : arr == 1 ? s.block_id : arr == 2 ? s.start : arr == 3 ? s.end : s.median);
  } else if (lane == kVlCount) {
    nw = (w & ~0xffu) | (static_cast<uint32_t>(s.cc) & 0xffu);
  } else if (lane == kVlId) {
    nw = static_cast<uint32_t>(s.id0);
  } else if (lane == kVlId + 1) {
    nw = static_cast<uint32_t>(s.id1);
  } else if (lane == kVlSeen) {
    nw = s.seen0;
  } else if (lane == kVlSeen + 1) {
    nw = s.seen1;
  } else if (lane == kVlDone) {
    nw = (w & 0xffff0000u) | (static_cast<uint32_t>(s.done0) & 0xffu) | ((static_cast<uint32_t>(s.done1) & 0xffu) << 8);
  }
  return nw;
}

// The step applied in place to the words w held one per lane (lane l holds
// word kVeilWord0 + l); called by whole waves
__device__ inline void veil_apply_wave(const VeilStep &s, uint32_t &w) {
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const uint32_t next = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute((lane + 1) * 4, static_cast<int>(w)));
  w = veil_apply(s, w, next, lane);
}

// ---- Veil eviction of one frame per call (pkv_evict_merge) ----------------
//
// Eviction workgroups cover kEvTiles of update_kernel's merge tiles (each
// thread kEvTiles groups, same roles), so that the per-workgroup reads (the
// record, the stored group ids) and the arrivals are fewer.
constexpr int kEvTiles = 3;
constexpr int kEvIdLoads = 2;  // 16-byte loads of stored group ids per thread
constexpr int kEvMaxFseq = 4 * kEvIdLoads * kUpdThreads;
__host__ __device__ inline int evict_tile_groups(int D) { return kEvTiles * merge_tile_groups(D); }

// One frame per call.  One wave-wide gather brings the record's decision
// words, the frame time and weight and the slots' counts while the frame's
// patch chunks (regular grid of patch 2) stream in; the step is decided in
// scalar registers, and only a continued block then reads its slot's sums,
// stored group ids (verified against the grid by a block-wide vote) and
// anchor positions.  A head this path does not cover (another strategy kind
// or patch size, a continued block whose stored ids are not the grid's)
// runs update_kernel's merge tiles instead; the choice is the same in every
// workgroup of the head.  Launched only where the frame's grid of width
// W = spatial width tiles into 2 x 2 patches with at most MTPA of them, with
// at most 2 accumulator slots, FSEQ <= kEvMaxFseq, head_dim >= 32 and
// 16-byte aligned frames, sums and group ids (pkv_evict_merge checks).
// The values the first reads need come as leading scalar arguments, which
// the build preloads into scalar registers (-amdgpu-kernarg-preload-count),
// so that the gather does not wait for a kernel-argument load; they repeat
// fields of a.
__global__ void __launch_bounds__(kUpdThreads)
    evict_kernel(const HeadState *states, const int64_t *t_vals, const float *weights, const int32_t *num_groups,
                 const float *weight_sum, int32_t n_merge, int32_t mma, UpdArgs a) {
  extern __shared__ __attribute__((aligned(16))) int32_t dyn[];
  __shared__ __attribute__((aligned(16))) UpdShared sh;
  __shared__ uint32_t vote[kUpdThreads / 64];
  constexpr int p = kPrePatch, kTok = kPreTok;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x / n_merge, tile = blockIdx.x % n_merge;
  const int64_t hs0 = static_cast<int64_t>(h) * mma;

  // One wave-wide gather brings every value the step needs, issued first
  // (its addresses need only the preloaded arguments): lane l < 39 reads
  // Veil word l of the record; the next lanes read the record's kind,
  // capacity, patch and block frames, the frame time (two words) and
  // weight, and the slots' group counts and weight sums (absent optional
  // inputs read a stand-in address).  Meanwhile the groups' patch chunks in
  // the frame stream in.
  constexpr int kGKind = kVeilWords, kGCap = kGKind + 1, kGPatch = kGKind + 2, kGBf = kGKind + 3, kGT = kGKind + 4,
                kGW = kGKind + 6, kGNg = kGKind + 7, kGWs = kGKind + 9;
  static_assert(kGWs + 2 <= 64, "one gathered value per lane");
  const int32_t *rec = reinterpret_cast<const int32_t *>(states + h);
  const int32_t *gp = rec + kVeilWord0 + min(lane, kVeilWords - 1);
  const int s1 = min(1, mma - 1);
  if (lane == kGKind) gp = rec;
  if (lane == kGCap) gp = rec + offsetof(HeadState, capacity) / 4;
  if (lane == kGPatch) gp = rec + offsetof(HeadState, patch_size) / 4;
  if (lane == kGBf) gp = rec + offsetof(HeadState, block_frames) / 4;
  if (lane == kGT || lane == kGT + 1) gp = reinterpret_cast<const int32_t *>(t_vals) + (lane - kGT);
  if (lane == kGW && weights) gp = reinterpret_cast<const int32_t *>(weights);
  if (lane == kGNg || lane == kGNg + 1) gp = num_groups + hs0 + (lane == kGNg ? 0 : s1);
  if ((lane == kGWs || lane == kGWs + 1) && weight_sum)
    gp = reinterpret_cast<const int32_t *>(weight_sum + hs0 + (lane == kGWs ? 0 : s1));
  uint32_t rw = static_cast<uint32_t>(*gp);
  __builtin_amdgcn_sched_barrier(0);

  const int FSEQ = a.FSEQ, D = a.D, MTPA = a.MTPA, MMA = mma, W = a.width;
  const int cols = W / p, grid_ng = FSEQ / (p * p);
  const pkv_merge_layer &ml = a.ml;
  const MergeLane ln0(a, tile * kEvTiles);
  const int c = ln0.c, is_v = ln0.is_v;
  int g[kEvTiles];
  bool own[kEvTiles];
#pragma unroll
  for (int j = 0; j < kEvTiles; ++j) {
    const MergeLane ln(a, tile * kEvTiles + j);
    g[j] = ln.g;
    own[j] = ln.own;
  }
  const bool meta_lane = !is_v && c == 0;  // writes the group's count and positions
  // (loaded through a buffer resource of the head's frame: 32-bit offsets)
  const __amdgpu_buffer_rsrc_t srsrc = buf_rsrc(
      reinterpret_cast<const char *>(is_v ? a.src.v : a.src.k) + static_cast<uint64_t>(h) * a.src_hb,
      static_cast<int>((FSEQ - 1) * a.src_tb + D * 2));
  uint4 x[kEvTiles][kTok];
#pragma unroll
  for (int j = 0; j < kEvTiles; ++j) {
    const int gc = min(g[j], grid_ng - 1);
    const int gbase = (gc / cols) * p * W + (gc % cols) * p;
#pragma unroll
    for (int m = 0; m < kTok; ++m) x[j][m] = bld16_nt(srsrc, c * 2 + (gbase + (m / p) * W + m % p) * a.src_tb);
  }
  // the chunk loads stay issued ahead of the first use of the gather
  __builtin_amdgcn_sched_barrier(0);
  const int32_t kind = static_cast<int8_t>(lane_word(rw, kGKind) & 0xff);
  const int32_t cap = lane_word(rw, kGCap), pch = lane_word(rw, kGPatch), bf = lane_word(rw, kGBf);
  const int64_t t = static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(lane_word(rw, kGT + 1))) << 32) |
                                         static_cast<uint32_t>(lane_word(rw, kGT)));
  const float fw = weights ? __builtin_bit_cast(float, lane_word(rw, kGW)) : 1.0f;
  const int32_t ng0 = lane_word(rw, kGNg), ng1 = lane_word(rw, kGNg + 1);
  const float ws0 = weight_sum ? __builtin_bit_cast(float, lane_word(rw, kGWs)) : 0.0f;
  const float ws1 = weight_sum ? __builtin_bit_cast(float, lane_word(rw, kGWs + 1)) : 0.0f;
  VeilWords vw;
  vw.count = static_cast<uint32_t>(lane_word(rw, kVlCount));
  vw.id0 = lane_word(rw, kVlId);
  vw.id1 = lane_word(rw, kVlId + 1);
  vw.seen0 = static_cast<uint32_t>(lane_word(rw, kVlSeen));
  vw.seen1 = static_cast<uint32_t>(lane_word(rw, kVlSeen + 1));
  vw.done = static_cast<uint32_t>(lane_word(rw, kVlDone));

  const bool veil = kind == SK_MERGE && pch == p;
  VeilStep s;
  s.d = skip_desc();
  if (veil) s = veil_decide(vw, bf, cap, static_cast<int32_t>(t));
  const FrameDesc d = s.d;
  const int slot = d.accum_slot, is_new = d.is_new_block, fin = d.finalize_idx;
  const bool merging = veil && d.kind == PKV_DST_MERGE_ACCUM && slot >= 0 && slot < MMA;
  const int64_t hs = hs0 + (merging ? slot : 0);

  // Arrival as soon as every wave holds its gather: the head's last
  // workgroup to arrive knows that no workgroup of the head reads the
  // record, the slot counts or the weight sums any more (nor, in a block
  // begun by this call, the slot's group ids), so its write-back waits for
  // nothing but its own work; the arrival's round trip overlaps the reads
  // below.
  __syncthreads();
  int early = 0;
  if (tid == 0) early = atomicAdd(a.early + static_cast<int64_t>(h) * kArriveStride, 1);

  // a continued block: its slot's sums, anchor positions and stored group
  // ids, the ids verified against the grid by a block-wide vote
  float4 acc[kEvTiles][2];
  int64_t apos[kEvTiles][3] = {};
  int ng = grid_ng;
  float wsum = 0.0f + fw;
  bool fast = veil;
  if (merging && !is_new) {
    int4 ids[kEvIdLoads];
    const int n4 = FSEQ / 4;
#pragma unroll
    for (int k = 0; k < kEvIdLoads; ++k)
      ids[k] = reinterpret_cast<const int4 *>(ml.accum_group_ids + hs * FSEQ)[min(tid + k * kUpdThreads, n4 - 1)];
    float *acc_sum = is_v ? ml.accum_sum_v : ml.accum_sum_k;
#pragma unroll
    for (int j = 0; j < kEvTiles; ++j) {
      const float4 *ap = reinterpret_cast<const float4 *>(acc_sum + (hs * MTPA + min(g[j], MTPA - 1)) * D + c);
      acc[j][0] = ap[0];
      acc[j][1] = ap[1];
    }
    if (meta_lane && fin >= 0) {
#pragma unroll
      for (int j = 0; j < kEvTiles; ++j)
#pragma unroll
        for (int e = 0; e < 3; ++e) apos[j][e] = ml.accum_pos[(hs * MTPA + min(g[j], MTPA - 1)) * 3 + e];
    }
    ng = min(slot ? ng1 : ng0, MTPA);
    wsum = (slot ? ws1 : ws0) + fw;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < kEvIdLoads; ++k) {
      const int i = tid + k * kUpdThreads;
      if (i < n4) {
        int y = (4 * i) / W, xx = (4 * i) % W;
        const int32_t v[4] = {ids[k].x, ids[k].y, ids[k].z, ids[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bad |= v[e] != (y / p) * cols + xx / p;
          if (++xx == W) {
            xx = 0;
            ++y;
          }
        }
      }
    }
    if (tid == 0) sh.last = early;
    fast = ng == grid_ng && !__syncthreads_or(bad);
  } else {
    if (tid == 0) sh.last = early;
    __syncthreads();
  }
  const bool last = uni(sh.last) == a.n_merge - 1;
  if (last && tid == 0) atomicExch(a.early + static_cast<int64_t>(h) * kArriveStride, 0);
  int ticket = 0;
  if (!fast) {  // update_kernel's merge tiles, with their own arrival (same in every workgroup of the head)
    upd_merge_wg(a, sh, dyn, h, tile, ticket, kEvTiles);
    upd_finish(a, sh, h, tile, ticket);
    return;
  }

  // the head's last workgroup writes the record's Veil words, the
  // descriptor and the slot's group count and weight sum first (ahead of
  // its accumulator stores)
  if (last) {
    if (wave == 0) {
      veil_apply_wave(s, rw);
      if (lane < kVeilWords) reinterpret_cast<uint32_t *>(a.states + h)[kVeilWord0 + lane] = rw;
    }
    if (tid == 0) {
      store_desc(a.desc, h, 0, h, d);
      if (merging) {
        if (is_new) ml.accum_num_groups[hs] = ng;
        if (ml.accum_weight_sum) ml.accum_weight_sum[hs] = wsum;
      }
    }
  }

  if (merging) {
    float *acc_sum = is_v ? ml.accum_sum_v : ml.accum_sum_k;
#pragma unroll
    for (int j = 0; j < kEvTiles; ++j) {
      if (!own[j]) continue;
      const int gj = g[j];
      float ax[8];
      if (is_new) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ax[e] = 0.0f;
      } else {
        ax[0] = acc[j][0].x; ax[1] = acc[j][0].y; ax[2] = acc[j][0].z; ax[3] = acc[j][0].w;
        ax[4] = acc[j][1].x; ax[5] = acc[j][1].y; ax[6] = acc[j][1].z; ax[7] = acc[j][1].w;
      }
      if (gj < ng) {
#pragma unroll
        for (int m = 0; m < kTok; ++m) {
          const uint32_t xw[4] = {x[j][m].x, x[j][m].y, x[j][m].z, x[j][m].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            ax[2 * e] += fw * bf16_to_f32(static_cast<uint16_t>(xw[e] & 0xffff));
            ax[2 * e + 1] += fw * bf16_to_f32(static_cast<uint16_t>(xw[e] >> 16));
          }
        }
      }
      float4 *ap = reinterpret_cast<float4 *>(acc_sum + (hs * MTPA + gj) * D + c);
      ap[0] = make_float4(ax[0], ax[1], ax[2], ax[3]);
      ap[1] = make_float4(ax[4], ax[5], ax[6], ax[7]);
      const int64_t py = (gj / cols) * p, px = (gj % cols) * p;
      // a block begun here: the group ids of the group's members, one
      // member per K-side thread (no workgroup of the head reads them in
      // this call)
      if (is_new && !is_v && c < 8 * kTok && gj < ng)
        ml.accum_group_ids[hs * FSEQ + (gj / cols) * p * W + (gj % cols) * p + (c / 8 / p) * W + (c / 8) % p] = gj;
      if (is_new && meta_lane) {
        ml.accum_tokens_per_group[hs * MTPA + gj] =
            gj < ng ? static_cast<float>(kTok) * static_cast<float>(bf) : 0.0f;
        if (gj < ng) {
          int64_t *pp = ml.accum_pos + (hs * MTPA + gj) * 3;
          pp[0] = t;
          pp[1] = py;
          pp[2] = px;
        }
      }
      if (fin >= 0 && fin < a.MMB && gj < ng) {
        // count * sum(w) for weighted merges, else the reference's count * block_frames
        const float div = static_cast<float>(kTok) * (a.weights ? wsum : static_cast<float>(bf));
        const float inv = div > 0.0f ? 1.0f / div : 0.0f;
        const int64_t hp = static_cast<int64_t>(h) * a.MMB + fin;
        uint4 ox;
        ox.x = pack_bf16x2(ax[0] * inv, ax[1] * inv);
        ox.y = pack_bf16x2(ax[2] * inv, ax[3] * inv);
        ox.z = pack_bf16x2(ax[4] * inv, ax[5] * inv);
        ox.w = pack_bf16x2(ax[6] * inv, ax[7] * inv);
        st16_nt((is_v ? ml.merge_v : ml.merge_k) + (hp * MTPA + gj) * D + c, ox);  // not read again in the call
        if (meta_lane) {
          int64_t *mp = ml.merge_pos + (hp * MTPA + gj) * 3;
          mp[0] = is_new ? t : apos[j][0];
          mp[1] = is_new ? py : apos[j][1];
          mp[2] = is_new ? px : apos[j][2];
        }
      }
    }
    if (fin >= 0 && fin < a.MMB && tile == 0 && tid == 0) ml.merge_token_count[static_cast<int64_t>(h) * a.MMB + fin] = ng;
  }

}

// The decision words after a step (the values veil_apply gives lanes
// kVlCount, kVlId, kVlSeen and kVlDone), for the next frame's decision
__device__ inline void veil_advance(VeilWords &v, const VeilStep &s) {
  if (!s.changes()) return;
  v.count = (v.count & ~0xffu) | (static_cast<uint32_t>(s.cc) & 0xffu);
  v.id0 = s.id0;
  v.id1 = s.id1;
  v.seen0 = s.seen0;
  v.seen1 = s.seen1;
  v.done = (v.done & 0xffff0000u) | (static_cast<uint32_t>(s.done0) & 0xffu) |
           ((static_cast<uint32_t>(s.done1) & 0xffu) << 8);
}

// ---- Veil eviction of several frames per call (pkv_evict_merge, F > 1) ------
//
// Each workgroup takes one merge tile (8 groups at head_dim 128; a thread
// is a group, K or V and an 8-wide chunk, as in update_kernel's tiles)
// through all F frames, with its group's sums of both accumulator slots in
// registers: a slot's sums are read once (when its first use in the call
// continues a block) and stored once, after the last frame.  The frames'
// patch chunks stream through a ring of kEfRing frames of non-temporal
// loads, issued before anything is decided.  The Veil steps are decided in
// scalar registers frame by frame (every wave, the same); a first pass
// over them finds the slots whose first use continues a block, whose
// stored group ids are then verified against the grid by a block-wide vote
// (as in evict_kernel).  The head's last workgroup to arrive applies every
// step to the record's Veil words and writes them, the descriptors and the
// slots' group counts and weight sums.  A head this path does not cover
// (another strategy kind or patch size, a continued block off the grid)
// runs update_kernel's merge tile, the same in every workgroup of the
// head.  Sums are added frame by frame and member by member, as one frame
// per call adds them: the results equal F calls of one frame bit for bit.
constexpr int kEfRing = 2;

// Groups per workgroup of evict_frames_kernel: the workgroups of one call
// all run at once, three per compute unit, and those on a unit with three
// take longer than those on a unit with two (one frame's copies at a time
// per workgroup).  Of the tile sizes up to merge_tile_groups(D) whose
// workgroups fit in one round, the one with the fewest groups on the
// busiest unit (ties: the larger tile); at 12 heads of 420 groups on 256
// units, 7 groups (720 workgroups, 21 groups per busiest unit) rather than
// 8 (636, 24).
static int frames_tile_groups(int H, int MTPA, int D) {
  static int cus[64];
  int dev = 0;
  const int full = merge_tile_groups(D);
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return full;
  if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 0;
  const int64_t n_cu = cus[dev];
  if (n_cu <= 0) return full;
  int best = full;
  int64_t best_load = -1;
  for (int g = full; g >= (full + 1) / 2; --g) {
    const int64_t wgs = static_cast<int64_t>(H) * ((MTPA + g - 1) / g);
    if (wgs > 3 * n_cu) break;
    const int64_t load = (wgs + n_cu - 1) / n_cu * g;
    if (best_load < 0 || load < best_load) {
      best_load = load;
      best = g;
    }
  }
  return best;
}

__global__ void __launch_bounds__(kUpdThreads)
    evict_frames_kernel(const HeadState *states, const int64_t *t_vals, const float *weights,
                        const int32_t *num_groups, const float *weight_sum, int32_t n_merge, int32_t mma, UpdArgs a) {
  extern __shared__ __attribute__((aligned(16))) int32_t dyn[];
  __shared__ __attribute__((aligned(16))) UpdShared sh;
  constexpr int p = kPrePatch, kTok = kPreTok;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x / n_merge, tile = blockIdx.x % n_merge;
  const int64_t hs0 = static_cast<int64_t>(h) * mma;
  const int F = a.F;

  // one wave-wide gather: lane l < 39 reads Veil word l of the record, the
  // next lanes the record's kind, capacity, patch and block frames and the
  // slots' group counts and weight sums (absent inputs read a stand-in)
  constexpr int kGKind = kVeilWords, kGCap = kGKind + 1, kGPatch = kGKind + 2, kGBf = kGKind + 3,
                kGNg = kGKind + 4, kGWs = kGKind + 6;
  static_assert(kGWs + 2 <= 64, "one gathered value per lane");
  const int32_t *rec = reinterpret_cast<const int32_t *>(states + h);
  const int32_t *gp = rec + kVeilWord0 + min(lane, kVeilWords - 1);
  const int s1 = min(1, mma - 1);
  if (lane == kGKind) gp = rec;
  if (lane == kGCap) gp = rec + offsetof(HeadState, capacity) / 4;
  if (lane == kGPatch) gp = rec + offsetof(HeadState, patch_size) / 4;
  if (lane == kGBf) gp = rec + offsetof(HeadState, block_frames) / 4;
  if (lane == kGNg || lane == kGNg + 1) gp = num_groups + hs0 + (lane == kGNg ? 0 : s1);
  if ((lane == kGWs || lane == kGWs + 1) && weight_sum)
    gp = reinterpret_cast<const int32_t *>(weight_sum + hs0 + (lane == kGWs ? 0 : s1));
  uint32_t rw = static_cast<uint32_t>(*gp);
  // frame f's time and weight in lane f (read with readlane: no load, and
  // so no wait, in the frame loop, whose waits would also wait for the
  // frames in flight)
  static_assert(kUpdMaxFrames <= 64, "one frame per lane");
  const int64_t t_lane = t_vals[min(lane, F - 1)];
  const float w_lane = weights ? weights[min(lane, F - 1)] : 1.0f;
  __builtin_amdgcn_sched_barrier(0);

  const int FSEQ = a.FSEQ, D = a.D, MTPA = a.MTPA, W = a.width;
  const int cols = W / p, grid_ng = FSEQ / (p * p);
  const pkv_merge_layer &ml = a.ml;
  // a tile is gpt groups (the host's choice, at most merge_tile_groups(D)):
  // lanes of the wave pairs' groups past gpt idle (no copies, no writes)
  const int cpt = D / 8, gpw = 64 / cpt;
  const int gpt = (MTPA + n_merge - 1) / n_merge;
  const int local = (wave >> 1) * gpw + lane / cpt;
  const int g = tile * gpt + local, c = (lane % cpt) * 8;
  const int is_v = uni(wave & 1);  // wave-uniform: a scalar buffer resource, no per-lane loop
  const bool own = lane / cpt < gpw && local < gpt && g < MTPA;
  const bool meta_lane = own && !is_v && c == 0;  // writes the group's count and positions
  // the group's members in every frame, copied into this wave's ring
  // slots in LDS (the dynamic LDS, which only the fallback path uses
  // otherwise): slot r of wave w holds member m of every lane at
  // ((r * 4 + w) * kTok + m) * 1 KB, lane l at +16 l.  One buffer resource
  // over the head's rows of all F frames (32-bit offsets).
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 srsrc;
  {
    const uint64_t addr = reinterpret_cast<uint64_t>(reinterpret_cast<const char *>(is_v ? a.src.v : a.src.k) +
                                                     static_cast<uint64_t>(h) * a.src_hb);
    srsrc[0] = static_cast<int>(addr & 0xffffffffu);
    srsrc[1] = static_cast<int>((addr >> 32) & 0xffffu);
    srsrc[2] = static_cast<int>(static_cast<int64_t>(F - 1) * a.src_fb + static_cast<int64_t>(FSEQ - 1) * a.src_tb +
                                D * 2);
    srsrc[3] = kRsrcWord3;
  }
  uint32_t toff[kTok];
  {
    const int gc = min(g, grid_ng - 1);
    const int gbase = (gc / cols) * p * W + (gc % cols) * p;
    // an idle lane's offset lies past the resource's end (the frames' bytes
    // are below 2^31): its copies read zeros and fetch nothing
#pragma unroll
    for (int m = 0; m < kTok; ++m)
      toff[m] = local < gpt ? c * 2 + (gbase + (m / p) * W + m % p) * a.src_tb : 0x80000000u;
  }
  const int wave_s = uni(wave);
  typedef __attribute__((address_space(3))) char lds_char_t;
  const uint32_t ring0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char_t *)dyn));
  // frame f (the last frame past the end) into ring slot r: kTok copies
  auto copy_frame = [&](int f, int r) {
    const uint32_t fo = static_cast<uint32_t>(min(f, F - 1)) * a.src_fb;
#pragma unroll
    for (int m = 0; m < kTok; ++m) {
      const uint32_t lds = ring0 + static_cast<uint32_t>(((r * 4 + wave_s) * kTok + m) * 1024);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                   :
                   : "s"(lds), "v"(fo + toff[m]), "s"(srsrc)
                   : "memory", "m0");
#pragma clang diagnostic pop
    }
  };
  auto ring_read = [&](int r, int m) {
    return *reinterpret_cast<const uint4 *>(reinterpret_cast<const char *>(dyn) +
                                            ((r * 4 + wave_s) * kTok + m) * 1024 + lane * 16);
  };
#pragma unroll
  for (int r = 0; r < kEfRing; ++r) copy_frame(r, r);
  __builtin_amdgcn_sched_barrier(0);

  const int32_t kind = static_cast<int8_t>(lane_word(rw, kGKind) & 0xff);
  const int32_t cap = lane_word(rw, kGCap), pch = lane_word(rw, kGPatch), bf = lane_word(rw, kGBf);
  const int32_t ng0 = lane_word(rw, kGNg), ng1 = lane_word(rw, kGNg + 1);
  const float ws0 = weight_sum ? __builtin_bit_cast(float, lane_word(rw, kGWs)) : 0.0f;
  const float ws1 = weight_sum ? __builtin_bit_cast(float, lane_word(rw, kGWs + 1)) : 0.0f;
  VeilWords vw;
  vw.count = static_cast<uint32_t>(lane_word(rw, kVlCount));
  vw.id0 = lane_word(rw, kVlId);
  vw.id1 = lane_word(rw, kVlId + 1);
  vw.seen0 = static_cast<uint32_t>(lane_word(rw, kVlSeen));
  vw.seen1 = static_cast<uint32_t>(lane_word(rw, kVlSeen + 1));
  vw.done = static_cast<uint32_t>(lane_word(rw, kVlDone));
  const bool veil = kind == SK_MERGE && pch == p;

  auto frame_t = [&](int f) {
    const uint64_t u = static_cast<uint64_t>(t_lane);
    return static_cast<int64_t>(
        (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), f))) << 32) |
        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), f)));
  };
  auto frame_w = [&](int f) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w_lane), f)); };

  // the slots whose first use in the call continues a block: only a slot
  // holding a block at the start can, so the steps are followed only until
  // each such slot's first use is known
  uint32_t cont = 0;
  if (veil) {
    VeilWords v = vw;
    uint32_t open = (vw.id0 != -1 ? 1u : 0u) | (vw.id1 != -1 && mma > 1 ? 2u : 0u);
    for (int f = 0; f < F && open; ++f) {
      const VeilStep s = veil_decide(v, bf, cap, static_cast<int32_t>(frame_t(f)));
      veil_advance(v, s);
      const int sl = s.d.accum_slot;
      if (!s.changes() || sl < 0 || sl >= mma || !(open & (1u << sl))) continue;
      if (!s.d.is_new_block) cont |= 1u << sl;
      open &= ~(1u << sl);
    }
  }

  // arrival as soon as every wave holds its gather (evict_kernel's
  // protocol): no workgroup of the head reads the record, the slot counts
  // or the weight sums after it; the stored group ids read below are
  // rewritten in this call only with the grid's ids, which they hold
  __syncthreads();
  int early = 0;
  if (tid == 0) early = atomicAdd(a.early + static_cast<int64_t>(h) * kArriveStride, 1);

  float ax[2][8];
  int64_t apos[2][3] = {};
  bool fast = veil;
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
    for (int e = 0; e < 8; ++e) ax[sl][e] = 0.0f;
    if (!(cont & (1u << sl))) continue;
    const int64_t hs = hs0 + sl;
    int4 ids[kEvIdLoads];
    const int n4 = FSEQ / 4;
#pragma unroll
    for (int k = 0; k < kEvIdLoads; ++k)
      ids[k] = reinterpret_cast<const int4 *>(ml.accum_group_ids + hs * FSEQ)[min(tid + k * kUpdThreads, n4 - 1)];
    const float *acc_sum = is_v ? ml.accum_sum_v : ml.accum_sum_k;
    const float4 *ap = reinterpret_cast<const float4 *>(acc_sum + (hs * MTPA + min(g, MTPA - 1)) * D + c);
    const float4 a0 = ap[0], a1 = ap[1];
    ax[sl][0] = a0.x; ax[sl][1] = a0.y; ax[sl][2] = a0.z; ax[sl][3] = a0.w;
    ax[sl][4] = a1.x; ax[sl][5] = a1.y; ax[sl][6] = a1.z; ax[sl][7] = a1.w;
    if (meta_lane) {
#pragma unroll
      for (int e = 0; e < 3; ++e) apos[sl][e] = ml.accum_pos[(hs * MTPA + min(g, MTPA - 1)) * 3 + e];
    }
    bool bad = min(sl ? ng1 : ng0, MTPA) != grid_ng;
#pragma unroll
    for (int k = 0; k < kEvIdLoads; ++k) {
      const int i = tid + k * kUpdThreads;
      if (i < n4) {
        int y = (4 * i) / W, xx = (4 * i) % W;
        const int32_t v[4] = {ids[k].x, ids[k].y, ids[k].z, ids[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bad |= v[e] != (y / p) * cols + xx / p;
          if (++xx == W) {
            xx = 0;
            ++y;
          }
        }
      }
    }
    fast = fast && !__syncthreads_or(bad);
  }
  if (tid == 0) sh.last = early;
  __syncthreads();
  const bool last = uni(sh.last) == a.n_merge - 1;
  if (last && tid == 0) atomicExch(a.early + static_cast<int64_t>(h) * kArriveStride, 0);
  if (!fast) {  // update_kernel's merge tile, with its own arrival (same in every workgroup of the head)
    __builtin_amdgcn_s_waitcnt(0xf70);  // vmcnt(0): the ring's copies landed before the tile reuses its LDS
    __syncthreads();
    int ticket = 0;
    upd_merge_wg(a, sh, dyn, h, tile, ticket, 1);
    upd_finish(a, sh, h, tile, ticket);
    return;
  }

  // every load so far complete here, once: the frame loop's waits are then
  // for the frames in flight only (a wait in the loop for a load from
  // before it would also wait for every frame issued since)
  __builtin_amdgcn_s_waitcnt(0xf70);  // vmcnt(0)
  static_assert(kMaxMergeBlocks < 15, "finalize index in four bits");
  VeilWords v = vw;
  uint32_t dec = 0;
  float wsum[2] = {ws0, ws1};
  int64_t tpos[2] = {0, 0};
  bool fresh[2] = {false, false};  // the slot's block began in this call (positions from tpos)
  uint32_t touched = 0;
  const int64_t py = (g / cols) * p, px = (g % cols) * p;
  for (int f0 = 0; f0 < F; f0 += kEfRing) {
#pragma unroll
    for (int r = 0; r < kEfRing; ++r) {
      const int f = f0 + r;
      if (f >= F) break;
      const int64_t t = frame_t(f);
      const float fw = frame_w(f);
      // frame f's copies complete: the (kEfRing - 1) frames after it may be in flight
      __builtin_amdgcn_s_waitcnt((((kEfRing - 1) * kTok) & 15) | (7 << 4) | (15 << 8) | ((((kEfRing - 1) * kTok) >> 4) << 14));
      asm volatile("" ::: "memory");
      uint4 xr[kTok];
#pragma unroll
      for (int m = 0; m < kTok; ++m) xr[m] = ring_read(r, m);
      VeilStep st;
      st.d = skip_desc();
      if (veil) st = veil_decide(v, bf, cap, static_cast<int32_t>(t));
      veil_advance(v, st);
      const FrameDesc d = st.d;
      const int slot = d.accum_slot, is_new = d.is_new_block, fin = d.finalize_idx;
      const bool merging = d.kind == PKV_DST_MERGE_ACCUM && slot >= 0 && slot < mma;
      // frame f's step in lane f, for the descriptors: changed (bit 0), slot
      // (bit 1), new block (bit 2), finalize index + 1 (bits 4..7)
      if (lane == f && d.kind == PKV_DST_MERGE_ACCUM)
        dec = 1u | (static_cast<uint32_t>(slot & 1) << 1) | (static_cast<uint32_t>(is_new) << 2) |
              (static_cast<uint32_t>(fin + 1) << 4);
      // a completed block enters the record's FIFO (the only step that
      // changes its arrays; the other words are set from the last step)
      if (last && wave_s == 0 && fin >= 0) veil_apply_wave(st, rw);
      auto on_slot = [&](auto sl_c) {
        constexpr int sl = decltype(sl_c)::value;
        const int64_t hs = hs0 + sl;
        if (is_new) {
#pragma unroll
          for (int e = 0; e < 8; ++e) ax[sl][e] = 0.0f;
          wsum[sl] = 0.0f;
          tpos[sl] = t;
          fresh[sl] = true;
        }
        touched |= 1u << sl;
        wsum[sl] = wsum[sl] + fw;
        if (!own) return;
        if (g < grid_ng) {
#pragma unroll
          for (int m = 0; m < kTok; ++m) {
            const uint32_t xw[4] = {xr[m].x, xr[m].y, xr[m].z, xr[m].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              ax[sl][2 * e] += fw * bf16_to_f32(static_cast<uint16_t>(xw[e] & 0xffff));
              ax[sl][2 * e + 1] += fw * bf16_to_f32(static_cast<uint16_t>(xw[e] >> 16));
            }
          }
        }
        // a block begun here: the group ids of the group's members (one
        // member per K-side thread), its count and anchor positions
        if (is_new && !is_v && c < 8 * kTok && g < grid_ng)
          ml.accum_group_ids[hs * FSEQ + (g / cols) * p * W + (g % cols) * p + (c / 8 / p) * W + (c / 8) % p] = g;
        if (is_new && meta_lane) {
          ml.accum_tokens_per_group[hs * MTPA + g] =
              g < grid_ng ? static_cast<float>(kTok) * static_cast<float>(bf) : 0.0f;
          if (g < grid_ng) {
            int64_t *pp = ml.accum_pos + (hs * MTPA + g) * 3;
            pp[0] = t;
            pp[1] = py;
            pp[2] = px;
          }
        }
        if (fin >= 0 && fin < a.MMB && g < grid_ng) {
          // count * sum(w) for weighted merges, else the reference's count * block_frames
          const float div = static_cast<float>(kTok) * (a.weights ? wsum[sl] : static_cast<float>(bf));
          const float inv = div > 0.0f ? 1.0f / div : 0.0f;
          const int64_t hp = static_cast<int64_t>(h) * a.MMB + fin;
          uint4 ox;
          ox.x = pack_bf16x2(ax[sl][0] * inv, ax[sl][1] * inv);
          ox.y = pack_bf16x2(ax[sl][2] * inv, ax[sl][3] * inv);
          ox.z = pack_bf16x2(ax[sl][4] * inv, ax[sl][5] * inv);
          ox.w = pack_bf16x2(ax[sl][6] * inv, ax[sl][7] * inv);
          // (non-temporal, as the sums below: results nothing in the launch
          // reads again; kept dirty in L2 they were written back at the
          // launch's end, after the last workgroup)
          st16_nt((is_v ? ml.merge_v : ml.merge_k) + (hp * MTPA + g) * D + c, ox);
          if (meta_lane) {
            int64_t *mp = ml.merge_pos + (hp * MTPA + g) * 3;
            mp[0] = fresh[sl] ? tpos[sl] : apos[sl][0];
            mp[1] = fresh[sl] ? py : apos[sl][1];
            mp[2] = fresh[sl] ? px : apos[sl][2];
          }
        }
      };
      if (merging) {
        if (slot) on_slot(std::integral_constant<int, 1>());
        else on_slot(std::integral_constant<int, 0>());
        if (fin >= 0 && fin < a.MMB && tile == 0 && tid == 0) ml.merge_token_count[static_cast<int64_t>(h) * a.MMB + fin] = grid_ng;
      }
      // ring slot r takes frame f + kEfRing (the last frame again past the
      // end: the same number of copies every frame keeps the waits exact),
      // once this wave's reads of the slot are complete
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      copy_frame(f + kEfRing, r);
    }
  }

  __builtin_amdgcn_s_waitcnt(0xf70);  // vmcnt(0): no copy lands in LDS after the workgroup ends
  // the slots' sums, once
  if (own) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      if (!(touched & (1u << sl))) continue;
      float *acc_sum = is_v ? ml.accum_sum_v : ml.accum_sum_k;
      float4 *ap = reinterpret_cast<float4 *>(acc_sum + ((hs0 + sl) * MTPA + g) * D + c);
      st16_nt(ap, make_uint4(__float_as_uint(ax[sl][0]), __float_as_uint(ax[sl][1]), __float_as_uint(ax[sl][2]),
                             __float_as_uint(ax[sl][3])));
      st16_nt(ap + 1, make_uint4(__float_as_uint(ax[sl][4]), __float_as_uint(ax[sl][5]), __float_as_uint(ax[sl][6]),
                                 __float_as_uint(ax[sl][7])));
    }
  }
  if (last) {
    // the record's words after the last step, and the frames' descriptors
    // (lane f writes frame f's)
    if (wave_s == 0) {
      if (lane == kVlCount) rw = (rw & ~0xffu) | (v.count & 0xffu);
      if (lane == kVlId) rw = static_cast<uint32_t>(v.id0);
      if (lane == kVlId + 1) rw = static_cast<uint32_t>(v.id1);
      if (lane == kVlSeen) rw = v.seen0;
      if (lane == kVlSeen + 1) rw = v.seen1;
      if (lane == kVlDone) rw = (rw & 0xffff0000u) | (v.done & 0xffffu);
      if (lane < kVeilWords) reinterpret_cast<uint32_t *>(a.states + h)[kVeilWord0 + lane] = rw;
      if (lane < F) {
        FrameDesc fd = skip_desc();
        if (dec & 1u) {
          fd.kind = PKV_DST_MERGE_ACCUM;
          fd.accum_slot = static_cast<int>((dec >> 1) & 1u);
          fd.is_new_block = static_cast<int>((dec >> 2) & 1u);
          fd.finalize_idx = static_cast<int>(dec >> 4) - 1;
          fd.local_idx = static_cast<int32_t>(t_lane) % bf;  // veil_decide's local index
        }
        store_desc(a.desc, h * F + lane, lane, h, fd);
      }
    }
    if (tid == 0) {
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        if (!(touched & (1u << sl))) continue;
        if (fresh[sl]) ml.accum_num_groups[hs0 + sl] = grid_ng;
        if (ml.accum_weight_sum) ml.accum_weight_sum[hs0 + sl] = wsum[sl];
      }
    }
  }
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

// Workspace of pkv_evict_merge: per head the two-level arrival counters of
// update_kernel's merge tiles (kArriveFan + 1 lines) and the eviction
// kernel's arrival counter (one line), each a 128-byte line.
static int64_t evict_ws_bytes(int H) {
  return static_cast<int64_t>(H) * (kArriveFan + 2) * kArriveStride * 4;
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

// Workspace of pkv_cache_update: the 8 descriptor arrays ([H*F] int32 each,
// 256-byte aligned) and the arrival counters (kArriveFan + 1 per head, one
// 128-byte line each).
static int64_t update_ws_bytes(int H, int F) {
  return 8 * align_up(static_cast<int64_t>(H) * F * 4, 256) +
         static_cast<int64_t>(H) * (kArriveFan + 1) * kArriveStride * 4;
}

int64_t pkv_cache_update_workspace_size(const pkv_geometry *geo, int32_t frames) {
  if (!geo || frames <= 0) return 0;
  return update_ws_bytes(geo->num_heads, frames);
}

int pkv_cache_update(const pkv_geometry *geo, const pkv_pools *pools, const pkv_update_args *a,
                     pkv_stream_t stream) {
  int rc = check_geometry(geo);
  if (rc) return rc;
  if (!pools || !a || !a->new_k || !a->new_v || !a->states_layer || !a->sink_caps_layer ||
      !a->committed_vc_layer || !a->workspace)
    return fail(PKV_ERR_INVALID, "cache_update: NULL argument");
  const int H = geo->num_heads, FSEQ = geo->frame_seqlen, D = geo->head_dim, F = a->frames;
  if (a->layer < 0 || a->layer >= geo->num_layers) return fail(PKV_ERR_INVALID, "cache_update: layer out of range");
  if (F <= 0 || F > geo->max_recent)
    return fail(PKV_ERR_UNSUPPORTED, "cache_update: frames per block (%d) must be in [1, max_recent=%d]", F,
                geo->max_recent);
  if (F > kUpdMaxFrames)
    return fail(PKV_ERR_UNSUPPORTED, "cache_update: %d frames per block exceed %d", F, kUpdMaxFrames);
  if (a->spatial_width <= 0) return fail(PKV_ERR_INVALID, "cache_update: spatial_width must be > 0");
  if (D / 8 > kUpdThreads) return fail(PKV_ERR_UNSUPPORTED, "cache_update: head_dim %d exceeds %d", D, 8 * kUpdThreads);
  const int64_t l = a->layer;
  const int MMA = geo->max_merge_active, MMB = geo->max_merge_blocks, MTPA = geo->max_merge_tokens;
  // merge heads: bit h of merge_heads, bit 63 standing for every head >= 63
  uint64_t mh_mask = a->merge_heads;
  if (H < 64) mh_mask &= (uint64_t{1} << H) - 1;
  const int n_mh = __builtin_popcountll(mh_mask & ~(uint64_t{1} << 63)) + ((mh_mask >> 63) & 1 ? H - 63 : 0);
  const bool merge = a->pass_kind == 1 && n_mh > 0;
  const int cpt = D / 8, per_tile = kUpdThreads / cpt;
  UpdArgs u;
  u.states = reinterpret_cast<HeadState *>(a->states_layer);
  u.sink_caps = a->sink_caps_layer;
  u.committed_vc = a->committed_vc_layer;
  u.vc = pools->valid_count + l * H * 3;
  u.src = FrameSrc{a->new_k, a->new_v, static_cast<int64_t>(FSEQ) * a->tok_stride, a->head_stride, a->tok_stride};
  u.pools = pool_ptrs(geo, pools);
  u.ml.accum_sum_k = pools->merge_accum_sum_k + l * H * MMA * MTPA * D;
  u.ml.accum_sum_v = pools->merge_accum_sum_v + l * H * MMA * MTPA * D;
  u.ml.accum_pos = pools->merge_accum_pos + l * H * MMA * MTPA * 3;
  u.ml.accum_group_ids = pools->merge_accum_group_ids + l * H * MMA * FSEQ;
  u.ml.accum_tokens_per_group = pools->merge_accum_tokens_per_group + l * H * MMA * MTPA;
  u.ml.accum_num_groups = pools->merge_accum_num_groups + l * H * MMA;
  u.ml.accum_weight_sum = pools->merge_accum_weight_sum ? pools->merge_accum_weight_sum + l * H * MMA : nullptr;
  u.ml.merge_k = pools->merge_k + l * H * MMB * MTPA * D;
  u.ml.merge_v = pools->merge_v + l * H * MMB * MTPA * D;
  u.ml.merge_pos = pools->merge_pos + l * H * MMB * MTPA * 3;
  u.ml.merge_token_count = pools->merge_token_count + l * H * MMB;
  char *w = static_cast<char *>(a->workspace);
  const int64_t dbytes = align_up(static_cast<int64_t>(H) * F * 4, 256);
  int32_t *dw[8];
  for (int i = 0; i < 8; ++i) dw[i] = reinterpret_cast<int32_t *>(w + i * dbytes);
  u.desc = pkv_state_desc{dw[0], dw[1], dw[2], dw[3], dw[4], dw[5], dw[6], dw[7]};
  u.arrive = reinterpret_cast<int32_t *>(w + 8 * dbytes);
  u.early = nullptr;
  const int64_t src_bytes = static_cast<int64_t>(F) * FSEQ * a->tok_stride * 2;
  const int64_t max_slots = std::max(std::max(geo->max_sink, geo->max_middle), geo->max_recent);
  if (src_bytes >= (int64_t{1} << 31) || max_slots * FSEQ * D * 2 >= (int64_t{1} << 31))
    return fail(PKV_ERR_UNSUPPORTED, "cache_update: the new frames or one head's pool exceed 2 GiB");
  u.src_fb = static_cast<uint32_t>(static_cast<int64_t>(FSEQ) * a->tok_stride * 2);
  u.src_hb = static_cast<uint32_t>(a->head_stride * 2);
  u.src_tb = static_cast<uint32_t>(a->tok_stride * 2);
  u.t0 = a->t0;
  u.t_vals = nullptr;
  u.weights = nullptr;
  u.counters = 1;
  u.layer = a->layer; u.H = H; u.F = F; u.FSEQ = FSEQ; u.D = D; u.width = a->spatial_width;
  u.max_sink = geo->max_sink; u.max_middle = geo->max_middle; u.max_recent = geo->max_recent;
  u.MMA = MMA; u.MMB = MMB; u.MTPA = MTPA;
  u.pass_kind = a->pass_kind; u.shift_pending = a->shift_pending;
  u.n_scat = (FSEQ + per_tile - 1) / per_tile;
  u.n_merge = 0;
  u.n_mh = merge ? n_mh : 0;
  u.merge_heads = mh_mask;
  size_t smem = 0;
  if (merge) {
    if (FSEQ > kMaxMergeFseq)
      return fail(PKV_ERR_UNSUPPORTED, "cache_update: frame_seqlen %d exceeds %d", FSEQ, kMaxMergeFseq);
    if (MTPA > kMaxMergeGroups)
      return fail(PKV_ERR_UNSUPPORTED, "cache_update: %d tokens per anchor exceed %d", MTPA, kMaxMergeGroups);
    if (MMA > kMaxMergeSlots)
      return fail(PKV_ERR_UNSUPPORTED, "cache_update: %d active merge blocks exceed %d", MMA, kMaxMergeSlots);
    if (D / 8 > 64) return fail(PKV_ERR_UNSUPPORTED, "cache_update: merges need head_dim <= 512, got %d", D);
    const int gpt = merge_tile_groups(D);
    u.n_merge = (MTPA + gpt - 1) / gpt;
    smem = static_cast<size_t>(merge_lds_words(FSEQ, MMA)) * sizeof(int32_t);
    if (smem > 65536 && hipFuncSetAttribute(reinterpret_cast<const void *>(update_kernel),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(smem)) != hipSuccess)
      return fail(PKV_ERR_HIP, "cache_update: cannot reserve %zu bytes of LDS", smem);
  }
  hipLaunchKernelGGL(update_kernel, dim3(u.n_mh * u.n_merge + H * u.n_scat), dim3(kUpdThreads), smem, as_stream(stream),
                     u);
  return check_launch("update_kernel");
}

int pkv_evict_merge(uint8_t *states, int32_t H, int32_t F, int32_t FSEQ, int32_t D, int32_t MMA, int32_t MMB,
                    int32_t MTPA, const int64_t *t_vals, const uint16_t *new_k, const uint16_t *new_v,
                    int32_t spatial_width, const float *frame_weights, const pkv_state_desc *desc,
                    const pkv_merge_layer *ml, void *workspace, pkv_stream_t stream) {
  if (H == 0 || F == 0) return PKV_OK;
  if (!states || !t_vals || !new_k || !new_v || !desc || !ml || !workspace || H < 0 || F < 0 || FSEQ <= 0 ||
      D <= 0 || MMA <= 0 || MMB <= 0 || MTPA <= 0)
    return fail(PKV_ERR_INVALID, "evict_merge: bad arguments");
  if (!desc->dst_kind || !desc->dst_slot || !desc->src_frame || !desc->src_head || !desc->merge_accum_slot ||
      !desc->merge_local_idx || !desc->merge_finalize_completed_idx || !desc->merge_is_new_block)
    return fail(PKV_ERR_INVALID, "evict_merge: NULL descriptor array");
  if (frame_weights && !ml->accum_weight_sum)
    return fail(PKV_ERR_INVALID, "evict_merge: weighted merge needs accum_weight_sum");
  if (spatial_width <= 0) return fail(PKV_ERR_INVALID, "evict_merge: spatial_width must be > 0");
  if (F > kUpdMaxFrames) return fail(PKV_ERR_UNSUPPORTED, "evict_merge: %d frames exceed %d", F, kUpdMaxFrames);
  if (D % 8 != 0 || D / 8 > 64)
    return fail(PKV_ERR_UNSUPPORTED, "evict_merge: head_dim %d must be a multiple of 8, at most 512", D);
  if (FSEQ > kMaxMergeFseq)
    return fail(PKV_ERR_UNSUPPORTED, "evict_merge: frame_seqlen %d exceeds %d", FSEQ, kMaxMergeFseq);
  if (MTPA > kMaxMergeGroups)
    return fail(PKV_ERR_UNSUPPORTED, "evict_merge: %d tokens per anchor exceed %d", MTPA, kMaxMergeGroups);
  if (MMA > kMaxMergeSlots)
    return fail(PKV_ERR_UNSUPPORTED, "evict_merge: %d active merge blocks exceed %d", MMA, kMaxMergeSlots);
  if (static_cast<int64_t>(F) * H * FSEQ * D * 2 >= (int64_t{1} << 31))
    return fail(PKV_ERR_UNSUPPORTED, "evict_merge: the new frames exceed 2 GiB");
  int32_t *arrive = static_cast<int32_t *>(workspace);
  UpdArgs u{};
  u.states = reinterpret_cast<HeadState *>(states);
  u.src = FrameSrc{new_k, new_v, static_cast<int64_t>(H) * FSEQ * D, static_cast<int64_t>(FSEQ) * D, D};
  u.ml = *ml;
  u.desc = *desc;
  u.arrive = arrive;
  u.early = arrive + static_cast<int64_t>(H) * (kArriveFan + 1) * kArriveStride;
  u.src_fb = static_cast<uint32_t>(static_cast<int64_t>(H) * FSEQ * D * 2);
  u.src_hb = static_cast<uint32_t>(static_cast<int64_t>(FSEQ) * D * 2);
  u.src_tb = static_cast<uint32_t>(D * 2);
  u.t0 = 0;
  u.t_vals = t_vals;
  u.weights = frame_weights;
  u.counters = 0;
  u.H = H; u.F = F; u.FSEQ = FSEQ; u.D = D; u.width = spatial_width;
  u.MMA = MMA; u.MMB = MMB; u.MTPA = MTPA;
  u.pass_kind = 1;
  u.n_scat = 0;
  u.n_mh = H;
  u.merge_heads = H >= 64 ? ~uint64_t{0} : (uint64_t{1} << H) - 1;
  // frames on a grid of 2 x 2 patches: evict_kernel (one frame) or
  // evict_frames_kernel (several), which still run update_kernel's merge
  // tile for heads their path does not cover
  auto al16 = [](const void *q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  const int W = spatial_width;
  const bool grid = MMA <= 2 && W <= FSEQ && FSEQ % W == 0 && W % 2 == 0 && (FSEQ / W) % 2 == 0 &&
                    FSEQ / 4 <= MTPA && FSEQ <= kEvMaxFseq && D >= 8 * kPreTok && al16(new_k) && al16(new_v) &&
                    al16(ml->accum_sum_k) && al16(ml->accum_sum_v) && al16(ml->accum_group_ids);
  const bool one = grid && F == 1, many = grid && F > 1;
  int gpt = one ? evict_tile_groups(D) : merge_tile_groups(D);
  if (many) gpt = frames_tile_groups(H, MTPA, D);
  u.n_merge = (MTPA + gpt - 1) / gpt;
  const void *kern = one ? reinterpret_cast<const void *>(evict_kernel)
                         : many ? reinterpret_cast<const void *>(evict_frames_kernel)
                                : reinterpret_cast<const void *>(update_kernel);
  size_t smem = static_cast<size_t>(merge_lds_words(FSEQ, MMA)) * sizeof(int32_t);
  if (many) smem = std::max(smem, static_cast<size_t>(kEfRing) * (kUpdThreads / 64) * kPreTok * 1024);
  if (smem > 65536 &&
      hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)) != hipSuccess)
    return fail(PKV_ERR_HIP, "evict_merge: cannot reserve %zu bytes of LDS", smem);
  if (one) {
    hipLaunchKernelGGL(evict_kernel, dim3(H * u.n_merge), dim3(kUpdThreads), smem, as_stream(stream), u.states,
                       u.t_vals, u.weights, u.ml.accum_num_groups, u.ml.accum_weight_sum, u.n_merge, u.MMA, u);
    return check_launch("evict_kernel");
  }
  if (many) {
    hipLaunchKernelGGL(evict_frames_kernel, dim3(H * u.n_merge), dim3(kUpdThreads), smem, as_stream(stream),
                       u.states, u.t_vals, u.weights, u.ml.accum_num_groups, u.ml.accum_weight_sum, u.n_merge, u.MMA,
                       u);
    return check_launch("evict_frames_kernel");
  }
  hipLaunchKernelGGL(update_kernel, dim3(H * u.n_merge), dim3(kUpdThreads), smem, as_stream(stream), u);
  return check_launch("update_kernel");
}

int64_t pkv_evict_merge_workspace_size(int32_t num_heads) {
  return num_heads > 0 ? evict_ws_bytes(num_heads) : 0;
}

}  // extern "C"
