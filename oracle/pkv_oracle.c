/*
 * pkv_oracle.c -- CPU restatement of the reference's pyramid KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels: it may be built and called by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg, and by nothing else.  The product path never
 * links or calls it.
 *
 * Every function restates one piece of IF-LAB-PKU/Pyramid-Forcing (paths
 * relative to the reference's pyramidkv/ directory) in the loop structure of
 * the reference, not of the HIP kernels, so that a mismatch between the two
 * shows up as a parity failure:
 *   orc_state_update  csrc/anchor_store_update.cu:43-313 (+ _mega_state_ref.py)
 *   orc_plan_multi    csrc/mega_plan.cc:63-80, 133-264, 513-616
 *   orc_pack          csrc/pyramidkv_pack.cu:28-185
 *   orc_update_frames csrc/pyramidkv_update.cu:21-110
 *   orc_merge_accum   csrc/mega_merge_accum.cu:52-252 (fp32, same add order)
 *   orc_rope_apply    rope.py:18-68 with the pack kernel's fp32 formula
 * Built with -ffp-contract=off: products and sums are rounded one at a time.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define MAX_PHASE 6
#define MAX_BUCKET 4
#define MAX_TKEYED 24
#define MAX_LAG 4
#define MAX_MBLOCKS 6
#define MAX_MACTIVE 2
#define MAX_MFRAMES 4

enum { SK_RECENT = 0, SK_CYCLIC = 1, SK_STRIDE = 2, SK_LAG = 3, SK_MERGE = 4 };
enum { DST_SKIP = -1, DST_MIDDLE = 1, DST_MERGE = 5 };

/* anchor_store.cuh:62-132 */
typedef struct {
  int8_t kind, sink_capacity, pad0[2];
  int32_t period, bucket_cap, interval, capacity, patch_size, block_frames;
  int32_t lag_offsets[MAX_LAG];
  int32_t lag_offset_count;
  int32_t cyclic_slot[MAX_PHASE * MAX_BUCKET];
  int32_t cyclic_t[MAX_PHASE * MAX_BUCKET];
  int8_t cyclic_cursor[MAX_PHASE];
  int32_t tkey_slot[MAX_TKEYED];
  int32_t tkey_t[MAX_TKEYED];
  int8_t tkey_count, tkey_head, pad1[2];
  int32_t mc_slot[MAX_MBLOCKS], mc_block[MAX_MBLOCKS], mc_start[MAX_MBLOCKS], mc_end[MAX_MBLOCKS],
      mc_median[MAX_MBLOCKS];
  int8_t mc_count, pad2[3];
  int32_t ma_block[MAX_MACTIVE], ma_slot[MAX_MACTIVE];
  int8_t ma_seen[MAX_MACTIVE][MAX_MFRAMES];
  int8_t ma_count[MAX_MACTIVE], pad3[2];
  int32_t cached_num_groups;
} State;

_Static_assert(sizeof(State) == 600, "PerHeadState is 600 bytes");

int64_t orc_state_size(void) { return (int64_t)sizeof(State); }

static float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round-to-nearest-even, NaN -> 0x7fc0 */
static uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* ---------------- state machine (anchor_store_update.cu) ---------------- */

typedef struct {
  int32_t kind, slot, accum, local, fin, isnew;
} Desc;

static Desc d_skip(void) {
  Desc d = {DST_SKIP, -1, -1, -1, -1, 0};
  return d;
}

static Desc upd_cyclic(State *s, int32_t t) { /* :43-61 */
  int32_t phase = t % s->period;
  int32_t cursor = s->cyclic_cursor[phase];
  int32_t slot = phase * s->bucket_cap + cursor;
  Desc d = d_skip();
  s->cyclic_slot[slot] = slot;
  s->cyclic_t[slot] = t;
  s->cyclic_cursor[phase] = (int8_t)((cursor + 1) % s->bucket_cap);
  d.kind = DST_MIDDLE;
  d.slot = slot;
  return d;
}

static Desc upd_stride_or_lag(State *s, int32_t t, int stride) { /* :63-110 */
  Desc d = d_skip();
  int32_t slot;
  if (stride && t % s->interval != 0) return d;
  slot = s->tkey_head;
  s->tkey_head = (int8_t)((slot + 1) % s->capacity);
  if (s->tkey_count < s->capacity) s->tkey_count = (int8_t)(s->tkey_count + 1);
  s->tkey_slot[slot] = slot;
  s->tkey_t[slot] = t;
  d.kind = DST_MIDDLE;
  d.slot = slot;
  return d;
}

static Desc upd_merge(State *s, int32_t t) { /* :122-231 */
  Desc d = d_skip();
  int32_t block_id, local_idx, accum = -1, isnew = 0, fin = -1;
  int i, j;
  if (s->block_frames <= 0) return d;
  block_id = t / s->block_frames;
  local_idx = t % s->block_frames;
  for (i = 0; i < MAX_MACTIVE; ++i)
    if (s->ma_block[i] == block_id) { accum = i; break; }
  if (accum == -1) {
    for (i = 0; i < MAX_MACTIVE; ++i)
      if (s->ma_block[i] == -1) { accum = i; break; }
    if (accum == -1) {
      accum = 0;
      s->ma_block[0] = -1;
      for (j = 0; j < MAX_MFRAMES; ++j) s->ma_seen[0][j] = 0;
      s->ma_count[0] = 0;
    }
    s->ma_block[accum] = block_id;
    for (j = 0; j < MAX_MFRAMES; ++j) s->ma_seen[accum][j] = 0;
    s->ma_count[accum] = 0;
    isnew = 1;
  }
  if (s->ma_seen[accum][local_idx] != 0) return d; /* duplicate -> SKIP */
  s->ma_seen[accum][local_idx] = 1;
  s->ma_count[accum] = (int8_t)(s->ma_count[accum] + 1);
  if (s->ma_count[accum] >= s->block_frames) {
    int32_t start_t = block_id * s->block_frames;
    int32_t end_t = start_t + s->block_frames - 1;
    int32_t median_t = (start_t + end_t) / 2;
    int32_t idx;
    if (s->mc_count < s->capacity) {
      idx = s->mc_count;
      s->mc_count = (int8_t)(s->mc_count + 1);
    } else {
      for (i = 1; i < s->capacity; ++i) {
        s->mc_slot[i - 1] = s->mc_slot[i];
        s->mc_block[i - 1] = s->mc_block[i];
        s->mc_start[i - 1] = s->mc_start[i];
        s->mc_end[i - 1] = s->mc_end[i];
        s->mc_median[i - 1] = s->mc_median[i];
      }
      idx = s->capacity - 1;
    }
    s->mc_slot[idx] = idx;
    s->mc_block[idx] = block_id;
    s->mc_start[idx] = start_t;
    s->mc_end[idx] = end_t;
    s->mc_median[idx] = median_t;
    s->ma_block[accum] = -1;
    for (j = 0; j < MAX_MFRAMES; ++j) s->ma_seen[accum][j] = 0;
    s->ma_count[accum] = 0;
    fin = idx;
  }
  d.kind = DST_MERGE;
  d.slot = -1;
  d.accum = accum;
  d.local = local_idx;
  d.fin = fin;
  d.isnew = isnew;
  return d;
}

/* desc: 8 arrays of H*F int32 back to back, in the order dst_kind, dst_slot,
 * src_frame, src_head, merge_accum_slot, merge_local_idx,
 * merge_finalize_completed_idx, merge_is_new_block (:233-313). */
void orc_state_update(uint8_t *states, int H, const int64_t *t_vals, int F, int pass_kind, int32_t *desc) {
  int h, f;
  const int N = H * F;
  for (h = 0; h < H; ++h) {
    State *s = (State *)(states + (size_t)h * sizeof(State));
    for (f = 0; f < F; ++f) {
      const int i = h * F + f;
      Desc d = d_skip();
      if (pass_kind == 1) {
        const int32_t t = (int32_t)t_vals[f];
        switch (s->kind) {
          case SK_CYCLIC: d = upd_cyclic(s, t); break;
          case SK_STRIDE: d = upd_stride_or_lag(s, t, 1); break;
          case SK_LAG: d = upd_stride_or_lag(s, t, 0); break;
          case SK_MERGE: d = upd_merge(s, t); break;
          default: break;
        }
      }
      desc[0 * N + i] = d.kind;
      desc[1 * N + i] = d.slot;
      desc[2 * N + i] = f;
      desc[3 * N + i] = h;
      desc[4 * N + i] = d.accum;
      desc[5 * N + i] = d.local;
      desc[6 * N + i] = d.fin;
      desc[7 * N + i] = d.isnew;
    }
  }
}

/* ---------------- planner (mega_plan.cc) ---------------- */

int64_t orc_map_sink_time(int64_t t, int mode, int cmin, int cmax, int lag) { /* :63-80 */
  if (mode == 1) {
    int64_t delta = t;
    int64_t out;
    if (delta < cmin) delta = cmin;
    if (delta > cmax) delta = cmax;
    out = t - delta;
    return out < 0 ? 0 : out;
  } else {
    int64_t out = t - lag;
    return out < 0 ? 0 : out;
  }
}

/* One layer.  vc [H,3] int64, mtc [H,MMB] int32.  Outputs as in
 * mega_plan_multi (:513-654): cu [C*H+1]; per-segment arrays [C*H*S].
 * Returns the packed-token total. */
int32_t orc_plan_multi(int H, int FSEQ, int max_sink, int max_middle, int max_recent, int MMB,
                       const uint8_t *states, const int64_t *vc, const int32_t *mtc, const int64_t *t_list,
                       int C, int sink_mode, int cmin, int cmax, int lag, int32_t *cu, int32_t *sk, int32_t *sg,
                       int32_t *sl, int32_t *dst, int64_t *traw, int64_t *tremap) {
  const int S = max_sink + max_middle + max_recent + MMB;
  const int N = C * H * S;
  int32_t run = 0;
  int c, h, i;
  for (i = 0; i < N; ++i) {
    sk[i] = -1; sg[i] = 0; sl[i] = 0; dst[i] = 0; traw[i] = -1; tremap[i] = -1;
  }
  for (i = 0; i < C * H + 1; ++i) cu[i] = 0;
  cu[0] = 0;
  for (c = 0; c < C; ++c) {
    const int64_t t_c = t_list[c];
    const int64_t sync_t = orc_map_sink_time(t_c, sink_mode, cmin, cmax, lag);
    for (h = 0; h < H; ++h) { /* emit_chunk_plan :154-262 */
      const State *s = (const State *)(states + (size_t)h * sizeof(State));
      const int base = c * H * S + h * S;
      int fp = 0;
      const int thresh = s->sink_capacity;
      const int recent_min_t = 2147483647;
      const int n_sink_raw = (int)vc[h * 3 + 0];
      const int n_sink = (thresh > 0 && thresh < n_sink_raw) ? thresh : n_sink_raw;
      const int n_recent = (int)vc[h * 3 + 2];
      int q, r;
      for (q = 0; q < n_sink && q < max_sink; ++q) {
        const int j = base + fp;
        sk[j] = 0; sg[j] = h * max_sink + q; sl[j] = FSEQ; dst[j] = run;
        traw[j] = q; tremap[j] = sync_t;
        run += FSEQ; ++fp;
      }
      for (r = 0; r < n_recent && r < max_recent; ++r) {
        const int j = base + fp;
        sk[j] = 2; sg[j] = h * max_recent + r; sl[j] = FSEQ; dst[j] = run;
        traw[j] = -1; tremap[j] = -1;
        run += FSEQ; ++fp;
      }
      if (s->kind == SK_CYCLIC) {
        const int period = s->period > 0 ? s->period : 1;
        const int bcap = s->bucket_cap > 0 ? s->bucket_cap : 1;
        const int phase = (int)(((t_c % period) + period) % period);
        const int b0 = phase * MAX_BUCKET;
        const int b1 = b0 + (bcap < MAX_BUCKET ? bcap : MAX_BUCKET);
        for (i = b0; i < b1; ++i) {
          int j;
          if (s->cyclic_slot[i] < 0) continue;
          if (s->cyclic_t[i] < thresh) continue;
          if (s->cyclic_t[i] >= recent_min_t) continue;
          j = base + fp;
          sk[j] = 1; sg[j] = h * max_middle + i; sl[j] = FSEQ; dst[j] = run;
          traw[j] = s->cyclic_t[i]; tremap[j] = sync_t;
          run += FSEQ; ++fp;
          if (fp >= S) break;
        }
      } else if (s->kind == SK_STRIDE || s->kind == SK_LAG) {
        const int tc = s->tkey_count;
        for (i = 0; i < tc && i < MAX_TKEYED; ++i) {
          int j;
          if (s->tkey_t[i] < thresh) continue;
          if (s->tkey_t[i] >= recent_min_t) continue;
          j = base + fp;
          sk[j] = 1; sg[j] = h * max_middle + i; sl[j] = FSEQ; dst[j] = run;
          traw[j] = s->tkey_t[i]; tremap[j] = (s->kind == SK_STRIDE) ? sync_t : -1;
          run += FSEQ; ++fp;
          if (fp >= S) break;
        }
      }
      if (s->kind == SK_MERGE) {
        const int mcc = s->mc_count;
        for (i = 0; i < mcc && i < MAX_MBLOCKS; ++i) {
          const int slot = s->mc_slot[i];
          int32_t tok;
          int j;
          if (slot < 0 || slot >= MMB) continue;
          if (s->mc_start[i] <= 0) continue;
          if (s->mc_end[i] >= recent_min_t) continue;
          tok = mtc[h * MMB + slot];
          if (tok <= 0) continue;
          if (fp >= S) break;
          j = base + fp;
          sk[j] = 3; sg[j] = h * MMB + slot; sl[j] = tok; dst[j] = run;
          traw[j] = 0; tremap[j] = s->mc_median[i];
          run += tok; ++fp;
        }
      }
      cu[c * H + h + 1] = run;
    }
  }
  return run;
}

/* ---------------- pack + RoPE (pyramidkv_pack.cu) ---------------- */

/* (kr*fr - ki*fi, kr*fi + ki*fr), each op rounded to fp32 (:154-160). */
static void rot_pair(uint16_t kr16, uint16_t ki16, float fr, float fi, uint16_t *outr, uint16_t *outi) {
  const float kr = bf2f(kr16), ki = bf2f(ki16);
  const float a = kr * fr, b = ki * fi, c = kr * fi, d = ki * fr;
  *outr = f2bf(a - b);
  *outi = f2bf(c + d);
}

static int clamp_row(int64_t v, int rows) {
  int r = (int)v;
  if (r < 0) r = 0;
  if (r >= rows) r = rows - 1;
  return r;
}

static void rope_row(const uint16_t *src, uint16_t *dst, int D, int64_t t, int64_t y, int64_t x, const float *ft,
                     int ft_rows, int ft_cols, const float *fy, int fy_rows, int fy_cols, const float *fx,
                     int fx_rows, int fx_cols) {
  const int half = D / 2;
  int p;
  for (p = 0; p < half; ++p) {
    float fr, fi;
    if (p < ft_cols) {
      const int row = clamp_row(t, ft_rows);
      fr = ft[row * ft_cols * 2 + p * 2];
      fi = ft[row * ft_cols * 2 + p * 2 + 1];
    } else if (p < ft_cols + fy_cols) {
      const int row = clamp_row(y, fy_rows);
      const int col = p - ft_cols;
      fr = fy[row * fy_cols * 2 + col * 2];
      fi = fy[row * fy_cols * 2 + col * 2 + 1];
    } else {
      const int row = clamp_row(x, fx_rows);
      const int col = p - ft_cols - fy_cols;
      fr = fx[row * fx_cols * 2 + col * 2];
      fi = fx[row * fx_cols * 2 + col * 2 + 1];
    }
    rot_pair(src[2 * p], src[2 * p + 1], fr, fi, &dst[2 * p], &dst[2 * p + 1]);
  }
}

/* pools: K/V pointers per kind (0 sink, 1 middle, 2 recent, 3 merge), pos
 * pointers per kind (nullable).  rope applied when tremap && ft. */
void orc_pack(const uint16_t *const *pk, const uint16_t *const *pv, const int64_t *const *ppos, int FSEQ, int MTPA,
              int D, const int32_t *sk, const int32_t *sg, const int32_t *sl, const int32_t *dst, int n_seg,
              const int64_t *tremap, const float *ft, int ft_rows, int ft_cols, const float *fy, int fy_rows,
              int fy_cols, const float *fx, int fx_rows, int fx_cols, uint16_t *k_out, uint16_t *v_out,
              int64_t *pos_out) {
  int seg;
  for (seg = 0; seg < n_seg; ++seg) {
    const int kind = sk[seg];
    int len, stride, tok;
    const uint16_t *src_k, *src_v;
    const int64_t *src_p = NULL;
    int fuse;
    int64_t tr;
    if (kind < 0) continue;
    len = sl[seg];
    if (len <= 0) continue;
    stride = (kind == 3) ? MTPA : FSEQ;
    src_k = pk[kind] + (int64_t)sg[seg] * stride * D;
    src_v = pv[kind] + (int64_t)sg[seg] * stride * D;
    if (ppos[kind]) src_p = ppos[kind] + (int64_t)sg[seg] * stride * 3;
    fuse = (tremap != NULL) && (ft != NULL) && (src_p != NULL);
    tr = fuse ? tremap[seg] : -1;
    for (tok = 0; tok < len; ++tok) {
      const uint16_t *kr = src_k + (int64_t)tok * D;
      uint16_t *ko = k_out + ((int64_t)dst[seg] + tok) * D;
      if (fuse) {
        int64_t t = src_p[tok * 3 + 0];
        if (tr >= 0) t = tr;
        rope_row(kr, ko, D, t, src_p[tok * 3 + 1], src_p[tok * 3 + 2], ft, ft_rows, ft_cols, fy, fy_rows, fy_cols,
                 fx, fx_rows, fx_cols);
      } else {
        memcpy(ko, kr, (size_t)D * 2);
      }
      memcpy(v_out + ((int64_t)dst[seg] + tok) * D, src_v + (int64_t)tok * D, (size_t)D * 2);
    }
    if (pos_out && src_p) memcpy(pos_out + (int64_t)dst[seg] * 3, src_p, (size_t)len * 3 * 8);
  }
}

void orc_rope_apply(const uint16_t *k, const int64_t *pos, int64_t n, int D, const float *ft, int ft_rows,
                    int ft_cols, const float *fy, int fy_rows, int fy_cols, const float *fx, int fx_rows,
                    int fx_cols, uint16_t *out) {
  int64_t i;
  for (i = 0; i < n; ++i)
    rope_row(k + i * D, out + i * D, D, pos[i * 3], pos[i * 3 + 1], pos[i * 3 + 2], ft, ft_rows, ft_cols, fy,
             fy_rows, fy_cols, fx, fx_rows, fx_cols);
}

/* ---------------- frame copy (pyramidkv_update.cu) ---------------- */

/* Kinds 0 / 1 / 2 name the sink / middle / recent pool; every other kind
 * (SKIP -1, and MERGE 5, which the reference's caller masks to -1 before the
 * op, _mega_cache.py:358-362) writes nothing, and so do slots outside the
 * pool (nslots[kind]) and sources outside [F, H].  Within that domain this
 * is the reference kernel's copy. */
void orc_update_frames(const uint16_t *new_k, const uint16_t *new_v, const int64_t *new_pos, int F, int H, int FSEQ,
                       int D, uint16_t *const *pk, uint16_t *const *pv, int64_t *const *ppos, const int64_t *nslots,
                       const int32_t *kind, const int32_t *slot_global, const int32_t *src_frame,
                       const int32_t *src_head, int n) {
  int op;
  for (op = 0; op < n; ++op) {
    const int k = kind[op];
    int64_t src, dstb;
    if (k < 0 || k > 2) continue;
    if (slot_global[op] < 0 || slot_global[op] >= nslots[k] || src_frame[op] < 0 || src_frame[op] >= F ||
        src_head[op] < 0 || src_head[op] >= H)
      continue;
    src = ((int64_t)src_frame[op] * H + src_head[op]) * FSEQ * D;
    dstb = (int64_t)slot_global[op] * FSEQ * D;
    memcpy(pk[k] + dstb, new_k + src, (size_t)FSEQ * D * 2);
    memcpy(pv[k] + dstb, new_v + src, (size_t)FSEQ * D * 2);
    if (new_pos && ppos[k])
      memcpy(ppos[k] + (int64_t)slot_global[op] * FSEQ * 3,
             new_pos + ((int64_t)src_frame[op] * H + src_head[op]) * FSEQ * 3, (size_t)FSEQ * 3 * 8);
  }
}

/* ---------------- Veil merge accumulate (mega_merge_accum.cu) ------------
 * One layer.  Loop structure of the reference kernel: frames in order, for
 * each head and dim the tokens in ascending order with one fp32 add into
 * the token's group accumulator (:193-209).  weights (nullable [F]) scale
 * each frame's contribution and turn the divisor into count * sum(w); the
 * reference operation is weights == NULL.  awsum (nullable) keeps the running
 * sum of the block's frame weights, 1 per frame without weights, so that
 * weighted and unweighted calls can continue each other's blocks.  The finalize uses the IEEE
 * reciprocal 1/div (the reference's --use_fast_math reciprocal is
 * approximate; 1/16 is exact either way). */
void orc_merge_accum(const uint8_t *states, int H, int F, int FSEQ, int D, int MMA, int MMB, int MTPA,
                     const uint16_t *new_k, const uint16_t *new_v, const int64_t *new_pos, const int32_t *dkind,
                     const int32_t *dslot, const int32_t *dfin, const int32_t *dnew, const float *weights,
                     float *sum_k, float *sum_v, int64_t *apos, int32_t *agid, float *atpg, int32_t *ang,
                     float *awsum, uint16_t *mk, uint16_t *mv, int64_t *mpos, int32_t *mtc) {
  int h, f, t, d, g;
  for (h = 0; h < H; ++h) {
    const State *s = (const State *)(states + (size_t)h * sizeof(State));
    const int32_t bf = s->block_frames;
    for (f = 0; f < F; ++f) {
      const int di = h * F + f;
      const int kind = dkind[di], slot = dslot[di], isnew = dnew[di], fin = dfin[di];
      const int64_t hs = (int64_t)h * MMA + slot;
      const int64_t pbase = ((int64_t)f * H + h) * FSEQ * 3;
      const float w = weights ? weights[f] : 1.0f;
      if (kind != DST_MERGE || slot < 0) continue;
      if (isnew) { /* :100-184 */
        const int32_t p = s->patch_size;
        int32_t maxy = -1, maxx = -1, cols, rows, ng;
        for (g = 0; g < MTPA; ++g)
          for (d = 0; d < D; ++d) {
            sum_k[(hs * MTPA + g) * D + d] = 0.0f;
            sum_v[(hs * MTPA + g) * D + d] = 0.0f;
          }
        for (t = 0; t < FSEQ; ++t) {
          const int32_t y = (int32_t)new_pos[pbase + t * 3 + 1], x = (int32_t)new_pos[pbase + t * 3 + 2];
          if (y > maxy) maxy = y;
          if (x > maxx) maxx = x;
        }
        cols = (maxx >= 0 && p > 0) ? (maxx / p + 1) : 1;
        rows = (maxy >= 0 && p > 0) ? (maxy / p + 1) : 1;
        ng = rows * cols;
        if (ng > MTPA) ng = MTPA;
        ang[hs] = ng;
        if (awsum) awsum[hs] = 0.0f;
        for (g = 0; g < MTPA; ++g) atpg[hs * MTPA + g] = 0.0f;
        for (t = 0; t < FSEQ; ++t) {
          const int32_t y = (int32_t)new_pos[pbase + t * 3 + 1], x = (int32_t)new_pos[pbase + t * 3 + 2];
          const int32_t py = p > 0 ? y / p : 0, px = p > 0 ? x / p : 0;
          int32_t gid = py * cols + px;
          if (gid < 0 || gid >= ng) gid = 0;
          agid[hs * FSEQ + t] = gid;
          atpg[hs * MTPA + gid] += 1.0f;
        }
        for (g = 0; g < ng; ++g) atpg[hs * MTPA + g] *= (float)bf;
        for (g = 0; g < ng; ++g) {
          apos[(hs * MTPA + g) * 3 + 0] = new_pos[pbase];
          apos[(hs * MTPA + g) * 3 + 1] = (g / cols) * p;
          apos[(hs * MTPA + g) * 3 + 2] = (g % cols) * p;
        }
      }
      { /* :193-209 */
        const int64_t kv = ((int64_t)f * H + h) * FSEQ;
        for (d = 0; d < D; ++d)
          for (t = 0; t < FSEQ; ++t) {
            const int32_t gid = agid[hs * FSEQ + t];
            const float kf = bf2f(new_k[(kv + t) * D + d]), vf = bf2f(new_v[(kv + t) * D + d]);
            if (weights) {
              sum_k[(hs * MTPA + gid) * D + d] += w * kf;
              sum_v[(hs * MTPA + gid) * D + d] += w * vf;
            } else {
              sum_k[(hs * MTPA + gid) * D + d] += kf;
              sum_v[(hs * MTPA + gid) * D + d] += vf;
            }
          }
        if (awsum) awsum[hs] += w;
      }
      if (fin >= 0) { /* :215-249 */
        const int32_t ng = ang[hs];
        const int64_t hp = (int64_t)h * MMB + fin;
        for (g = 0; g < ng; ++g) {
          float div;
          float inv;
          if (weights) {
            int32_t cnt = 0;
            for (t = 0; t < FSEQ; ++t) cnt += (agid[hs * FSEQ + t] == g);
            div = (float)cnt * awsum[hs];
          } else {
            div = atpg[hs * MTPA + g];
          }
          inv = div > 0.0f ? 1.0f / div : 0.0f;
          for (d = 0; d < D; ++d) {
            mk[(hp * MTPA + g) * D + d] = f2bf(sum_k[(hs * MTPA + g) * D + d] * inv);
            mv[(hp * MTPA + g) * D + d] = f2bf(sum_v[(hs * MTPA + g) * D + d] * inv);
          }
          mpos[(hp * MTPA + g) * 3 + 0] = apos[(hs * MTPA + g) * 3 + 0];
          mpos[(hp * MTPA + g) * 3 + 1] = apos[(hs * MTPA + g) * 3 + 1];
          mpos[(hp * MTPA + g) * 3 + 2] = apos[(hs * MTPA + g) * 3 + 2];
        }
        mtc[hp] = ng;
      }
    }
  }
}
