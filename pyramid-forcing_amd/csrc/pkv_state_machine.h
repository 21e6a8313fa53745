// Per-(layer, head) strategy state machines: Wave (cyclic), Anchor (stride),
// lag and Veil (merge).  One thread owns one HeadState and walks the frames
// of a block in order.  Semantics follow
// pyramidkv/csrc/anchor_store_update.cu:43-231 (and its Python mirror
// pyramidkv/_mega_state_ref.py:116-236), including the completed-FIFO
// slot-id shift on merge eviction (anchor_store_update.cu:196-214).
#pragma once

#include "pkv_common.h"

namespace pkv {

struct FrameDesc {
  int32_t kind, slot, accum_slot, local_idx, finalize_idx, is_new_block;
};

__device__ inline FrameDesc skip_desc() { return FrameDesc{PKV_DST_SKIP, -1, -1, -1, -1, 0}; }

// Wave: phase = t % period, ring of bucket_cap entries per phase
// (anchor_store_update.cu:43-61).
__device__ inline FrameDesc sm_cyclic(HeadState &s, int32_t t) {
  if (s.period <= 0 || s.period > kMaxPhase || s.bucket_cap <= 0 || t < 0) return skip_desc();
  const int32_t phase = t % s.period;
  const int32_t cursor = s.cyclic_cursor[phase];
  const int32_t slot = phase * s.bucket_cap + cursor;
  if (cursor < 0 || slot >= kMaxPhase * kMaxBucket) return skip_desc();
  s.cyclic_slot[slot] = slot;
  s.cyclic_t[slot] = t;
  s.cyclic_cursor[phase] = static_cast<int8_t>((cursor + 1) % s.bucket_cap);
  FrameDesc d = skip_desc();
  d.kind = PKV_DST_MIDDLE;
  d.slot = slot;
  return d;
}

// Anchor (stride) and lag: ring FIFO keyed by t; stride keeps only
// t % interval == 0 (anchor_store_update.cu:63-110).
__device__ inline FrameDesc sm_tkeyed(HeadState &s, int32_t t, bool filter) {
  if (s.capacity <= 0 || (filter && s.interval <= 0)) return skip_desc();
  if (filter && (t % s.interval) != 0) return skip_desc();
  const int32_t slot = s.tkey_head;
  if (slot < 0 || slot >= kMaxTKeyed) return skip_desc();
  s.tkey_head = static_cast<int8_t>((slot + 1) % s.capacity);
  if (s.tkey_count < s.capacity) s.tkey_count = static_cast<int8_t>(s.tkey_count + 1);
  s.tkey_slot[slot] = slot;
  s.tkey_t[slot] = t;
  FrameDesc d = skip_desc();
  d.kind = PKV_DST_MIDDLE;
  d.slot = slot;
  return d;
}

__device__ inline void clear_active(HeadState &s, int a) {
  s.merge_active_block_id[a] = -1;
  for (int j = 0; j < kMaxMergeBlockFrames; ++j) s.merge_active_seen[a][j] = 0;
  s.merge_active_complete_count[a] = 0;
}

// Guards on out-of-range parameters (period, capacities, slot ids) turn a
// frame into SKIP where the reference would index past the record; the
// host-side state builders reject such parameters before they get here.
//
// Veil: block = t / block_frames; find or allocate an accumulating slot
// (evicting slot 0 when both are busy), drop duplicates, finalize into the
// completed FIFO when every frame of the block was seen
// (anchor_store_update.cu:122-231).
__device__ inline FrameDesc sm_merge(HeadState &s, int32_t t) {
  if (s.block_frames <= 0) return skip_desc();
  if (s.block_frames > kMaxMergeBlockFrames || s.capacity <= 0 || s.capacity > kMaxMergeBlocks || t < 0)
    return skip_desc();
  const int32_t block_id = t / s.block_frames;
  const int32_t local_idx = t % s.block_frames;
  int32_t a = -1;
  for (int i = 0; i < kMaxMergeActive; ++i)
    if (s.merge_active_block_id[i] == block_id) { a = i; break; }
  int32_t is_new = 0;
  if (a == -1) {
    for (int i = 0; i < kMaxMergeActive; ++i)
      if (s.merge_active_block_id[i] == -1) { a = i; break; }
    if (a == -1) {
      a = 0;
      clear_active(s, 0);
    }
    clear_active(s, a);
    s.merge_active_block_id[a] = block_id;
    is_new = 1;
  }
  if (s.merge_active_seen[a][local_idx] != 0) return skip_desc();
  s.merge_active_seen[a][local_idx] = 1;
  s.merge_active_complete_count[a] = static_cast<int8_t>(s.merge_active_complete_count[a] + 1);

  int32_t fin = -1;
  if (s.merge_active_complete_count[a] >= s.block_frames) {
    const int32_t start_t = block_id * s.block_frames;
    const int32_t end_t = start_t + s.block_frames - 1;
    const int32_t median_t = (start_t + end_t) / 2;
    int32_t idx;
    if (s.merge_completed_count < s.capacity) {
      idx = s.merge_completed_count;
      s.merge_completed_count = static_cast<int8_t>(s.merge_completed_count + 1);
    } else {
      for (int i = 1; i < s.capacity; ++i) {
        s.merge_completed_slot[i - 1] = s.merge_completed_slot[i];
        s.merge_completed_block_id[i - 1] = s.merge_completed_block_id[i];
        s.merge_completed_start_t[i - 1] = s.merge_completed_start_t[i];
        s.merge_completed_end_t[i - 1] = s.merge_completed_end_t[i];
        s.merge_completed_median_t[i - 1] = s.merge_completed_median_t[i];
      }
      idx = s.capacity - 1;
    }
    s.merge_completed_slot[idx] = idx;
    s.merge_completed_block_id[idx] = block_id;
    s.merge_completed_start_t[idx] = start_t;
    s.merge_completed_end_t[idx] = end_t;
    s.merge_completed_median_t[idx] = median_t;
    s.merge_active_block_id[a] = -1;
    for (int j = 0; j < kMaxMergeBlockFrames; ++j) s.merge_active_seen[a][j] = 0;
    s.merge_active_complete_count[a] = 0;
    fin = idx;
  }
  FrameDesc d;
  d.kind = PKV_DST_MERGE_ACCUM;
  d.slot = -1;
  d.accum_slot = a;
  d.local_idx = local_idx;
  d.finalize_idx = fin;
  d.is_new_block = is_new;
  return d;
}

__device__ inline FrameDesc sm_step(HeadState &s, int32_t t) {
  switch (s.kind) {
    case SK_CYCLIC: return sm_cyclic(s, t);
    case SK_STRIDE: return sm_tkeyed(s, t, true);
    case SK_LAG: return sm_tkeyed(s, t, false);
    case SK_MERGE: return sm_merge(s, t);
    default: return skip_desc();
  }
}

// Write the 8 descriptor outputs of frame f of head h (index h*F+f).
__device__ inline void store_desc(const pkv_state_desc &o, int idx, int f, int h, const FrameDesc &d) {
  o.dst_kind[idx] = d.kind;
  o.dst_slot[idx] = d.slot;
  o.src_frame[idx] = f;
  o.src_head[idx] = h;
  o.merge_accum_slot[idx] = d.accum_slot;
  o.merge_local_idx[idx] = d.local_idx;
  o.merge_finalize_completed_idx[idx] = d.finalize_idx;
  o.merge_is_new_block[idx] = d.is_new_block;
}

// Run the state machine of head h over t_vals[0..F) (pass 1 = clean);
// noisy passes emit SKIP and leave the state untouched
// (anchor_store_update.cu:257-269).  The record is processed in place.
__device__ inline void run_head(HeadState *states, int h, const int64_t *t_vals, int F,
                                int pass_kind, const pkv_state_desc &out) {
  HeadState &s = states[h];
  for (int f = 0; f < F; ++f) {
    FrameDesc d = skip_desc();
    if (pass_kind == 1) d = sm_step(s, static_cast<int32_t>(t_vals[f]));
    store_desc(out, h * F + f, f, h, d);
  }
}

}  // namespace pkv
