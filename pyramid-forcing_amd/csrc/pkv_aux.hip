// Data-movement ops of the reference's _ops.py surface and its legacy
// planner, for gfx950:
//   scatter_copy               pointer-list gather into a workspace (scatter_copy.cu:13-47)
//   apply_pos_override         pos[i, 0] = val over index ranges (scatter_copy.cu:53-71)
//   refresh_readout_layout     K/V gather + history time map + frame ids (scatter_copy.cu:77-168)
//   anchor_store_write_frames  frame -> store slot copy (scatter_copy.cu:170-225)
//   pyramidkv_plan             legacy 3-segment plan (pyramidkv_plan.cc:46-133), built on the device
//
// Copies move 16-byte vectors when the source, destination and length allow
// it (4-byte words, then bytes otherwise) and split every segment over
// several workgroups.  Descriptors that point outside the destination
// (checked against the extents the caller passes) are skipped instead of
// being followed.

#include "pkv_common.h"

namespace pkv {

constexpr int kAuxThreads = 256;
constexpr int kAuxSplit = 16;  // workgroups per segment (grid.y)

// Copy `bytes` bytes from src to dst; this workgroup handles the share
// selected by (part, parts).
__device__ inline void copy_share(const char *src, char *dst, int64_t bytes, int part, int parts) {
  const uintptr_t align = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                          static_cast<uintptr_t>(bytes);
  const int64_t step = static_cast<int64_t>(parts) * blockDim.x;
  const int64_t first = static_cast<int64_t>(part) * blockDim.x + threadIdx.x;
  if ((align & 15) == 0) {
    const uint4 *s = reinterpret_cast<const uint4 *>(src);
    uint4 *d = reinterpret_cast<uint4 *>(dst);
    const int64_t n = bytes / 16;
    // four loads in flight before the stores
    for (int64_t i = first; i < n; i += 4 * step) {
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (i + u * step < n) v[u] = s[i + u * step];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (i + u * step < n) d[i + u * step] = v[u];
    }
  } else if ((align & 3) == 0) {
    const int32_t *s = reinterpret_cast<const int32_t *>(src);
    int32_t *d = reinterpret_cast<int32_t *>(dst);
    const int64_t n = bytes / 4;
    for (int64_t i = first; i < n; i += step) d[i] = s[i];
  } else {
    for (int64_t i = first; i < bytes; i += step) dst[i] = src[i];
  }
}

__global__ void __launch_bounds__(kAuxThreads) scatter_copy_kernel(const int64_t *src_ptrs, const int64_t *lengths,
                                                                   const int64_t *offsets, int n, char *dst,
                                                                   int64_t dst_rows, int64_t row_bytes) {
  const int seg = blockIdx.x;
  if (seg >= n) return;
  const int64_t len = lengths[seg], off = offsets[seg];
  if (len <= 0 || off < 0 || off + len > dst_rows) return;
  const char *src = reinterpret_cast<const char *>(src_ptrs[seg]);
  copy_share(src, dst + off * row_bytes, len * row_bytes, blockIdx.y, gridDim.y);
}

__global__ void __launch_bounds__(kAuxThreads) pos_override_kernel(int64_t *pos, int64_t rows, const int64_t *starts,
                                                                   const int64_t *ends, const int64_t *vals, int m) {
  const int r = blockIdx.x;
  if (r >= m) return;
  int64_t s = starts[r], e = ends[r];
  const int64_t v = vals[r];
  if (s < 0) s = 0;
  if (e > rows) e = rows;
  for (int64_t i = s + static_cast<int64_t>(blockIdx.y) * blockDim.x + threadIdx.x; i < e;
       i += static_cast<int64_t>(gridDim.y) * blockDim.x)
    pos[i * 3] = v;
}

// history time map of refresh_readout_layout (scatter_copy.cu:138-160):
// mode 1 clamps the relative time, mode 2 compresses what exceeds the limit
// by the soft factor (round half to even), the result is clamped at 0
__device__ inline int64_t map_history_t(int64_t src_t, int64_t current_t, int mode, int64_t rel_max, float soft) {
  int64_t rel = current_t - src_t;
  if (rel < 0) rel = 0;
  int64_t mapped = src_t;
  if (mode == 1) {
    if (rel > rel_max) rel = rel_max;
    mapped = current_t - rel;
  } else if (mode == 2) {
    if (rel > rel_max) rel = rel_max + static_cast<int64_t>(rintf(__fmul_rn(static_cast<float>(rel - rel_max), soft)));
    mapped = current_t - rel;
  }
  return mapped < 0 ? 0 : mapped;
}

__global__ void __launch_bounds__(kAuxThreads) refresh_kernel(pkv_refresh_args a) {
  const int seg = blockIdx.x;
  if (seg >= a.n_segments) return;
  const int64_t len = a.lengths[seg], off = a.offsets[seg];
  if (len <= 0 || off < 0 || off + len > a.dst_rows) return;
  const char *sk = reinterpret_cast<const char *>(a.src_ptrs_k[seg]);
  const char *sv = reinterpret_cast<const char *>(a.src_ptrs_v[seg]);
  const int64_t *sp = reinterpret_cast<const int64_t *>(a.src_ptrs_pos[seg]);
  char *dk = static_cast<char *>(a.dst_k) + off * a.row_bytes;
  char *dv = static_cast<char *>(a.dst_v) + off * a.row_bytes;
  copy_share(sk, dk, len * a.row_bytes, blockIdx.y, gridDim.y);
  copy_share(sv, dv, len * a.row_bytes, blockIdx.y, gridDim.y);
  const int64_t flag = a.flags[seg];
  const bool do_map = (flag & 1) != 0, physical = (flag & 2) != 0, override_t = (flag & 4) != 0;
  const int64_t rope_t = a.dynamic_rope_t[seg];
  int64_t *op = a.dst_pos + off * 3;
  int64_t *of = a.dst_frame_ids + off;
  for (int64_t row = static_cast<int64_t>(blockIdx.y) * blockDim.x + threadIdx.x; row < len;
       row += static_cast<int64_t>(gridDim.y) * blockDim.x) {
    const int64_t src_t = sp[row * 3];
    int64_t t = src_t;
    if (override_t)
      t = rope_t;
    else if (do_map && a.history_relative_t_max > 0)
      t = map_history_t(src_t, a.current_t, a.history_mode_code, a.history_relative_t_max, a.history_soft_factor);
    op[row * 3] = t;
    op[row * 3 + 1] = sp[row * 3 + 1];
    op[row * 3 + 2] = sp[row * 3 + 2];
    of[row] = physical ? src_t : t;
  }
}

__global__ void __launch_bounds__(kAuxThreads) write_frames_kernel(const char *k_seq, const char *v_seq,
                                                                   const int64_t *pos_seq, int64_t src_frames,
                                                                   const int64_t *frame_desc, int n, char *store_k,
                                                                   char *store_v, int64_t *store_pos,
                                                                   int64_t capacity, int64_t frame_seqlen,
                                                                   int64_t row_bytes) {
  const int fr = blockIdx.x;
  if (fr >= n) return;
  const int64_t src_frame = frame_desc[2 * fr], slot = frame_desc[2 * fr + 1];
  if (src_frame < 0 || slot < 0 || src_frame >= src_frames || slot >= capacity) return;
  const int64_t fbytes = frame_seqlen * row_bytes;
  copy_share(k_seq + src_frame * fbytes, store_k + slot * fbytes, fbytes, blockIdx.y, gridDim.y);
  copy_share(v_seq + src_frame * fbytes, store_v + slot * fbytes, fbytes, blockIdx.y, gridDim.y);
  const int64_t *sp = pos_seq + src_frame * frame_seqlen * 3;
  int64_t *dp = store_pos + slot * frame_seqlen * 3;
  for (int64_t i = static_cast<int64_t>(blockIdx.y) * blockDim.x + threadIdx.x; i < frame_seqlen * 3;
       i += static_cast<int64_t>(gridDim.y) * blockDim.x)
    dp[i] = sp[i];
}

// Legacy plan: per (layer, head) three segments in the order sink, recent,
// middle; a segment covers slots 0..valid_count-1 of its pool
// (seg_length = valid_count * FSEQ, slot_global = (l*H + h) * max_slots).
// One workgroup; block-wide exclusive scan over the (layer, head) totals.
constexpr int kLegacyThreads = 1024;
__global__ void __launch_bounds__(kLegacyThreads) plan_legacy_kernel(int L, int H, int FSEQ, int ms, int mm, int mr,
                                                                     const int64_t *vc, int32_t *cu, int32_t *sk,
                                                                     int32_t *sg, int32_t *sl, int32_t *dst) {
  __shared__ int32_t part[kLegacyThreads];
  const int tid = threadIdx.x;
  const int n = L * H;
  const int per = (n + kLegacyThreads - 1) / kLegacyThreads;
  const int q0 = tid * per, q1 = min(n, q0 + per);
  const int order[3] = {0, 2, 1};
  const int slots[3] = {ms, mm, mr};
  int32_t acc = 0;
  for (int q = q0; q < q1; ++q)
    for (int k = 0; k < 3; ++k) {
      const int64_t v = vc[q * 3 + order[k]];
      if (v > 0) acc += static_cast<int32_t>(v) * FSEQ;
    }
  part[tid] = acc;
  __syncthreads();
  for (int off = 1; off < kLegacyThreads; off <<= 1) {
    const int32_t v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int32_t run = part[tid] - acc;
  if (tid == 0) cu[0] = 0;
  for (int q = q0; q < q1; ++q) {
    for (int k = 0; k < 3; ++k) {
      const int kind = order[k];
      const int d = q * 3 + k;
      const int64_t v = vc[q * 3 + kind];
      if (v <= 0) {
        sk[d] = PKV_SEG_INACTIVE;
        sg[d] = 0;
        sl[d] = 0;
        dst[d] = 0;
        continue;
      }
      const int32_t tokens = static_cast<int32_t>(v) * FSEQ;
      sk[d] = kind;
      sg[d] = q * slots[kind];
      sl[d] = tokens;
      dst[d] = run;
      run += tokens;
    }
    cu[q + 1] = run;
  }
}

static dim3 split_grid(int n) { return dim3(static_cast<unsigned>(n), kAuxSplit); }

}  // namespace pkv

using namespace pkv;

extern "C" {

int pkv_scatter_copy(const int64_t *src_ptrs, const int64_t *lengths, const int64_t *offsets, int32_t n_segments,
                     void *dst, int64_t dst_rows, int64_t row_bytes, pkv_stream_t stream) {
  if (n_segments == 0) return PKV_OK;
  if (n_segments < 0 || !src_ptrs || !lengths || !offsets || !dst || row_bytes <= 0 || dst_rows < 0)
    return fail(PKV_ERR_INVALID, "scatter_copy: bad arguments");
  hipLaunchKernelGGL(scatter_copy_kernel, split_grid(n_segments), dim3(kAuxThreads), 0, as_stream(stream), src_ptrs,
                     lengths, offsets, n_segments, static_cast<char *>(dst), dst_rows, row_bytes);
  return check_launch("scatter_copy_kernel");
}

int pkv_pos_override(int64_t *pos, int64_t rows, const int64_t *starts, const int64_t *ends, const int64_t *vals,
                     int32_t n_ranges, pkv_stream_t stream) {
  if (n_ranges == 0) return PKV_OK;
  if (n_ranges < 0 || !pos || !starts || !ends || !vals || rows < 0)
    return fail(PKV_ERR_INVALID, "apply_pos_override: bad arguments");
  hipLaunchKernelGGL(pos_override_kernel, dim3(static_cast<unsigned>(n_ranges), 4), dim3(kAuxThreads), 0,
                     as_stream(stream), pos, rows, starts, ends, vals, n_ranges);
  return check_launch("pos_override_kernel");
}

int pkv_refresh_readout(const pkv_refresh_args *a, pkv_stream_t stream) {
  if (!a) return fail(PKV_ERR_INVALID, "refresh_readout_layout: NULL arguments");
  if (a->n_segments == 0) return PKV_OK;
  if (a->n_segments < 0 || !a->src_ptrs_k || !a->src_ptrs_v || !a->src_ptrs_pos || !a->offsets || !a->lengths ||
      !a->flags || !a->dynamic_rope_t || !a->dst_k || !a->dst_v || !a->dst_pos || !a->dst_frame_ids ||
      a->row_bytes <= 0 || a->dst_rows < 0)
    return fail(PKV_ERR_INVALID, "refresh_readout_layout: bad arguments");
  hipLaunchKernelGGL(refresh_kernel, split_grid(a->n_segments), dim3(kAuxThreads), 0, as_stream(stream), *a);
  return check_launch("refresh_kernel");
}

int pkv_anchor_store_write_frames(const void *k_seq, const void *v_seq, const int64_t *pos_seq, int64_t src_frames,
                                  const int64_t *frame_desc, int32_t n_frames, void *store_k, void *store_v,
                                  int64_t *store_pos, int64_t capacity, int64_t frame_seqlen, int64_t row_bytes,
                                  pkv_stream_t stream) {
  if (n_frames == 0) return PKV_OK;
  if (n_frames < 0 || !k_seq || !v_seq || !pos_seq || !frame_desc || !store_k || !store_v || !store_pos ||
      frame_seqlen <= 0 || row_bytes <= 0)
    return fail(PKV_ERR_INVALID, "anchor_store_write_frames: bad arguments");
  hipLaunchKernelGGL(write_frames_kernel, split_grid(n_frames), dim3(kAuxThreads), 0, as_stream(stream),
                     static_cast<const char *>(k_seq), static_cast<const char *>(v_seq), pos_seq, src_frames,
                     frame_desc, n_frames, static_cast<char *>(store_k), static_cast<char *>(store_v), store_pos,
                     capacity, frame_seqlen, row_bytes);
  return check_launch("write_frames_kernel");
}

int pkv_plan_legacy(const pkv_geometry *geo, const int64_t *valid_count, int32_t *cu_seqlens_k, int32_t *src_kind,
                    int32_t *src_slot_global, int32_t *seg_lengths, int32_t *dst_token_offsets,
                    pkv_stream_t stream) {
  int rc = check_geometry(geo);
  if (rc) return rc;
  if (!valid_count || !cu_seqlens_k || !src_kind || !src_slot_global || !seg_lengths || !dst_token_offsets)
    return fail(PKV_ERR_INVALID, "pyramidkv_plan: NULL argument");
  hipLaunchKernelGGL(plan_legacy_kernel, dim3(1), dim3(kLegacyThreads), 0, as_stream(stream), geo->num_layers,
                     geo->num_heads, geo->frame_seqlen, geo->max_sink, geo->max_middle, geo->max_recent, valid_count,
                     cu_seqlens_k, src_kind, src_slot_global, seg_lengths, dst_token_offsets);
  return check_launch("plan_legacy_kernel");
}

}  // extern "C"
