/*
 * pyramidkv_hip.h -- C ABI of the MI355X (gfx950) pyramid KV-cache hot path.
 *
 * Every entry point takes plain device pointers, extents and a hipStream_t
 * (passed as an opaque pointer), enqueues its kernels on that stream, and
 * returns PKV_OK (0) or a negative pkv_status.  The library never allocates
 * device memory and never synchronises the stream, with one documented
 * exception (pkv_plan_multi reads back the packed-token total when the
 * static bound cannot rule out a workspace overflow).  Error text of the
 * last failing call on the calling thread is returned by pkv_last_error().
 *
 * bf16 tensors are passed as uint16_t bit patterns.  Shapes use the
 * reference's conventions: L layers, H heads, D head_dim, FSEQ tokens per
 * latent frame, pools laid out [L, H, slots, FSEQ, D] (K/V) and
 * [L, H, slots, FSEQ, 3] (int64 positions), merge anchors
 * [L, H, MMB, MTPA, D] with MMB = 6 finalized anchors, MMA = 2 accumulating
 * blocks and MTPA = 420 tokens per anchor.
 *
 * Reference interfaces replaced (IF-LAB-PKU/Pyramid-Forcing):
 *   pkv_perhead_state_size   scatter_copy_bind.cpp:405-407  (mega_state_perhead_size)
 *   pkv_state_update         anchor_store_update.cu:324-374 (launch_mega_state_update)
 *   pkv_update_frames        pyramidkv_update.cu:115-189    (launch_pyramidkv_update)
 *   pkv_merge_accum          mega_merge_accum.cu:268-340    (launch_mega_merge_accum)
 *   pkv_plan_multi           mega_plan.cc:286-407, 513-654  (mega_plan / mega_plan_multi)
 *   pkv_pack                 pyramidkv_pack.cu:189-311      (launch_pyramidkv_pack)
 *   pkv_plan_pack            _mega_cache.py:461-523 (plan -> layer offset -> pack of attend)
 *   pkv_scatter_copy         scatter_copy.cu:13-47, scatter_copy_bind.cpp:451-465 (scatter_copy)
 *   pkv_pos_override         scatter_copy.cu:53-71, scatter_copy_bind.cpp:467-479 (apply_pos_override)
 *   pkv_refresh_readout      scatter_copy.cu:77-168, scatter_copy_bind.cpp:527-627 (refresh_readout_layout)
 *   pkv_anchor_store_write_frames  scatter_copy.cu:170-225, scatter_copy_bind.cpp:629-683
 *   pkv_plan_legacy          pyramidkv_plan.cc:46-133 (pyramidkv_plan)
 *   pkv_rope_apply           rope.py:18-68, triton_rope.py:17-247 (apply_rope_to_flat_k)
 *   pkv_ragged_attn_fwd      _mega_cache.py:540-559, flash_attn_varlen_func (flash-attn 2.8.3)
 *   pkv_cache_update         _mega_cache.py:136-414 (MegaCache.update: sink/recent routing,
 *                            noisy/clean commit, mega_state_update, pyramidkv_update,
 *                            mega_merge_accum), fused into three launches
 * (paths are relative to pyramidkv/csrc/ or pyramidkv/ of the reference.)
 */
#ifndef PYRAMIDKV_HIP_H
#define PYRAMIDKV_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKV_ABI_VERSION 3

typedef void *pkv_stream_t; /* hipStream_t; NULL selects the null stream */

enum pkv_status {
  PKV_OK = 0,
  PKV_ERR_INVALID = -1,     /* bad argument (shape, pointer, range) */
  PKV_ERR_HIP = -2,         /* a HIP runtime call failed */
  PKV_ERR_CAPACITY = -3,    /* packed tokens exceed the pack workspace */
  PKV_ERR_UNSUPPORTED = -4  /* valid request this build does not implement */
};

/* Destination kinds written by the state machine (anchor_store_update.cu:33-41). */
#define PKV_DST_SKIP (-1)
#define PKV_DST_SINK 0
#define PKV_DST_MIDDLE 1
#define PKV_DST_RECENT 2
#define PKV_DST_MERGE_ACCUM 5

/* Segment kinds written by the planner (mega_plan.cc:30-37). */
#define PKV_SEG_INACTIVE (-1)
#define PKV_SEG_SINK 0
#define PKV_SEG_MIDDLE 1
#define PKV_SEG_RECENT 2
#define PKV_SEG_MERGE 3

int pkv_abi_version(void);
/* sizeof(PerHeadState) of the byte-level state record: 600 (anchor_store.cuh:62-139). */
int64_t pkv_perhead_state_size(void);
const char *pkv_last_error(void);

/* ---- shared geometry / pool descriptors -------------------------------- */

typedef struct pkv_geometry {
  int32_t num_layers, num_heads, head_dim, frame_seqlen;
  int32_t max_sink, max_middle, max_recent;
  int32_t max_merge_blocks;  /* MMB (6) */
  int32_t max_merge_active;  /* MMA (2) */
  int32_t max_merge_tokens;  /* MTPA (420) */
  int64_t max_pack_tokens;   /* capacity of k_flat_out / v_flat_out / pos_flat_out */
} pkv_geometry;

typedef struct pkv_pools {
  uint16_t *sink_k, *sink_v, *middle_k, *middle_v, *recent_k, *recent_v;
  int64_t *sink_pos, *middle_pos, *recent_pos;
  uint16_t *merge_k, *merge_v;
  int64_t *merge_pos;
  int32_t *merge_token_count;          /* [L,H,MMB] */
  float *merge_accum_sum_k;            /* [L,H,MMA,MTPA,D] */
  float *merge_accum_sum_v;
  int64_t *merge_accum_pos;            /* [L,H,MMA,MTPA,3] */
  int32_t *merge_accum_group_ids;      /* [L,H,MMA,FSEQ] */
  float *merge_accum_tokens_per_group; /* [L,H,MMA,MTPA] */
  int32_t *merge_accum_num_groups;     /* [L,H,MMA] */
  float *merge_accum_weight_sum;       /* [L,H,MMA] running sum of frame weights */
  int64_t *valid_count;                /* [L,H,3] frames held per kind */
  uint16_t *k_flat_out, *v_flat_out;   /* [max_pack_tokens, D] */
  int64_t *pos_flat_out;               /* [max_pack_tokens, 3] */
} pkv_pools;

/* 8 descriptor outputs of the state machine, each [H*F] int32, index h*F+f. */
typedef struct pkv_state_desc {
  int32_t *dst_kind, *dst_slot, *src_frame, *src_head;
  int32_t *merge_accum_slot, *merge_local_idx;
  int32_t *merge_finalize_completed_idx, *merge_is_new_block;
} pkv_state_desc;

/* mega_state_update: mutate H PerHeadState records (one layer) for the
 * frames new_t_vals[0..F) (device int64) and emit descriptors.
 * pass_kind 0 = noisy (state untouched, all SKIP), 1 = clean. */
int pkv_state_update(uint8_t *states, int32_t num_heads,
                     const int64_t *new_t_vals, int32_t frames_in_block,
                     int32_t pass_kind, const pkv_state_desc *desc,
                     pkv_stream_t stream);

/* pyramidkv_update: copy frame (src_frame, src_head) of new_k/new_v
 * [F,H,FSEQ,D] (and new_pos [F,H,FSEQ,3] when non-NULL) into pool slot
 * dst_slot_global of pool dst_kind (0 sink / 1 middle / 2 recent).  Any
 * other kind (SKIP -1; MERGE 5, which the reference's caller masks to -1
 * first, _mega_cache.py:358-362, while its kernel would route it to the
 * recent pool) writes nothing, and so do slots outside the pool and sources
 * outside [frames_in_block, H]. */
int pkv_update_frames(const pkv_geometry *geo, const pkv_pools *pools,
                      const uint16_t *new_k, const uint16_t *new_v,
                      const int64_t *new_pos, int32_t frames_in_block,
                      const int32_t *dst_kind, const int32_t *dst_slot_global,
                      const int32_t *src_frame, const int32_t *src_head,
                      int32_t n_writes, pkv_stream_t stream);

/* One layer's slices of the merge accumulators and anchor pools. */
typedef struct pkv_merge_layer {
  float *accum_sum_k, *accum_sum_v;   /* [H,MMA,MTPA,D] */
  int64_t *accum_pos;                 /* [H,MMA,MTPA,3] */
  int32_t *accum_group_ids;           /* [H,MMA,FSEQ] */
  float *accum_tokens_per_group;      /* [H,MMA,MTPA] */
  int32_t *accum_num_groups;          /* [H,MMA] */
  float *accum_weight_sum;            /* [H,MMA] running sum of the block's frame weights (1 per
                                         unweighted frame); NULL ok when weights == NULL */
  uint16_t *merge_k, *merge_v;        /* [H,MMB,MTPA,D] */
  int64_t *merge_pos;                 /* [H,MMB,MTPA,3] */
  int32_t *merge_token_count;         /* [H,MMB] */
} pkv_merge_layer;

/* mega_merge_accum (Veil): for each merge descriptor (kind 5) in frame
 * order, zero + group a new block, add the frame's K/V into its 2x2-patch
 * fp32 group sums, and on finalize write bf16(sum / divisor) into the anchor
 * pool.  frame_weights (device fp32 [F], nullable) turns the block mean into
 * a weighted mean sum(w*x) / (count * sum(w)); NULL means w == 1, which is
 * the reference operation.  workspace: pkv_merge_workspace_size(H, F, FSEQ,
 * MTPA) bytes of device scratch (per-frame group member lists). */
int64_t pkv_merge_workspace_size(int32_t H, int32_t F, int32_t FSEQ, int32_t MTPA);

int pkv_merge_accum(const uint8_t *states, int32_t H, int32_t F, int32_t FSEQ,
                    int32_t D, int32_t MMA, int32_t MMB, int32_t MTPA,
                    const uint16_t *new_k, const uint16_t *new_v,
                    const int64_t *new_pos, const int32_t *desc_dst_kind,
                    const int32_t *desc_merge_accum_slot,
                    const int32_t *desc_merge_finalize_completed_idx,
                    const int32_t *desc_merge_is_new_block,
                    const float *frame_weights, const pkv_merge_layer *ml,
                    void *workspace, pkv_stream_t stream);

/* pkv_merge_accum without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * scratch is a static device array of PKV_MERGE_STATIC_SCRATCH_BYTES per
 * device (held until the process ends); calls needing more
 * (pkv_merge_workspace_size(H, F, FSEQ, MTPA) above the limit: about H * F
 * <= 130 at FSEQ 1560) return PKV_ERR_CAPACITY.  Same kernels and results as
 * pkv_merge_accum.  Calls that overlap on one device race on the array.
 * The array's device address is looked up on the first call on each device
 * and kept for the process; like every device pointer the process holds, it
 * does not survive hipDeviceReset of that device (do not call this entry
 * point after one). */
#define PKV_MERGE_STATIC_SCRATCH_BYTES (1 << 20)

int pkv_merge_accum_static(const uint8_t *states, int32_t H, int32_t F, int32_t FSEQ,
                           int32_t D, int32_t MMA, int32_t MMB, int32_t MTPA,
                           const uint16_t *new_k, const uint16_t *new_v,
                           const int64_t *new_pos, const int32_t *desc_dst_kind,
                           const int32_t *desc_merge_accum_slot,
                           const int32_t *desc_merge_finalize_completed_idx,
                           const int32_t *desc_merge_is_new_block,
                           const float *frame_weights, const pkv_merge_layer *ml,
                           pkv_stream_t stream);

/* Dynamic-RoPE remap configuration (mega_plan.cc:63-114). */
typedef struct pkv_remap {
  int32_t sink_mode_code;      /* 0 lag, 1 window_clamp */
  int32_t sink_clamp_min, sink_clamp_max, decoupled_sink_lag;
  int32_t hist_mode_code;      /* accepted, ignored by the planner (mega_plan.cc:259) */
  int32_t hist_relative_t_max;
  double hist_soft_factor;
} pkv_remap;

/* Plan outputs (device). cu [C*H+1]; the rest [C*H*S], S = max_sink +
 * max_middle + max_recent + MMB. */
typedef struct pkv_plan_out {
  int32_t *cu_seqlens_k, *src_kind, *src_slot_global, *seg_lengths,
      *dst_token_offsets;
  int64_t *anchor_t_raw, *anchor_t_remap;
} pkv_plan_out;

/* mega_plan_multi on the device: one layer's states [H*600] bytes,
 * valid_count slice [H,3] int64, merge_token_count slice [H,MMB] int32,
 * current_t_list host int64 [num_chunks].  When num_chunks exceeds what the
 * pack workspace is sized for, the total is read back and
 * PKV_ERR_CAPACITY is returned if it overflows (mega_plan.cc:618-629).
 * total_tokens_out (device int32, nullable) receives cu[C*H]. */
int pkv_plan_multi(const pkv_geometry *geo, const uint8_t *states_layer,
                   const int64_t *valid_count_layer,
                   const int32_t *merge_token_count_layer,
                   const int64_t *current_t_list, int32_t num_chunks,
                   const pkv_remap *remap, const pkv_plan_out *out,
                   int32_t *total_tokens_out, pkv_stream_t stream);

/* 3D RoPE tables: fp32 [rows, cols*2] (re, im interleaved) for the t, y
 * and x axes.  All three present, or the struct pointer NULL. */
typedef struct pkv_rope_tables {
  const float *ft, *fy, *fx;
  int32_t ft_rows, ft_cols, fy_rows, fy_cols, fx_rows, fx_cols;
} pkv_rope_tables;

/* pyramidkv_pack: gather segments from the four pools into the flat
 * workspaces; K gets 3D RoPE at (tremap >= 0 ? tremap : pos.t, y, x) when
 * anchor_t_remap and rope are non-NULL.  src_slot_global is already
 * layer-offset (_mega_attention.py:516-552). */
int pkv_pack(const pkv_geometry *geo, const pkv_pools *pools,
             const int32_t *src_kind, const int32_t *src_slot_global,
             const int32_t *seg_lengths, const int32_t *dst_token_offsets,
             int32_t n_segments, const int64_t *anchor_t_remap,
             const pkv_rope_tables *rope, pkv_stream_t stream);

/* MegaCache.attend's K/V side in two launches and no host sync: the
 * device plan of mega_plan_multi for layer `layer` with the per-kind layer
 * offset of _layer_offset_slot_global folded into src_slot_global
 * (mega_plan.cc:513-654, _mega_attention.py:349-385), then pyramidkv_pack
 * with fused RoPE (rope may be NULL: pure gather) into pools->k/v/pos_flat_out
 * (pyramidkv_pack.cu:189-311; caller _mega_cache.py:461-523).  plan_ws holds
 * caller-owned device buffers of C*H+1 / C*H*S entries; cu_seqlens_k
 * receives the per-(chunk, head) offsets the attention reads.  Same
 * capacity check and error text as pkv_plan_multi. */
int pkv_plan_pack(const pkv_geometry *geo, const pkv_pools *pools,
                  const uint8_t *states_layer, int32_t layer,
                  const int64_t *current_t_list, int32_t num_chunks,
                  const pkv_remap *remap, const pkv_rope_tables *rope,
                  const pkv_plan_out *plan_ws, pkv_stream_t stream);

/* scatter_copy: segment i copies lengths[i] rows of row_bytes bytes from
 * the device address src_ptrs[i] to dst rows offsets[i].. (all int64 device
 * arrays).  Segments whose rows fall outside [0, dst_rows) are skipped. */
int pkv_scatter_copy(const int64_t *src_ptrs, const int64_t *lengths,
                     const int64_t *offsets, int32_t n_segments, void *dst,
                     int64_t dst_rows, int64_t row_bytes, pkv_stream_t stream);

/* apply_pos_override: pos[i, 0] = vals[r] for starts[r] <= i < ends[r]
 * (pos [rows, 3] int64; ranges clipped to [0, rows)). */
int pkv_pos_override(int64_t *pos, int64_t rows, const int64_t *starts,
                     const int64_t *ends, const int64_t *vals, int32_t n_ranges,
                     pkv_stream_t stream);

/* refresh_readout_layout: per segment, copy lengths[i] rows of K and V from
 * the device addresses src_ptrs_k/v[i] to dst rows offsets[i].., and write
 * dst_pos / dst_frame_ids from the int64 [len, 3] positions at
 * src_ptrs_pos[i]: flags bit 2 sets t = dynamic_rope_t[i]; otherwise bit 0
 * applies the history time map (mode 0 none, 1 relative_clamp, 2
 * relative_softcap) relative to current_t; bit 1 makes the frame id the
 * source t instead of the written t.  Segments outside [0, dst_rows) are
 * skipped. */
typedef struct pkv_refresh_args {
  const int64_t *src_ptrs_k, *src_ptrs_v, *src_ptrs_pos;
  const int64_t *offsets, *lengths, *flags, *dynamic_rope_t;
  void *dst_k, *dst_v;
  int64_t *dst_pos, *dst_frame_ids;
  int64_t dst_rows, row_bytes, current_t, history_relative_t_max;
  int32_t n_segments, history_mode_code;
  float history_soft_factor;
} pkv_refresh_args;
int pkv_refresh_readout(const pkv_refresh_args *args, pkv_stream_t stream);

/* anchor_store_write_frames: frame_desc [n, 2] int64 (source frame, store
 * slot); copies a frame of frame_seqlen rows of K, V (row_bytes each) and
 * its [frame_seqlen, 3] int64 positions into the slot.  Descriptors with a
 * negative field, a source frame >= src_frames or a slot >= capacity are
 * skipped. */
int pkv_anchor_store_write_frames(const void *k_seq, const void *v_seq,
                                  const int64_t *pos_seq, int64_t src_frames,
                                  const int64_t *frame_desc, int32_t n_frames,
                                  void *store_k, void *store_v, int64_t *store_pos,
                                  int64_t capacity, int64_t frame_seqlen,
                                  int64_t row_bytes, pkv_stream_t stream);

/* pyramidkv_plan (legacy): over all L*H heads, three segments each in the
 * order sink, recent, middle covering slots 0..valid_count-1; outputs cu
 * [L*H+1] and [3*L*H] descriptor arrays (int32, device). */
int pkv_plan_legacy(const pkv_geometry *geo, const int64_t *valid_count,
                    int32_t *cu_seqlens_k, int32_t *src_kind,
                    int32_t *src_slot_global, int32_t *seg_lengths,
                    int32_t *dst_token_offsets, pkv_stream_t stream);

/* apply_rope_to_flat_k: out[n, D] = rot(k[n, D], pos[n, 3]); out may equal k. */
int pkv_rope_apply(const uint16_t *k, const int64_t *pos, int64_t n_tokens,
                   int32_t head_dim, const pkv_rope_tables *rope, uint16_t *out,
                   pkv_stream_t stream);

/* Ragged-cache attention, non-causal, bf16 in/out, fp32 softmax+accumulate.
 * Query sequence b (0..num_batches) owns rows cu_seqlens_q[b]..[b+1] of q,
 * head h (0..num_heads_q) at column offset h*q_head_stride.  With
 * kv_per_head != 0 the key sequence of (b, h) is rows
 * cu_seqlens_k[b*num_heads_q + h] .. +1 of k/v (per-head ragged KV, the
 * layout pyramidkv_pack produces); otherwise rows cu_seqlens_k[b]..[b+1]
 * at column offset h*kv_head_stride (flash-attn varlen).  Strides are in
 * elements.  max_seqlen_q bounds the query-tile grid. */
typedef struct pkv_attn_args {
  const uint16_t *q, *k, *v;
  uint16_t *o;
  const int32_t *cu_seqlens_q, *cu_seqlens_k;
  int32_t num_batches, num_heads_q, head_dim, kv_per_head;
  int64_t q_tok_stride, q_head_stride;
  int64_t kv_tok_stride, kv_head_stride;
  int64_t o_tok_stride, o_head_stride;
  int32_t max_seqlen_q;
  float softmax_scale;
  int32_t causal; /* must be 0 */
} pkv_attn_args;

/* Launches of head_dim 128 with at least 1,024 query tiles of 384 rows run
 * one workgroup per compute unit, claiming tiles from counters in a static
 * device array: one 128-byte block per stream, taken on the stream's first
 * such launch (launches on different streams may overlap); past 64 streams
 * on a device they run one tile per workgroup.  Nothing is allocated. */
int pkv_ragged_attn_fwd(const pkv_attn_args *args, pkv_stream_t stream);

/* The same attention with a device workspace (replaces the same call,
 * _mega_cache.py:540-559).  Launches of head_dim 128 with fewer than 1,024
 * query tiles of 384 rows (and at most 1,024 sequences) -- one layer's heads
 * per call, as MegaCache.attend makes them -- split each sequence's keys
 * into chunks so that the (query tile, chunk) items fill every compute unit
 * evenly, and merge a query tile's chunks in a second launch, in chunk order
 * (deterministic).  Other launches, or a workspace smaller than
 * pkv_ragged_attn_workspace_size(), run as pkv_ragged_attn_fwd.  The
 * workspace needs no initialisation; calls sharing one must be ordered (one
 * stream). */
int64_t pkv_ragged_attn_workspace_size(void);
int pkv_ragged_attn_fwd_ws(const pkv_attn_args *args, void *workspace, int64_t workspace_bytes,
                           pkv_stream_t stream);

/* ---- fused MegaCache.update -------------------------------------------- */

/* Bytes of device workspace pkv_cache_update needs for F frames per block.
 * The workspace starts with the 8 state-machine descriptor arrays of the
 * last call (pkv_state_desc order, each [H*F] int32, 256-byte aligned),
 * followed by H int32 arrival counters.  The counters must be zero before the
 * first call (allocate the workspace zero-filled); every call leaves them
 * zero.  Calls that share one workspace must be ordered (one stream). */
int64_t pkv_cache_update_workspace_size(const pkv_geometry *geo, int32_t frames);

typedef struct pkv_update_args {
  int32_t layer;
  int32_t frames;            /* F = L_in / FSEQ, 1 <= F <= max_recent */
  int64_t t0;                /* current_start / FSEQ */
  int32_t pass_kind;         /* 0 noisy, 1 clean */
  int32_t shift_pending;     /* 1: this block's recent shift is already in the pool */
  int32_t spatial_width;     /* W of the (y, x) = (tok / W, tok % W) grid */
  int32_t reserved;          /* 0 */
  const uint16_t *new_k;     /* [L_in, H, D] rows, token stride tok_stride */
  const uint16_t *new_v;
  int64_t tok_stride;        /* elements between consecutive tokens (H*D) */
  int64_t head_stride;       /* elements between heads within a token (D) */
  uint8_t *states_layer;     /* [H*600] */
  const int64_t *sink_caps_layer; /* [H] */
  int64_t *committed_vc_layer;    /* [H,3] */
  void *workspace;           /* pkv_cache_update_workspace_size bytes */
  uint64_t merge_heads;      /* bit h: head h is a Veil head, whose clean passes accumulate
                                merges (bit 63 stands for every head >= 63); 0: none */
} pkv_update_args;

/* Veil eviction in one launch: pkv_state_update (clean pass) of H records
 * for the frames t_vals[0..F) followed by pkv_merge_accum of those frames
 * at the grid positions (t_vals[f], tok / W, tok % W) -- the positions
 * MegaCache.update gives its frames (_mega_cache.py:203-215) -- with
 * optional frame weights.  Results equal the two calls in sequence on those
 * positions; new_k/new_v are [F, H, FSEQ, D] bf16, 1 <= F <= 64 (several
 * frames per call read each frame once and keep the fp32 sums on chip; the
 * results equal F one-frame calls bit for bit).  It has no counterpart
 * in the reference, which evicts through mega_state_update
 * (anchor_store_update.cu:257-269) and mega_merge_accum
 * (mega_merge_accum.cu:52-340); it is for callers that evict frames
 * outside MegaCache.update.  workspace: pkv_evict_merge_workspace_size
 * bytes of arrival counters, zero-filled before first use; every call
 * leaves them zero.  Calls that share a workspace must not overlap. */
int pkv_evict_merge(uint8_t *states, int32_t num_heads, int32_t frames, int32_t frame_seqlen, int32_t head_dim,
                    int32_t max_merge_active, int32_t max_merge_blocks, int32_t max_merge_tokens,
                    const int64_t *t_vals, const uint16_t *new_k, const uint16_t *new_v, int32_t spatial_width,
                    const float *frame_weights, const pkv_state_desc *desc, const pkv_merge_layer *ml,
                    void *workspace, pkv_stream_t stream);
/* Workspace bytes pkv_evict_merge needs for num_heads heads. */
int64_t pkv_evict_merge_workspace_size(int32_t num_heads);

/* MegaCache.update of one layer (_mega_cache.py:136-414) in one launch:
 * sink / recent routing of the F new frames with the recent FIFO shift, the
 * state machine and middle-pool writes of a clean pass, the Veil merge
 * accumulate (the pkv_merge_accum semantics, unweighted) and the counter
 * commit.  Positions are the grid (t0 + f, tok / W, tok % W). */
int pkv_cache_update(const pkv_geometry *geo, const pkv_pools *pools,
                     const pkv_update_args *args, pkv_stream_t stream);

/*
 * Row operations of the causal DiT block around the cache, for the
 * end-to-end rollout (replacing the eager PyTorch chains of
 * wan/modules/model.py:70-99 WanRMSNorm / WanLayerNorm and the modulation
 * and gated residuals of wan/modules/causal_model.py:395-420).  Rows are
 * contiguous runs of `cols` values; one wave reduces one row in registers.
 *
 * pkv_dit_layer_norm: out[r] = bf16(LN(x[r]) * m + a), LN without affine
 *   weights (biased variance, eps inside the square root); m = 1 + mul when
 *   mul_plus_one (modulation: norm(x) * (1 + scale) + shift), else mul
 *   (LayerNorm affine weight); mul and add may be NULL (1 and 0).  x fp32
 *   [rows, cols], cols a multiple of 4 and at most 4096.
 * pkv_dit_rms_norm: out[r] = bf16(x[r] * rsqrt(mean(x[r]^2) + eps) * w) in
 *   fp32; x bf16 with a row stride (a column slice of a wider tensor),
 *   cols and strides multiples of 8, cols at most 8192; weight may be NULL.
 * pkv_dit_residual: x[r, c] += float(y[r, c]) * gate[c] in fp32 (gate may be
 *   NULL), in place; x fp32 [rows, cols], y bf16 with a row stride.
 * pkv_dit_gelu_tanh: out = bf16(gelu_tanh(float(x))) elementwise, n a
 *   multiple of 8.
 * pkv_dit_residual_layer_norm: pkv_dit_residual, then pkv_dit_layer_norm of
 *   the updated rows, in one pass over x (the residual update followed by
 *   the next norm of causal_model.py:395-420); same results as the two
 *   calls in sequence.
 */
int pkv_dit_layer_norm(const float *x, int64_t rows, int32_t cols, const float *mul,
                       const float *add, int32_t mul_plus_one, float eps, uint16_t *out,
                       pkv_stream_t stream);
int pkv_dit_rms_norm(const uint16_t *x, int64_t x_row_stride, int64_t rows, int32_t cols,
                     const float *weight, float eps, uint16_t *out, int64_t out_row_stride,
                     pkv_stream_t stream);
int pkv_dit_residual(float *x, int64_t rows, int32_t cols, const uint16_t *y,
                     int64_t y_row_stride, const float *gate, pkv_stream_t stream);
int pkv_dit_gelu_tanh(const uint16_t *x, int64_t n, uint16_t *out, pkv_stream_t stream);
int pkv_dit_residual_layer_norm(float *x, int64_t rows, int32_t cols, const uint16_t *y,
                                int64_t y_row_stride, const float *gate, const float *mul,
                                const float *add, int32_t mul_plus_one, float eps, uint16_t *out,
                                pkv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PYRAMIDKV_HIP_H */
