// Internal definitions shared by the gfx950 kernels of the pyramid KV-cache path.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "pyramidkv_hip.h"

namespace pkv {

// Compile-time bounds of the per-head strategy record
// (reference: pyramidkv/csrc/anchor_store.cuh:39-45, 145-148).
constexpr int kMaxPhase = 6;
constexpr int kMaxBucket = 4;
constexpr int kMaxTKeyed = 24;
constexpr int kMaxLagOffsets = 4;
constexpr int kMaxMergeBlocks = 6;
constexpr int kMaxMergeActive = 2;
constexpr int kMaxMergeBlockFrames = 4;
constexpr int kMaxMergeTokens = 420;

enum : int8_t { SK_RECENT = 0, SK_CYCLIC = 1, SK_STRIDE = 2, SK_LAG = 3, SK_MERGE = 4 };

// Byte-level state record of one (layer, head).  The field order and sizes
// are the ABI the reference's Python side serialises with a numpy
// structured dtype (anchor_store.cuh:62-132, _mega_state_ops.py:36-77), so
// it is kept identical; natural alignment gives the same 600-byte layout.
struct HeadState {
  int8_t kind;
  int8_t sink_capacity;
  int8_t pad0[2];
  int32_t period;
  int32_t bucket_cap;
  int32_t interval;
  int32_t capacity;
  int32_t patch_size;
  int32_t block_frames;
  int32_t lag_offsets[kMaxLagOffsets];
  int32_t lag_offset_count;
  int32_t cyclic_slot[kMaxPhase * kMaxBucket];
  int32_t cyclic_t[kMaxPhase * kMaxBucket];
  int8_t cyclic_cursor[kMaxPhase];
  int32_t tkey_slot[kMaxTKeyed];
  int32_t tkey_t[kMaxTKeyed];
  int8_t tkey_count;
  int8_t tkey_head;
  int8_t pad1[2];
  int32_t merge_completed_slot[kMaxMergeBlocks];
  int32_t merge_completed_block_id[kMaxMergeBlocks];
  int32_t merge_completed_start_t[kMaxMergeBlocks];
  int32_t merge_completed_end_t[kMaxMergeBlocks];
  int32_t merge_completed_median_t[kMaxMergeBlocks];
  int8_t merge_completed_count;
  int8_t pad2[3];
  int32_t merge_active_block_id[kMaxMergeActive];
  int32_t merge_active_slot[kMaxMergeActive];
  int8_t merge_active_seen[kMaxMergeActive][kMaxMergeBlockFrames];
  int8_t merge_active_complete_count[kMaxMergeActive];
  int8_t pad3[2];
  int32_t cached_num_groups;
};

static_assert(sizeof(HeadState) == 600, "HeadState must be 600 bytes");
static_assert(sizeof(HeadState) % 8 == 0, "records are copied as 8-byte words");
static_assert(offsetof(HeadState, cyclic_cursor) == 240, "layout");
static_assert(offsetof(HeadState, tkey_slot) == 248, "layout");
static_assert(offsetof(HeadState, tkey_count) == 440, "layout");
static_assert(offsetof(HeadState, merge_completed_slot) == 444, "layout");
static_assert(offsetof(HeadState, merge_completed_count) == 564, "layout");
static_assert(offsetof(HeadState, merge_active_block_id) == 568, "layout");
static_assert(offsetof(HeadState, cached_num_groups) == 596, "layout");

// ---- bf16 <-> fp32 ----------------------------------------------------------

__host__ __device__ inline float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN -> quiet NaN 0x7fc0), the
// rounding torch and __float2bfloat16 use.
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) |
         (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// Read of a workgroup-uniform value that no thread writes while the kernel
// runs (written by an earlier launch), through the constant address space:
// the compiler issues it as a scalar load, which keeps it out of the vector
// registers and lets several such reads share one wait.
template <typename T>
__device__ inline T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(p);
}

// Copy of n 8-byte words from global memory into LDS by the whole workgroup:
// each thread issues kBatch reads before its LDS writes, so a batch costs one
// memory round trip.  The reads are unconditional (indices past the end read
// the last word): guarded reads sit in separate blocks, and at their joins
// the compiler waits for each read before issuing the next.
template <int kBatch = 4>
__device__ inline void stage_words(uint2 *lds, const uint2 *g, int n) {
  for (int i0 = 0; i0 < n; i0 += kBatch * static_cast<int>(blockDim.x)) {
    uint2 v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int i = i0 + static_cast<int>(threadIdx.x) + k * static_cast<int>(blockDim.x);
      v[k] = g[i < n ? i : n - 1];
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int i = i0 + static_cast<int>(threadIdx.x) + k * static_cast<int>(blockDim.x);
      if (i < n) lds[i] = v[k];
    }
  }
}

// ---- error plumbing (host) --------------------------------------------------

void set_error(const char *fmt, ...);
int fail(int status, const char *fmt, ...);
int check_launch(const char *what);
// PKV_OK or PKV_ERR_INVALID with a message for a malformed geometry
int check_geometry(const pkv_geometry *g);

inline hipStream_t as_stream(pkv_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace pkv
