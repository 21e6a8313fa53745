// Planner, pack and 3D RoPE kernels for gfx950.
//
// The planner runs on the device: one workgroup walks the (chunk, head)
// pairs of a layer call, emits each pair's ordered segment list and
// computes the global offsets with a block-wide exclusive scan, so the plan
// never leaves the GPU (the reference builds it on the host after three
// blocking device-to-host copies, mega_plan.cc:557-568).
//
// The pack kernel is a persistent gather: each work item is (segment,
// 64-token tile); 16 lanes move one 256-byte K row with 16-byte loads, the
// same lanes rotate their 4 complex pairs in registers, V and positions are
// copied alongside.

#include "pkv_common.h"

namespace pkv {

// ---------------------------------------------------------------------------
// dynamic-RoPE time remaps (mega_plan.cc:63-114, rope.py:86-134)
// ---------------------------------------------------------------------------
__host__ __device__ inline int64_t map_sink_time(int64_t t, int mode, int cmin, int cmax, int lag) {
  if (mode == 1) {
    int64_t d = t;
    if (d < cmin) d = cmin;
    if (d > cmax) d = cmax;
    const int64_t out = t - d;
    return out < 0 ? 0 : out;
  }
  const int64_t out = t - lag;
  return out < 0 ? 0 : out;
}

constexpr int kMaxPlanChunks = 64;
constexpr int kPlanThreads = 1024;
constexpr int kMaxPlanPairs = 4096;

struct PlanParams {
  int H, S, FSEQ, max_sink, max_middle, max_recent, MMB, C;
  int32_t slot_off[4];  // per-kind layer offset added to src_slot_global (0 for the reference op)
  int64_t t[kMaxPlanChunks];
  int64_t sync_t[kMaxPlanChunks];
};

// Inclusive prefix sum over the 64 lanes of a wave by DPP: row shifts 1, 2,
// 4, 8 scan each 16-lane row, then lane 15 of rows 0 and 2 is added to rows
// 1 and 3 (row_bcast:15) and lane 31 to rows 2 and 3 (row_bcast:31).  Lanes
// whose source lies outside the row (or rows the mask leaves out) add 0.
__device__ inline int32_t wave_incl_sum(int32_t x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

// Per-(chunk, head) quantities shared by the pair's candidate segments.
struct PairCtx {
  int thresh, n_sink, n_recent, kind_s, b0, b1, tc, mcc;
  int64_t sync_t;
};

__device__ inline PairCtx pair_ctx(const PlanParams &p, const HeadState &s, const int64_t *vc_h, int c) {
  PairCtx x;
  const int64_t t_c = p.t[c];
  x.sync_t = p.sync_t[c];
  x.thresh = s.sink_capacity;
  const int n_sink_raw = static_cast<int>(vc_h[0]);
  x.n_sink = (x.thresh > 0 && x.thresh < n_sink_raw) ? x.thresh : n_sink_raw;
  x.n_recent = static_cast<int>(vc_h[2]);
  x.kind_s = s.kind;
  const int period = s.period > 0 ? s.period : 1;
  const int bucket_cap = s.bucket_cap > 0 ? s.bucket_cap : 1;
  // the reference's ((t % period) + period) % period; 32-bit when t fits
  const int phase = (t_c >= 0 && t_c <= 0x7fffffff)
                        ? static_cast<int>(static_cast<uint32_t>(t_c) % static_cast<uint32_t>(period))
                        : static_cast<int>(((t_c % period) + period) % period);
  x.b0 = phase * kMaxBucket;
  x.b1 = x.b0 + (bucket_cap < kMaxBucket ? bucket_cap : kMaxBucket);
  x.tc = s.tkey_count;
  x.mcc = s.merge_completed_count;
  return x;
}

// Candidate j of a pair in the reference's fixed order sink -> recent ->
// middle (Wave bucket of the current phase, or the Anchor/lag ring in slot
// order) -> merge anchors (mega_plan.cc:133-264).
struct Cand {
  bool valid;
  int kind, sg, len;
  int64_t traw, tremap;
};

__device__ inline Cand eval_cand(const PlanParams &p, const HeadState &s, const int32_t *mtc_h, const PairCtx &x,
                                 int h, int j) {
  const int32_t recent_min_t = 0x7fffffff;
  const int c_sink = p.max_sink, c_rec = c_sink + p.max_recent, c_mid = c_rec + kMaxTKeyed,
            n_cand = c_mid + kMaxMergeBlocks;
  Cand d{false, PKV_SEG_INACTIVE, 0, 0, -1, -1};
  if (j < c_sink) {
    d.valid = j < x.n_sink;
    d.kind = PKV_SEG_SINK;
    d.sg = p.slot_off[0] + h * p.max_sink + j;
    d.len = p.FSEQ;
    d.traw = j;
    d.tremap = x.sync_t;
  } else if (j < c_rec) {
    const int r = j - c_sink;
    d.valid = r < x.n_recent;
    d.kind = PKV_SEG_RECENT;
    d.sg = p.slot_off[2] + h * p.max_recent + r;
    d.len = p.FSEQ;
  } else if (j < c_mid) {
    const int i = j - c_rec;
    d.kind = PKV_SEG_MIDDLE;
    d.len = p.FSEQ;
    if (x.kind_s == SK_CYCLIC) {
      const int idx = x.b0 + i;
      if (idx < x.b1 && idx < kMaxPhase * kMaxBucket) {
        const int32_t t = s.cyclic_t[idx];
        d.valid = s.cyclic_slot[idx] >= 0 && t >= x.thresh && t < recent_min_t;
        d.sg = p.slot_off[1] + h * p.max_middle + idx;
        d.traw = t;
        d.tremap = x.sync_t;
      }
    } else if (x.kind_s == SK_STRIDE || x.kind_s == SK_LAG) {
      if (i < x.tc) {
        const int32_t t = s.tkey_t[i];
        d.valid = t >= x.thresh && t < recent_min_t;
        d.sg = p.slot_off[1] + h * p.max_middle + i;
        d.traw = t;
        d.tremap = x.kind_s == SK_STRIDE ? x.sync_t : -1;
      }
    }
  } else if (j < n_cand) {
    const int i = j - c_mid;
    if (x.kind_s == SK_MERGE && i < x.mcc) {
      const int slot = s.merge_completed_slot[i];
      if (slot >= 0 && slot < p.MMB && s.merge_completed_start_t[i] > 0 && s.merge_completed_end_t[i] < recent_min_t) {
        const int32_t tok = mtc_h[slot];
        d.valid = tok > 0;
        d.kind = PKV_SEG_MERGE;
        d.sg = p.slot_off[3] + h * p.MMB + slot;
        d.len = tok;
        d.traw = 0;
        d.tremap = s.merge_completed_median_t[i];
      }
    }
  }
  return d;
}

__device__ inline void put_seg(const pkv_plan_out &o, int i, const Cand &d, int32_t dst) {
  o.src_kind[i] = d.kind;
  o.src_slot_global[i] = d.sg;
  o.seg_lengths[i] = d.len;
  o.dst_token_offsets[i] = dst;
  o.anchor_t_raw[i] = d.traw;
  o.anchor_t_remap[i] = d.tremap;
}

__device__ inline void put_inactive(const pkv_plan_out &o, int i) {
  put_seg(o, i, Cand{false, PKV_SEG_INACTIVE, 0, 0, -1, -1}, 0);
}

// Segment emission for one (chunk c, head h) by one wave (the general path,
// for any number of candidates).  Every lane evaluates one candidate; a
// candidate's position is the number of valid candidates before it (ballot
// popcount), positions >= S are dropped (the reference stops appending at
// S), and the destination offsets are a wave prefix sum of the lengths.
// Returns the pair's token total (uniform over the wave).
template <bool kWrite>
__device__ int32_t emit_pair(const PlanParams &p, const HeadState &s, const int64_t *vc_h, const int32_t *mtc_h,
                             int c, int h, int base, int32_t dst0, const pkv_plan_out &o) {
  const int lane = threadIdx.x & 63;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int S = p.S;
  const PairCtx x = pair_ctx(p, s, vc_h, c);
  const int n_cand = p.max_sink + p.max_recent + kMaxTKeyed + kMaxMergeBlocks;
  int fp = 0;
  int32_t run = 0;
  for (int j0 = 0; j0 < n_cand; j0 += 64) {
    const Cand d = eval_cand(p, s, mtc_h, x, h, j0 + lane);
    const uint64_t mask = __ballot(d.valid);
    const int pos = fp + __popcll(mask & below);
    const bool emit = d.valid && pos < S;
    const int32_t l = emit ? d.len : 0;
    const int32_t incl = wave_incl_sum(l);
    if (kWrite && emit) put_seg(o, base + pos, d, dst0 + run + incl - l);
    run += __shfl(incl, 63);
    fp = min(S, fp + __popcll(mask));
  }
  if (kWrite)
    for (int i = fp + lane; i < S; i += 64) put_inactive(o, base + i);
  return run;
}

// One workgroup.  The layer's state records, counters and merge token counts
// are staged in LDS with coalesced reads (when they fit).
//  - One-pass form (at most 64 candidates and segments per pair, at most 64
//    pairs): each wave evaluates the candidates of up to kPlanRegRounds pairs
//    once and keeps them in registers; one barrier publishes the pair totals,
//    every wave scans those 64 values itself and writes its segments.
//  - General form: a count-only pass gives every pair its token total, a
//    block-wide exclusive scan turns those into offsets, and a second pass
//    re-evaluates each pair's segments and writes them.
constexpr int kPlanStageHeads = 48;  // heads whose records are staged in LDS
constexpr int kPlanRegRounds = 4;    // pairs per wave held in registers by the one-pass form

__global__ void __launch_bounds__(kPlanThreads) plan_kernel(PlanParams p, const HeadState *states,
                                                            const int64_t *vc, const int32_t *mtc,
                                                            pkv_plan_out o, int32_t *total_out) {
  __shared__ int32_t len[kMaxPlanPairs];
  __shared__ int32_t part[1];
  __shared__ __attribute__((aligned(16))) HeadState s_states[kPlanStageHeads];
  __shared__ int64_t s_vc[kPlanStageHeads * 3];
  __shared__ int32_t s_mtc[kPlanStageHeads * kMaxMergeBlocks];
  const int tid = threadIdx.x;
  const int pairs = p.C * p.H;
  const bool staged = p.H <= kPlanStageHeads && p.MMB <= kMaxMergeBlocks;
  if (staged) {
    // every read is issued before the LDS writes (one memory round trip for
    // up to 4 * kPlanThreads record words); the counters fit one per thread
    static_assert(kPlanStageHeads * 3 <= kPlanThreads && kPlanStageHeads * kMaxMergeBlocks <= kPlanThreads &&
                      kPlanStageHeads * sizeof(HeadState) / 8 <= 4 * kPlanThreads,
                  "staging sizes");
    const int nvc = p.H * 3, nmtc = p.H * p.MMB;
    const int nw = p.H * static_cast<int>(sizeof(HeadState)) / 8;
    const uint2 *g = reinterpret_cast<const uint2 *>(states);
    uint2 *l = reinterpret_cast<uint2 *>(s_states);
    // reads with clamped indices, unconditional except the merge counts
    // (which may be empty), issued last: a wait the compiler places after a
    // guarded read then delays no other read
    uint2 w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = g[min(tid + k * kPlanThreads, nw - 1)];
    const int64_t v = vc[min(tid, nvc - 1)];
    int32_t m = 0;
    if (nmtc > 0) m = mtc[min(tid, nmtc - 1)];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (tid + k * kPlanThreads < nw) l[tid + k * kPlanThreads] = w[k];
    if (tid < nvc) s_vc[tid] = v;
    if (tid < nmtc) s_mtc[tid] = m;
  }
  __syncthreads();
  const HeadState *st = staged ? s_states : states;
  const int64_t *vcs = staged ? s_vc : vc;
  const int32_t *mts = staged ? s_mtc : mtc;
  const int wave = tid >> 6, n_waves = blockDim.x >> 6, lane = tid & 63;
  const int n_cand = p.max_sink + p.max_recent + kMaxTKeyed + kMaxMergeBlocks;
  // (the one-pass form reads the staged copies by their LDS arrays, so that
  // the compiler issues LDS reads rather than generic ones)
  if (staged && n_cand <= 64 && p.S <= 64 && pairs <= 64 && pairs <= n_waves * kPlanRegRounds) {
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    Cand cd[kPlanRegRounds];
    int pos[kPlanRegRounds], excl[kPlanRegRounds], nv[kPlanRegRounds];
    bool emit[kPlanRegRounds];
#pragma unroll
    for (int r = 0; r < kPlanRegRounds; ++r) {
      const int q = wave + r * n_waves;
      emit[r] = false;
      pos[r] = excl[r] = nv[r] = 0;
      if (q < pairs) {  // uniform over the wave
        const int c = q / p.H, h = q % p.H;
        const PairCtx x = pair_ctx(p, s_states[h], s_vc + h * 3, c);
        cd[r] = eval_cand(p, s_states[h], s_mtc + h * p.MMB, x, h, lane);
        const uint64_t mask = __ballot(cd[r].valid);
        pos[r] = __popcll(mask & below);
        emit[r] = cd[r].valid && pos[r] < p.S;
        const int32_t l = emit[r] ? cd[r].len : 0;
        const int32_t incl = wave_incl_sum(l);
        excl[r] = incl - l;
        nv[r] = min(p.S, __popcll(mask));
        if (lane == 63) len[q] = incl;
      }
    }
    __syncthreads();
    const int32_t v = lane < pairs ? len[lane] : 0;
    const int32_t incl = wave_incl_sum(v);  // lane q: end offset of pair q
    const int32_t total = __shfl(incl, 63);
    if (tid == 0) {
      o.cu_seqlens_k[0] = 0;
      if (total_out) *total_out = total;
    }
#pragma unroll
    for (int r = 0; r < kPlanRegRounds; ++r) {
      const int q = wave + r * n_waves;
      if (q >= pairs) continue;  // uniform over the wave
      const int32_t end = __shfl(incl, q);
      const int32_t base = __shfl(incl - v, q);
      const int i0 = q * p.S;
      if (emit[r]) put_seg(o, i0 + pos[r], cd[r], base + excl[r]);
      if (lane >= nv[r] && lane < p.S) put_inactive(o, i0 + lane);
      if (lane == 0) o.cu_seqlens_k[q + 1] = end;
    }
    return;
  }
  for (int q = wave; q < pairs; q += n_waves) {
    const int c = q / p.H, h = q % p.H;
    const int32_t n = emit_pair<false>(p, st[h], vcs + h * 3, mts + h * p.MMB, c, h, q * p.S, 0, o);
    if (lane == 0) len[q] = n;
  }
  __syncthreads();
  // exclusive scan of len[0..pairs) in 64-pair chunks: each wave scans its
  // chunks with lane shuffles, wave 0 scans the chunk totals, and every
  // element gets its chunk's base (two barriers)
  __shared__ int32_t ctot[kMaxPlanPairs / 64];
  const int n_chunks = (pairs + 63) / 64;
  for (int ch = wave; ch < n_chunks; ch += n_waves) {
    const int q = ch * 64 + lane;
    const int32_t v = q < pairs ? len[q] : 0;
    const int32_t incl = wave_incl_sum(v);
    if (q < pairs) len[q] = incl - v;
    if (lane == 63) ctot[ch] = incl;
  }
  __syncthreads();
  if (wave == 0) {
    int32_t run = 0;
    for (int c0 = 0; c0 < n_chunks; c0 += 64) {
      const int ch = c0 + lane;
      const int32_t v = ch < n_chunks ? ctot[ch] : 0;
      const int32_t incl = wave_incl_sum(v);
      if (ch < n_chunks) ctot[ch] = run + incl - v;
      run += __shfl(incl, 63);
    }
    if (lane == 0) part[0] = run;
  }
  __syncthreads();
  for (int q = tid; q < pairs; q += blockDim.x) len[q] += ctot[q >> 6];
  __syncthreads();
  if (tid == 0) o.cu_seqlens_k[0] = 0;
  for (int q = wave; q < pairs; q += n_waves) {
    const int c = q / p.H, h = q % p.H;
    const int32_t b = len[q];
    const int32_t n = emit_pair<true>(p, st[h], vcs + h * 3, mts + h * p.MMB, c, h, q * p.S, b, o);
    if (lane == 0) o.cu_seqlens_k[q + 1] = b + n;
  }
  if (tid == 0 && total_out) *total_out = part[0];
}

// ---------------------------------------------------------------------------
// 3D RoPE on one 16-byte chunk (8 bf16 = 4 complex pairs) of a K row
// (pyramidkv_pack.cu:114-161, rope.py:18-68)
// ---------------------------------------------------------------------------
struct Rope {
  const float *ft, *fy, *fx;
  int ft_rows, ft_cols, fy_rows, fy_cols, fx_rows, fx_cols;
};

__device__ inline int clamp_row(int64_t v, int rows) {
  int r = static_cast<int>(v);
  if (r < 0) r = 0;
  if (r >= rows) r = rows - 1;
  return r;
}

// The complex product is evaluated as (kr*fr - ki*fi, kr*fi + ki*fr) with
// every product and sum individually rounded (explicit round-to-nearest
// operations, no FMA contraction), the formula the CPU restatement uses;
// results round to bf16 RNE.
__device__ inline uint4 rope_chunk(uint4 raw, int chunk, int64_t t, int64_t y, int64_t x, const Rope &r) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  uint32_t o[4];
  const int rt = clamp_row(t, r.ft_rows), ry = clamp_row(y, r.fy_rows), rx = clamp_row(x, r.fx_rows);
  const int fy_end = r.ft_cols + r.fy_cols;
  for (int e = 0; e < 4; ++e) {
    const int pidx = chunk * 4 + e;
    const float *tab;
    if (pidx < r.ft_cols)
      tab = r.ft + (static_cast<int64_t>(rt) * r.ft_cols + pidx) * 2;
    else if (pidx < fy_end)
      tab = r.fy + (static_cast<int64_t>(ry) * r.fy_cols + (pidx - r.ft_cols)) * 2;
    else
      tab = r.fx + (static_cast<int64_t>(rx) * r.fx_cols + (pidx - fy_end)) * 2;
    const float2 f = *reinterpret_cast<const float2 *>(tab);
    const float kr = bf16_to_f32(static_cast<uint16_t>(w[e] & 0xffff));
    const float ki = bf16_to_f32(static_cast<uint16_t>(w[e] >> 16));
    const float a = __fmul_rn(kr, f.x), b = __fmul_rn(ki, f.y);
    const float c = __fmul_rn(kr, f.y), d = __fmul_rn(ki, f.x);
    o[e] = pack_bf16x2(__fsub_rn(a, b), __fadd_rn(c, d));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// The table entry of complex pair e of a chunk: pairs [0, ft_cols) use the
// t table, the next fy_cols the y table, the rest the x table; sel names
// the coordinate (0 t, 1 y, 2 x) whose clamped row indexes it.
struct PairTab {
  const float *p;  // table base + 2 * column
  int stride;      // floats per table row
  int sel;
};
__device__ inline PairTab pair_tab(int chunk, int e, const Rope &r) {
  const int pidx = chunk * 4 + e, fy_end = r.ft_cols + r.fy_cols;
  if (pidx < r.ft_cols) return PairTab{r.ft + 2 * pidx, 2 * r.ft_cols, 0};
  if (pidx < fy_end) return PairTab{r.fy + 2 * (pidx - r.ft_cols), 2 * r.fy_cols, 1};
  return PairTab{r.fx + 2 * (pidx - fy_end), 2 * r.fx_cols, 2};
}

// f32 pair -> bf16x2 by the hardware round-to-nearest-even conversion, with
// any NaN half replaced by 0x7fc0: the same bits as pack_bf16x2
__device__ inline uint32_t cvt_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffu) > 0x7f80u) u = (u & 0xffff0000u) | 0x7fc0u;
  if ((u & 0x7fff0000u) > 0x7f800000u) u = (u & 0xffffu) | 0x7fc00000u;
  return u;
}

// rope_chunk with the table entries of the chunk's 4 pairs resolved
// (tabs) and the clamped rows of the token's (t, y, x) given
__device__ inline uint4 rope_chunk_rows(uint4 raw, const PairTab (&tabs)[4], const int (&rows)[3]) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float2 f[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = tabs[e].sel == 0 ? rows[0] : (tabs[e].sel == 1 ? rows[1] : rows[2]);
    f[e] = *reinterpret_cast<const float2 *>(tabs[e].p + row * tabs[e].stride);
  }
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float kr = bf16_to_f32(static_cast<uint16_t>(w[e] & 0xffff));
    const float ki = bf16_to_f32(static_cast<uint16_t>(w[e] >> 16));
    const float a = __fmul_rn(kr, f[e].x), b = __fmul_rn(ki, f[e].y);
    const float c = __fmul_rn(kr, f[e].y), d = __fmul_rn(ki, f[e].x);
    o[e] = cvt_bf16x2(__fsub_rn(a, b), __fadd_rn(c, d));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ inline uint4 ld16(const uint16_t *p) { return *reinterpret_cast<const uint4 *>(p); }

__device__ inline void st16(uint16_t *p, uint4 v) { *reinterpret_cast<uint4 *>(p) = v; }
// streaming store (non-temporal): the flat K/V of one layer call is larger
// than the caches, so its lines are not kept
__device__ inline void st16_nt(uint16_t *p, uint4 v) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(p));
}

// ---------------------------------------------------------------------------
// pack
// ---------------------------------------------------------------------------
constexpr int kPackTok = 64;
constexpr int kPackThreads = 256;
constexpr int kPackPer = 4;  // 16-byte chunks per thread per round

struct PackArgs {
  const uint16_t *k[4], *v[4];
  const int64_t *pos[4];
  int64_t slots[4];
  uint16_t *k_out, *v_out;
  int64_t *pos_out;
  const int32_t *kind, *sg, *len, *dst;
  const int64_t *tremap;
  Rope rope;
  int fuse;  // rope tables + tremap present
  int n_seg, tiles_per_seg, FSEQ, MTPA, D;
  int64_t capacity;
};

__global__ void __launch_bounds__(kPackThreads) pack_kernel(PackArgs a) {
  // clamped RoPE table rows (t, y, x) of the tile's tokens
  __shared__ int s_rows[kPackTok][3];
  const int items = a.n_seg * a.tiles_per_seg;
  const int cpt = a.D / 8;
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    const int seg = it / a.tiles_per_seg, tile = it % a.tiles_per_seg;
    // every descriptor field is read before the first test, by scalar loads
    // in one round trip (seg < n_seg, so all of them are in bounds; the
    // descriptors do not change while the kernel runs)
    const int kind = ld_uniform(a.kind + seg);
    const int len = ld_uniform(a.len + seg);
    const int64_t sg = ld_uniform(a.sg + seg);
    const int64_t dst = ld_uniform(a.dst + seg);
    const int64_t tr_seg = a.fuse ? ld_uniform(a.tremap + seg) : -1;
    if (kind < 0 || kind > 3) continue;
    if (len <= 0 || tile * kPackTok >= len) continue;
    const int stride = (kind == PKV_SEG_MERGE) ? a.MTPA : a.FSEQ;
    // a segment starts at its slot and may run on through the following
    // slots of the pool (the legacy plan's whole-pool segments), never past
    // the pool's end
    if (sg < 0 || sg * stride + len > a.slots[kind] * stride || dst < 0 || dst + len > a.capacity || !a.k[kind])
      continue;
    const uint16_t *sk = a.k[kind] + sg * stride * a.D;
    const uint16_t *sv = a.v[kind] + sg * stride * a.D;
    const int64_t *sp = a.pos[kind] ? a.pos[kind] + sg * stride * 3 : nullptr;
    uint16_t *ok = a.k_out + dst * a.D;
    uint16_t *ov = a.v_out + dst * a.D;
    const bool rope = a.fuse && sp;  // uniform over the workgroup
    const int64_t tr = rope ? tr_seg : -1;
    // segments up to tiles_per_seg tiles long (every frame or merge anchor)
    // take one pass; longer ones are walked tiles_per_seg tiles at a time
    for (int tok0 = tile * kPackTok; tok0 < len; tok0 += a.tiles_per_seg * kPackTok) {
      const int ntok = min(kPackTok, len - tok0);
      const int n_items = ntok * cpt;
      if (rope) {
        // the tile's table rows, one thread per token (the positions are
        // read once per token instead of once per chunk)
        __syncthreads();  // the previous tile's readers are done
        for (int i = threadIdx.x; i < ntok; i += blockDim.x) {
          const int64_t *pp = sp + static_cast<int64_t>(tok0 + i) * 3;
          s_rows[i][0] = clamp_row(tr >= 0 ? tr : pp[0], a.rope.ft_rows);
          s_rows[i][1] = clamp_row(pp[1], a.rope.fy_rows);
          s_rows[i][2] = clamp_row(pp[2], a.rope.fx_rows);
        }
        __syncthreads();
      }
      // all of this thread's chunks of a round are loaded before any store
      // (up to kPackPer 16-byte K and V reads in flight per thread; one round
      // covers the tile for head_dim <= 128)
      for (int base = 0; base < n_items; base += kPackPer * kPackThreads) {
        uint4 kk[kPackPer], vv[kPackPer];
#pragma unroll
        for (int u = 0; u < kPackPer; ++u) {
          const int i = base + threadIdx.x + u * kPackThreads;
          if (i < n_items) {
            const int64_t e = static_cast<int64_t>(tok0 + i / cpt) * a.D + (i % cpt) * 8;
            kk[u] = ld16(sk + e);
            vv[u] = ld16(sv + e);
          }
        }
#pragma unroll
        for (int u = 0; u < kPackPer; ++u) {
          const int i = base + threadIdx.x + u * kPackThreads;
          if (i >= n_items) continue;
          const int tl = i / cpt, ch = i % cpt;
          const int64_t e = static_cast<int64_t>(tok0 + tl) * a.D + ch * 8;
          uint4 k4 = kk[u];
          if (rope) {
            const int rows[3] = {s_rows[tl][0], s_rows[tl][1], s_rows[tl][2]};
            PairTab t4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) t4[q] = pair_tab(ch, q, a.rope);
            k4 = rope_chunk_rows(k4, t4, rows);
          }
          st16_nt(ok + e, k4);
          st16_nt(ov + e, vv[u]);
        }
      }
      if (a.pos_out && sp) {
        int64_t *op = a.pos_out + dst * 3;
        for (int i = threadIdx.x; i < ntok * 3; i += blockDim.x) {
          const int64_t e = static_cast<int64_t>(tok0) * 3 + i;
          op[e] = sp[e];
        }
      }
    }  // tiles of a long segment
  }
}

__global__ void __launch_bounds__(kPackThreads) rope_kernel(const uint16_t *k, const int64_t *pos, int64_t n,
                                                            int D, Rope r, uint16_t *out) {
  const int cpt = D / 8;
  const int64_t total = n * cpt;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t tok = i / cpt;
    const int ch = static_cast<int>(i % cpt);
    const int64_t *pp = pos + tok * 3;
    const uint4 kk = ld16(k + tok * D + ch * 8);
    st16(out + tok * D + ch * 8, rope_chunk(kk, ch, pp[0], pp[1], pp[2], r));
  }
}

static int make_rope(const pkv_rope_tables *t, int D, Rope &r, const char *who) {
  if (!t->ft || !t->fy || !t->fx)
    return fail(PKV_ERR_INVALID, "%s: the t, y and x RoPE tables must all be given", who);
  if (t->ft_cols + t->fy_cols + t->fx_cols != D / 2)
    return fail(PKV_ERR_INVALID, "%s: RoPE table columns %d+%d+%d != head_dim/2 = %d", who, t->ft_cols,
                t->fy_cols, t->fx_cols, D / 2);
  if (t->ft_rows <= 0 || t->fy_rows <= 0 || t->fx_rows <= 0)
    return fail(PKV_ERR_INVALID, "%s: RoPE tables must have rows", who);
  if (t->ft_cols < 0 || t->fy_cols < 0 || t->fx_cols < 0)
    return fail(PKV_ERR_INVALID, "%s: negative RoPE table columns", who);
  r = Rope{t->ft, t->fy, t->fx, t->ft_rows, t->ft_cols, t->fy_rows, t->fy_cols, t->fx_rows, t->fx_cols};
  return PKV_OK;
}

}  // namespace pkv

using namespace pkv;

// Plan launch shared by mega_plan_multi (slot_layer < 0: per-layer slot ids,
// the reference op's output) and the fused plan + pack (slot ids offset to
// layer slot_layer of the [L, H, slots] pools).
static int plan_launch(const pkv_geometry *geo, const uint8_t *states_layer, const int64_t *valid_count_layer,
                       const int32_t *merge_token_count_layer, const int64_t *current_t_list, int32_t num_chunks,
                       const pkv_remap *remap, const pkv_plan_out *out, int32_t *total_tokens_out, int slot_layer,
                       hipStream_t st) {
  if (!geo || !states_layer || !valid_count_layer || !merge_token_count_layer || !current_t_list || !remap ||
      !out)
    return fail(PKV_ERR_INVALID, "mega_plan_multi: NULL argument");
  if (num_chunks <= 0) return fail(PKV_ERR_INVALID, "mega_plan_multi: empty current_t_list");
  if (num_chunks > kMaxPlanChunks)
    return fail(PKV_ERR_UNSUPPORTED, "mega_plan_multi: %d chunks exceed %d", num_chunks, kMaxPlanChunks);
  const int H = geo->num_heads;
  if (num_chunks * H > kMaxPlanPairs)
    return fail(PKV_ERR_UNSUPPORTED, "mega_plan_multi: %d (chunk, head) pairs exceed %d", num_chunks * H,
                kMaxPlanPairs);
  PlanParams p;
  p.H = H;
  p.S = geo->max_sink + geo->max_middle + geo->max_recent + geo->max_merge_blocks;
  p.FSEQ = geo->frame_seqlen;
  p.max_sink = geo->max_sink;
  p.max_middle = geo->max_middle;
  p.max_recent = geo->max_recent;
  p.MMB = geo->max_merge_blocks;
  p.C = num_chunks;
  const int32_t lay = slot_layer > 0 ? slot_layer : 0;
  p.slot_off[0] = lay * H * geo->max_sink;
  p.slot_off[1] = lay * H * geo->max_middle;
  p.slot_off[2] = lay * H * geo->max_recent;
  p.slot_off[3] = lay * H * geo->max_merge_blocks;
  for (int c = 0; c < num_chunks; ++c) {
    p.t[c] = current_t_list[c];
    p.sync_t[c] = map_sink_time(current_t_list[c], remap->sink_mode_code, remap->sink_clamp_min,
                                remap->sink_clamp_max, remap->decoupled_sink_lag);
  }
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, st, p,
                     reinterpret_cast<const HeadState *>(states_layer), valid_count_layer,
                     merge_token_count_layer, *out, total_tokens_out);
  int rc = check_launch("plan_kernel");
  if (rc) return rc;
  // Static bound on the packed tokens: every (chunk, head) emits at most S
  // segments of at most max(FSEQ, MTPA) tokens.  Only when that bound can
  // exceed the workspace is the actual total read back (one sync).
  const int64_t seg_max = geo->frame_seqlen > geo->max_merge_tokens ? geo->frame_seqlen : geo->max_merge_tokens;
  const int64_t bound = static_cast<int64_t>(num_chunks) * H *
                        ((geo->max_sink + geo->max_middle + geo->max_recent) * static_cast<int64_t>(geo->frame_seqlen) +
                         geo->max_merge_blocks * seg_max);
  if (bound > geo->max_pack_tokens) {
    // the actual total needs a host read; a stream under graph capture
    // cannot synchronise, so say why instead of invalidating the capture
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(PKV_ERR_UNSUPPORTED,
                  "mega_plan_multi: %d chunks may pack up to %lld tokens, more than the pack workspace (%lld), "
                  "and the actual total cannot be read back during graph capture: capture at most "
                  "max_attend_chunks chunks with frame_seqlen >= max_merge_tokens (%d)",
                  num_chunks, static_cast<long long>(bound), static_cast<long long>(geo->max_pack_tokens),
                  geo->max_merge_tokens);
    int32_t total = 0;
    if (hipMemcpyAsync(&total, out->cu_seqlens_k + num_chunks * H, sizeof(int32_t), hipMemcpyDeviceToHost, st) !=
            hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return fail(PKV_ERR_HIP, "mega_plan_multi: readback of the packed total failed");
    if (total > geo->max_pack_tokens)
      return fail(PKV_ERR_CAPACITY,
                  "mega_plan_multi: packed tokens (%d) exceed pack-workspace capacity (%lld). Either reduce "
                  "chunks (%d) or rebuild the manager with a larger max_attend_chunks.",
                  total, static_cast<long long>(geo->max_pack_tokens), num_chunks);
  }
  return PKV_OK;
}

extern "C" {

int pkv_plan_multi(const pkv_geometry *geo, const uint8_t *states_layer, const int64_t *valid_count_layer,
                   const int32_t *merge_token_count_layer, const int64_t *current_t_list, int32_t num_chunks,
                   const pkv_remap *remap, const pkv_plan_out *out, int32_t *total_tokens_out,
                   pkv_stream_t stream) {
  return plan_launch(geo, states_layer, valid_count_layer, merge_token_count_layer, current_t_list, num_chunks,
                     remap, out, total_tokens_out, -1, as_stream(stream));
}

int pkv_pack(const pkv_geometry *geo, const pkv_pools *pools, const int32_t *src_kind,
             const int32_t *src_slot_global, const int32_t *seg_lengths, const int32_t *dst_token_offsets,
             int32_t n_segments, const int64_t *anchor_t_remap, const pkv_rope_tables *rope,
             pkv_stream_t stream) {
  if (!geo || !pools) return fail(PKV_ERR_INVALID, "pyramidkv_pack: NULL geometry/pools");
  if (n_segments == 0) return PKV_OK;
  if (n_segments < 0 || !src_kind || !src_slot_global || !seg_lengths || !dst_token_offsets)
    return fail(PKV_ERR_INVALID, "pyramidkv_pack: bad descriptors");
  if (geo->head_dim % 8) return fail(PKV_ERR_INVALID, "pyramidkv_pack: head_dim must be a multiple of 8");
  if (!pools->k_flat_out || !pools->v_flat_out) return fail(PKV_ERR_INVALID, "pyramidkv_pack: no flat outputs");
  PackArgs a;
  const int64_t lh = static_cast<int64_t>(geo->num_layers) * geo->num_heads;
  a.k[0] = pools->sink_k; a.v[0] = pools->sink_v; a.pos[0] = pools->sink_pos; a.slots[0] = lh * geo->max_sink;
  a.k[1] = pools->middle_k; a.v[1] = pools->middle_v; a.pos[1] = pools->middle_pos; a.slots[1] = lh * geo->max_middle;
  a.k[2] = pools->recent_k; a.v[2] = pools->recent_v; a.pos[2] = pools->recent_pos; a.slots[2] = lh * geo->max_recent;
  a.k[3] = pools->merge_k; a.v[3] = pools->merge_v; a.pos[3] = pools->merge_pos; a.slots[3] = lh * geo->max_merge_blocks;
  a.k_out = pools->k_flat_out;
  a.v_out = pools->v_flat_out;
  a.pos_out = pools->pos_flat_out;
  a.kind = src_kind;
  a.sg = src_slot_global;
  a.len = seg_lengths;
  a.dst = dst_token_offsets;
  a.tremap = anchor_t_remap;
  a.fuse = 0;
  if (anchor_t_remap && rope) {
    int rc = make_rope(rope, geo->head_dim, a.rope, "pyramidkv_pack");
    if (rc) return rc;
    a.fuse = 1;
  }
  a.n_seg = n_segments;
  a.FSEQ = geo->frame_seqlen;
  a.MTPA = geo->max_merge_tokens;
  a.D = geo->head_dim;
  a.capacity = geo->max_pack_tokens;
  const int seg_max = geo->frame_seqlen > geo->max_merge_tokens ? geo->frame_seqlen : geo->max_merge_tokens;
  a.tiles_per_seg = (seg_max + kPackTok - 1) / kPackTok;
  const int64_t items = static_cast<int64_t>(n_segments) * a.tiles_per_seg;
  if (items > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "pyramidkv_pack: too many segments");
  const int grid = static_cast<int>(items);  // one workgroup per (segment, tile); inactive ones exit at once
  hipLaunchKernelGGL(pack_kernel, dim3(grid), dim3(kPackThreads), 0, as_stream(stream), a);
  return check_launch("pack_kernel");
}

int pkv_plan_pack(const pkv_geometry *geo, const pkv_pools *pools, const uint8_t *states_layer, int32_t layer,
                  const int64_t *current_t_list, int32_t num_chunks, const pkv_remap *remap,
                  const pkv_rope_tables *rope, const pkv_plan_out *plan_ws, pkv_stream_t stream) {
  if (!geo || !pools || !plan_ws || !pools->valid_count || !pools->merge_token_count)
    return fail(PKV_ERR_INVALID, "plan_pack: NULL argument");
  if (layer < 0 || layer >= geo->num_layers) return fail(PKV_ERR_INVALID, "plan_pack: layer out of range");
  const int H = geo->num_heads;
  const int S = geo->max_sink + geo->max_middle + geo->max_recent + geo->max_merge_blocks;
  hipStream_t st = as_stream(stream);
  int rc = plan_launch(geo, states_layer, pools->valid_count + static_cast<int64_t>(layer) * H * 3,
                       pools->merge_token_count + static_cast<int64_t>(layer) * H * geo->max_merge_blocks,
                       current_t_list, num_chunks, remap, plan_ws, nullptr, layer, st);
  if (rc) return rc;
  return pkv_pack(geo, pools, plan_ws->src_kind, plan_ws->src_slot_global, plan_ws->seg_lengths,
                  plan_ws->dst_token_offsets, num_chunks * H * S, rope ? plan_ws->anchor_t_remap : nullptr, rope,
                  stream);
}

int pkv_rope_apply(const uint16_t *k, const int64_t *pos, int64_t n_tokens, int32_t head_dim,
                   const pkv_rope_tables *rope, uint16_t *out, pkv_stream_t stream) {
  if (n_tokens == 0) return PKV_OK;
  if (!k || !pos || !rope || !out || n_tokens < 0 || head_dim <= 0 || head_dim % 8)
    return fail(PKV_ERR_INVALID, "rope_apply: bad arguments");
  Rope r;
  int rc = make_rope(rope, head_dim, r, "rope_apply");
  if (rc) return rc;
  const int64_t work = n_tokens * (head_dim / 8);
  int64_t blocks = (work + kPackThreads - 1) / kPackThreads;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(rope_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kPackThreads), 0, as_stream(stream), k,
                     pos, n_tokens, head_dim, r, out);
  return check_launch("rope_kernel");
}

}  // extern "C"
