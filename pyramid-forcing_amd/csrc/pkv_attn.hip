// Ragged-cache attention for gfx950: bf16 inputs, fp32 online softmax and
// accumulation, MFMA v_mfma_f32_32x32x16_bf16.  Replaces the reference's
// flash_attn_varlen_func call (pyramidkv/_mega_cache.py:540-559).
// head_dim 128 runs attn_p3_kernel (384 query rows per workgroup, three
// wave groups rotating between matrix work, exponentials and data movement)
// on launches of at least kP3MinGrid of its workgroups, else attn_pp_kernel
// (256 rows, two groups alternating between matrix work and data
// movement), both described at the kernel; head_dim 64 runs
// attn_fwd_kernel, described here.
//
// Work decomposition.  A workgroup of 8 waves owns 256 query rows (32 per
// wave) of one (query sequence, head) pair and streams that pair's keys in
// tiles of 64 through double-buffered LDS, one barrier per tile; one
// workgroup per CU, so every SIMD runs two waves (each within 256 registers)
// whose MFMA and softmax phases interleave.  All 512 threads stage both K and
// V: 16-byte buffer loads bounded at the sequence's last row (rows past the
// end read as zero), issued two iterations before their store, stored
// row-major into LDS with 16-byte stores.  Each staged tile serves 256 query
// rows, which halves the load and LDS-store traffic per flop of a 128-row
// workgroup.  The order of the work items balances the XCDs (balanced_item).
// In a sequence's last, partial query tile the waves without query rows only
// stage their share of the tiles, which leaves their SIMDs' matrix cores and
// the LDS read bandwidth to the waves that have rows.
//
// Software pipelining.  Iteration j computes S(j+1) = K(j+1) Q^T while the
// softmax of S(j), computed one iteration earlier, runs in the same basic
// block, then O += V(j)^T P(j).  K and V tiles therefore sit in LDS one tile
// apart (K(j+1) and V(j) during iteration j), in separate double buffers,
// still with one barrier per tile.
//
// Operand arrangement.  The wave computes S^T = K * Q^T (A = K rows read
// from LDS, B = Q^T kept in registers), so the 32x32 MFMA result gives every
// lane one query column and 16 keys of it: lane half hf holds keys
// {8*(i/4) + 4*hf + i%4 : i < 16} of a 32-key block.  O^T = V^T * P^T then
// takes P^T straight from those registers as the B operand (for each 16-key
// step, the lane's 8 keys in that order) and V^T as the A operand, read from
// the row-major V tile with the LDS transpose read ds_read_b64_tr_b16: in
// every 16-lane group, lane j addresses V[k0 + j/4][d0 + 4*(j%4)] and lane i
// receives V[k0 + r][d0 + i] for r = 0..3, i.e. one dim and four keys.
// O^T's accumulator again gives every lane one query column, so the row
// statistics need one half-wave exchange (v_permlane32_swap) and the rescale
// of O is lane-local.
//
// Softmax runs in the log2 domain (the scale is folded into one FMA before
// v_exp_f32).  Fast pass: each query row's reference m is the maximum of its
// first key tile and never moves, so the loop has no running maximum and O
// is never rescaled; P = 2^(S*c - m) stays below 2^kHeadroom unless a later
// key scores kHeadroom (log2 units) above the first tile.  A lane detects
// that from its probability sums (a P at or above the bound makes its sum
// reach it); the workgroup then recomputes its rows in a slow pass with the
// classic moving maximum and rescaled O.  Either way the final O / l is the
// exact softmax, with P rounded to bf16 for the P*V product and the row sums
// taken over the same rounded values (v_dot2c_f32_bf16 against (1, 1)), so
// numerator and denominator use identical weights.

#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "pkv_common.h"

namespace pkv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kBK = 64;  // keys per LDS tile
constexpr float kHeadroom = 64.0f;  // bound of log2(P) in the fast pass
// head_dim-128 kernels: a row sum in [2^kHeadroom, 2^kRebaseMax) after a
// tile is rescaled in place; one at or above 2^kRebaseMax (or not finite)
// sends the workgroup to the slow pass
constexpr float kRebaseMax = 96.0f;
constexpr int kSchedMax = 1024;  // sequences the XCD-balanced schedule handles

struct AttnParams {
  const uint16_t *q, *k, *v;
  uint16_t *o;
  const int32_t *cu_q, *cu_k;
  int Hq, kv_per_head, q_tiles, n_wg;
  int64_t q_tok, q_head, kv_tok, kv_head, o_tok, o_head;
  float scale_log2;
  // key-split launches (attn_p3_kernel<true> + attn_combine_kernel): the
  // per-item partial results and item records in the caller's workspace
  float *part;
  int4 *rec;
  int n_seq, n_cu;
  // queue launches of attn_p3_kernel<false> (one workgroup per compute
  // unit, items claimed from per-XCD counters): this stream's counter
  // block; null = one item per workgroup
  int *queue;
};

// Consecutive workgroup ids are dispatched round-robin over the 8 XCDs;
// renumber them so that XCD x runs the contiguous index range
// [start_x, start_x + count_x) of the work list, in increasing order.
__device__ inline int xcd_remap(int i, int n) {
  const int xcd = i % 8, k = i / 8;
  const int base = n / 8, rem = n % 8;
  return xcd < rem ? xcd * (base + 1) + k : rem * (base + 1) + (xcd - rem) * base + k;
}

// Work list of (sequence, query tile) items, computed by every workgroup in
// its prologue (a few microseconds, no workspace, no extra launch).  A
// sequence's cost is its query tiles times its key tiles.  Sequences are
// ranked by cost (largest first, ties by index) and dealt to 8 bins in snake
// order (ranks 0..7 to bins 0..7, ranks 8..15 to bins 7..0, ...), each bin
// keeping the ranked order; the list is the bins' items concatenated, a
// sequence's query tiles consecutive.  With xcd_remap each XCD then runs one
// bin: balanced work per XCD (its own L2 holds the keys its query tiles
// share) and the longest sequences first.  Every step is parallel over the
// sequences.  Returns false when this workgroup has no item.  scratch:
// 4 * kSchedMax ints of LDS, 16-byte aligned; every thread of the workgroup
// must call it.
__device__ inline int snake_bin(int p) { return ((p >> 3) & 1) ? 7 - (p & 7) : (p & 7); }

__device__ bool balanced_item(const int32_t *cu_q, const int32_t *cu_k, int Hq, int n_seq, int kv_per_head, int bq,
                              int c, int *scratch, int &seq_out, int &qt_out) {
  int *cost = scratch, *order = scratch + kSchedMax, *qts = scratch + 2 * kSchedMax, *off = scratch + 3 * kSchedMax;
  __shared__ int res[2];
  __shared__ int btot[8];
  const int n4 = (n_seq + 3) & ~3;
  for (int s = threadIdx.x; s < n4; s += blockDim.x) {
    int nq = 0, cs = -1;  // padding entries rank after every sequence
    if (s < n_seq) {
      const int b = s / Hq;
      nq = (cu_q[b + 1] - cu_q[b] + bq - 1) / bq;
      const int kv = kv_per_head ? s : b;
      cs = nq * ((cu_k[kv + 1] - cu_k[kv] + 63) / 64 + 1);  // +1: fixed cost per query tile
    }
    qts[s] = nq;
    cost[s] = cs;
  }
  if (threadIdx.x < 8) btot[threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    res[0] = -1;
    res[1] = 0;
  }
  __syncthreads();
  // rank = number of sequences before s in (cost desc, index asc) order;
  // the costs are read four at a time (the same address across the wave)
  for (int s = threadIdx.x; s < n_seq; s += blockDim.x) {
    const int cs = cost[s];
    int r = 0;
    const int4 *c4 = reinterpret_cast<const int4 *>(cost);
#pragma unroll 4
    for (int t4 = 0; t4 < n4 / 4; ++t4) {
      const int4 v = c4[t4];
      const int t = 4 * t4;
      r += (v.x > cs) || (v.x == cs && t < s);
      r += (v.y > cs) || (v.y == cs && t + 1 < s);
      r += (v.z > cs) || (v.z == cs && t + 2 < s);
      r += (v.w > cs) || (v.w == cs && t + 3 < s);
    }
    order[r] = s;
  }
  __syncthreads();
  // rank p: its bin, its item offset within the bin, the bin totals
  for (int p = threadIdx.x; p < n_seq; p += blockDim.x) {
    const int x = snake_bin(p), k = p >> 3;
    int o = 0;
#pragma unroll 4
    for (int kk = 0; kk < k; ++kk) o += qts[order[8 * kk + ((kk & 1) ? 7 - x : x)]];
    off[p] = o;
    atomicAdd(&btot[x], qts[order[p]]);
  }
  __syncthreads();
  for (int p = threadIdx.x; p < n_seq; p += blockDim.x) {
    const int x = snake_bin(p);
    int base = off[p];
    for (int xx = 0; xx < x; ++xx) base += btot[xx];
    const int sq = order[p];
    if (c >= base && c < base + qts[sq]) {
      res[0] = sq;
      res[1] = c - base;
    }
  }
  __syncthreads();
  seq_out = res[0];
  qt_out = res[1];
  return seq_out >= 0;
}

// ---- queue launches --------------------------------------------------------
// In a launch of one workgroup per item, the dispatcher hands an XCD's
// workgroups out in order, each to a shader engine it picks in turn; a
// workgroup whose engine has no free compute unit holds back every later
// one, so a unit that frees early can sit idle for tens of microseconds
// (measured: 2.3% of every unit's time over a rollout's attention, plus the
// ragged end of the launch).  A queue launch instead starts one workgroup
// per compute unit; each claims items one at a time from a counter of its
// own XCD's bin of the XCD-balanced order (the work list above, bin x =
// what XCD x runs in a launch of one workgroup per item) and, once that bin
// is empty, from the other bins in turn, so that units never wait on the
// dispatcher and a slower XCD's last items go to faster ones.
//
// Counter block (kQueueInts ints): claims of bin x at [x], x = 0..7;
// workgroups finished at [8].  The last workgroup to finish sets the block
// back to zero, so consecutive launches on one stream share it.
constexpr int kQueueInts = 32;

// The work list in bin-major order: bin x holds entries [start[x],
// start[x + 1]), each a sequence and the query tiles of the bin before it.
struct QueueTable {
  int seq[kSchedMax];
  int pre[kSchedMax];
  int start[9];
  int total[8];
};

// Builds the table from cu_q / cu_k (every workgroup, once per launch;
// every thread calls it).  scratch: 4 * kSchedMax ints of LDS.
__device__ void queue_table(const int32_t *cu_q, const int32_t *cu_k, int Hq, int n_seq, int kv_per_head, int bq,
                            int *scratch, QueueTable &tab) {
  int *cost = scratch, *order = scratch + kSchedMax, *qts = scratch + 2 * kSchedMax, *tq = scratch + 3 * kSchedMax;
  const int n4 = (n_seq + 3) & ~3;
  for (int s = threadIdx.x; s < n4; s += blockDim.x) {
    int nq = 0, cs = -1;  // padding entries rank after every sequence
    if (s < n_seq) {
      const int b = s / Hq;
      nq = (cu_q[b + 1] - cu_q[b] + bq - 1) / bq;
      const int kv = kv_per_head ? s : b;
      cs = nq * ((cu_k[kv + 1] - cu_k[kv] + 63) / 64 + 1);  // the cost balanced_item ranks by
    }
    qts[s] = nq;
    cost[s] = cs;
  }
  if (threadIdx.x < 9) {
    // bin x: one entry per full row of 8 ranks, and one in the last, partial
    // row when the snake order reaches it (rows run 0..7 and 7..0 in turn)
    const int rows = n_seq >> 3, rem = n_seq & 7;
    int st = 0;
    for (int x = 0; x < static_cast<int>(threadIdx.x); ++x) st += rows + ((rows & 1) ? (7 - x < rem) : (x < rem));
    tab.start[threadIdx.x] = st;
  }
  __syncthreads();
  for (int s = threadIdx.x; s < n_seq; s += blockDim.x) {
    const int cs = cost[s];
    int r = 0;
    const int4 *c4 = reinterpret_cast<const int4 *>(cost);
#pragma unroll 4
    for (int t4 = 0; t4 < n4 / 4; ++t4) {
      const int4 v = c4[t4];
      const int t = 4 * t4;
      r += (v.x > cs) || (v.x == cs && t < s);
      r += (v.y > cs) || (v.y == cs && t + 1 < s);
      r += (v.z > cs) || (v.z == cs && t + 2 < s);
      r += (v.w > cs) || (v.w == cs && t + 3 < s);
    }
    order[r] = s;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < n_seq; r += blockDim.x) {
    const int e = tab.start[snake_bin(r)] + (r >> 3);
    tab.seq[e] = order[r];
    tq[e] = qts[order[r]];
  }
  __syncthreads();
  if (threadIdx.x < 8) {
    int run = 0;
    for (int e = tab.start[threadIdx.x]; e < tab.start[threadIdx.x + 1]; ++e) {
      tab.pre[e] = run;
      run += tq[e];
    }
    tab.total[threadIdx.x] = run;
  }
  __syncthreads();
}

// Claims the next item (thread 0; the result reaches every thread): from
// this XCD's bin, else from bins x + 1, x + 2, ... (mod 8).  `spent` (thread
// 0's) holds the bins found empty.  The first barrier also ends the last
// item: no wave still reads its tiles when the next item's copies begin.
__device__ bool queue_next(int *queue, const QueueTable &tab, unsigned &spent, int &seq, int &qt) {
  __shared__ int pick[2];
  __syncthreads();
  if (threadIdx.x == 0) {
    int sq = -1, t = 0;
    const int x = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 7;  // HW_REG_XCC_ID, bits 3:0
    for (int d = 0; d < 8 && sq < 0; ++d) {
      const int y = (x + d) & 7;
      if (spent & (1u << y)) continue;
      const int n_y = tab.total[y];
      const int i = n_y > 0 ? __hip_atomic_fetch_add(queue + y, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
      if (i >= n_y) {
        spent |= 1u << y;
        continue;
      }
      // the bin's last entry whose tiles start at or before item i
      int lo = tab.start[y], hi = tab.start[y + 1] - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tab.pre[mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      sq = tab.seq[lo];
      t = i - tab.pre[lo];
    }
    pick[0] = sq;
    pick[1] = t;
  }
  __syncthreads();
  seq = pick[0];
  qt = pick[1];
  return seq >= 0;
}

// Counts the workgroup out; the last one clears the counters for the next
// launch on the stream (its acquire sees every other workgroup's claims).
__device__ void queue_done(int *queue) {
  if (threadIdx.x == 0) {
    const int d = __hip_atomic_fetch_add(queue + 8, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (d == static_cast<int>(gridDim.x) - 1) {
      for (int y = 0; y < 9; ++y) __hip_atomic_store(queue + y, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// One item of a key-split launch: query tile qt of sequence seq against key
// tiles [t_lo, t_hi) (32 keys each) of its k chunks (chunk j); the items of
// sequence seq are numbered base + j * nq + qt.
struct SplitItem {
  int seq, qt, j, k, nq, base, t_lo, t_hi;
};

constexpr int kSplitRows = 384;  // query rows per item (attn_p3_kernel's workgroup)
constexpr int kSplitKeys = 32;   // keys per key tile (attn_p3_kernel's kPK)

// Key-split plan, computed by every workgroup of the launch in its prologue
// (the same on each, from cu_q / cu_k alone).  Sequence s has nq_s query tiles
// of kSplitRows rows and nkt_s key tiles; its keys split into
// k_s = ceil(nkt_s / C) chunks of equal length (+-1 tile).  The chunk length
// C is chosen among ceil(nkt_max / k), k = 1 .. kSplitMaxChunks, as the one
// with the least estimated time ceil(items / n_cu) * (C + kSplitItemTiles)
// (rounds of items over the compute units, each item's fixed cost counted
// as kSplitItemTiles key tiles; fewer items on ties) among those with at
// most n_items items.  Items are ranked by chunk length (longest first, ties
// by sequence index), and a sequence's items ordered (chunk, query tile):
// the query tiles of one chunk are consecutive, so they run at the same time
// on one XCD and read the same keys through its L2.  Returns false when item
// c does not exist.  scratch: 6 * kSchedMax ints of LDS, 16-byte aligned;
// every thread must call it.
constexpr int kSplitMaxChunks = 8;
constexpr int kSplitItemTiles = 8;
__device__ bool split_item(const AttnParams &p, int n_items, int c, int *scratch, SplitItem &out) {
  const int n_seq = p.n_seq;
  int *nq = scratch, *nkt = scratch + kSchedMax, *cost = scratch + 2 * kSchedMax;
  int *order = scratch + 3 * kSchedMax, *items = scratch + 4 * kSchedMax, *kk = scratch + 5 * kSchedMax;
  __shared__ int acc[3];
  __shared__ SplitItem res;
  const int n4 = (n_seq + 3) & ~3;
  if (threadIdx.x == 0) {
    acc[0] = 1;  // largest nkt (at least 1)
    acc[1] = 0;
    res.seq = -1;
  }
  __syncthreads();
  for (int s = threadIdx.x; s < n4; s += blockDim.x) {
    int q = 0, t = 0;
    if (s < n_seq) {
      const int b = s / p.Hq;
      q = (p.cu_q[b + 1] - p.cu_q[b] + kSplitRows - 1) / kSplitRows;
      const int kv = p.kv_per_head ? s : b;
      t = (p.cu_k[kv + 1] - p.cu_k[kv] + kSplitKeys - 1) / kSplitKeys;
      if (q > 0) atomicMax(&acc[0], t);
    }
    nq[s] = q;
    nkt[s] = t;
  }
  __syncthreads();
  // chunk length: the candidate of least estimated time
  const int nkt_max = acc[0];
  int C = nkt_max;
  int64_t best = -1;
  for (int k1 = 1; k1 <= kSplitMaxChunks; ++k1) {
    const int cand = (nkt_max + k1 - 1) / k1;
    if (k1 > 1 && cand == (nkt_max + k1 - 2) / (k1 - 1)) continue;  // same length as k1 - 1
    if (threadIdx.x == 0) acc[1] = 0;
    __syncthreads();
    int part = 0;
    for (int s = threadIdx.x; s < n_seq; s += blockDim.x) part += nq[s] * max(1, (nkt[s] + cand - 1) / cand);
    if (part) atomicAdd(&acc[1], part);
    __syncthreads();
    const int n_it = acc[1];
    __syncthreads();
    if (n_it > n_items) break;  // more chunks only add items
    const int64_t t = static_cast<int64_t>((n_it + p.n_cu - 1) / p.n_cu) * (cand + kSplitItemTiles);
    if (best < 0 || t < best) {
      best = t;
      C = cand;
    }
  }
  for (int s = threadIdx.x; s < n4; s += blockDim.x) {
    int k = 1, cs = -1;
    if (s < n_seq && nq[s] > 0) {
      k = max(1, (nkt[s] + C - 1) / C);
      cs = (nkt[s] + k - 1) / k + 1;  // +1: fixed cost per item
    }
    kk[s] = k;
    cost[s] = cs;
    items[s] = s < n_seq ? nq[s] * k : 0;
  }
  __syncthreads();
  // rank = sequences before s in (cost desc, index asc) order
  for (int s = threadIdx.x; s < n_seq; s += blockDim.x) {
    const int cs = cost[s];
    int r = 0;
    for (int t = 0; t < n_seq; ++t) r += (cost[t] > cs) || (cost[t] == cs && t < s);
    order[r] = s;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < n_seq; r += blockDim.x) {
    int base = 0;
    for (int rr = 0; rr < r; ++rr) base += items[order[rr]];
    const int s = order[r];
    if (c >= base && c < base + items[s]) {
      const int local = c - base, q = nq[s], k = kk[s];
      res.seq = s;
      res.j = local / q;
      res.qt = local % q;
      res.k = k;
      res.nq = q;
      res.base = base;
      res.t_lo = static_cast<int>(static_cast<int64_t>(res.j) * nkt[s] / k);
      res.t_hi = static_cast<int>(static_cast<int64_t>(res.j + 1) * nkt[s] / k);
    }
  }
  __syncthreads();
  out = res;
  __syncthreads();  // the scratch is reused by the caller
  return out.seq >= 0;
}

__device__ inline uint4 ldg16(const uint16_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// Buffer resource word 3 for gfx9-family raw buffers (32-bit data format,
// no swizzle); out-of-range loads return zero.
constexpr int kRsrcWord3 = 0x00020000;
__device__ inline uint4 bload16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ inline bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// transpose read of 4 x 16 bits (see the operand arrangement above)
__device__ inline i16x4 lds_tr16(const uint16_t *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)((__attribute__((address_space(3))) char *)(p)));
}

// max / sum of x over lanes l and l^32 (v_permlane32_swap exchanges the two
// half-waves of its operands)
__device__ inline float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// x + the sum of the 8 bf16 values of p (two accumulation chains)
__device__ inline float bf16x8_sum(bf16x8 p, float x) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 one;
  one[0] = static_cast<__bf16>(1.0f);
  one[1] = one[0];
  const bf16x2 p0 = {p[0], p[1]}, p1 = {p[2], p[3]}, p2 = {p[4], p[5]}, p3 = {p[6], p[7]};
  const float a = __builtin_amdgcn_fdot2_f32_bf16(p0, one, x, false);
  const float b = __builtin_amdgcn_fdot2_f32_bf16(p1, one, 0.0f, false);
  return __builtin_amdgcn_fdot2_f32_bf16(p3, one, __builtin_amdgcn_fdot2_f32_bf16(p2, one, a, false), false) + b;
}

// x + the sum of the 8 bf16 values of p in one chain of four dot products
// (the running row sum itself is the accumulator: no partial sums to add)
__device__ inline float bf16x8_acc(bf16x8 p, float x) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 one;
  one[0] = static_cast<__bf16>(1.0f);
  one[1] = one[0];
  const bf16x2 p0 = {p[0], p[1]}, p1 = {p[2], p[3]}, p2 = {p[4], p[5]}, p3 = {p[6], p[7]};
  x = __builtin_amdgcn_fdot2_f32_bf16(p0, one, x, false);
  x = __builtin_amdgcn_fdot2_f32_bf16(p1, one, x, false);
  x = __builtin_amdgcn_fdot2_f32_bf16(p2, one, x, false);
  return __builtin_amdgcn_fdot2_f32_bf16(p3, one, x, false);
}

__device__ inline float half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int D>
__global__ void __launch_bounds__(kThreads, 1) attn_fwd_kernel(AttnParams p) {
  constexpr int BQ = 32 * kWaves;
  constexpr int DS = D / 16;  // k-steps of the QK^T product
  constexpr int DB = D / 32;  // 32-row blocks of O^T
  // LDS row strides (elements).  K rows are read 16 bytes per lane, 32
  // rows at a time: +16 B per row puts 16 consecutive rows on distinct
  // banks.  V rows are read by the transpose read, 4 rows x 64 B per 32
  // lanes: +64 B per row puts those 4 rows on distinct banks.
  constexpr int RS = D + 8;
  constexpr int RSV = D + 32;
  constexpr int KCH = D / 8;  // 16-byte chunks per row
  constexpr int LD = kBK * KCH / kThreads;  // 16-byte loads per thread per tile, each of K and V
  static_assert(LD * kThreads == kBK * KCH && LD <= 4, "tile split");
  static_assert(2 * kBK * RS * 2 >= 4 * kSchedMax * 4, "schedule scratch fits in the K tiles");
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBK * RS];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kBK * RSV];

  int seq, qt;
  const int n_seq = p.n_wg / p.q_tiles;
  if (n_seq <= kSchedMax) {
    // the schedule's scratch is the K tiles, not yet in use
    // (its last barrier orders every scratch read before the first K store)
    if (!balanced_item(p.cu_q, p.cu_k, p.Hq, n_seq, p.kv_per_head, BQ, xcd_remap(blockIdx.x, p.n_wg),
                       reinterpret_cast<int *>(&Ks[0][0]), seq, qt))
      return;
  } else {
    const int wg = xcd_remap(blockIdx.x, p.n_wg);
    seq = wg / p.q_tiles;
    qt = wg % p.q_tiles;
  }
  const int b = seq / p.Hq, h = seq % p.Hq;
  const int q_begin = p.cu_q[b];
  const int Lq = p.cu_q[b + 1] - q_begin;
  const int q0 = qt * BQ;
  if (q0 >= Lq) return;
  const int kv_idx = p.kv_per_head ? seq : b;
  const int k_begin = p.cu_k[kv_idx];
  const int Lk = p.cu_k[kv_idx + 1] - k_begin;

  const uint16_t *qp = p.q + static_cast<int64_t>(q_begin) * p.q_tok + h * p.q_head;
  const int64_t kv_off = static_cast<int64_t>(k_begin) * p.kv_tok + (p.kv_per_head ? 0 : h * p.kv_head);
  const uint16_t *kp = p.k + kv_off;
  const uint16_t *vp = p.v + kv_off;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lq = lane & 31, hf = lane >> 5;
  const int row_q = q0 + wave * 32 + lq;
  // the wave holds query rows (a partial last query tile leaves the later
  // waves without any); decided on a scalar copy of the wave index, so the
  // branch is uniform
  const bool wave_rows = q0 + __builtin_amdgcn_readfirstlane(wave) * 32 < Lq;
  const float c = p.scale_log2;

  // ---- Q^T operand, resident for the whole key loop
  bf16x8 qr[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row_q < Lq) v = ldg16(qp + static_cast<int64_t>(row_q) * p.q_tok + 16 * s + 8 * hf);
    qr[s] = as_bf16x8(v);
  }
  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  // ---- K/V staging through buffer resources based at the tile's first row
  // and bounded at the sequence's last row: rows past Lk read as zero
  // without a branch, no access can leave the sequence, and offsets stay
  // within one tile whatever the sequence length
  const int64_t row_elems = p.kv_tok;
  const int row_bytes = static_cast<int>(row_elems) * 2;
  // Two register sets of staged K and V rows; see the loop below for which
  // tiles they hold.  A tile at or past the sequence's end gets a resource
  // with no records: its loads return zero without touching memory, so every
  // tile is loaded unconditionally (no branch around a load keeps the
  // compiler's outstanding-load accounting exact, and each wait covers only
  // the rows that are about to be stored).
  uint4 sk[2][LD], sv[2][LD];
  // S^T for the 32 keys kb*32.. of the K tile in buf
  auto qk = [&](int buf, int kb) {
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4 *>(&Ks[buf][(kb * 32 + lq) * RS + 16 * s + 8 * hf]));
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qr[s], acc, 0, 0, 0);
    }
    return acc;
  };

  // V^T fragment addresses: key row 4*hf + (lane%16)/4 (+8 for the second
  // half of a 16-key step), dim column 16*((lane/16)%2) + 4*(lane%4)
  const int v_row = 4 * hf + ((lane & 15) >> 2);
  const int v_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // resource for the rows of tile kt of a K or V sequence
  auto tile_rsrc = [&](const uint16_t *seq_base, int kt) {
    const int64_t first = static_cast<int64_t>(kt) * kBK;
    const int64_t left = (static_cast<int64_t>(Lk) - first) * row_elems * 2;
    const int nrec = static_cast<int>(left <= 0 ? 0 : (left < 0x7fffffff ? left : 0x7fffffff));
    const int64_t base = left <= 0 ? 0 : first * row_elems;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(seq_base + base), 0, nrec, kRsrcWord3);
  };
  auto load_rows = [&](const uint16_t *seq_base, int kt, uint4 (&x4)[LD]) {
    const __amdgpu_buffer_rsrc_t r = tile_rsrc(seq_base, kt);
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int idx = tid + i * kThreads;
      x4[i] = bload16(r, (idx / KCH) * row_bytes + (idx % KCH) * 16);
    }
  };
  auto load_k = [&](int kt, uint4 (&k4)[LD]) { load_rows(kp, kt, k4); };
  auto load_v = [&](int kt, uint4 (&v4)[LD]) { load_rows(vp, kt, v4); };
  auto store_k = [&](int buf, const uint4 (&k4)[LD]) {
#pragma unroll
    for (int r = 0; r < LD; ++r) {
      const int idx = tid + r * kThreads;
      *reinterpret_cast<uint4 *>(&Ks[buf][(idx / KCH) * RS + (idx % KCH) * 8]) = k4[r];
    }
  };
  auto store_v = [&](int buf, const uint4 (&v4)[LD]) {
#pragma unroll
    for (int r = 0; r < LD; ++r) {
      const int idx = tid + r * kThreads;
      *reinterpret_cast<uint4 *>(&Vs[buf][(idx / KCH) * RSV + (idx % KCH) * 8]) = v4[r];
    }
  };

  // scores of keys past the sequence's end in the tile at key kb0 -> -inf
  auto mask = [&](f32x16 &c0, f32x16 &c1, int kb0) {
    if (kb0 + kBK > Lk) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb0 + 8 * (i / 4) + 4 * hf + (i % 4);
        if (key >= Lk) c0[i] = -INFINITY;
        if (key + 32 >= Lk) c1[i] = -INFINITY;
      }
    }
  };
  // the row maximum of a tile (scaled to the log2 domain)
  auto tile_max = [&](const f32x16 &c0, const f32x16 &c1) {
    float mq[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      mq[r] = fmaxf(c0[r], c1[r]);
#pragma unroll
      for (int i = r + 4; i < 16; i += 4) mq[r] = fmaxf(mq[r], fmaxf(c0[i], c1[i]));
    }
    return half_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) * c;
  };
  // P = 2^(S*c - mr) as bf16 B operands (for each 16-key step, the lane's 8
  // keys in the operand order); returns the lane's sum of its 32 P
  auto probs = [&](const f32x16 &c0, const f32x16 &c1, float mr, bf16x8 (&pb)[4]) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const float sv_ = ks < 2 ? c0[8 * ks + jj] : c1[8 * (ks - 2) + jj];
        pb[ks][jj] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(sv_, c, -mr)));
      }
    return bf16x8_sum(pb[0], 0.0f) + bf16x8_sum(pb[2], bf16x8_sum(pb[1], 0.0f) + bf16x8_sum(pb[3], 0.0f));
  };
  // O^T += V^T P^T from V tile buffer vb
  auto pv = [&](int vb, const bf16x8 (&pb)[4]) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint16_t *vptr = &Vs[vb][(16 * ks + v_row) * RSV + db * 32 + v_col];
        const i16x4 lo = lds_tr16(vptr), hi = lds_tr16(vptr + 8 * RSV);
        const i16x4 a8[2] = {lo, hi};
        const bf16x8 a = __builtin_bit_cast(bf16x8, a8);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ks], o[db], 0, 0, 0);
      }
  };

  __shared__ int ovf_any;
  if (tid == 0) ovf_any = 0;
  const int n_pairs = (Lk + 2 * kBK - 1) / (2 * kBK);
  if (n_pairs > 0) {
    // prologue: K0 -> Ks[0], V0 -> Vs[0], K1 -> Ks[1]; register set 0
    // holds (K2, V1), set 1 (K3, V2); S(0) from Ks[0]
    load_k(0, sk[0]);
    load_v(0, sv[0]);
    store_k(0, sk[0]);
    store_v(0, sv[0]);
    load_k(1, sk[1]);
    store_k(1, sk[1]);
    __builtin_amdgcn_sched_barrier(0);
    load_k(2, sk[0]);
    load_v(1, sv[0]);
    __builtin_amdgcn_sched_barrier(0);
    load_k(3, sk[1]);
    load_v(2, sv[1]);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    bool ovf = false;
    if (wave_rows) {
      f32x16 sa0 = qk(0, 0), sa1 = qk(0, 1), sb0, sb1;
      mask(sa0, sa1, 0);
      m = tile_max(sa0, sa1);  // finite: the first tile holds key 0

      // iteration j: Ks[(j+1)%2] = K(j+1), Vs[j%2] = V(j), (c0, c1) = S(j);
      // register set j%2 holds (K(j+2), V(j+1)), stored now, then refilled
      // with (K(j+4), V(j+3)); S(j+1) is computed while S(j) goes through the
      // exponentials, then O += V(j)^T P(j)
      auto step = [&](int j, f32x16 &c0, f32x16 &c1, f32x16 &n0, f32x16 &n1, uint4 (&k4)[LD],
                      uint4 (&v4)[LD]) {
        __syncthreads();
        store_k(j & 1, k4);
        store_v((j + 1) & 1, v4);
        load_k(j + 4, k4);
        load_v(j + 3, v4);
        mask(c0, c1, j * kBK);
        // ---- one block: S(j+1) MFMAs interleaved with the exponentials of S(j)
        n0 = qk((j + 1) & 1, 0);
        n1 = qk((j + 1) & 1, 1);
        bf16x8 pb[4];
        const float ps = probs(c0, c1, m, pb);
        l += ps;
        ovf |= !(ps < exp2f(kHeadroom));
        pv(j & 1, pb);
      };
      for (int pr = 0; pr < n_pairs; ++pr) {
        step(2 * pr, sa0, sa1, sb0, sb1, sk[0], sv[0]);
        step(2 * pr + 1, sb0, sb1, sa0, sa1, sk[1], sv[1]);
      }
    } else {
      // no query row in this wave: stage its share of every tile, with the
      // same barriers as the steps above
      for (int pr = 0; pr < n_pairs; ++pr) {
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
          const int j = 2 * pr + hs;
          __syncthreads();
          store_k(j & 1, sk[hs]);
          store_v((j + 1) & 1, sv[hs]);
          load_k(j + 4, sk[hs]);
          load_v(j + 3, sv[hs]);
        }
      }
    }
    if (ovf) ovf_any = 1;
    __syncthreads();
    if (ovf_any) {
      // ---- slow pass: a later key outscored the first tile by kHeadroom.
      // One tile at a time through buffer 0, online softmax with a moving
      // maximum and O rescaled when it moves.
      m = -INFINITY;
      l = 0.0f;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
      for (int kt = 0; kt < 2 * n_pairs; ++kt) {
        __syncthreads();
        load_k(kt, sk[0]);
        load_v(kt, sv[0]);
        store_k(0, sk[0]);
        store_v(0, sv[0]);
        __syncthreads();
        if (!wave_rows) continue;
        f32x16 c0 = qk(0, 0), c1 = qk(0, 1);
        mask(c0, c1, kt * kBK);
        const float m_new = fmaxf(m, tile_max(c0, c1));
        const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
        m = m_new;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        bf16x8 pb[4];
        l = l * alpha + probs(c0, c1, m, pb);
        pv(0, pb);
      }
    }
  }

  // ---- epilogue: O = O^T / l, rows of 4 consecutive dims per store
  uint16_t *op = p.o + static_cast<int64_t>(q_begin) * p.o_tok + h * p.o_head;
  const float lt = half_sum(l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (row_q < Lq) {
    uint16_t *orow = op + static_cast<int64_t>(row_q) * p.o_tok;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<__bf16>(o[db][4 * g + e] * inv);
        *reinterpret_cast<bf16x4 *>(orow + d) = v;
      }
  }
}

// ---------------------------------------------------------------------------
// Two-group ping-pong kernel (head_dim 128)
// ---------------------------------------------------------------------------
// The 8 waves form two groups of four, one wave of each group per SIMD
// (wave w runs on SIMD w % 4; group 0 = waves 0-3, group 1 = waves 4-7).
// Keys stream in tiles of 32.  Every tile takes four barrier-separated
// intervals, and the two groups run the same per-tile program one interval
// apart, so in every interval one wave of each SIMD issues matrix
// instructions while the other moves data:
//
//   interval    group 0                           group 1
//   I0          S(t+1) = K(t+1) Q^T, P(t) = exp   K(t+1) LDS -> regs, DMA K(t+4)
//   I1          V(t) LDS -> regs, DMA K(t+4)      S(t+1), P(t)
//   I2          O += V(t)^T P(t)                  V(t) LDS -> regs, DMA V(t+3)
//   I3          K(t+2) LDS -> regs, DMA V(t+3)    O += V(t)^T P(t)
//
// The exponentials of P(t) are interleaved with the MFMAs of S(t+1) in the
// same wave.  K and V tiles reach LDS through buffer loads that write LDS
// directly (no staging registers), four slots per operand, each slot a
// separate LDS array so the compiler's wait-count bookkeeping can tell the
// slots apart.  Each wave copies 4 rows of each tile; rows are 256 bytes
// with the 16-byte chunks XOR-swizzled (K: chunk ^ (row % 16), V: chunk ^
// 4 * (row % 4)) so that the fragment reads of 32 rows (K) and the transpose
// reads of 8 rows (V) spread over all banks.  A wave waits for its own
// copies (vmcnt) before the barrier that precedes the first read of that
// tile by any wave.  Softmax, the fast / slow pass split and the operand
// arrangement are those of attn_fwd_kernel.
constexpr int kPK = 32;                 // keys per tile
constexpr int kPRow = 256;              // LDS bytes per key row (128 bf16)
constexpr int kPTileElems = kPK * 128;  // bf16 elements per tile
static_assert(kPK == kSplitKeys, "the key-split plan counts attn_p3_kernel's key tiles");

typedef __attribute__((address_space(3))) char lds_char;
typedef int i32x4 __attribute__((ext_vector_type(4)));

template <int N>
using ic = std::integral_constant<int, N>;

// s_waitcnt on vmcnt only (gfx9 encoding: vmcnt[3:0] | expcnt 7 << 4 |
// lgkmcnt 15 << 8 | vmcnt[5:4] << 14)
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// workgroup barrier that no instruction is moved across (memory operations
// by the compiler fence, everything else by the scheduling barriers), so each
// interval's instructions stay between its two barriers
__device__ inline void pp_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

__global__ void __launch_bounds__(kThreads, 1) attn_pp_kernel(AttnParams p) {
  constexpr int D = 128;
  __shared__ __attribute__((aligned(16))) uint16_t Ka[kPTileElems], Kb[kPTileElems], Kc[kPTileElems], Kd[kPTileElems];
  __shared__ __attribute__((aligned(16))) uint16_t Va[kPTileElems], Vb[kPTileElems], Vc[kPTileElems], Vd[kPTileElems];
  __shared__ __attribute__((aligned(16))) int sched[4 * kSchedMax];
  auto kslot = [&](auto s) -> uint16_t * {
    constexpr int S = decltype(s)::value & 3;
    if constexpr (S == 0) return Ka;
    else if constexpr (S == 1) return Kb;
    else if constexpr (S == 2) return Kc;
    else return Kd;
  };
  auto vslot = [&](auto s) -> uint16_t * {
    constexpr int S = decltype(s)::value & 3;
    if constexpr (S == 0) return Va;
    else if constexpr (S == 1) return Vb;
    else if constexpr (S == 2) return Vc;
    else return Vd;
  };

  int seq, qt;
  const int n_seq = p.n_wg / p.q_tiles;
  if (n_seq <= kSchedMax) {
    if (!balanced_item(p.cu_q, p.cu_k, p.Hq, n_seq, p.kv_per_head, 32 * kWaves, xcd_remap(blockIdx.x, p.n_wg),
                       sched, seq, qt))
      return;
  } else {
    const int wg = xcd_remap(blockIdx.x, p.n_wg);
    seq = wg / p.q_tiles;
    qt = wg % p.q_tiles;
  }
  const int b = seq / p.Hq, h = seq % p.Hq;
  const int q_begin = p.cu_q[b];
  const int Lq = p.cu_q[b + 1] - q_begin;
  const int q0 = qt * 32 * kWaves;
  if (q0 >= Lq) return;
  const int kv_idx = p.kv_per_head ? seq : b;
  const int k_begin = p.cu_k[kv_idx];
  const int Lk = p.cu_k[kv_idx + 1] - k_begin;
  const uint16_t *qp = p.q + static_cast<int64_t>(q_begin) * p.q_tok + h * p.q_head;
  const int64_t kv_off = static_cast<int64_t>(k_begin) * p.kv_tok + (p.kv_per_head ? 0 : h * p.kv_head);
  const uint16_t *kp = p.k + kv_off;
  const uint16_t *vp = p.v + kv_off;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int grp = wave_s >> 2, wq = wave_s & 3;
  const int lq = lane & 31, hf = lane >> 5;
  const int row_q = q0 + wave * 32 + lq;
  const bool wave_rows = q0 + wave_s * 32 < Lq;
  const float c = p.scale_log2;

  bf16x8 qr[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row_q < Lq) v = ldg16(qp + static_cast<int64_t>(row_q) * p.q_tok + 16 * s + 8 * hf);
    qr[s] = as_bf16x8(v);
  }
  // Q is in registers before the first tile copy is issued: the compiler,
  // which cannot see the copies, then has no load of its own pending in the
  // key loop, where a wait for one would also wait for every copy in flight
  wait_vm<0>();
  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  const int nT = (Lk + kPK - 1) / kPK;

  // ---- tile copies: buffer resources based at the tile's first row and
  // bounded at the sequence's last row (rows past the end, and tiles past
  // the end, copy zeros)
  const int64_t row_elems = p.kv_tok;
  const int row_bytes = static_cast<int>(row_elems) * 2;
  // this wave copies rows 16*grp + 4*wq .. +3 of every tile; lane i the
  // 16-byte position i % 16 of row i / 16 of them
  const int dma_row = 16 * grp + 4 * wq + (lane >> 4);
  const int dma_pos = lane & 15;
  const int k_voff = dma_row * row_bytes + 16 * (dma_pos ^ (dma_row & 15));
  const int v_voff = dma_row * row_bytes + 16 * (dma_pos ^ (4 * (dma_row & 3)));
  const int dma_lds = (16 * grp + 4 * wq) * kPRow;
  // The copies are issued as inline assembly: the compiler then inserts no
  // wait of its own before the LDS reads of the slots (its bookkeeping
  // cannot follow the slots around the loop and waits far too early).  Every
  // wait for them is explicit; the compiler's waits for its own loads stay
  // correct, since those only ever have more, not fewer, loads after them.
  auto dma = [&](const uint16_t *base, int kt, uint16_t *slot, int voff) {
    const int64_t first = static_cast<int64_t>(kt) * kPK;
    const int64_t left = (static_cast<int64_t>(Lk) - first) * row_elems * 2;
    const int nrec = static_cast<int>(left <= 0 ? 0 : (left < 0x7fffffff ? left : 0x7fffffff));
    const uint64_t addr = reinterpret_cast<uint64_t>(base + (left <= 0 ? 0 : first * row_elems));
    i32x4 rsrc;
    rsrc[0] = static_cast<int>(addr & 0xffffffffu);
    rsrc[1] = static_cast<int>((addr >> 32) & 0xffffu);
    rsrc[2] = nrec;
    rsrc[3] = kRsrcWord3;
    const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char *)slot)) + dma_lds;
    // m0 is reserved to the compiler, which uses it nowhere else in this
    // kernel (the listing has no other m0 access)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
#pragma clang diagnostic pop
  };
  auto dma_k = [&](uint16_t *slot, int kt) { dma(kp, kt, slot, k_voff); };
  auto dma_v = [&](uint16_t *slot, int kt) { dma(vp, kt, slot, v_voff); };

  // ---- fragment reads
  // K: step s reads row lq, 16-byte chunk 2s + hf (swizzled)
  int kaddr[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) kaddr[s] = lq * kPRow + 16 * ((2 * s + hf) ^ (lq & 15));
  // V^T: key row 4*hf + (lane%16)/4 (+8, +16*ks), dims 32*db + v_col..+3
  const int v_row = 4 * hf + ((lane & 15) >> 2);
  const int v_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  int vaddr[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
    vaddr[db] = v_row * kPRow + 16 * ((4 * db + v_col / 8) ^ (4 * (v_row & 3))) + 2 * (v_col % 8);
  uint4 kreg[8];
  i16x4 vreg[2][4][2];
  auto load_k = [&](const uint16_t *slot) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
      kreg[s] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const char *>(slot) + kaddr[s]);
  };
  auto load_v = [&](const uint16_t *slot) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint16_t *ptr = reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(slot) + vaddr[db] +
                                                                 ks * 16 * kPRow);
        vreg[ks][db][0] = lds_tr16(ptr);
        vreg[ks][db][1] = lds_tr16(ptr + 8 * kPRow / 2);
      }
  };
  // S^T of the 32 keys in kreg
  auto gemm0 = [&](f32x16 &acc) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kreg[s]), qr[s], acc, 0, 0, 0);
  };
  // O^T += V^T P^T
  auto gemm1 = [&](const bf16x8 (&pb)[2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const i16x4 a8[2] = {vreg[ks][db][0], vreg[ks][db][1]};
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a8), pb[ks], o[db], 0, 0, 0);
      }
  };
  // keys past the sequence's end in the tile at key kb0 -> -inf
  // (a branch the compiler does not flatten: the volatile asm cannot be
  // speculated, so full tiles skip the compares)
  auto mask = [&](f32x16 &s, int kb0) {
    if (kb0 + kPK > Lk) {
      asm volatile("");
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (kb0 + 8 * (i / 4) + 4 * hf + (i % 4) >= Lk) s[i] = -INFINITY;
    }
  };
  auto tile_max = [&](const f32x16 &s) {
    float mq[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) mq[r] = fmaxf(fmaxf(s[r], s[r + 4]), fmaxf(s[r + 8], s[r + 12]));
    return half_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) * c;
  };
  // slow pass: P = 2^(S*c - mr) as the two 16-key B operands; returns the
  // lane's sum
  auto probs = [&](const f32x16 &s, float mr, bf16x8 (&pb)[2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        pb[ks][jj] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(s[8 * ks + jj], c, -mr)));
    return bf16x8_sum(pb[0], 0.0f) + bf16x8_sum(pb[1], 0.0f);
  };
  // fast pass: P = 2^(S*c - m) against the row's reference m, added to the
  // running sum (one chain of dot products)
  auto probs_fast = [&](const f32x16 &s, bf16x8 (&pb)[2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        pb[ks][jj] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(s[8 * ks + jj], c, -m)));
    l = bf16x8_acc(pb[1], bf16x8_acc(pb[0], l));
  };

  __shared__ int ovf_any;
  if (tid == 0) ovf_any = 0;
  bool ovf = false;
  if (nT > 0) {
    // prologue: copies of K0, K1, V0, K2, V1, K3, V2 (the order in which the
    // loop's iterations -4 .. -1 would have issued them), S(0), m and K(1)
    dma_k(Ka, 0);
    dma_k(Kb, 1);
    dma_v(Va, 0);
    dma_k(Kc, 2);
    dma_v(Vb, 1);
    dma_k(Kd, 3);
    wait_vm<4>();
    __syncthreads();  // ovf_any initialised, K0 and K1 complete
    f32x16 sa, sb;
    if (wave_rows) {
      load_k(Ka);
      gemm0(sa);
      mask(sa, 0);
      m = tile_max(sa);  // finite: the first tile holds key 0
      load_k(Kb);
    }
    dma_v(Vc, 2);
    wait_vm<4>();  // V0 complete
    pp_barrier();
    // group 1 runs every interval one barrier later than group 0
    if (grp == 1) pp_barrier();

    bf16x8 pb[2];
    // A row whose sum reached 2^kHeadroom met a key that far above its
    // reference: after the tile's P*V product (I3) both lanes of the row scale O
    // and their sums by the larger sum's power of two (exact) and raise the
    // row's reference by as much.  A sum at or above 2^kRebaseMax, or not
    // finite, leaves the workgroup to the slow pass.
    auto rebase = [&]() {
      const float lmax = half_max(l);
      if (!(lmax < exp2f(kRebaseMax))) {
        ovf = true;
      } else if (!(lmax < exp2f(kHeadroom))) {
        const int e = __builtin_amdgcn_frexp_expf(lmax);
        const float f = __builtin_amdgcn_ldexpf(1.0f, -e);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= f;
        l *= f;
        m += static_cast<float>(e);
      }
    };
    auto iter = [&](auto tt_c, int t) {
      constexpr int TT = decltype(tt_c)::value;
      f32x16 &scur = (TT & 1) ? sb : sa;
      f32x16 &snext = (TT & 1) ? sa : sb;
      // I0: S(t+1) MFMAs with P(t)'s exponentials in their shadow (the
      // compiler's own interleaving: pinning one MFMA between every two
      // exponentials with scheduling-group barriers ran 0.8% slower)
      gemm0(snext);
      probs_fast(scur, pb);
      pp_barrier();
      // I1: V(t) to registers, copy of K(t+4); K(t+2) complete after the wait
      load_v(vslot(ic<TT>()));
      dma_k(kslot(ic<TT>()), t + 4);
      wait_vm<4>();
      pp_barrier();
      // I2: O += V(t)^T P(t); keys of S(t+1) past the end masked
      gemm1(pb);
      mask(snext, (t + 1) * kPK);
      pp_barrier();
      // I3: K(t+2) to registers, copy of V(t+3); V(t+1) complete after the
      // wait; rows whose sum reached 2^kHeadroom rebased
      load_k(kslot(ic<TT + 2>()));
      dma_v(vslot(ic<TT + 3>()), t + 3);
      if (__builtin_amdgcn_ballot_w64(!(l < exp2f(kHeadroom))) != 0) rebase();
      wait_vm<4>();
      pp_barrier();
    };
    // The loops run a multiple of 4 iterations (the slots cycle with period
    // 4 and the unrolled body has no exit in the middle, which keeps every
    // value in one register assignment): iterations past the last tile copy
    // zero rows and mask every key.  A wave without query rows (a sequence's
    // last, partial query tile) only copies its share of every tile, with the
    // same waits and barriers.
    auto copy_only = [&](auto tt_c, int t) {
      constexpr int TT = decltype(tt_c)::value;
      pp_barrier();
      dma_k(kslot(ic<TT>()), t + 4);
      wait_vm<4>();
      pp_barrier();
      pp_barrier();
      dma_v(vslot(ic<TT + 3>()), t + 3);
      wait_vm<4>();
      pp_barrier();
    };
    if (wave_rows) {
      for (int t0 = 0; t0 < nT; t0 += 4) {
        iter(ic<0>(), t0);
        iter(ic<1>(), t0 + 1);
        iter(ic<2>(), t0 + 2);
        iter(ic<3>(), t0 + 3);
      }
    } else {
      for (int t0 = 0; t0 < nT; t0 += 4) {
        copy_only(ic<0>(), t0);
        copy_only(ic<1>(), t0 + 1);
        copy_only(ic<2>(), t0 + 2);
        copy_only(ic<3>(), t0 + 3);
      }
    }
    if (grp == 0) pp_barrier();
    wait_vm<0>();  // no copy may land in LDS after the workgroup ends
    // every tile's sums were rebased below 2^kHeadroom (or flagged)
    ovf = ovf || !(l < exp2f(kHeadroom));
    if (ovf) ovf_any = 1;
    __syncthreads();
    if (ovf_any) {
      // ---- slow pass (a later key outscored the first tile by kHeadroom):
      // one tile at a time through slots Ka / Va, online softmax with a
      // moving maximum and O rescaled when it moves
      m = -INFINITY;
      l = 0.0f;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
      for (int kt = 0; kt < nT; ++kt) {
        dma_k(Ka, kt);
        dma_v(Va, kt);
        wait_vm<0>();
        __syncthreads();
        if (wave_rows) {
          load_k(Ka);
          load_v(Va);
          f32x16 s;
          gemm0(s);
          mask(s, kt * kPK);
          const float m_new = fmaxf(m, tile_max(s));
          const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
          m = m_new;
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
          bf16x8 pq[2];
          l = l * alpha + probs(s, m, pq);
          gemm1(pq);
        }
        __syncthreads();
      }
    }
  }

  // ---- epilogue: O = O^T / l
  uint16_t *op = p.o + static_cast<int64_t>(q_begin) * p.o_tok + h * p.o_head;
  const float lt = half_sum(l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (row_q < Lq) {
    uint16_t *orow = op + static_cast<int64_t>(row_q) * p.o_tok;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<__bf16>(o[db][4 * g + e] * inv);
        *reinterpret_cast<bf16x4 *>(orow + d) = v;
      }
  }
}

// ---------------------------------------------------------------------------
// Three-group kernel (head_dim 128, large launches): attn_p3_kernel
// ---------------------------------------------------------------------------
// A workgroup of 12 waves owns 384 query rows (32 per wave) of one (query
// sequence, head) pair; waves w, w+4 and w+8 share a SIMD (wave w runs on
// SIMD w % 4), and group g is waves 4g..4g+3, one wave per SIMD.  Each K/V
// tile copied into LDS feeds 384 query rows: attention at full load runs at
// a power-limited clock, and moving tiles from L2 into LDS is a large part of
// its power (timing-only variants of attn_pp_kernel that skip a quarter of
// the copies ran 12% faster at the same MFMA busy fraction), so the tile
// feeds as many rows as the register file holds (three waves of at most 168
// registers per SIMD).  A launch with fewer than kP3MinGrid such workgroups
// runs attn_pp_kernel instead: its 256-row workgroups put more CUs to work
// when the grid does not cover the chip several times (one layer's 12 heads
// in a rollout step are 156 workgroups here, 228 there).
//
// Keys stream in tiles of 32.  Each tile takes six barrier-separated
// intervals; group g runs local interval k of tile t in global interval
// 6t + k + 2g:
//
//   local   work                                        LDS reads
//   L0      P(t) = exp(S(t)) (mask, row sums)
//   L1      V(t)^T fragments                                8 KB
//   L2      O += V(t)^T P(t)                     (8 MFMA)
//   L3      copy of V(t+3) (groups 0, 1)
//   L4      K(t+1) fragments; copy of K(t+4) (groups 0, 1) 8 KB
//   L5      S(t+1) = K(t+1) Q^T                  (8 MFMA)
//
// The three groups are in local intervals {0, 2, 4} or {1, 3, 5} at any
// time, so in every global interval exactly one wave of each SIMD issues
// matrix instructions, one reads 8 KB of fragments and one computes
// exponentials or waits.  (Mixing 4 KB of K and 4 KB of V reads in every
// interval ran 6% slower; moving half of the exponentials beside the V^T
// reads, 10% slower.)
//
// The tile copies and the swizzled LDS rows are those of attn_pp_kernel,
// with the four slots per operand in one 64 KB array.  Groups 0 and 1 copy 4
// rows each of every tile (two copies per wave per tile) and wait for all
// but their 4 newest copies at the end of every interval: a copy is complete
// 12 intervals after it was issued, and every copy is issued at least 14
// intervals before the first read of its tile (group 1's V copy at global
// 6t+5, V(t+3) first read at 6t+19) and after the reads of the tile its slot
// held were consumed.  The operand arrangement and the slow pass are those
// of attn_fwd_kernel.
//
// Softmax (both head_dim-128 kernels): P = 2^(S*c - m) in fp32 from the
// exact bf16 products (scaling Q by c in bf16 instead would move a score by
// ~2^-9 |q| |k|, several times P's own rounding for keys of large norm),
// with each row's reference m fixed at its first tile's maximum; the row
// sum is one chain of v_dot2c_f32_bf16 into the running sum.  After each
// tile's P*V product a ballot over the sums finds rows whose sum reached
// 2^kHeadroom (a key that far above the reference): only those rows rescale
// O and their sums by an exact power of two and raise m (rebase); the
// workgroup recomputes in the slow pass only when a sum reached
// 2^kRebaseMax or is not finite.  Against per-tile partial sums and
// per-tile checks, config 2 ran 2% faster; a row with a key 70 log2 units
// above its first tile costs one rebase instead of a recompute of its
// workgroup.
constexpr int kP3Waves = 12;
constexpr int kP3Threads = 64 * kP3Waves;
constexpr int kP3Rows = 32 * kP3Waves;
constexpr int kP3MinGrid = 1024;  // workgroups: four per CU
// a key-split item's partial result: per wave its lanes' 64 O^T values
// (16 float4 per lane, lane-minor) and then per wave and lane (r, l)
constexpr int kPartOFloats = kP3Waves * 16 * 64 * 4;
constexpr int kPartFloats = kPartOFloats + kP3Waves * 64 * 2;

static_assert(kP3Rows == kSplitRows, "a key-split item is one attn_p3_kernel workgroup");

// A sequence's last query tile holds Lq mod 384 rows -- 72 of the 4,680 of a
// rollout's query chunk -- so in the plain work shape three of its twelve
// waves have rows, and the tile took 82% of a full workgroup's time for 19%
// of its work.  Tiles of at most kTailRows rows instead split their keys
// within the workgroup: wave w takes row block w >> 2 (32 rows) against key
// quarter w & 3, so each SIMD runs one quarter's keys for up to three row
// blocks.  Each quarter streams its tiles through its own two K and two V
// slots (waves 0-7 copy: wave w < 4 the K tiles of quarter w, wave 4 + w
// its V tiles; K runs a tile ahead of V, so that a step's score MFMAs are
// those of the next tile and overlap its softmax, and one-dword touches
// four tiles ahead bring the keys into L2), with the classic online
// softmax (moving maximum; O rescaled only when a row's maximum grows, so
// no slow pass).  Quarters 1-3 then hand (O, m, l) through LDS to quarter
// 0, which merges them and writes the rows.
constexpr int kTailRows = 96;
constexpr int kTailMinTiles = 8;

__device__ __attribute__((always_inline)) inline void tail_item(const AttnParams &p, uint16_t *kv,
                                                                const uint16_t *qp, const uint16_t *kp,
                                                                const uint16_t *vp, int q_begin, int Lq, int q0,
                                                                int h, int Lk) {
  // opaque per item: nothing derived from the lane is hoisted out of a queue
  // launch's item loop (where it would stay live through every item)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qtr = wave & 3, rb = wave >> 2;
  const int lq = lane & 31, hf = lane >> 5;
  const int row_q = q0 + rb * 32 + lq;
  const bool rows = q0 + rb * 32 < Lq;
  const float c = p.scale_log2;
  const int nT = (Lk + kPK - 1) / kPK;
  // this SIMD's key quarter and the length of the longest
  const int t_lo = qtr * nT / 4, t_hi = (qtr + 1) * nT / 4;
  const int len = (nT + 3) / 4;
  const int kq0 = t_lo * kPK;
  const int Lkq = min(t_hi * kPK, Lk) - kq0;
  auto slot = [&](int q, int kind, int j) { return kv + ((q * 2 + kind) * 2 + j) * kPTileElems; };

  bf16x8 qr[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row_q < Lq) v = ldg16(qp + static_cast<int64_t>(row_q) * p.q_tok + 16 * s + 8 * hf);
    qr[s] = as_bf16x8(v);
  }
  wait_vm<0>();
  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  // copies: wave w < 8 copies the K (w < 4) or V (w >= 4) tiles of quarter
  // w & 3, all 32 rows (8 instructions of 4 rows), into slot j
  const bool copier = wave < 8;
  const int cq = wave & 3, ckind = wave >> 2;
  const int c_lo = cq * nT / 4, c_hi = (cq + 1) * nT / 4;
  const int64_t row_elems = p.kv_tok;
  const int row_bytes = static_cast<int>(row_elems) * 2;
  const uint16_t *cbase = (ckind ? vp : kp) + static_cast<int64_t>(c_lo) * kPK * row_elems;
  const int cLk = min(c_hi * kPK, Lk) - c_lo * kPK;
  const int drow = lane >> 4, dpos = lane & 15;
  auto copy_tile = [&](int i, int j) {
    const int64_t first = static_cast<int64_t>(i) * kPK;
    const int64_t left = (static_cast<int64_t>(cLk) - first) * row_elems * 2;
    const int nrec = static_cast<int>(left <= 0 ? 0 : (left < 0x7fffffff ? left : 0x7fffffff));
    const uint64_t addr = reinterpret_cast<uint64_t>(cbase + (left <= 0 ? 0 : first * row_elems));
    i32x4 rsrc;
    rsrc[0] = static_cast<int>(addr & 0xffffffffu);
    rsrc[1] = static_cast<int>((addr >> 32) & 0xffffu);
    rsrc[2] = nrec;
    rsrc[3] = kRsrcWord3;
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char *)slot(cq, ckind, j)));
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      const int r = 4 * ch + drow;
      const int sw = ckind ? (dpos ^ (4 * (r & 3))) : (dpos ^ (r & 15));
      const int voff = r * row_bytes + 16 * sw;
      const uint32_t lds = lds0 + ch * 4 * kPRow;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                   :
                   : "s"(lds), "v"(voff), "s"(rsrc)
                   : "memory", "m0");
#pragma clang diagnostic pop
    }
  };

  // fragment reads (the main kernel's addressing, on this quarter's slots).
  // K chunk 2s + hf of row lq sits at 16 * ((2s + hf) ^ (lq & 15)) within
  // the row, which is kaddr0 ^ (s << 5); the V transpose reads of column
  // block db sit at vaddr0 ^ (db << 6).  Both are recomputed every step
  // from bases the compiler cannot hoist, which keeps twelve addresses out
  // of the registers.
  const int kaddr0 = lq * kPRow + 16 * (hf ^ (lq & 15));
  const int v_row = 4 * hf + ((lane & 15) >> 2);
  const int v_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int vaddr0 = v_row * kPRow + 16 * ((v_col / 8) ^ (4 * (v_row & 3))) + 2 * (v_col % 8);
  static_assert(kPRow == 256, "the XOR forms assume 256-byte rows");

  // touch: one dword per 64 bytes of tile i of this wave's quarter and kind,
  // copied into a 256-byte LDS sink that nothing reads, so that the tile is
  // in L2 when its copy is issued (the quarters read keys that the
  // sequence's other query tiles have not reached yet)
  __shared__ __attribute__((aligned(16))) uint32_t sink[64];
  const uint32_t sink0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char *)sink));
  auto touch_tile = [&](int i) {
    const int64_t first = static_cast<int64_t>(i) * kPK;
    const int64_t left = (static_cast<int64_t>(cLk) - first) * row_elems * 2;
    // always two loads (the waits count them); past the quarter's keys they
    // have no records and read nothing
    const int nrec = static_cast<int>(left <= 0 ? 0 : (left < 0x7fffffff ? left : 0x7fffffff));
    const uint64_t addr = reinterpret_cast<uint64_t>(cbase + (left <= 0 ? 0 : first * row_elems));
    i32x4 rsrc;
    rsrc[0] = static_cast<int>(addr & 0xffffffffu);
    rsrc[1] = static_cast<int>((addr >> 32) & 0xffffu);
    rsrc[2] = nrec;
    rsrc[3] = kRsrcWord3;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int voff = (16 * u + (lane >> 2)) * row_bytes + 64 * (lane & 3);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                   :
                   : "s"(sink0), "v"(voff), "s"(rsrc)
                   : "memory", "m0");
#pragma clang diagnostic pop
    }
  };
  // K runs one tile ahead of V: step i reads K tile i + 1 (the scores of
  // the next step, whose MFMAs overlap this step's softmax) and V tile i,
  // while the copies of K tile i + 2 and V tile i + 1 fill the other slots
  auto scores = [&](const uint16_t *ks) {
    int ka = kaddr0;
    asm volatile("" : "+v"(ka));
    uint4 kreg[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
      kreg[s] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const char *>(ks) + (ka ^ (s << 5)));
    f32x16 sc;
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kreg[s]), qr[s], sc, 0, 0, 0);
    return sc;
  };
  const int nq = t_hi - t_lo;  // this quarter's tiles (len or len - 1)
  if (copier) {
    copy_tile(0, 0);
    if (ckind == 0) copy_tile(1, 1);
    wait_vm<0>();
  }
  __syncthreads();
  f32x16 sc = {};
  if (rows && nq > 0) sc = scores(slot(qtr, 0, 0));
  for (int i = 0; i < len; ++i) {
    if (copier) wait_vm<2>();  // the copies of the last step (its touches may be in flight)
    __syncthreads();           // ... are visible, and the slots they replace are read
    if (copier) {
      copy_tile(ckind ? i + 1 : i + 2, ckind ? (i + 1) & 1 : i & 1);
      touch_tile(i + 4);
    }
    if (rows && i < nq) {
      const f32x16 sn = scores(slot(qtr, 0, (i + 1) & 1));  // unused past the quarter's end
      const uint16_t *vs = slot(qtr, 1, i & 1);
      const int kb0 = i * kPK;
      if (kb0 + kPK > Lkq) {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (kb0 + 8 * (e / 4) + 4 * hf + (e % 4) >= Lkq) sc[e] = -INFINITY;
      }
      float mq[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) mq[r] = fmaxf(fmaxf(sc[r], sc[r + 4]), fmaxf(sc[r + 8], sc[r + 12]));
      const float m_new = fmaxf(m, half_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) * c);
      if (__builtin_amdgcn_ballot_w64(m_new > m) != 0) {  // some row's maximum grew
        const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - m_new);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
        l *= alpha;
        m = m_new;
      }
      bf16x8 pb[2];
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          pb[ks2][jj] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(sc[8 * ks2 + jj], c, -m)));
      l = bf16x8_acc(pb[1], bf16x8_acc(pb[0], l));
      int va = vaddr0;
      asm volatile("" : "+v"(va));
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {  // one key half at a time (16 registers of V fragments)
        i16x4 vreg[4][2];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const uint16_t *ptr = reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(vs) +
                                                                   (va ^ (db << 6)) + ks2 * 16 * kPRow);
          vreg[db][0] = lds_tr16(ptr);
          vreg[db][1] = lds_tr16(ptr + 8 * kPRow / 2);
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const i16x4 a8[2] = {vreg[db][0], vreg[db][1]};
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a8), pb[ks2], o[db], 0, 0, 0);
        }
      }
      sc = sn;
    }
  }
  if (copier) wait_vm<0>();
  __syncthreads();  // every copy landed and every slot read: the slots hold the merge

  // merge quarters 1-3 into quarter 0 (in quarter order, one at a time
  // through the first 50 KB of the slots)
  float *xo = reinterpret_cast<float *>(kv);
  float2 *xml = reinterpret_cast<float2 *>(xo + 3 * 16 * 64 * 4);
  // the lane index again, rather than keeping tid & 63 live through the loop
  int ln = threadIdx.x;
  asm volatile("" : "+v"(ln));
  ln &= 63;
  for (int qq = 1; qq < 4; ++qq) {
    if (qtr == qq && rows) {
      float4 *po = reinterpret_cast<float4 *>(xo) + rb * 16 * 64 + ln;
#pragma unroll
      for (int e = 0; e < 16; ++e)
        po[e * 64] = make_float4(o[e / 4][4 * (e % 4)], o[e / 4][4 * (e % 4) + 1], o[e / 4][4 * (e % 4) + 2],
                                 o[e / 4][4 * (e % 4) + 3]);
      xml[rb * 64 + ln] = make_float2(m, l);
    }
    __syncthreads();
    if (qtr == 0 && rows) {
      const float2 ml = xml[rb * 64 + ln];
      const float M = fmaxf(m, ml.x);
      const float a0 = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
      const float a1 = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - M);
      const float4 *po = reinterpret_cast<const float4 *>(xo) + rb * 16 * 64 + ln;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float4 v = po[e * 64];
        o[e / 4][4 * (e % 4)] = fmaf(o[e / 4][4 * (e % 4)], a0, v.x * a1);
        o[e / 4][4 * (e % 4) + 1] = fmaf(o[e / 4][4 * (e % 4) + 1], a0, v.y * a1);
        o[e / 4][4 * (e % 4) + 2] = fmaf(o[e / 4][4 * (e % 4) + 2], a0, v.z * a1);
        o[e / 4][4 * (e % 4) + 3] = fmaf(o[e / 4][4 * (e % 4) + 3], a0, v.w * a1);
      }
      l = fmaf(l, a0, ml.y * a1);
      m = M;
    }
    __syncthreads();
  }
  if (qtr != 0 || !rows) return;
  const float lt = half_sum(l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (row_q < Lq) {
    uint16_t *orow = p.o + static_cast<int64_t>(q_begin + row_q) * p.o_tok + h * p.o_head;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<__bf16>(o[db][4 * g + e] * inv);
        *reinterpret_cast<bf16x4 *>(orow + d) = v;
      }
  }
}

// SPLIT: the workgroup runs item xcd_remap(blockIdx.x) of the key-split plan
// (split_item): one query tile against one chunk of its sequence's keys.
// An item whose sequence has one chunk writes O as the plain kernel does;
// otherwise it writes its partial result (unnormalised O^T, the reference r
// its probabilities were taken against -- 0, m, or the slow pass's final
// maximum -- and the row sum l, per lane) to part slot c, and
// attn_combine_kernel merges a query tile's chunks.  Every workgroup writes
// its item's record (k = 0 when the item does not exist).
// One work item of attn_p3_kernel: query tile qt (kP3Rows rows) of
// sequence seq against all of its keys, or, in a key-split launch, against
// the chunk of keys that `it` names.  Every wave takes every barrier of the
// item; waves leave only after the item's last barrier.
template <bool SPLIT>
__device__ __attribute__((always_inline)) inline void p3_item(const AttnParams &p, uint16_t *kv, int seq, int qt,
                                                              const SplitItem &it) {
  auto kslot = [&](auto s) -> uint16_t * { return kv + (decltype(s)::value & 3) * kPTileElems; };
  auto vslot = [&](auto s) -> uint16_t * { return kv + (4 + (decltype(s)::value & 3)) * kPTileElems; };
  uint16_t *const Ka = kslot(ic<0>()), *const Kb = kslot(ic<1>()), *const Kc = kslot(ic<2>()), *const Kd = kslot(ic<3>());
  uint16_t *const Va = vslot(ic<0>()), *const Vb = vslot(ic<1>()), *const Vc = vslot(ic<2>());
  const int b = seq / p.Hq, h = seq % p.Hq;
  const int q_begin = p.cu_q[b];
  const int Lq = p.cu_q[b + 1] - q_begin;
  const int q0 = qt * kP3Rows;
  if (q0 >= Lq) return;
  const int kv_idx = p.kv_per_head ? seq : b;
  int k_begin = p.cu_k[kv_idx];
  int Lk = p.cu_k[kv_idx + 1] - k_begin;
  if constexpr (SPLIT) {  // this item's chunk of the keys
    const int lo = min(it.t_lo * kPK, Lk), hi = min(it.t_hi * kPK, Lk);
    k_begin += lo;
    Lk = hi - lo;
  }
  const uint16_t *qp = p.q + static_cast<int64_t>(q_begin) * p.q_tok + h * p.q_head;
  const int64_t kv_off = static_cast<int64_t>(k_begin) * p.kv_tok + (p.kv_per_head ? 0 : h * p.kv_head);
  const uint16_t *kp = p.k + kv_off;
  const uint16_t *vp = p.v + kv_off;

  // opaque per item: nothing derived from the lane is hoisted out of a queue
  // launch's item loop (where it would stay live through every item)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int grp = wave_s >> 2, wq = wave_s & 3;
  const bool copier = grp < 2;
  const int lq = lane & 31, hf = lane >> 5;
  const int row_q = q0 + wave * 32 + lq;
  const bool wave_rows = q0 + wave_s * 32 < Lq;
  const float c = p.scale_log2;

  if constexpr (!SPLIT) {
    if (Lq - q0 <= kTailRows && (Lk + kPK - 1) / kPK >= kTailMinTiles) {
      tail_item(p, kv, qp, kp, vp, q_begin, Lq, q0, h, Lk);
      return;
    }
  }

  bf16x8 qr[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row_q < Lq) v = ldg16(qp + static_cast<int64_t>(row_q) * p.q_tok + 16 * s + 8 * hf);
    qr[s] = as_bf16x8(v);
  }
  // Q is in registers before the first tile copy is issued: the compiler,
  // which cannot see the copies, then has no load of its own pending in the
  // key loop, where a wait for one would also wait for every copy in flight
  wait_vm<0>();
  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  float ref = 0.0f;  // the reference P was taken against (partial results of key-split items)
  const int nT = (Lk + kPK - 1) / kPK;

  // ---- tile copies (groups 0 and 1): buffer resources based at the tile's
  // first row and bounded at the sequence's last row (rows past the end, and
  // tiles past the end, copy zeros); this wave copies rows 16*grp + 4*wq ..
  // +3 of every tile, lane i the 16-byte position i % 16 of row i / 16 of them
  const int64_t row_elems = p.kv_tok;
  const int row_bytes = static_cast<int>(row_elems) * 2;
  const int dma_row = 16 * grp + 4 * wq + (lane >> 4);
  const int dma_pos = lane & 15;
  const int k_voff = dma_row * row_bytes + 16 * (dma_pos ^ (dma_row & 15));
  const int v_voff = dma_row * row_bytes + 16 * (dma_pos ^ (4 * (dma_row & 3)));
  const int dma_lds = (16 * grp + 4 * wq) * kPRow;
  // The copies are issued as inline assembly: the compiler then inserts no
  // wait of its own before the LDS reads of the slots (its bookkeeping
  // cannot follow the slots around the loop and waits far too early).  Every
  // wait for them is explicit; the compiler's waits for its own loads stay
  // correct, since those only ever have more, not fewer, loads after them.
  auto dma = [&](const uint16_t *base, int kt, uint16_t *slot, int voff) {
    const int64_t first = static_cast<int64_t>(kt) * kPK;
    const int64_t left = (static_cast<int64_t>(Lk) - first) * row_elems * 2;
    const int nrec = static_cast<int>(left <= 0 ? 0 : (left < 0x7fffffff ? left : 0x7fffffff));
    const uint64_t addr = reinterpret_cast<uint64_t>(base + (left <= 0 ? 0 : first * row_elems));
    i32x4 rsrc;
    rsrc[0] = static_cast<int>(addr & 0xffffffffu);
    rsrc[1] = static_cast<int>((addr >> 32) & 0xffffu);
    rsrc[2] = nrec;
    rsrc[3] = kRsrcWord3;
    const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char *)slot)) + dma_lds;
    // m0 is reserved to the compiler, which uses it nowhere else in this
    // kernel (the listing has no other m0 access)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
#pragma clang diagnostic pop
  };
  auto dma_k = [&](uint16_t *slot, int kt) { dma(kp, kt, slot, k_voff); };
  auto dma_v = [&](uint16_t *slot, int kt) { dma(vp, kt, slot, v_voff); };

  // ---- fragment reads
  // K: step s reads row lq, 16-byte chunk 2s + hf (swizzled)
  int kaddr[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) kaddr[s] = lq * kPRow + 16 * ((2 * s + hf) ^ (lq & 15));
  const int v_row = 4 * hf + ((lane & 15) >> 2);
  const int v_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  int vaddr[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
    vaddr[db] = v_row * kPRow + 16 * ((4 * db + v_col / 8) ^ (4 * (v_row & 3))) + 2 * (v_col % 8);
  uint4 kreg[8];
  i16x4 vreg[2][4][2];
  // K fragments of steps 4*H .. 4*H+3
  auto load_k_half = [&](const uint16_t *slot, auto h_c) {
    constexpr int H = decltype(h_c)::value;
#pragma unroll
    for (int s = 4 * H; s < 4 * H + 4; ++s)
      kreg[s] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const char *>(slot) + kaddr[s]);
  };
  // V^T fragments of key step KS (keys 16*KS .. +15)
  auto load_v_half = [&](const uint16_t *slot, auto ks_c) {
    constexpr int KS = decltype(ks_c)::value;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const uint16_t *ptr =
          reinterpret_cast<const uint16_t *>(reinterpret_cast<const char *>(slot) + vaddr[db] + KS * 16 * kPRow);
      vreg[KS][db][0] = lds_tr16(ptr);
      vreg[KS][db][1] = lds_tr16(ptr + 8 * kPRow / 2);
    }
  };
  auto gemm0 = [&](f32x16 &acc) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kreg[s]), qr[s], acc, 0, 0, 0);
  };
  auto gemm1 = [&](const bf16x8 (&pb)[2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const i16x4 a8[2] = {vreg[ks][db][0], vreg[ks][db][1]};
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a8), pb[ks], o[db], 0, 0, 0);
      }
  };
  auto mask = [&](f32x16 &s, int kb0) {
    if (kb0 + kPK > Lk) {
      asm volatile("");
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (kb0 + 8 * (i / 4) + 4 * hf + (i % 4) >= Lk) s[i] = -INFINITY;
    }
  };
  auto tile_max = [&](const f32x16 &s) {
    float mq[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) mq[r] = fmaxf(fmaxf(s[r], s[r + 4]), fmaxf(s[r + 8], s[r + 12]));
    return half_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) * c;
  };
  // slow pass: P = 2^(S*c - m), returns the lane's sum
  auto probs = [&](const f32x16 &s, float mr, bf16x8 (&pb)[2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        pb[ks][jj] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(s[8 * ks + jj], c, -mr)));
    return bf16x8_sum(pb[0], 0.0f) + bf16x8_sum(pb[1], 0.0f);
  };
  // fast pass: P = 2^(S*c - m) against the row's reference m, added to the
  // running sum (one chain of dot products)
  auto probs_fast = [&](const f32x16 &s, bf16x8 (&pb)[2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        pb[ks][jj] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(s[8 * ks + jj], c, -m)));
    l = bf16x8_acc(pb[1], bf16x8_acc(pb[0], l));
  };
  // end of an interval: this wave's copies older than its 4 newest are
  // complete, then the workgroup barrier
  auto step = [&]() {
    wait_vm<4>();
    pp_barrier();
  };

  __shared__ int ovf_any;
  if (tid == 0) ovf_any = 0;
  bool ovf = false;
  if (nT > 0) {
    // prologue: copies of K0, V0, K1, V1, K2, V2, K3 (the order in which the
    // loop's tiles -4 .. -1 would have issued them), S(0) and m
    if (copier) {
      dma_k(Ka, 0);
      dma_v(Va, 0);
      dma_k(Kb, 1);
      dma_v(Vb, 1);
      dma_k(Kc, 2);
      dma_v(Vc, 2);
      dma_k(Kd, 3);
    }
    wait_vm<5>();     // K0 and V0 complete
    __syncthreads();  // ovf_any initialised
    f32x16 s;
    if (wave_rows) {
      load_k_half(Ka, ic<0>());
      load_k_half(Ka, ic<1>());
      gemm0(s);
      mask(s, 0);
      m = tile_max(s);  // finite: the first tile holds key 0
    }
    // P < 2^kHeadroom unless a later key scores that far above the row's
    // reference, which its sum shows after the tile (rebase)
    // group g runs two intervals behind group g - 1
    for (int i = 0; i < grp; ++i) {
      step();
      step();
    }

    bf16x8 pb[2];
    // A row whose sum reached 2^kHeadroom met a key that far above its
    // reference: after the tile's P*V product both lanes of the row scale O
    // and their sums by the larger sum's power of two (exact) and raise the
    // row's reference by as much.  A sum at or above 2^kRebaseMax, or not
    // finite, leaves the workgroup to the slow pass.
    auto rebase = [&]() {
      const float lmax = half_max(l);
      if (!(lmax < exp2f(kRebaseMax))) {
        ovf = true;
      } else if (!(lmax < exp2f(kHeadroom))) {
        const int e = __builtin_amdgcn_frexp_expf(lmax);
        const float f = __builtin_amdgcn_ldexpf(1.0f, -e);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= f;
        l *= f;
        m += static_cast<float>(e);
      }
    };
    auto iter = [&](auto tt_c, int t) {
      constexpr int TT = decltype(tt_c)::value;
      // L0: P(t)
      mask(s, t * kPK);
      probs_fast(s, pb);
      // the row sums are taken here, not sunk to a later interval where P
      // would have to stay live
      asm volatile("" : "+v"(l));
      step();
      // L1: V(t) fragments
      load_v_half(vslot(ic<TT>()), ic<0>());
      load_v_half(vslot(ic<TT>()), ic<1>());
      step();
      // L2: O += V(t)^T P(t)
      gemm1(pb);
      step();
      // L3: copy of V(t+3); rows whose sum reached 2^kHeadroom rebased
      if (copier) dma_v(vslot(ic<TT + 3>()), t + 3);
      if (__builtin_amdgcn_ballot_w64(!(l < exp2f(kHeadroom))) != 0) rebase();
      step();
      // L4: K(t+1) fragments, copy of K(t+4)
      load_k_half(kslot(ic<TT + 1>()), ic<0>());
      load_k_half(kslot(ic<TT + 1>()), ic<1>());
      if (copier) dma_k(kslot(ic<TT>()), t + 4);
      step();
      // L5: S(t+1)
      gemm0(s);
      step();
    };
    // waves without query rows (a sequence's last, partial query tile) only
    // copy their rows of every tile, with the same waits and barriers
    auto copy_only = [&](auto tt_c, int t) {
      constexpr int TT = decltype(tt_c)::value;
      step();
      step();
      step();
      if (copier) dma_v(vslot(ic<TT + 3>()), t + 3);
      step();
      if (copier) dma_k(kslot(ic<TT>()), t + 4);
      step();
      step();
    };
    // a multiple of 4 tiles (the slots cycle with period 4): tiles past the
    // last copy zero rows and mask every key
    if (wave_rows) {
      for (int t0 = 0; t0 < nT; t0 += 4) {
        iter(ic<0>(), t0);
        iter(ic<1>(), t0 + 1);
        iter(ic<2>(), t0 + 2);
        iter(ic<3>(), t0 + 3);
      }
    } else {
      for (int t0 = 0; t0 < nT; t0 += 4) {
        copy_only(ic<0>(), t0);
        copy_only(ic<1>(), t0 + 1);
        copy_only(ic<2>(), t0 + 2);
        copy_only(ic<3>(), t0 + 3);
      }
    }
    for (int i = grp; i < 2; ++i) {
      step();
      step();
    }
    wait_vm<0>();  // no copy may land in LDS after the workgroup ends
    // every tile's sums were rebased below 2^kHeadroom (or flagged)
    ovf = ovf || !(l < exp2f(kHeadroom));
    ref = m;
    if (ovf) ovf_any = 1;
    __syncthreads();
    if (ovf_any) {
      // ---- slow pass (a later key outscored the first tile by kHeadroom):
      // one tile at a time through slots Ka / Va, online softmax with a
      // moving maximum and O rescaled when it moves
      m = -INFINITY;
      l = 0.0f;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
      for (int kt = 0; kt < nT; ++kt) {
        if (copier) {
          dma_k(Ka, kt);
          dma_v(Va, kt);
        }
        wait_vm<0>();
        __syncthreads();
        if (wave_rows) {
          // V^T fragments only after the S product (K fragments no longer live)
          load_k_half(Ka, ic<0>());
          load_k_half(Ka, ic<1>());
          f32x16 s2;
          gemm0(s2);
          mask(s2, kt * kPK);
          const float m_new = fmaxf(m, tile_max(s2));
          const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
          m = m_new;
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
          bf16x8 pq[2];
          l = l * alpha + probs(s2, m, pq);
          asm volatile("" ::: "memory");
          load_v_half(Va, ic<0>());
          load_v_half(Va, ic<1>());
          gemm1(pq);
        }
        __syncthreads();
      }
      ref = m;
    }
  }

  if constexpr (SPLIT) {
    if (it.k > 1) {
      // partial result of this chunk, in the lane layout attn_combine_kernel reads
      if (!wave_rows) return;
      float *slot = p.part + static_cast<int64_t>(xcd_remap(blockIdx.x, p.n_wg)) * kPartFloats;
      float4 *po = reinterpret_cast<float4 *>(slot) + wave * 16 * 64 + lane;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        po[j * 64] = make_float4(o[j / 4][4 * (j % 4)], o[j / 4][4 * (j % 4) + 1], o[j / 4][4 * (j % 4) + 2],
                                 o[j / 4][4 * (j % 4) + 3]);
      reinterpret_cast<float2 *>(slot + kPartOFloats)[wave * 64 + lane] = make_float2(ref, l);
      return;
    }
  }

  // ---- epilogue: O = O^T / l
  uint16_t *op = p.o + static_cast<int64_t>(q_begin) * p.o_tok + h * p.o_head;
  const float lt = half_sum(l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  int rq = row_q;  // the row's offset computed again, not kept from the Q load through the key loop
  asm volatile("" : "+v"(rq));
  if (rq < Lq) {
    uint16_t *orow = op + static_cast<int64_t>(rq) * p.o_tok;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<__bf16>(o[db][4 * g + e] * inv);
        *reinterpret_cast<bf16x4 *>(orow + d) = v;
      }
  }
}

template <bool SPLIT>
__global__ void __launch_bounds__(kP3Threads, 1) attn_p3_kernel(AttnParams p) {
  // the eight tile slots (K 0-3, V 4-7) in one 64 KB array at the start of
  // LDS, so that every fragment read addresses its slot by an immediate
  // offset; the work-list scratch of the prologue shares it (no copy is
  // issued before the work list is read)
  // (a tail item uses sixteen slots: its own K and V pairs per key quarter)
  __shared__ __attribute__((aligned(16))) uint16_t kv[16 * kPTileElems];
  static_assert(8 * kPTileElems * 2 >= 6 * kSchedMax * 4, "work-list scratch fits in the tile slots");
  int *sched = reinterpret_cast<int *>(kv);
  if constexpr (SPLIT) {
    SplitItem it{};
    const int c = xcd_remap(blockIdx.x, p.n_wg);
    const bool ok = split_item(p, p.n_wg, c, sched, it);
    if (threadIdx.x == 0) p.rec[c] = ok ? make_int4(it.seq, it.qt, it.j | (it.k << 16), it.nq) : make_int4(0, 0, 0, 0);
    if (!ok) return;
    p3_item<true>(p, kv, it.seq, it.qt, it);
  } else {
    const int n_seq = p.n_wg / p.q_tiles;
    __shared__ QueueTable tab;
    if (p.queue) queue_table(p.cu_q, p.cu_k, p.Hq, n_seq, p.kv_per_head, kP3Rows, sched, tab);
    unsigned spent = 0;  // queue mode: the bins this workgroup found empty (thread 0)
    for (bool first = true;; first = false) {
      int seq, qt;
      if (p.queue) {
        if (!queue_next(p.queue, tab, spent, seq, qt)) break;
      } else {
        // one item per workgroup, in the XCD-balanced order
        if (!first) break;
        if (n_seq <= kSchedMax) {
          if (!balanced_item(p.cu_q, p.cu_k, p.Hq, n_seq, p.kv_per_head, kP3Rows, xcd_remap(blockIdx.x, p.n_wg),
                             sched, seq, qt))
            break;
        } else {
          const int wg = xcd_remap(blockIdx.x, p.n_wg);
          seq = wg / p.q_tiles;
          qt = wg % p.q_tiles;
        }
      }
      p3_item<false>(p, kv, seq, qt, SplitItem{});
    }
    if (p.queue) queue_done(p.queue);
  }
}

// Second launch of a key-split attention: item c with chunk j = 0 of a
// split query tile (k > 1 chunks) merges the partial results of items
// c + j' * nq, j' = 0 .. k-1, in that order: with M the largest reference,
// O = sum_j' 2^(r_j' - M) O_j' / sum_j' 2^(r_j' - M) l_j' (fp32), written
// as attn_p3_kernel's epilogue writes it.  Other items exit at once.
__global__ void __launch_bounds__(kP3Threads) attn_combine_kernel(AttnParams p) {
  const int c = blockIdx.x;
  const int4 r = p.rec[c];
  const int k = r.z >> 16, j = r.z & 0xffff;
  if (k <= 1 || j != 0) return;
  const int seq = r.x, qt = r.y, nq = r.w;
  const int b = seq / p.Hq, h = seq % p.Hq;
  const int q_begin = p.cu_q[b];
  const int Lq = p.cu_q[b + 1] - q_begin;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lq = lane & 31, hf = lane >> 5;
  const int q0 = qt * kP3Rows;
  if (q0 + wave * 32 >= Lq) return;
  auto slot = [&](int jj) { return p.part + static_cast<int64_t>(c + jj * nq) * kPartFloats; };
  float M = -INFINITY;
  for (int jj = 0; jj < k; ++jj) M = fmaxf(M, reinterpret_cast<const float2 *>(slot(jj) + kPartOFloats)[wave * 64 + lane].x);
  float l = 0.0f;
  float4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int jj = 0; jj < k; ++jj) {
    const float *sp = slot(jj);
    const float2 rl = reinterpret_cast<const float2 *>(sp + kPartOFloats)[wave * 64 + lane];
    const float w = __builtin_amdgcn_exp2f(rl.x - M);
    l = fmaf(w, rl.y, l);
    const float4 *po = reinterpret_cast<const float4 *>(sp) + wave * 16 * 64 + lane;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float4 v = po[i * 64];
      acc[i].x = fmaf(w, v.x, acc[i].x);
      acc[i].y = fmaf(w, v.y, acc[i].y);
      acc[i].z = fmaf(w, v.z, acc[i].z);
      acc[i].w = fmaf(w, v.w, acc[i].w);
    }
  }
  const float lt = half_sum(l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  const int row_q = q0 + wave * 32 + lq;
  if (row_q < Lq) {
    uint16_t *orow = p.o + static_cast<int64_t>(q_begin + row_q) * p.o_tok + h * p.o_head;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        const float4 v = acc[4 * db + g];
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        bf16x4 o4;
        o4[0] = static_cast<__bf16>(v.x * inv);
        o4[1] = static_cast<__bf16>(v.y * inv);
        o4[2] = static_cast<__bf16>(v.z * inv);
        o4[3] = static_cast<__bf16>(v.w * inv);
        *reinterpret_cast<bf16x4 *>(orow + d) = o4;
      }
  }
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// Queue counter blocks: a file-scope array on each device, kQueueSlots
// blocks of kQueueInts ints.  A stream takes a block on its first queue
// launch on a device (cleared there, in stream order, by a one-workgroup
// kernel) and keeps it, so launches on one stream reuse it in turn and
// launches on different streams never share one.  Past kQueueSlots streams
// on a device, launches run one item per workgroup.
constexpr int kQueueSlots = 64;
__device__ __attribute__((aligned(256))) int g_attn_queue[kQueueSlots * kQueueInts];

__global__ void queue_clear_kernel(int *q) {
  if (threadIdx.x < kQueueInts) q[threadIdx.x] = 0;
}

static int *queue_for(hipStream_t st) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, int *> blocks;
  static int *base[64];
  static int used[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  // the array's address on this device (the host-side name is not one),
  // looked up on every call: after a device reset the array is a new one,
  // and every block of it is taken afresh
  void *ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_attn_queue)) != hipSuccess || !ptr) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (base[dev] != static_cast<int *>(ptr)) {
    for (auto it = blocks.begin(); it != blocks.end();) it = it->first.first == dev ? blocks.erase(it) : std::next(it);
    base[dev] = static_cast<int *>(ptr);
    used[dev] = 0;
  }
  const auto key = std::make_pair(dev, st);
  const auto found = blocks.find(key);
  if (found != blocks.end()) return found->second;
  if (used[dev] >= kQueueSlots) return nullptr;
  int *q = base[dev] + used[dev] * kQueueInts;
  hipLaunchKernelGGL(queue_clear_kernel, dim3(1), dim3(64), 0, st, q);
  if (hipGetLastError() != hipSuccess) return nullptr;
  ++used[dev];
  blocks.emplace(key, q);
  return q;
}

// Items a key-split launch may have: three per compute unit.
static int64_t split_items() { return 3 * static_cast<int64_t>(device_cus()); }
static int64_t split_ws_bytes(int64_t items) {
  return items * (static_cast<int64_t>(kPartFloats) * 4 + static_cast<int64_t>(sizeof(int4)));
}

// Key-split launch (head_dim 128): attn_p3_kernel<true> over n items, then
// attn_combine_kernel.  Returns -1 when the launch does not qualify (the
// caller then runs the plain kernels).
static int launch_split(const pkv_attn_args *a, void *ws, int64_t ws_bytes, hipStream_t st) {
  const int64_t seqs = static_cast<int64_t>(a->num_batches) * a->num_heads_q;
  const int64_t q_tiles = (a->max_seqlen_q + kP3Rows - 1) / kP3Rows;
  const int64_t n = split_items();
  // small launches only: those the 12-wave kernel would not fill the chip with
  // per-head keys only (the cache's attention; a shared key sequence, as in
  // cross-attention to a short text context, gains nothing from splitting)
  if (!ws || a->head_dim != 128 || !a->kv_per_head || n <= 0 || seqs > kSchedMax ||
      seqs * q_tiles >= kP3MinGrid || seqs * q_tiles > n || ws_bytes < split_ws_bytes(n))
    return -1;
  AttnParams p{};
  p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o;
  p.cu_q = a->cu_seqlens_q; p.cu_k = a->cu_seqlens_k;
  p.Hq = a->num_heads_q;
  p.kv_per_head = a->kv_per_head;
  p.q_tiles = static_cast<int>(q_tiles);
  p.n_wg = static_cast<int>(n);
  p.n_seq = static_cast<int>(seqs);
  p.n_cu = device_cus();
  p.q_tok = a->q_tok_stride; p.q_head = a->q_head_stride;
  p.kv_tok = a->kv_tok_stride; p.kv_head = a->kv_head_stride;
  p.o_tok = a->o_tok_stride; p.o_head = a->o_head_stride;
  p.scale_log2 = a->softmax_scale * 1.4426950408889634f;
  p.part = static_cast<float *>(ws);
  p.rec = reinterpret_cast<int4 *>(static_cast<char *>(ws) + n * static_cast<int64_t>(kPartFloats) * 4);
  hipLaunchKernelGGL(attn_p3_kernel<true>, dim3(p.n_wg), dim3(kP3Threads), 0, st, p);
  int rc = check_launch("attn_p3_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(p.n_wg), dim3(kP3Threads), 0, st, p);
  return check_launch("attn_combine_kernel");
}

template <int D>
static int launch_attn(const pkv_attn_args *a, hipStream_t st) {
  constexpr int BQ = 32 * kWaves;
  AttnParams p{};
  p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o;
  p.cu_q = a->cu_seqlens_q; p.cu_k = a->cu_seqlens_k;
  p.Hq = a->num_heads_q;
  p.kv_per_head = a->kv_per_head;
  // head_dim 128: attn_p3_kernel (384 query rows per workgroup) when its
  // grid has at least kP3MinGrid workgroups, else attn_pp_kernel
  const int64_t seqs = static_cast<int64_t>(a->num_batches) * a->num_heads_q;
  const bool p3 = D == 128 && seqs * ((a->max_seqlen_q + kP3Rows - 1) / kP3Rows) >= kP3MinGrid;
  const int bq = p3 ? kP3Rows : BQ;
  p.q_tiles = (a->max_seqlen_q + bq - 1) / bq;
  const int64_t n = static_cast<int64_t>(p.q_tiles) * a->num_batches * a->num_heads_q;
  if (n > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: grid too large");
  p.n_wg = static_cast<int>(n);
  p.q_tok = a->q_tok_stride; p.q_head = a->q_head_stride;
  p.kv_tok = a->kv_tok_stride; p.kv_head = a->kv_head_stride;
  p.o_tok = a->o_tok_stride; p.o_head = a->o_head_stride;
  p.scale_log2 = a->softmax_scale * 1.4426950408889634f;
  if (p.n_wg == 0) return PKV_OK;
  if (p3) {
    // a queue launch (one workgroup per compute unit) when the XCD-balanced
    // work list covers the sequences and this stream has a counter block
    const int cus = device_cus();
    p.queue = seqs <= kSchedMax && cus > 0 && p.n_wg > cus ? queue_for(st) : nullptr;
    hipLaunchKernelGGL(attn_p3_kernel<false>, dim3(p.queue ? cus : p.n_wg), dim3(kP3Threads), 0, st, p);
    return check_launch("attn_p3_kernel");
  }
  if (D == 128) {
    hipLaunchKernelGGL(attn_pp_kernel, dim3(p.n_wg), dim3(kThreads), 0, st, p);
    return check_launch("attn_pp_kernel");
  }
  hipLaunchKernelGGL((attn_fwd_kernel<D>), dim3(p.n_wg), dim3(kThreads), 0, st, p);
  return check_launch("attn_fwd_kernel");
}

}  // namespace pkv

using namespace pkv;

// checks shared by both entry points; 1 = nothing to do
static int attn_check(const pkv_attn_args *a) {
  if (!a || !a->q || !a->k || !a->v || !a->o || !a->cu_seqlens_q || !a->cu_seqlens_k)
    return fail(PKV_ERR_INVALID, "ragged_attn: NULL argument");
  if (a->causal) return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: causal masking is not implemented (causal=False only)");
  if (a->num_batches < 0 || a->num_heads_q <= 0 || a->max_seqlen_q < 0)
    return fail(PKV_ERR_INVALID, "ragged_attn: bad sizes");
  if (a->num_batches == 0 || a->max_seqlen_q == 0) return 1;
  if ((a->q_tok_stride & 7) || (a->q_head_stride & 7) || (a->kv_tok_stride & 7) || (a->kv_head_stride & 7) ||
      (a->o_tok_stride & 3) || (a->o_head_stride & 3))
    return fail(PKV_ERR_INVALID, "ragged_attn: strides must keep 16-byte rows aligned");
  if (a->kv_tok_stride * 2 * kBK > 0x7fffffff)
    return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: kv token stride too large");
  if (a->head_dim != 128 && a->head_dim != 64)
    return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: head_dim %d (supported: 64, 128)", a->head_dim);
  return 0;
}

extern "C" int64_t pkv_ragged_attn_workspace_size(void) {
  const int64_t n = split_items();
  return n > 0 ? split_ws_bytes(n) : 0;
}

extern "C" int pkv_ragged_attn_fwd_ws(const pkv_attn_args *a, void *workspace, int64_t workspace_bytes,
                                      pkv_stream_t stream) {
  const int rc = attn_check(a);
  if (rc) return rc < 0 ? rc : PKV_OK;
  const int s = launch_split(a, workspace, workspace_bytes, as_stream(stream));
  if (s >= 0) return s;
  return pkv_ragged_attn_fwd(a, stream);
}

extern "C" int pkv_ragged_attn_fwd(const pkv_attn_args *a, pkv_stream_t stream) {
  if (!a || !a->q || !a->k || !a->v || !a->o || !a->cu_seqlens_q || !a->cu_seqlens_k)
    return fail(PKV_ERR_INVALID, "ragged_attn: NULL argument");
  if (a->causal) return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: causal masking is not implemented (causal=False only)");
  if (a->num_batches < 0 || a->num_heads_q <= 0 || a->max_seqlen_q < 0)
    return fail(PKV_ERR_INVALID, "ragged_attn: bad sizes");
  if (a->num_batches == 0 || a->max_seqlen_q == 0) return PKV_OK;
  const int64_t align_mask = 7;
  if ((a->q_tok_stride & align_mask) || (a->q_head_stride & align_mask) || (a->kv_tok_stride & align_mask) ||
      (a->kv_head_stride & align_mask) || (a->o_tok_stride & 3) || (a->o_head_stride & 3))
    return fail(PKV_ERR_INVALID, "ragged_attn: strides must keep 16-byte rows aligned");
  // buffer offsets within one 64-row tile are 32-bit
  if (a->kv_tok_stride * 2 * kBK > 0x7fffffff)
    return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: kv token stride too large");
  hipStream_t st = as_stream(stream);
  switch (a->head_dim) {
    case 128: return launch_attn<128>(a, st);
    case 64: return launch_attn<64>(a, st);
    default: return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: head_dim %d (supported: 64, 128)", a->head_dim);
  }
}
