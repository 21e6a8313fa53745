// Ragged-cache attention for gfx950: bf16 inputs, fp32 online softmax and
// accumulation, MFMA v_mfma_f32_32x32x16_bf16.
//
// Work decomposition.  A workgroup (4 waves) owns 32*QB*4 query rows of one
// (query sequence, head) pair and streams that pair's keys through LDS in
// tiles of 64.  Each wave owns 32*QB query rows.
//
// Operand arrangement.  The wave computes S^T = K * Q^T (A = K rows read from
// LDS, B = Q^T kept in registers for the whole loop), so the 32x32 MFMA
// result gives every lane one query column and 16 keys of it.  The
// probabilities are then consumed as the B operand of O^T = V^T * P^T
// straight from registers: for a k-step of 16 keys, lane half hf holds keys
// {16ks + 8*(j/4) + 4*hf + j%4 : j < 8}, and V^T is stored in LDS with the
// two middle bits of each 16-key group swapped so those 8 keys are one
// contiguous 16-byte read.  O^T's accumulator again gives every lane one
// query column, so the running max / sum and the rescale of O are lane-local
// (one xor-32 exchange per row statistic).
//
// Softmax runs in the log2 domain, s' = s * scale * log2(e), exp2 via
// v_exp_f32; P is rounded to bf16 before the P*V product, row sums use the
// unrounded fp32 values (the flash-attention scheme).

#include "pkv_common.h"

namespace pkv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = 64 * kAttnWaves;
constexpr int kBK = 64;  // keys per LDS tile

struct AttnParams {
  const uint16_t *q, *k, *v;
  uint16_t *o;
  const int32_t *cu_q, *cu_k;
  int Hq, kv_per_head, q_tiles, n_wg;
  int64_t q_tok, q_head, kv_tok, kv_head, o_tok, o_head;
  float scale_log2;
};

// Consecutive workgroup ids are dispatched round-robin over the 8 XCDs;
// renumber them so that the query tiles of one sequence (which share its
// keys) run on the same XCD and share its L2.
__device__ inline int xcd_remap(int i, int n) {
  const int xcd = i % 8, k = i / 8;
  const int base = n / 8, rem = n % 8;
  return xcd < rem ? xcd * (base + 1) + k : rem * (base + 1) + (xcd - rem) * base + k;
}

__device__ inline bool tid_in_range(int n) { return static_cast<int>(threadIdx.x) < n; }

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

__device__ inline float xor32(float x) { return __shfl_xor(x, 32); }

// max / sum of x over lanes l and l^32 (v_permlane32_swap exchanges the two
// half-waves of its operands)
__device__ inline float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// position of key k (0..63) of a tile inside its V^T row: swap bits 2 and 3
__device__ inline int vt_pos(int k) { return (k & ~0xC) | ((k & 4) << 1) | ((k & 8) >> 1); }

template <int D, int QB>
__global__ void __launch_bounds__(kAttnThreads) attn_fwd_kernel(AttnParams p) {
  constexpr int BQ = 32 * QB * kAttnWaves;
  constexpr int DS = D / 16;  // k-steps of the QK^T product
  constexpr int DB = D / 32;  // 32-row blocks of O^T
  constexpr int KS = D + 8;   // K row stride in LDS (elements); +16 B kills bank conflicts
  constexpr int VS = kBK + 8; // V^T row stride in LDS (elements)
  constexpr int KCH = D / 8;  // 16-byte chunks per K/V row
  constexpr int KLD = kBK * KCH / kAttnThreads;  // 16-byte K loads per thread per tile
  static_assert(KLD * kAttnThreads == kBK * KCH, "tile split");
  constexpr int VGRP = kBK / 4;                   // 4-key groups per tile
  static_assert(VGRP * KCH <= kAttnThreads, "V split");
  const bool v_owner = tid_in_range(VGRP * KCH);
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBK * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VS];

  const int wg = xcd_remap(blockIdx.x, p.n_wg);
  const int seq = wg / p.q_tiles, qt = wg % p.q_tiles;
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
  const int wq0 = q0 + wave * 32 * QB;

  // ---- Q^T operand, resident for the whole key loop
  bf16x8 qr[QB][DS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = wq0 + qb * 32 + lq;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (row < Lq) v = ldg16(qp + static_cast<int64_t>(row) * p.q_tok + 16 * s + 8 * hf);
      qr[qb][s] = as_bf16x8(v);
    }
  }

  f32x16 o[QB][DB];
  float m[QB], l[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m[qb] = -INFINITY;
    l[qb] = 0.0f;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[qb][db][i] = 0.0f;
  }

  // ---- global -> register staging of one K/V tile
  uint4 kreg[KLD], vreg[4];
  const int vgrp = tid % VGRP, vch = tid / VGRP;  // V: 4 keys x 8 dims per thread
  auto load_tile = [&](int kt) {
    const int kbase = kt * kBK;
#pragma unroll
    for (int r = 0; r < KLD; ++r) {
      const int idx = tid + r * kAttnThreads;
      const int row = idx / KCH, ch = idx % KCH;
      const int key = kbase + row;
      kreg[r] = key < Lk ? ldg16(kp + static_cast<int64_t>(key) * p.kv_tok + ch * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = kbase + vgrp * 4 + j;
      vreg[j] = (v_owner && key < Lk) ? ldg16(vp + static_cast<int64_t>(key) * p.kv_tok + vch * 8)
                                      : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int r = 0; r < KLD; ++r) {
      const int idx = tid + r * kAttnThreads;
      const int row = idx / KCH, ch = idx % KCH;
      *reinterpret_cast<uint4 *>(&Ks[row * KS + ch * 8]) = kreg[r];
    }
    if (!v_owner) return;
    // transpose 4 keys x 8 dims into 8 rows of 4 keys
    const uint32_t w0[4] = {vreg[0].x, vreg[0].y, vreg[0].z, vreg[0].w};
    const uint32_t w1[4] = {vreg[1].x, vreg[1].y, vreg[1].z, vreg[1].w};
    const uint32_t w2[4] = {vreg[2].x, vreg[2].y, vreg[2].z, vreg[2].w};
    const uint32_t w3[4] = {vreg[3].x, vreg[3].y, vreg[3].z, vreg[3].w};
    const int col = vt_pos(vgrp * 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // dims 2e (low halves) and 2e+1 (high halves)
      const uint32_t lo01 = (w0[e] & 0xffffu) | (w1[e] << 16);
      const uint32_t lo23 = (w2[e] & 0xffffu) | (w3[e] << 16);
      const uint32_t hi01 = (w0[e] >> 16) | (w1[e] & 0xffff0000u);
      const uint32_t hi23 = (w2[e] >> 16) | (w3[e] & 0xffff0000u);
      *reinterpret_cast<uint2 *>(&Vt[(vch * 8 + 2 * e) * VS + col]) = make_uint2(lo01, lo23);
      *reinterpret_cast<uint2 *>(&Vt[(vch * 8 + 2 * e + 1) * VS + col]) = make_uint2(hi01, hi23);
    }
  };

  const int n_tiles = (Lk + kBK - 1) / kBK;
  if (n_tiles > 0) load_tile(0);
  for (int kt = 0; kt < n_tiles; ++kt) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (kt + 1 < n_tiles) load_tile(kt + 1);

    const int kbase = kt * kBK;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kb0 = kbase + kb * 32;
      if (kb0 >= Lk) break;
      // ---- S^T = K Q^T for 32 keys
      f32x16 sacc[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[qb][i] = 0.0f;
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4 *>(&Ks[(kb * 32 + lq) * KS + 16 * s + 8 * hf]));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          sacc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qr[qb][s], sacc[qb], 0, 0, 0);
      }

      // ---- online softmax over the 32 keys
      const bool full = kb0 + 32 <= Lk;
      bf16x8 pb[2][QB];  // [ks][qb]
      bool rescale = false;
      float alpha[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float sv = sacc[qb][i] * p.scale_log2;
          if (!full) {
            const int key = kb0 + 8 * (i / 4) + 4 * hf + (i % 4);
            if (key >= Lk) sv = -INFINITY;
          }
          sacc[qb][i] = sv;
          mx = fmaxf(mx, sv);
        }
        mx = fmaxf(mx, xor32(mx));
        const float mnew = fmaxf(m[qb], mx);
        const float mref = mnew == -INFINITY ? 0.0f : mnew;
        alpha[qb] = __builtin_amdgcn_exp2f(m[qb] - mref);
        rescale |= mnew > m[qb];
        m[qb] = mnew;
        float ps = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          bf16x8 v;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float e = __builtin_amdgcn_exp2f(sacc[qb][8 * ks + j] - mref);
            ps += e;
            v[j] = static_cast<__bf16>(e);
          }
          pb[ks][qb] = v;
        }
        l[qb] = l[qb] * alpha[qb] + ps;
      }
      if (__any(rescale)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[qb][db][i] *= alpha[qb];
      }

      // ---- O^T += V^T P^T
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16x8 a =
              as_bf16x8(*reinterpret_cast<const uint4 *>(&Vt[(db * 32 + lq) * VS + kb * 32 + 16 * ks + 8 * hf]));
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ks][qb], o[qb][db], 0, 0, 0);
        }
    }
  }

  // ---- epilogue: O = O^T / l, rows of 4 consecutive dims per store
  uint16_t *op = p.o + static_cast<int64_t>(q_begin) * p.o_tok + h * p.o_head;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float lt = l[qb] + xor32(l[qb]);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int row = wq0 + qb * 32 + lq;
    if (row >= Lq) continue;
    uint16_t *orow = op + static_cast<int64_t>(row) * p.o_tok;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<__bf16>(o[qb][db][4 * g + e] * inv);
        *reinterpret_cast<bf16x4 *>(orow + d) = v;
      }
  }
}

// ---------------------------------------------------------------------------
// Two waves per SIMD.  A workgroup of 8 waves owns 256 query rows (32 per
// wave) of one (query sequence, head) pair, so every SIMD runs two waves
// whose MFMA and softmax phases overlap; each wave stays within 256
// registers.  K and V^T tiles of 64 keys are double-buffered in LDS with one
// barrier per tile: waves 0-3 stage K rows (16-byte loads), waves 4-7 stage V
// and transpose it in registers.  Global loads for tile t+2 are issued while
// tile t is consumed.  Inside a tile the QK^T product of the second 32-key
// block is issued before the softmax of the first.
//
// The softmax keeps its running maximum in log2 units and moves it only when
// a new block exceeds it by more than kLazy (probabilities stay <= 2^kLazy,
// far inside fp32 and bf16 range); O and the row sums are rescaled only
// then.  The final O / l is the exact softmax either way.
// ---------------------------------------------------------------------------
constexpr int kWaves2 = 4;
constexpr float kLazy = 8.0f;

template <int D, int W>
__global__ void __launch_bounds__(64 * W, 2) attn_fwd2_kernel(AttnParams p) {
  constexpr int BQ = 32 * W;
  constexpr int HT = 32 * W;  // threads per staging role (half the workgroup)
  constexpr int DS = D / 16;
  constexpr int DB = D / 32;
  constexpr int KS = D + 8;
  constexpr int VS = kBK + 8;
  constexpr int KCH = D / 8;
  constexpr int KLD = kBK * KCH / HT;  // 16-byte K loads per thread of the K half
  static_assert(KLD * HT == kBK * KCH, "K tile split");
  constexpr int VGRP = kBK / 4;
  constexpr int VPAIRS = VGRP * KCH;    // (4-key group, 16-byte chunk) pairs of the V half
  constexpr int VPP = (VPAIRS + HT - 1) / HT;  // pairs per thread
  static_assert(VPP * 4 <= 8 && KLD <= 8, "staging registers");
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBK * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][D * VS];

  const int wg = xcd_remap(blockIdx.x, p.n_wg);
  const int seq = wg / p.q_tiles, qt = wg % p.q_tiles;
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
  const float c = p.scale_log2;

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

  // K/V reads go through buffer resources bounded at the sequence's last
  // row: rows past Lk read as zero without a branch, and no access can leave
  // the sequence.
  const int64_t kv_bytes = static_cast<int64_t>(Lk) * p.kv_tok * 2;
  const int nrec = static_cast<int>(kv_bytes < 0x7fffffff ? kv_bytes : 0x7fffffff);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(kp), 0, nrec, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(vp), 0, nrec, kRsrcWord3);
  const int row_bytes = static_cast<int>(p.kv_tok) * 2;

  // staging roles, decided per wave (readfirstlane makes the uniformity
  // visible to the compiler, so each role keeps its own scalar resource)
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const bool k_loader = wave_u < W / 2;
  const int vt = tid - HT;
  uint4 st[8];

  auto load_tile = [&](int kt) {
    const int kbase = kt * kBK;
    if (k_loader) {
#pragma unroll
      for (int r = 0; r < KLD; ++r) {
        const int idx = tid + r * HT;
        const int row = idx / KCH, ch = idx % KCH;
        st[r] = bload16(rk, (kbase + row) * row_bytes + ch * 16);
      }
    } else {
#pragma unroll
      for (int pp = 0; pp < VPP; ++pp) {
        const int pair = vt + pp * HT;
        if (VPAIRS % HT == 0 || pair < VPAIRS) {
          const int vgrp = pair % VGRP, vch = pair / VGRP;
#pragma unroll
          for (int j = 0; j < 4; ++j) st[pp * 4 + j] = bload16(rv, (kbase + vgrp * 4 + j) * row_bytes + vch * 16);
        }
      }
    }
  };
  auto store_tile = [&](int buf) {
    if (k_loader) {
#pragma unroll
      for (int r = 0; r < KLD; ++r) {
        const int idx = tid + r * HT;
        const int row = idx / KCH, ch = idx % KCH;
        *reinterpret_cast<uint4 *>(&Ks[buf][row * KS + ch * 8]) = st[r];
      }
    } else {
#pragma unroll
      for (int pp = 0; pp < VPP; ++pp) {
        const int pair = vt + pp * HT;
        if (VPAIRS % HT == 0 || pair < VPAIRS) {
          const int vgrp = pair % VGRP, vch = pair / VGRP;
          const uint4 *q4 = st + pp * 4;
          const uint32_t w0[4] = {q4[0].x, q4[0].y, q4[0].z, q4[0].w};
          const uint32_t w1[4] = {q4[1].x, q4[1].y, q4[1].z, q4[1].w};
          const uint32_t w2[4] = {q4[2].x, q4[2].y, q4[2].z, q4[2].w};
          const uint32_t w3[4] = {q4[3].x, q4[3].y, q4[3].z, q4[3].w};
          const int col = vt_pos(vgrp * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t lo01 = (w0[e] & 0xffffu) | (w1[e] << 16);
            const uint32_t lo23 = (w2[e] & 0xffffu) | (w3[e] << 16);
            const uint32_t hi01 = (w0[e] >> 16) | (w1[e] & 0xffff0000u);
            const uint32_t hi23 = (w2[e] >> 16) | (w3[e] & 0xffff0000u);
            *reinterpret_cast<uint2 *>(&Vt[buf][(vch * 8 + 2 * e) * VS + col]) = make_uint2(lo01, lo23);
            *reinterpret_cast<uint2 *>(&Vt[buf][(vch * 8 + 2 * e + 1) * VS + col]) = make_uint2(hi01, hi23);
          }
        }
      }
    }
  };

  auto qk = [&](int buf, int kb) {
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4 *>(&Ks[buf][(kb * 32 + lq) * KS + 16 * s + 8 * hf]));
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qr[s], acc, 0, 0, 0);
    }
    return acc;
  };

  // softmax of one 64-key tile (two 32-key S^T blocks) and O^T += V^T P^T
  auto consume = [&](f32x16 s0, f32x16 s1, int buf, int kb0) {
    if (kb0 + kBK > Lk) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb0 + 8 * (i / 4) + 4 * hf + (i % 4);
        if (key >= Lk) s0[i] = -INFINITY;
        if (key + 32 >= Lk) s1[i] = -INFINITY;
      }
    }
    float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, fmaxf(s0[i], s1[i]));
    mx = half_max(mx) * c;
    const bool move = mx > m + kLazy || m == -INFINITY;
    float alpha = 1.0f;
    if (move) {
      alpha = __builtin_amdgcn_exp2f(m - mx);
      m = mx;
    }
    float ps = 0.0f;
    bf16x8 pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sv = ks < 2 ? s0[8 * ks + j] : s1[8 * (ks - 2) + j];
        const float e = __builtin_amdgcn_exp2f(fmaf(sv, c, -m));
        ps += e;
        pb[ks][j] = static_cast<__bf16>(e);
      }
    l = l * alpha + ps;
    if (__any(move)) {
      // in place (tied operands), so the accumulators keep their registers
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) asm volatile("v_mul_f32_e32 %0, %1, %0" : "+v"(o[db][i]) : "v"(alpha));
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16x8 a =
            as_bf16x8(*reinterpret_cast<const uint4 *>(&Vt[buf][(db * 32 + lq) * VS + 16 * ks + 8 * hf]));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ks], o[db], 0, 0, 0);
      }
  };

  const int n_tiles = (Lk + kBK - 1) / kBK;
  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
    if (n_tiles > 1) load_tile(1);
  }
  for (int kt = 0; kt < n_tiles; ++kt) {
    const int buf = kt & 1;
    __syncthreads();
    if (kt + 1 < n_tiles) store_tile(buf ^ 1);
    if (kt + 2 < n_tiles) load_tile(kt + 2);
    const f32x16 s0 = qk(buf, 0);
    const f32x16 s1 = qk(buf, 1);
    consume(s0, s1, buf, kt * kBK);
  }

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

template <int D>
static int launch_attn2(const pkv_attn_args *a, hipStream_t st) {
  constexpr int BQ = 32 * kWaves2;
  AttnParams p;
  p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o;
  p.cu_q = a->cu_seqlens_q; p.cu_k = a->cu_seqlens_k;
  p.Hq = a->num_heads_q;
  p.kv_per_head = a->kv_per_head;
  p.q_tiles = (a->max_seqlen_q + BQ - 1) / BQ;
  const int64_t n = static_cast<int64_t>(p.q_tiles) * a->num_batches * a->num_heads_q;
  if (n > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: grid too large");
  p.n_wg = static_cast<int>(n);
  p.q_tok = a->q_tok_stride; p.q_head = a->q_head_stride;
  p.kv_tok = a->kv_tok_stride; p.kv_head = a->kv_head_stride;
  p.o_tok = a->o_tok_stride; p.o_head = a->o_head_stride;
  p.scale_log2 = a->softmax_scale * 1.4426950408889634f;
  if (p.n_wg == 0) return PKV_OK;
  hipLaunchKernelGGL((attn_fwd2_kernel<D, kWaves2>), dim3(p.n_wg), dim3(64 * kWaves2), 0, st, p);
  return check_launch("attn_fwd2_kernel");
}

template <int D, int QB>
static int launch_attn(const pkv_attn_args *a, hipStream_t st) {
  constexpr int BQ = 32 * QB * kAttnWaves;
  AttnParams p;
  p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o;
  p.cu_q = a->cu_seqlens_q; p.cu_k = a->cu_seqlens_k;
  p.Hq = a->num_heads_q;
  p.kv_per_head = a->kv_per_head;
  p.q_tiles = (a->max_seqlen_q + BQ - 1) / BQ;
  const int64_t n = static_cast<int64_t>(p.q_tiles) * a->num_batches * a->num_heads_q;
  if (n > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: grid too large");
  p.n_wg = static_cast<int>(n);
  p.q_tok = a->q_tok_stride; p.q_head = a->q_head_stride;
  p.kv_tok = a->kv_tok_stride; p.kv_head = a->kv_head_stride;
  p.o_tok = a->o_tok_stride; p.o_head = a->o_head_stride;
  p.scale_log2 = a->softmax_scale * 1.4426950408889634f;
  if (p.n_wg == 0) return PKV_OK;
  hipLaunchKernelGGL((attn_fwd_kernel<D, QB>), dim3(p.n_wg), dim3(kAttnThreads), 0, st, p);
  return check_launch("attn_fwd_kernel");
}

}  // namespace pkv

using namespace pkv;

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
  hipStream_t st = as_stream(stream);
  switch (a->head_dim) {
    case 128: return launch_attn2<128>(a, st);
    case 64: return launch_attn2<64>(a, st);
    default: return fail(PKV_ERR_UNSUPPORTED, "ragged_attn: head_dim %d (supported: 64, 128)", a->head_dim);
  }
}
