// Row operations of the causal DiT block that drives the pyramid cache in the
// end-to-end rollout (wan/modules/causal_model.py:395-420 of the reference):
// LayerNorm with modulation or affine weights, RMSNorm of q and k
// (wan/modules/model.py:70-99), the gated residual updates of the fp32
// residual stream, and the tanh GELU of the feed-forward.  Each is one
// launch instead of the chain of elementwise and reduction kernels that
// eager PyTorch runs for it.
//
// The row kernels give one wave to a row: lane i holds the 16-byte vectors
// i, i + 64, ... of the row in registers (up to kMaxVec of them), the sums
// are wave reductions, and the row is read from memory once.  LayerNorm
// takes the mean first and then the sum of squared deviations (two-pass in
// registers), so a large mean does not cancel the variance.

#include "pkv_common.h"

namespace pkv {

constexpr int kDitRowsPerBlock = 4;  // one wave per row
constexpr int kMaxVec = 16;          // 16-byte vectors per lane: rows up to 4096 fp32 / 8192 bf16

__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

__device__ inline float4 ld_f4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// a + float(b) * gate[4j..4j+3] with one rounding per element (fma), or
// a + float(b) without a gate: the residual update of 4 columns, shared by
// the residual kernel and the fused residual + LayerNorm so both round alike
__device__ inline float4 residual4(float4 a, uint2 b, const float *gate, int j) {
  const float y0 = bf16_to_f32(static_cast<uint16_t>(b.x & 0xffff)), y1 = bf16_to_f32(static_cast<uint16_t>(b.x >> 16));
  const float y2 = bf16_to_f32(static_cast<uint16_t>(b.y & 0xffff)), y3 = bf16_to_f32(static_cast<uint16_t>(b.y >> 16));
  if (gate) {
    const float4 g = ld_f4(gate + 4 * j);
    return make_float4(__fmaf_rn(y0, g.x, a.x), __fmaf_rn(y1, g.y, a.y), __fmaf_rn(y2, g.z, a.z),
                       __fmaf_rn(y3, g.w, a.w));
  }
  return make_float4(__fadd_rn(a.x, y0), __fadd_rn(a.y, y1), __fadd_rn(a.z, y2), __fadd_rn(a.w, y3));
}

// out[r, :] = bf16(LN(x[r, :]) * m + a), LN without affine weights; m =
// (one_plus ? 1 + mul : mul) and a = add, each optional (1 and 0).  kRes
// first applies the residual update x[r, :] += float(y[r, :]) * gate in
// registers and writes the updated row back, so the row is read once.
template <int K, bool kRes>
__global__ void __launch_bounds__(64 * kDitRowsPerBlock) ln_mod_kernel(float *x, int64_t rows, int C,
                                                                       const float *mul, const float *add,
                                                                       int one_plus, float eps, uint16_t *out,
                                                                       const uint16_t *y, int64_t y_stride,
                                                                       const float *gate) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kDitRowsPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  float *xr = x + r * C;
  const int nv = C / 4;
  float4 v[K];
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int j = lane + 64 * k;
    v[k] = j < nv ? ld_f4(xr + 4 * j) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (kRes && j < nv) {
      v[k] = residual4(v[k], *reinterpret_cast<const uint2 *>(y + r * y_stride + 4 * j), gate, j);
      *reinterpret_cast<float4 *>(xr + 4 * j) = v[k];
    }
    s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
  }
  const float mean = wave_sum(s) / static_cast<float>(C);
  float q = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int j = lane + 64 * k;
    if (j < nv) {
      const float a = v[k].x - mean, b = v[k].y - mean, c = v[k].z - mean, d = v[k].w - mean;
      q += (a * a + b * b) + (c * c + d * d);
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / static_cast<float>(C) + eps);
  uint16_t *orow = out + r * C;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int j = lane + 64 * k;
    if (j >= nv) continue;
    float y[4] = {(v[k].x - mean) * rstd, (v[k].y - mean) * rstd, (v[k].z - mean) * rstd, (v[k].w - mean) * rstd};
    if (mul) {
      const float4 m = ld_f4(mul + 4 * j);
      const float mm[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] *= one_plus ? 1.0f + mm[e] : mm[e];
    }
    if (add) {
      const float4 a = ld_f4(add + 4 * j);
      y[0] += a.x;
      y[1] += a.y;
      y[2] += a.z;
      y[3] += a.w;
    }
    *reinterpret_cast<uint2 *>(orow + 4 * j) = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
  }
}

// out[r, :] = bf16(x * rsqrt(mean(x^2) + eps) * w) in fp32, x bf16
template <int K>
__global__ void __launch_bounds__(64 * kDitRowsPerBlock) rms_kernel(const uint16_t *x, int64_t x_stride, int64_t rows,
                                                                    int C, const float *w, float eps,
                                                                    uint16_t *out, int64_t out_stride) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kDitRowsPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  const uint16_t *xr = x + r * x_stride;
  const int nv = C / 8;
  uint4 v[K];
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int j = lane + 64 * k;
    v[k] = j < nv ? *reinterpret_cast<const uint4 *>(xr + 8 * j) : make_uint4(0, 0, 0, 0);
    const uint32_t wd[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = bf16_to_f32(static_cast<uint16_t>(wd[e] & 0xffff));
      const float b = bf16_to_f32(static_cast<uint16_t>(wd[e] >> 16));
      s += a * a + b * b;
    }
  }
  const float rn = rsqrtf(wave_sum(s) / static_cast<float>(C) + eps);
  uint16_t *orow = out + r * out_stride;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int j = lane + 64 * k;
    if (j >= nv) continue;
    const uint32_t wd[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a = bf16_to_f32(static_cast<uint16_t>(wd[e] & 0xffff)) * rn;
      float b = bf16_to_f32(static_cast<uint16_t>(wd[e] >> 16)) * rn;
      if (w) {
        a *= w[8 * j + 2 * e];
        b *= w[8 * j + 2 * e + 1];
      }
      o[e] = pack_bf16x2(a, b);
    }
    *reinterpret_cast<uint4 *>(orow + 8 * j) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// x[r, c] += float(y[r, c]) * gate[c] (gate optional: 1), 4 columns per thread
__global__ void __launch_bounds__(256) residual_kernel(float *x, int64_t rows, int C, const uint16_t *y,
                                                       int64_t y_stride, const float *gate) {
  const int nv = C / 4;
  const int64_t total = rows * nv;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / nv;
    const int j = static_cast<int>(i % nv);
    const float4 a = ld_f4(x + r * C + 4 * j);
    const uint2 b = *reinterpret_cast<const uint2 *>(y + r * y_stride + 4 * j);
    *reinterpret_cast<float4 *>(x + r * C + 4 * j) = residual4(a, b, gate, j);
  }
}

// out = bf16(0.5 x (1 + tanh(u))), u = sqrt(2 / pi) (x + 0.044715 x^3), in fp32, 8 values per thread.
// 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)), so the value is x / (1 + 2^(t)) with
// t = -2 log2(e) u: one v_exp_f32 and one v_rcp_f32 (each within about 1 ulp
// of fp32, far below the bf16 rounding of the result) instead of a library
// tanh.  Large |u| give x (t -> -inf) or a signed zero (t -> +inf).
__device__ inline float gelu_tanh_f32(float x) {
  constexpr float kC1 = -2.0f * 1.4426950408889634f * 0.7978845608028654f;  // -2 log2(e) sqrt(2/pi)
  constexpr float kC3 = kC1 * 0.044715f;
  const float t = x * fmaf(kC3, x * x, kC1);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// f32 pair -> bf16x2 by the hardware round-to-nearest-even conversion (NaN
// halves to 0x7fc0, as pack_bf16x2)
__device__ inline uint32_t cvt_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffu) > 0x7f80u) u = (u & 0xffff0000u) | 0x7fc0u;
  if ((u & 0x7fff0000u) > 0x7f800000u) u = (u & 0xffffu) | 0x7fc00000u;
  return u;
}

__global__ void __launch_bounds__(256) gelu_tanh_kernel(const uint16_t *x, int64_t n8, uint16_t *out) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n8;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint4 v = *reinterpret_cast<const uint4 *>(x + 8 * i);
    const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float f[2] = {bf16_to_f32(static_cast<uint16_t>(wd[e] & 0xffff)), bf16_to_f32(static_cast<uint16_t>(wd[e] >> 16))};
      o[e] = cvt_bf16x2(gelu_tanh_f32(f[0]), gelu_tanh_f32(f[1]));
    }
    *reinterpret_cast<uint4 *>(out + 8 * i) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

static int row_grid(int64_t rows);

// LayerNorm rows (kRes: after the residual update from y and gate)
template <bool kRes>
static int launch_ln_k(float *x, int64_t rows, int cols, const float *mul, const float *add, int mul_plus_one,
                       float eps, uint16_t *out, const uint16_t *y, int64_t y_stride, const float *gate, hipStream_t st,
                       const char *who) {
  const int vec = (cols / 4 + 63) / 64;
  const dim3 grid(row_grid(rows)), block(64 * kDitRowsPerBlock);
  if (vec <= 4)
    hipLaunchKernelGGL((ln_mod_kernel<4, kRes>), grid, block, 0, st, x, rows, cols, mul, add, mul_plus_one, eps, out, y,
                       y_stride, gate);
  else if (vec <= 8)
    hipLaunchKernelGGL((ln_mod_kernel<8, kRes>), grid, block, 0, st, x, rows, cols, mul, add, mul_plus_one, eps, out, y,
                       y_stride, gate);
  else if (vec <= kMaxVec)
    hipLaunchKernelGGL((ln_mod_kernel<kMaxVec, kRes>), grid, block, 0, st, x, rows, cols, mul, add, mul_plus_one, eps,
                       out, y, y_stride, gate);
  else
    return fail(PKV_ERR_UNSUPPORTED, "%s: cols (%d) above %d", who, cols, 64 * 4 * kMaxVec);
  return check_launch("ln_mod_kernel");
}

static int launch_ln(float *x, int64_t rows, int cols, const float *mul, const float *add, int mul_plus_one, float eps,
                     uint16_t *out, const uint16_t *y, int64_t y_stride, const float *gate, hipStream_t st,
                     const char *who) {
  return y ? launch_ln_k<true>(x, rows, cols, mul, add, mul_plus_one, eps, out, y, y_stride, gate, st, who)
           : launch_ln_k<false>(x, rows, cols, mul, add, mul_plus_one, eps, out, y, y_stride, gate, st, who);
}

static int row_grid(int64_t rows) {
  const int64_t g = (rows + kDitRowsPerBlock - 1) / kDitRowsPerBlock;
  return static_cast<int>(g);
}

static int flat_grid(int64_t items) {
  int64_t g = (items + 255) / 256;
  if (g > 65536) g = 65536;
  return static_cast<int>(g < 1 ? 1 : g);
}

}  // namespace pkv

using namespace pkv;

extern "C" int pkv_dit_layer_norm(const float *x, int64_t rows, int32_t cols, const float *mul, const float *add,
                                  int32_t mul_plus_one, float eps, uint16_t *out, pkv_stream_t stream) {
  if (rows == 0) return PKV_OK;
  if (!x || !out || rows < 0 || cols <= 0) return fail(PKV_ERR_INVALID, "dit_layer_norm: bad arguments");
  if (cols % 4) return fail(PKV_ERR_INVALID, "dit_layer_norm: cols (%d) must be a multiple of 4", cols);
  if (rows > 0x7fffffffLL * kDitRowsPerBlock) return fail(PKV_ERR_UNSUPPORTED, "dit_layer_norm: too many rows");
  return launch_ln(const_cast<float *>(x), rows, cols, mul, add, mul_plus_one, eps, out, nullptr, 0, nullptr,
                   as_stream(stream), "dit_layer_norm");
}

extern "C" int pkv_dit_residual_layer_norm(float *x, int64_t rows, int32_t cols, const uint16_t *y,
                                           int64_t y_row_stride, const float *gate, const float *mul,
                                           const float *add, int32_t mul_plus_one, float eps, uint16_t *out,
                                           pkv_stream_t stream) {
  if (rows == 0) return PKV_OK;
  if (!x || !y || !out || rows < 0 || cols <= 0) return fail(PKV_ERR_INVALID, "dit_residual_layer_norm: bad arguments");
  if (cols % 4 || y_row_stride % 4 || y_row_stride < cols)
    return fail(PKV_ERR_INVALID, "dit_residual_layer_norm: cols and the row stride must be multiples of 4 (cols %d)",
                cols);
  if (rows > 0x7fffffffLL * kDitRowsPerBlock)
    return fail(PKV_ERR_UNSUPPORTED, "dit_residual_layer_norm: too many rows");
  return launch_ln(x, rows, cols, mul, add, mul_plus_one, eps, out, y, y_row_stride, gate, as_stream(stream),
                   "dit_residual_layer_norm");
}

extern "C" int pkv_dit_rms_norm(const uint16_t *x, int64_t x_row_stride, int64_t rows, int32_t cols, const float *weight,
                                float eps, uint16_t *out, int64_t out_row_stride, pkv_stream_t stream) {
  if (rows == 0) return PKV_OK;
  if (!x || !out || rows < 0 || cols <= 0) return fail(PKV_ERR_INVALID, "dit_rms_norm: bad arguments");
  if (cols % 8 || x_row_stride % 8 || out_row_stride % 8 || x_row_stride < cols || out_row_stride < cols)
    return fail(PKV_ERR_INVALID, "dit_rms_norm: cols and row strides must be multiples of 8 (cols %d)", cols);
  if (rows > 0x7fffffffLL * kDitRowsPerBlock) return fail(PKV_ERR_UNSUPPORTED, "dit_rms_norm: too many rows");
  const int vec = (cols / 8 + 63) / 64;
  hipStream_t st = as_stream(stream);
  const dim3 grid(row_grid(rows)), block(64 * kDitRowsPerBlock);
  if (vec <= 4)
    hipLaunchKernelGGL(rms_kernel<4>, grid, block, 0, st, x, x_row_stride, rows, cols, weight, eps, out, out_row_stride);
  else if (vec <= kMaxVec)
    hipLaunchKernelGGL(rms_kernel<kMaxVec>, grid, block, 0, st, x, x_row_stride, rows, cols, weight, eps, out,
                       out_row_stride);
  else
    return fail(PKV_ERR_UNSUPPORTED, "dit_rms_norm: cols (%d) above %d", cols, 64 * 8 * kMaxVec);
  return check_launch("rms_kernel");
}

extern "C" int pkv_dit_residual(float *x, int64_t rows, int32_t cols, const uint16_t *y, int64_t y_row_stride,
                                const float *gate, pkv_stream_t stream) {
  if (rows == 0) return PKV_OK;
  if (!x || !y || rows < 0 || cols <= 0) return fail(PKV_ERR_INVALID, "dit_residual: bad arguments");
  if (cols % 4 || y_row_stride % 4 || y_row_stride < cols)
    return fail(PKV_ERR_INVALID, "dit_residual: cols and the row stride must be multiples of 4 (cols %d)", cols);
  hipLaunchKernelGGL(residual_kernel, dim3(flat_grid(rows * (cols / 4))), dim3(256), 0, as_stream(stream), x, rows,
                     cols, y, y_row_stride, gate);
  return check_launch("residual_kernel");
}

extern "C" int pkv_dit_gelu_tanh(const uint16_t *x, int64_t n, uint16_t *out, pkv_stream_t stream) {
  if (n == 0) return PKV_OK;
  if (!x || !out || n < 0) return fail(PKV_ERR_INVALID, "dit_gelu_tanh: bad arguments");
  if (n % 8) return fail(PKV_ERR_INVALID, "dit_gelu_tanh: n (%lld) must be a multiple of 8", static_cast<long long>(n));
  hipLaunchKernelGGL(gelu_tanh_kernel, dim3(flat_grid(n / 8)), dim3(256), 0, as_stream(stream), x, n / 8, out);
  return check_launch("gelu_tanh_kernel");
}
