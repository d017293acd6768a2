// Elementwise layer glue of the Llama forward: residual add + RMSNorm,
// SiLU(gate) * up, and SiLU(gate) * up with the post-attention RMSNorm's row
// scale applied to a gate/up projection of the unnormalised residual stream.
//
// Numerics follow transformers' Llama modules as lm/forward.py:56,64-65
// calls them: the residual add rounds to the activation type, RMSNorm
// normalises in fp32 (x * rsqrt(mean(x^2) + eps)), rounds to the
// activation type and then multiplies by the weight; SiLU is computed in
// fp32, rounded, then multiplied by `up` and rounded again.
#include "common.h"

#include <math.h>

namespace specdec {

constexpr int kNormThreads = 256;

// One workgroup per row, the row held in registers (PER values per thread,
// dim <= kNormThreads * PER).  If delta is non-null: hidden <- hidden + delta
// (rounded to T) first.  Then out <- weight * T(hidden * rsqrt(mean + eps)).
constexpr int kNormPer = 32;  // largest PER: dim <= 8192

template <typename T, int PER>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(T *__restrict__ hidden, const T *__restrict__ delta,
                                                                   const T *__restrict__ weight, T *__restrict__ out,
                                                                   int64_t dim, float eps) {
  __shared__ float red[kNormThreads / kWave];
  const int64_t row = blockIdx.x;
  T *h = hidden + row * dim;
  const T *dl = delta ? delta + row * dim : h;  // h stands in when there is no delta
  T *y = out + row * dim;
  const int tid = threadIdx.x;
  // every load is issued before the first store and without a branch
  // (indices clamped into the row), so the row costs one memory round trip
  float v[PER], w[PER], dv[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int64_t i = min(tid + (int64_t)k * kNormThreads, dim - 1);
    v[k] = to_f32(h[i]);
    w[k] = to_f32(weight[i]);
    dv[k] = to_f32(dl[i]);
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int64_t i = tid + (int64_t)k * kNormThreads;
    if (delta) {
      const T s = from_f32<T>(v[k] + dv[k]);
      if (i < dim) h[i] = s;
      v[k] = to_f32(s);
    }
    if (i >= dim) v[k] = 0.0f;
    ss += v[k] * v[k];
  }
  ss = block_sum(ss, red);
  const float inv = rsqrtf(ss / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int64_t i = tid + (int64_t)k * kNormThreads;
    if (i < dim) y[i] = from_f32<T>(w[k] * to_f32(from_f32<T>(v[k] * inv)));
  }
}

// ---- rows of 16-byte vectors -------------------------------------------
// Element e of a 16-byte vector of T.
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
template <typename T> __device__ __forceinline__ float vec_elem(const u32x4 &v, int e);
template <> __device__ __forceinline__ float vec_elem<float>(const u32x4 &v, int e) {
  const unsigned u = v[e];  // (a vector element straight inside __builtin_bit_cast reads element 0)
  return __builtin_bit_cast(float, u);
}
template <> __device__ __forceinline__ float vec_elem<__hip_bfloat16>(const u32x4 &v, int e) {
  return __uint_as_float((e & 1) ? (v[e >> 1] & 0xFFFF0000u) : (v[e >> 1] << 16));
}
template <typename T> __device__ __forceinline__ void vec_set(u32x4 &v, int e, T x);
template <> __device__ __forceinline__ void vec_set<float>(u32x4 &v, int e, float x) {
  v[e] = __builtin_bit_cast(unsigned, x);
}
template <> __device__ __forceinline__ void vec_set<__hip_bfloat16>(u32x4 &v, int e, __hip_bfloat16 x) {
  const unsigned b = __builtin_bit_cast(unsigned short, x), sh = 16 * (e & 1);
  v[e >> 1] = (v[e >> 1] & ~(0xFFFFu << sh)) | (b << sh);
}

// One wave per row, the row as 16-byte vectors in registers (NV per lane):
// the same arithmetic as add_rmsnorm_kernel, with the sum of squares
// reduced across the wave (no LDS, no barrier) -- the decode-size case,
// where a launch is a few microseconds of latency.  Needs dim a multiple
// of 16 / sizeof(T) and 16-byte aligned rows.
template <typename T, int NV>
__global__ __launch_bounds__(kWave) void add_rmsnorm_wave_kernel(T *__restrict__ hidden, const T *__restrict__ delta,
                                                                 const T *__restrict__ weight, T *__restrict__ out,
                                                                 int64_t dim, float eps) {
  constexpr int E = 16 / sizeof(T);
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x, nvec = (int)(dim / E);
  u32x4 *h = reinterpret_cast<u32x4 *>(hidden + row * dim);
  const u32x4 *dl = delta ? reinterpret_cast<const u32x4 *>(delta + row * dim) : h;
  const u32x4 *w = reinterpret_cast<const u32x4 *>(weight);
  u32x4 *y = reinterpret_cast<u32x4 *>(out + row * dim);
  u32x4 hv[NV], dv[NV], wv[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {  // every load first, indices clamped into the row
    const int i = min(lane + kWave * k, nvec - 1);
    hv[k] = h[i];
    dv[k] = dl[i];
    wv[k] = w[i];
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const bool in = lane + kWave * k < nvec;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float x = vec_elem<T>(hv[k], e);
      if (delta) {
        const T s = from_f32<T>(x + vec_elem<T>(dv[k], e));
        vec_set<T>(hv[k], e, s);
        x = to_f32(s);
      }
      ss += in ? x * x : 0.0f;
    }
    if (delta && in) h[lane + kWave * k] = hv[k];
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if (lane + kWave * k >= nvec) continue;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < E; ++e)
      vec_set<T>(o, e, from_f32<T>(vec_elem<T>(wv[k], e) * to_f32(from_f32<T>(vec_elem<T>(hv[k], e) * inv))));
    y[lane + kWave * k] = o;
  }
}

// SiLU(gate) * up over 16-byte vectors: thread i of row r handles elements
// 8i .. 8i+7 (bf16; 4 for fp32), one load of each operand.
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(const T *__restrict__ gu, T *__restrict__ out,
                                                            int64_t inter) {
  constexpr int E = 16 / sizeof(T);
  const int64_t r = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= inter / E) return;
  const u32x4 g = reinterpret_cast<const u32x4 *>(gu + r * 2 * inter)[i];
  const u32x4 u = reinterpret_cast<const u32x4 *>(gu + r * 2 * inter + inter)[i];
  u32x4 o;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float x = vec_elem<T>(g, e);
    const T a = from_f32<T>(x / (1.0f + expf(-x)));
    vec_set<T>(o, e, from_f32<T>(to_f32(a) * vec_elem<T>(u, e)));
  }
  reinterpret_cast<u32x4 *>(out + r * inter)[i] = o;
}

// The post-attention RMSNorm finished after the gate/up projection instead of
// before it.  With s = rsqrt(mean(x^2) + eps) and g the norm weight,
//   (g * (x * s)) @ W^T = s * (x @ (W diag(g))^T),
// so the projection reads the residual stream x itself, with g folded into
// W's columns, and this kernel scales each gate and up value by its row's s
// (rounded to T, as a projection's output is) before SiLU(gate) * up.
//
// Each wave reduces its row's sum of squares itself: lane l adds the row's
// 16-byte vectors l, l+64, l+128, ... in order, then wave_sum_dpp (lane moves
// in a fixed pattern, no LDS).  Every wave of every call therefore computes
// the same s for the same row, whatever the grid and the number of rows,
// with no barrier.  NV vectors per lane are in flight per pass over the row.
template <typename T, int NV>
__global__ __launch_bounds__(256) void rms_silu_mul_vec_kernel(const T *__restrict__ gu, const T *__restrict__ hidden,
                                                                T *__restrict__ out, int64_t inter, int64_t dim,
                                                                float eps) {
  constexpr int E = 16 / sizeof(T);
  const int64_t r = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = i < inter / E;
  const int64_t ic = live ? i : 0;  // dead lanes still take part in the wave's reduction
  const u32x4 g = reinterpret_cast<const u32x4 *>(gu + r * 2 * inter)[ic];
  const u32x4 u = reinterpret_cast<const u32x4 *>(gu + r * 2 * inter + inter)[ic];
  const u32x4 *h = reinterpret_cast<const u32x4 *>(hidden + r * dim);
  const int nvec = (int)(dim / E);
  if constexpr (sizeof(T) == 2) {
    // bf16: the helpers linear_silu_kernel shares (same bits for a row)
    const float s = row_rms_scale_bf16<NV>(h, nvec, (int)dim, eps, lane);
    if (!live) return;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < E; ++e)
      vec_set<T>(o, e, __builtin_bit_cast(T, silu_mul_scaled_bf16(vec_elem<T>(g, e), vec_elem<T>(u, e), s)));
    reinterpret_cast<u32x4 *>(out + r * inter)[i] = o;
    return;
  }
  float ss = 0.0f;
  for (int base = 0; base < nvec; base += kWave * NV) {
    u32x4 hv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) hv[k] = h[min(base + lane + kWave * k, nvec - 1)];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const bool in = base + lane + kWave * k < nvec;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float x = vec_elem<T>(hv[k], e);
        ss += in ? x * x : 0.0f;
      }
    }
  }
  ss = wave_sum_dpp(ss);
  const float s = rsqrtf(ss / (float)dim + eps);
  if (!live) return;
  u32x4 o;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float x = to_f32(from_f32<T>(s * vec_elem<T>(g, e)));
    const float up = to_f32(from_f32<T>(s * vec_elem<T>(u, e)));
    const T a = from_f32<T>(x / (1.0f + expf(-x)));
    vec_set<T>(o, e, from_f32<T>(to_f32(a) * up));
  }
  reinterpret_cast<u32x4 *>(out + r * inter)[i] = o;
}

// The same for any dim, inter and alignment, one element per thread: lane l
// adds elements l, l+64, ... of the row.
template <typename T>
__global__ __launch_bounds__(256) void rms_silu_mul_kernel(const T *__restrict__ gu, const T *__restrict__ hidden,
                                                           T *__restrict__ out, int64_t inter, int64_t dim,
                                                           float eps) {
  const int64_t r = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  float ss = 0.0f;
  for (int64_t j = lane; j < dim; j += kWave) {
    const float x = to_f32(hidden[r * dim + j]);
    ss += x * x;
  }
  ss = wave_sum_dpp(ss);
  const float s = rsqrtf(ss / (float)dim + eps);
  if (c >= inter) return;
  const float x = to_f32(from_f32<T>(s * to_f32(gu[r * 2 * inter + c])));
  const float up = to_f32(from_f32<T>(s * to_f32(gu[r * 2 * inter + inter + c])));
  const T a = from_f32<T>(x / (1.0f + expf(-x)));
  out[r * inter + c] = from_f32<T>(to_f32(a) * up);
}

template <typename T>
__global__ void silu_mul_kernel(const T *__restrict__ gu, T *__restrict__ out, int64_t rows, int64_t inter) {
  const int64_t total = rows * inter;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / inter, c = i - r * inter;
    const float g = to_f32(gu[r * 2 * inter + c]);
    const T a = from_f32<T>(g / (1.0f + expf(-g)));
    out[i] = from_f32<T>(to_f32(a) * to_f32(gu[r * 2 * inter + inter + c]));
  }
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

template <typename T>
static void launch_add_rmsnorm(T *hidden, const T *delta, const T *weight, T *out, int64_t rows, int64_t dim,
                               float eps, hipStream_t s) {
  constexpr int E = 16 / sizeof(T);
  const int64_t nvec = dim / E;
  if (dim % E == 0 && nvec <= 8 * kWave && aligned16(hidden) && aligned16(weight) && aligned16(out) &&
      (!delta || aligned16(delta))) {
    dim3 grid((unsigned)rows), block(kWave);
    if (nvec <= 2 * kWave) add_rmsnorm_wave_kernel<T, 2><<<grid, block, 0, s>>>(hidden, delta, weight, out, dim, eps);
    else if (nvec <= 4 * kWave) add_rmsnorm_wave_kernel<T, 4><<<grid, block, 0, s>>>(hidden, delta, weight, out, dim, eps);
    else add_rmsnorm_wave_kernel<T, 8><<<grid, block, 0, s>>>(hidden, delta, weight, out, dim, eps);
    return;
  }
  dim3 grid((unsigned)rows), block(kNormThreads);
  if (dim <= 4 * kNormThreads)
    add_rmsnorm_kernel<T, 4><<<grid, block, 0, s>>>(hidden, delta, weight, out, dim, eps);
  else if (dim <= 8 * kNormThreads)
    add_rmsnorm_kernel<T, 8><<<grid, block, 0, s>>>(hidden, delta, weight, out, dim, eps);
  else if (dim <= 16 * kNormThreads)
    add_rmsnorm_kernel<T, 16><<<grid, block, 0, s>>>(hidden, delta, weight, out, dim, eps);
  else
    add_rmsnorm_kernel<T, kNormPer><<<grid, block, 0, s>>>(hidden, delta, weight, out, dim, eps);
}

}  // namespace specdec

using namespace specdec;

SPECDEC_API int specdec_add_rmsnorm(void *hidden, const void *delta, const void *weight, void *out, int dtype,
                                    int64_t rows, int64_t dim, float eps, void *stream) {
  if (rows < 0 || dim <= 0) return SPECDEC_EINVAL;
  if (dim > (int64_t)kNormThreads * kNormPer) return SPECDEC_EUNSUPPORTED;
  if (rows == 0) return SPECDEC_OK;
  if (!hidden || !weight || !out) return SPECDEC_EINVAL;
  hipStream_t s = as_stream(stream);
  if (dtype == SPECDEC_BF16) {
    launch_add_rmsnorm<__hip_bfloat16>((__hip_bfloat16 *)hidden, (const __hip_bfloat16 *)delta,
                                       (const __hip_bfloat16 *)weight, (__hip_bfloat16 *)out, rows, dim, eps, s);
  } else if (dtype == SPECDEC_F32) {
    launch_add_rmsnorm<float>((float *)hidden, (const float *)delta, (const float *)weight, (float *)out, rows, dim,
                              eps, s);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}

SPECDEC_API int specdec_silu_mul(const void *gate_up, void *out, int dtype, int64_t rows, int64_t inter,
                                 void *stream) {
  if (rows < 0 || inter <= 0) return SPECDEC_EINVAL;
  if (rows == 0) return SPECDEC_OK;
  if (!gate_up || !out) return SPECDEC_EINVAL;
  hipStream_t s = as_stream(stream);
  const int E = (dtype == SPECDEC_BF16) ? 8 : 4;
  if ((dtype == SPECDEC_BF16 || dtype == SPECDEC_F32) && inter % E == 0 && rows <= 65535 &&
      aligned16(gate_up) && aligned16(out)) {
    dim3 grid((unsigned)((inter / E + 255) / 256), (unsigned)rows), block(256);
    if (dtype == SPECDEC_BF16)
      silu_mul_vec_kernel<__hip_bfloat16><<<grid, block, 0, s>>>((const __hip_bfloat16 *)gate_up,
                                                                 (__hip_bfloat16 *)out, inter);
    else
      silu_mul_vec_kernel<float><<<grid, block, 0, s>>>((const float *)gate_up, (float *)out, inter);
    return launch_status();
  }
  int64_t blocks = (rows * inter + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (dtype == SPECDEC_BF16) {
    silu_mul_kernel<__hip_bfloat16><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        (const __hip_bfloat16 *)gate_up, (__hip_bfloat16 *)out, rows, inter);
  } else if (dtype == SPECDEC_F32) {
    silu_mul_kernel<float><<<dim3((unsigned)blocks), dim3(256), 0, s>>>((const float *)gate_up, (float *)out, rows,
                                                                       inter);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}

namespace specdec {

template <typename T>
static void launch_rms_silu_mul(const T *gate_up, const T *hidden, T *out, int64_t rows, int64_t inter, int64_t dim,
                                float eps, hipStream_t s) {
  constexpr int E = 16 / sizeof(T);
  if (inter % E == 0 && dim % E == 0 && aligned16(gate_up) && aligned16(hidden) && aligned16(out)) {
    const int64_t nvec = dim / E;
    dim3 grid((unsigned)((inter / E + 255) / 256), (unsigned)rows), block(256);
    if (nvec <= 2 * kWave)
      rms_silu_mul_vec_kernel<T, 2><<<grid, block, 0, s>>>(gate_up, hidden, out, inter, dim, eps);
    else if (nvec <= 4 * kWave)
      rms_silu_mul_vec_kernel<T, 4><<<grid, block, 0, s>>>(gate_up, hidden, out, inter, dim, eps);
    else
      rms_silu_mul_vec_kernel<T, 8><<<grid, block, 0, s>>>(gate_up, hidden, out, inter, dim, eps);
    return;
  }
  dim3 grid((unsigned)((inter + 255) / 256), (unsigned)rows), block(256);
  rms_silu_mul_kernel<T><<<grid, block, 0, s>>>(gate_up, hidden, out, inter, dim, eps);
}

}  // namespace specdec

SPECDEC_API int specdec_rms_silu_mul(const void *gate_up, const void *hidden, void *out, int dtype, int64_t rows,
                                     int64_t inter, int64_t dim, float eps, void *stream) {
  if (rows < 0 || inter <= 0 || dim <= 0 || rows > 65535 || inter > ((int64_t)1 << 30)) return SPECDEC_EINVAL;
  if (rows == 0) return SPECDEC_OK;
  if (!gate_up || !hidden || !out) return SPECDEC_EINVAL;
  hipStream_t s = as_stream(stream);
  if (dtype == SPECDEC_BF16) {
    launch_rms_silu_mul<__hip_bfloat16>((const __hip_bfloat16 *)gate_up, (const __hip_bfloat16 *)hidden,
                                        (__hip_bfloat16 *)out, rows, inter, dim, eps, s);
  } else if (dtype == SPECDEC_F32) {
    launch_rms_silu_mul<float>((const float *)gate_up, (const float *)hidden, (float *)out, rows, inter, dim, eps, s);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}
