// Elementwise layer glue of the Llama forward, fused so a layer is nine
// launches: residual add + RMSNorm, and SiLU(gate) * up.
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

template <typename T>
static void launch_add_rmsnorm(T *hidden, const T *delta, const T *weight, T *out, int64_t rows, int64_t dim,
                               float eps, hipStream_t s) {
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
  int64_t blocks = (rows * inter + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t s = as_stream(stream);
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
