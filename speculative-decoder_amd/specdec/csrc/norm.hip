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

// One workgroup per row, the row held in registers (kNormPer values per
// thread, dim <= kNormThreads * kNormPer).  If delta is non-null:
// hidden <- hidden + delta (rounded to T) first.  Then
// out <- weight * T(hidden * rsqrt(mean + eps)).
constexpr int kNormPer = 32;

template <typename T>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(T *__restrict__ hidden, const T *__restrict__ delta,
                                                                   const T *__restrict__ weight, T *__restrict__ out,
                                                                   int64_t dim, float eps) {
  __shared__ float red[kNormThreads / kWave];
  const int64_t row = blockIdx.x;
  T *h = hidden + row * dim;
  const T *dl = delta ? delta + row * dim : nullptr;
  T *y = out + row * dim;
  const int tid = threadIdx.x;
  float v[kNormPer], w[kNormPer];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) {
    const int64_t i = tid + (int64_t)k * kNormThreads;
    v[k] = 0.0f;
    w[k] = 0.0f;
    if (i < dim) {
      float x = to_f32(h[i]);
      if (dl) {
        const T s = from_f32<T>(x + to_f32(dl[i]));
        h[i] = s;
        x = to_f32(s);
      }
      v[k] = x;
      w[k] = to_f32(weight[i]);
    }
    ss += v[k] * v[k];
  }
  ss = block_sum(ss, red);
  const float inv = rsqrtf(ss / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) {
    const int64_t i = tid + (int64_t)k * kNormThreads;
    if (i < dim) y[i] = from_f32<T>(w[k] * to_f32(from_f32<T>(v[k] * inv)));
  }
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
  dim3 grid((unsigned)rows), block(kNormThreads);
  hipStream_t s = as_stream(stream);
  if (dtype == SPECDEC_BF16) {
    add_rmsnorm_kernel<__hip_bfloat16><<<grid, block, 0, s>>>(
        (__hip_bfloat16 *)hidden, (const __hip_bfloat16 *)delta, (const __hip_bfloat16 *)weight,
        (__hip_bfloat16 *)out, dim, eps);
  } else if (dtype == SPECDEC_F32) {
    add_rmsnorm_kernel<float><<<grid, block, 0, s>>>((float *)hidden, (const float *)delta, (const float *)weight,
                                                     (float *)out, dim, eps);
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
