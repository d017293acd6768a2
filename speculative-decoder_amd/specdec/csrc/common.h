// Shared helpers for the gfx950 kernels of libspecdec.so: status codes,
// stream casts, wavefront (64-lane) and workgroup reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../../include/specdec.h"

#define SPECDEC_API extern "C" __attribute__((visibility("default")))

namespace specdec {

constexpr int kWave = 64;

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPECDEC_OK : SPECDEC_EHIP;
}

// Compute units of the current device (0 if it cannot be read), looked up
// once per device.
inline int cu_count() {
  static int counts[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    counts[dev] = n;
  }
  return counts[dev];
}

// RoPE + paged append of a call's new tokens (cache.hip): q rotated in place
// and k rotated, both written back / into the pools, v copied; with kv_only
// the q heads are left untouched.
int launch_rope_append(void *qkv, int dtype, int64_t token_stride, int32_t H, int32_t Hkv, int32_t d,
                       const float *cos_t, const float *sin_t, const int32_t *meta, int32_t batch, int32_t width,
                       const int32_t *tables, int64_t table_stride, int32_t bs, void *k_pool, void *v_pool,
                       bool kv_only, hipStream_t s);
// A draft decode step's attention as split partials
// (attention_decode_parts_kernel, folded by linear_parts_kernel): 4, 8 or
// 16 one-wave workgroups per (row, kv head), each leaving per query head
// kDecPart floats: m, l, two unused, then the 64 dims of O not divided by l
// (16-byte aligned).  With kDecWaves of them the fold has the bits of
// attention_decode_kernel's.
constexpr int kDecWaves = 4;
constexpr int kDecMaxParts = 16;
constexpr int kDecPart = 4 + 64;

// The same for the k and v heads only of a prompt-sized bf16 call (head_dim
// 64, block_size % 16 == 0), one workgroup per 16-position group and kv
// head, V stored in 8-byte runs (cache.hip).
int launch_rope_append_groups(void *qkv, int64_t token_stride, int32_t H, int32_t Hkv, const float *cos_t,
                              const float *sin_t, const int32_t *meta, int32_t batch, int32_t width,
                              const int32_t *tables, int64_t table_stride, int32_t bs, void *k_pool, void *v_pool,
                              hipStream_t s);

// ---- element conversion -------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(double x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(__hip_bfloat16 x) { return __bfloat162float(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ double from_f32<double>(float x) { return x; }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float x) {
  return __float2bfloat16(x);  // round to nearest even
}

// ---- RoPE -----------------------------------------------------------------
// transformers' q * cos + rotate_half(q) * sin for one (x1, x2) pair, with
// each product and each sum rounded on its own, as the separate elementwise
// ops of the reference round them.  hipcc contracts a * b - c * d into a
// fused multiply-add by default (one rounding fewer, so a nearly cancelling
// pair can land one bf16 step away once rounded), so contraction is
// switched off for these four products and two sums.
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float &y1, float &y2) {
#pragma clang fp contract(off)
  const float x1c = x1 * c, x2s = x2 * s, x2c = x2 * c, x1s = x1 * s;
  y1 = x1c - x2s;
  y2 = x2c + x1s;
}

// ---- wavefront reductions (all 64 lanes participate) --------------------
template <typename T> __device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
// The same sum through DPP lane moves instead of LDS permutes: within each
// row of 16 lanes, partners at xor 1, xor 2 (quad permutes), then the mirror
// in 8 and in 16 lanes, so every lane of a row holds the row's sum; then the
// four row sums are read into scalar registers and added as (r0 + r1) +
// (r2 + r3).  Each step adds a pair of equal-bit operands in both lanes, so
// every lane returns the same bits, in an order fixed by the lane layout.
template <int CTRL> __device__ __forceinline__ float dpp_partner_add(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true);
  return v + __int_as_float(moved);
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_partner_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]: xor 1
  v = dpp_partner_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]: xor 2
  v = dpp_partner_add<0x141>(v);  // row_half_mirror: lane i <-> 7 - i
  v = dpp_partner_add<0x140>(v);  // row_mirror: lane i <-> 15 - i
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}
// argmax of (value, index) pairs: the larger value, the lower index among
// equal values
__device__ __forceinline__ void argmax_keep(float &best, int &best_i, float v, int i) {
  if (v > best || (v == best && i < best_i)) {
    best = v;
    best_i = i;
  }
}

// The same reductions through DPP row moves (xor 1, xor 2, the half-row and
// row mirrors), then the four row results read into scalars and combined in
// row order: every lane returns the same value, in a fixed order.
template <int CTRL> __device__ __forceinline__ int dpp_move(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

template <int CTRL> __device__ __forceinline__ float dpp_max_step(float v) {
  return fmaxf(v, __int_as_float(dpp_move<CTRL>(__float_as_int(v))));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = dpp_max_step<0xB1>(v);
  v = dpp_max_step<0x4E>(v);
  v = dpp_max_step<0x141>(v);
  v = dpp_max_step<0x140>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

template <int CTRL> __device__ __forceinline__ void dpp_argmax_step(float &best, int &best_i) {
  const float ob = __int_as_float(dpp_move<CTRL>(__float_as_int(best)));
  const int oi = dpp_move<CTRL>(best_i);
  argmax_keep(best, best_i, ob, oi);
}

__device__ __forceinline__ void wave_argmax_dpp(float &best, int &best_i) {
  dpp_argmax_step<0xB1>(best, best_i);
  dpp_argmax_step<0x4E>(best, best_i);
  dpp_argmax_step<0x141>(best, best_i);
  dpp_argmax_step<0x140>(best, best_i);
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best), 0));
  int bi = __builtin_amdgcn_readlane(best_i, 0);
#pragma unroll
  for (int row = 1; row < 4; ++row)
    argmax_keep(b, bi, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best), 16 * row)),
                __builtin_amdgcn_readlane(best_i, 16 * row));
  best = b;
  best_i = bi;
}

template <typename T> __device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, kWave));
  return v;
}

// ---- the post-attention norm finished after the gate/up projection -------
// (rms_silu_mul_vec_kernel in norm.hip and linear_silu_kernel in linear.hip
// share these, so a row's activation has the same bits from either.)
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

// s = rsqrt(mean(h^2) + eps) of one bf16 row of `dim` elements stored as
// nvec 16-byte vectors: lane l adds the squares of its vectors l, l + 64,
// ... (NV per pass) in order, eight elements each in order, then
// wave_sum_dpp -- one fixed order, so every wave that computes it gets the
// same bits.  Contraction is off: each square and each sum is rounded on
// its own wherever the function is inlined.
template <int NV>
__device__ __forceinline__ void row_squares_pass_bf16(const u32x4 (&hv)[NV], int base, int nvec, int lane,
                                                      float &ss) {
#pragma clang fp contract(off)
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const bool in = base + lane + kWave * k < nvec;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const unsigned w = hv[k][e >> 1];
      const float x = __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
      const float sq = x * x;
      ss += in ? sq : 0.0f;
    }
  }
}
template <int NV>
__device__ __forceinline__ void row_pass_loads(const u32x4 *h, int base, int nvec, int lane, u32x4 (&hv)[NV]) {
#pragma unroll
  for (int k = 0; k < NV; ++k) hv[k] = h[min(base + lane + kWave * k, nvec - 1)];
}
// The rest of the row after its first pass (hv: that pass's vectors, which
// a caller may have loaded early), then the wave sum and the scale.
template <int NV>
__device__ __forceinline__ float row_rms_scale_bf16_from(const u32x4 *h, const u32x4 (&hv)[NV], int nvec, int dim,
                                                         float eps, int lane) {
#pragma clang fp contract(off)
  float ss = 0.0f;
  row_squares_pass_bf16<NV>(hv, 0, nvec, lane, ss);
  for (int base = kWave * NV; base < nvec; base += kWave * NV) {
    u32x4 hn[NV];
    row_pass_loads<NV>(h, base, nvec, lane, hn);
    row_squares_pass_bf16<NV>(hn, base, nvec, lane, ss);
  }
  ss = wave_sum_dpp(ss);
  return rsqrtf(ss / (float)dim + eps);
}
template <int NV>
__device__ __forceinline__ float row_rms_scale_bf16(const u32x4 *h, int nvec, int dim, float eps, int lane) {
  u32x4 hv[NV];
  row_pass_loads<NV>(h, 0, nvec, lane, hv);
  return row_rms_scale_bf16_from<NV>(h, hv, nvec, dim, eps, lane);
}

// SiLU(bf16(s g)) * bf16(s u), rounded to bf16 (raw bits): the gate and up
// values scaled by the row's norm scale and rounded as a projection's output
// is, then transformers' act_fn(gate) * up with each step rounded to bf16.
// SiLU(x) = x / (1 + e^-x) is taken as x * rcp(1 + 2^(-x log2 e)) on the
// hardware exp2 and reciprocal (about 1 ulp each, so the fp32 value is within
// a few ulp of the quotient and rounds to the same bf16 but for ties): a
// short dependent chain at the end of the MLP kernels, where an IEEE divide
// and a library exp made a chain of tens of instructions on few live lanes.
__device__ __forceinline__ unsigned short silu_mul_scaled_bf16(float g, float u, float s) {
#pragma clang fp contract(off)
  const float x = to_f32(from_f32<__hip_bfloat16>(s * g));
  const float up = to_f32(from_f32<__hip_bfloat16>(s * u));
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
  const __hip_bfloat16 a = from_f32<__hip_bfloat16>(x * __builtin_amdgcn_rcpf(1.0f + e));
  return __builtin_bit_cast(unsigned short, from_f32<__hip_bfloat16>(to_f32(a) * up));
}

// Workgroup-wide sum with a fixed reduction order (lane tree, then waves in
// index order), so repeated launches give identical bits.
// `scratch` holds at least blockDim.x / 64 elements.
template <typename T> __device__ T block_sum(T v, T *scratch) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  T total = T(0);
  for (int w = 0; w < nw; ++w) total += scratch[w];
  return total;
}

template <typename T> __device__ T block_max(T v, T *scratch) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  T m = scratch[0];
  for (int w = 1; w < nw; ++w) m = fmax(m, scratch[w]);
  return m;
}

// Exclusive scan of one value per thread across the workgroup, fixed order.
// Returns the exclusive prefix; *total receives the sum of all values.
// `scratch` holds at least blockDim.x / 64 + 1 elements.
template <typename T> __device__ T block_exclusive_scan(T v, T *scratch, T *total) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  // inclusive scan inside the wave (Hillis-Steele over shuffles)
  T x = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    T y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == kWave - 1) scratch[wid] = x;
  __syncthreads();
  T wave_prefix = T(0), all = T(0);
  for (int w = 0; w < nw; ++w) {
    if (w < wid) wave_prefix += scratch[w];
    all += scratch[w];
  }
  *total = all;
  // exclusive prefix taken from the neighbour's inclusive value rather than
  // x - v, which would round differently from a true prefix sum
  T excl = __shfl_up(x, 1, kWave);
  if (lane == 0) excl = T(0);
  return wave_prefix + excl;
}

}  // namespace specdec
