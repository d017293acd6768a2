// Accept-reject kernels: temperature softmax / one-hot argmax, the fused
// accept test + residual + inverse-CDF sample, the accept stage alone, the
// inverse-CDF sampler alone, and a one-hot writer.
//
// Reference semantics: lm/sampling.py:13-18 (probabilities),
// spec/accept.py:18-26 (residual), :29-35 (inverse CDF), :44-79 (accept).
//
// Layout: one workgroup per row (softmax) or per batch entry (accept).  Rows
// are walked in tiles of 4 elements per thread, so every load instruction
// is a coalesced 16-byte-per-lane read.  The inverse-CDF search accumulates
// the CDF in fp64 tile by tile (a fixed-order workgroup reduction per tile
// and a running carry), finds the tile whose end prefix passes the target,
// and scans only that tile element by element.  Re-reads of a row within
// one workgroup hit L2.
#include "common.h"

#include <float.h>
#include <math.h>

#include <initializer_list>

namespace specdec {

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

constexpr int kAcceptThreads = 1024;
constexpr int kSoftmaxThreads = 1024;

template <typename T> struct Tiny;
template <> struct Tiny<float> { static constexpr float v = FLT_MIN; };
template <> struct Tiny<double> { static constexpr double v = DBL_MIN; };

// Round an fp64 running sum to the element type: prefixes of an fp32 cumsum
// are accumulated in fp64 and rounded once per prefix.
__device__ __forceinline__ float round_to(double x, float) { return static_cast<float>(x); }
__device__ __forceinline__ double round_to(double x, double) { return x; }

// ------------------------------------------------------------ softmax ----
// One workgroup per row.  Rows of up to kSoftPer * 1024 elements (49152, the
// vocab) are read once into registers -- every load issued before the first
// use, so the row costs one memory round trip -- and written from there;
// longer rows take the streaming loop below.  Register element k of thread
// tid is row index k * 1024 + tid (coalesced 4-byte accesses), or, VEC (fp32
// rows of 16-byte aligned vectors), element k % 4 of the 16-byte vector
// (k / 4) * 1024 + tid: a quarter of the memory instructions.
constexpr int kSoftPer = 48;

// argmax with the first index among equal maxima
__device__ __forceinline__ void argmax_merge(float &best, int &best_i, float v, int i) {
  if (v > best || (v == best && i < best_i)) {
    best = v;
    best_i = i;
  }
}

__device__ __forceinline__ int block_argmax(float best, int best_i, float *red_f, int *red_i) {
  for (int o = kWave / 2; o > 0; o >>= 1) argmax_merge(best, best_i, __shfl_xor(best, o, kWave), __shfl_xor(best_i, o, kWave));
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  if (lane == 0) {
    red_f[wid] = best;
    red_i[wid] = best_i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) argmax_merge(best, best_i, red_f[w], red_i[w]);
    red_i[0] = best_i;
  }
  __syncthreads();
  return red_i[0];
}

template <typename TIn, bool UNIT_T = false, bool VEC = false>
__global__ __launch_bounds__(kSoftmaxThreads) void probabilities_kernel(
    const TIn *__restrict__ logits, int64_t row_stride, int64_t vocab, float temperature,
    float *__restrict__ out, int64_t out_stride, int64_t *__restrict__ index_out, int64_t index_stride) {
  __shared__ float red_f[kSoftmaxThreads / kWave];
  __shared__ int red_i[kSoftmaxThreads / kWave];
  const int64_t row = blockIdx.x;
  const TIn *x = logits + row * row_stride;
  float *y = out + row * out_stride;
  const int tid = threadIdx.x;
  constexpr float kLog2e = 1.4426950408889634f;
  const bool fits = vocab <= (int64_t)kSoftPer * kSoftmaxThreads;
  // row index of register element k
  auto at = [&](int k) -> int {
    return VEC ? 4 * ((k >> 2) * kSoftmaxThreads + tid) + (k & 3) : k * kSoftmaxThreads + tid;
  };
  // the row into v[]: indices past the row read its last element (VEC: its
  // last 4), so the loads need no branch
  auto load_row = [&](float (&v)[kSoftPer]) {
    if constexpr (VEC) {
      const float4 *x4 = reinterpret_cast<const float4 *>(x);
      const int lastv = (int)(vocab / 4) - 1;
#pragma unroll
      for (int kk = 0; kk < kSoftPer / 4; ++kk) {
        const float4 f = x4[min(kk * kSoftmaxThreads + tid, lastv)];
        v[4 * kk] = f.x, v[4 * kk + 1] = f.y, v[4 * kk + 2] = f.z, v[4 * kk + 3] = f.w;
      }
    } else {
      const int last = (int)vocab - 1;
#pragma unroll
      for (int k = 0; k < kSoftPer; ++k) v[k] = to_f32(x[min(k * kSoftmaxThreads + tid, last)]);
    }
  };

  if (temperature == 0.0f) {
    // one_hot(argmax(logits)) of the raw logits
    float best = -INFINITY;
    int best_i = INT32_MAX;
    if (fits) {
      float v[kSoftPer];
      load_row(v);
#pragma unroll
      for (int k = 0; k < kSoftPer; ++k) {
        const int i = at(k);
        if (i < vocab) argmax_merge(best, best_i, v[k], i);
      }
    } else {
      for (int64_t i = tid; i < vocab; i += blockDim.x) argmax_merge(best, best_i, to_f32(x[i]), (int)i);
    }
    const int hot = block_argmax(best, best_i, red_f, red_i);
    if (index_out && tid == 0) index_out[row * index_stride] = hot;
    if constexpr (VEC) {
      float4 *y4 = reinterpret_cast<float4 *>(y);
      for (int i4 = tid; i4 < (int)(vocab / 4); i4 += kSoftmaxThreads) {
        const int i = 4 * i4;
        y4[i4] = make_float4(i == hot ? 1.0f : 0.0f, i + 1 == hot ? 1.0f : 0.0f, i + 2 == hot ? 1.0f : 0.0f,
                             i + 3 == hot ? 1.0f : 0.0f);
      }
    } else {
      for (int64_t i = tid; i < vocab; i += blockDim.x) y[i] = (i == hot) ? 1.0f : 0.0f;
    }
    return;
  }

  // softmax(logits.float() / T): exp(v - m) is evaluated as
  // 2^((v - m) * log2 e) on the hardware exp2 (about 1e-6 relative for the
  // shifts that matter)
  // x / 1 is x exactly (NaN and infinities too), so the temperature-1
  // instance (UNIT_T) skips the divisions
  if (fits) {
    float v[kSoftPer];
    load_row(v);
    float m = -INFINITY, sum = 0.0f;
    if constexpr (UNIT_T) {
      // positions past the vocab hold copies of its last elements (the clamp
      // above): they leave the max alone, and their terms are zeroed below
      // (adding +0 to the sum changes no bit, as the exp2(-inf) = 0 of a
      // masked score would not)
#pragma unroll
      for (int k = 0; k < kSoftPer; ++k) m = fmaxf(m, v[k]);
      const float mg = block_max(m, red_f);
#pragma unroll
      for (int k = 0; k < kSoftPer; ++k) {
        const float e = __builtin_amdgcn_exp2f((v[k] - mg) * kLog2e);
        v[k] = at(k) < vocab ? e : 0.0f;
        sum += v[k];
      }
    } else {
#pragma unroll
      for (int k = 0; k < kSoftPer; ++k) {
        v[k] = (at(k) < vocab) ? v[k] / temperature : -INFINITY;
        m = fmaxf(m, v[k]);
      }
      const float mg = block_max(m, red_f);
#pragma unroll
      for (int k = 0; k < kSoftPer; ++k) {
        v[k] = __builtin_amdgcn_exp2f((v[k] - mg) * kLog2e);
        sum += v[k];
      }
    }
    const float inv = 1.0f / block_sum(sum, red_f);
    if constexpr (VEC) {
      float4 *y4 = reinterpret_cast<float4 *>(y);
#pragma unroll
      for (int kk = 0; kk < kSoftPer / 4; ++kk) {
        const int i4 = kk * kSoftmaxThreads + tid;
        if (i4 < (int)(vocab / 4))
          y4[i4] = make_float4(v[4 * kk] * inv, v[4 * kk + 1] * inv, v[4 * kk + 2] * inv, v[4 * kk + 3] * inv);
      }
    } else {
#pragma unroll
      for (int k = 0; k < kSoftPer; ++k) {
        const int i = at(k);
        if (i < vocab) y[i] = v[k] * inv;
      }
    }
    return;
  }
  // streaming: a running (max, sum) per thread, merged across the workgroup,
  // then a second pass that writes
  float m = -INFINITY, sum = 0.0f;
  for (int64_t i = tid; i < vocab; i += blockDim.x) {
    const float v = UNIT_T ? to_f32(x[i]) : to_f32(x[i]) / temperature;
    if (v > m) {
      sum = (m == -INFINITY) ? 0.0f : sum * __builtin_amdgcn_exp2f((m - v) * kLog2e);
      m = v;
    }
    sum += __builtin_amdgcn_exp2f((v - m) * kLog2e);
  }
  const float mg = block_max(m, red_f);
  sum = (m == -INFINITY) ? 0.0f : sum * __builtin_amdgcn_exp2f((m - mg) * kLog2e);
  const float inv = 1.0f / block_sum(sum, red_f);
  for (int64_t i = tid; i < vocab; i += blockDim.x)
    y[i] = __builtin_amdgcn_exp2f(((UNIT_T ? to_f32(x[i]) : to_f32(x[i]) / temperature) - mg) * kLog2e) * inv;
}

// ------------------------------------------- accept stage (per batch) ----
// Leading-accept count and the zero-q flag for batch entry b.  Runs on one
// thread; k is small (the draft length).
template <typename T>
__device__ __forceinline__ void accept_stage(const T *p, const T *q, int64_t p_bs, int64_t p_rs,
                                             int64_t q_bs, int64_t q_rs, const int64_t *draft,
                                             const T *u_accept, int64_t b, int64_t k, int64_t vocab,
                                             int64_t *n_out, int64_t *bad_out) {
  int64_t n = k, bad = 0;
  for (int64_t t = 0; t < k; ++t) {
    const int64_t x = draft[b * k + t];
    if (x < 0 || x >= vocab) { bad = 1; n = (n == k) ? t : n; continue; }
    const T px = p[b * p_bs + t * p_rs + x];
    const T qx = q[b * q_bs + t * q_rs + x];
    if (!(qx > T(0))) bad = 1;
    const T u = u_accept[b * k + t];
    // u < p/q written as a product, as the reference does
    if (n == k && !(u * qx < px)) n = t;
  }
  *n_out = n;
  *bad_out = bad;
}

// Inverse-CDF sample of one row whose element i is produced by `elem(i)`:
// the index of the first prefix sum (accumulated in fp64, rounded to T)
// that exceeds target = T(u * T(total)), clamped to vocab-1.
// Tile j covers elements [j*TILE, (j+1)*TILE), 4 consecutive per thread.
// Every prefix is computed one way only: the carry into the tile, plus a
// fixed-order workgroup exclusive scan of the per-thread sums, plus the
// thread's own elements in order.  Pass 1 runs that over every tile and
// keeps the prefix at each tile's end; pass 2 recomputes the one tile whose
// end prefix first exceeds the target -- the same arithmetic, so the same
// bits -- and counts its prefixes that do not.
constexpr int kCdfPerThread = 4;
constexpr int kMaxTiles = 64;  // vocab <= 64 * 4 * blockDim.x

template <typename T, typename Elem>
__device__ double cdf_tile(Elem elem, int64_t vocab, int64_t tile, int j, double carry, T target, double *scratch,
                           double *s_end, int *count) {
  const int tid = threadIdx.x;
  const int64_t base = j * tile + (int64_t)tid * kCdfPerThread;
  T v[kCdfPerThread];
  double local = 0.0;
#pragma unroll
  for (int e = 0; e < kCdfPerThread; ++e) {
    v[e] = base + e < vocab ? elem(base + e) : T(0);
    local += (double)v[e];
  }
  double unused;
  double run = carry + block_exclusive_scan(local, scratch, &unused);
  int c = 0;
#pragma unroll
  for (int e = 0; e < kCdfPerThread; ++e) {
    if (base + e >= vocab) break;
    run += (double)v[e];
    if (round_to(run, T()) <= target) ++c;
    if (base + e == min(vocab, (j + 1) * tile) - 1) *s_end = run;  // the tile's last element
  }
  *count = c;
  __syncthreads();
  return *s_end;
}

template <typename T, typename Elem>
__device__ int64_t inverse_cdf_row(Elem elem, int64_t vocab, T u, double *scratch, double *carry) {
  __shared__ double s_end;
  const int64_t tile = (int64_t)blockDim.x * kCdfPerThread;
  const int ntiles = (int)((vocab + tile - 1) / tile);
  double acc = 0.0;
  int count;
  for (int j = 0; j < ntiles; ++j) {
    acc = cdf_tile<T>(elem, vocab, tile, j, acc, T(0), scratch, &s_end, &count);
    if (threadIdx.x == 0) carry[j] = acc;  // prefix at the end of tile j
    __syncthreads();
  }
  const T target = u * round_to(acc, T());
  int jt = ntiles;
  for (int j = 0; j < ntiles; ++j)
    if (round_to(carry[j], T()) > target) { jt = j; break; }
  if (jt == ntiles) return vocab - 1;
  cdf_tile<T>(elem, vocab, tile, jt, jt == 0 ? 0.0 : carry[jt - 1], target, scratch, &s_end, &count);
  const int64_t idx = jt * tile + (int64_t)block_sum((double)count, scratch);
  return idx > vocab - 1 ? vocab - 1 : idx;
}

// fp32 rows of up to kRegTiles * 4096 elements: the whole row stays in
// registers, in runs.  The row is three chunks of 16384 elements; thread t
// owns the contiguous run 16t .. 16t+15 of each chunk, and vals[j][e] is
// element (j / 4) * 16384 + 16t + 4 (j % 4) + e.  A run is summed
// sequentially in fp64, one workgroup exclusive scan per chunk (the three
// interleaved) gives every thread the prefix at the start of its runs, and
// the answer is the number of prefixes (rounded to fp32) that do not
// exceed the target, which is taken from the prefix of the last element
// computed the same way.
constexpr int kRegTiles = 12;  // rows up to 49152 elements
constexpr int kChunkTiles = 4;
constexpr int kChunk = kChunkTiles * kAcceptThreads * kCdfPerThread;  // 16384
constexpr int kRun = kChunk / kAcceptThreads;                          // 16 per thread
constexpr int kChunks = kRegTiles / kChunkTiles;                       // 3

// A row read through a raw buffer descriptor of `elems` fp32 elements:
// loads past its end return 0 (the hardware range check on the vector
// offset), so the register-resident kernels load a whole row with no clamp,
// no select and no branch between the loads.  Word 3 is the gfx9-family
// descriptor format for untyped dword access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_buffer(const float *row, unsigned elems) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(row), 0, (int)(elems * 4u), 0x00020000);
}

// Element index of vals[j][e] for thread tid.
__device__ __forceinline__ int run_elem(int j, int tid, int e) {
  return (j / kChunkTiles) * kChunk + kRun * tid + kCdfPerThread * (j % kChunkTiles) + e;
}

// vals[j][0..3] of a row for thread tid: one 16-byte load when the row
// length is a multiple of 4 (a load then never straddles the row's end),
// else four 4-byte loads.  A wave's 16-byte loads cover 64 runs 64 bytes
// apart; its four loads of a chunk together read every byte of 4 KB.
template <bool VEC4>
__device__ __forceinline__ void load_run(__amdgpu_buffer_rsrc_t rb, int j, int tid, float (&out)[kCdfPerThread]) {
  const unsigned off = (unsigned)run_elem(j, tid, 0) * 4u;
  if (VEC4) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0);
#pragma unroll
    for (int e = 0; e < kCdfPerThread; ++e) out[e] = __builtin_bit_cast(float, (unsigned)v[e]);
  } else {
#pragma unroll
    for (int e = 0; e < kCdfPerThread; ++e)
      out[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, off + 4u * e, 0, 0));
  }
}

__device__ __forceinline__ int64_t inverse_cdf_regs(const float (&vals)[kRegTiles][kCdfPerThread], int64_t vocab,
                                                     float u, double *scratch) {
  __shared__ double s_wave[kAcceptThreads / kWave][kChunks];  // each wave's inclusive run-sum total, per chunk
  __shared__ double s_total;
  // the runs of chunks 1 and 2 wait out the scans here, each thread in its
  // own column (element m of thread t at [m][t]: no bank conflicts, no
  // barrier), which frees their registers
  __shared__ float s_park[kChunks - 1][kRun][kAcceptThreads];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const int nchunks = (int)((vocab + kChunk - 1) / kChunk);
  auto elem = [&](int c, int m) -> float {
    return c == 0 ? vals[m / kCdfPerThread][m % kCdfPerThread] : s_park[c - 1][m][tid];
  };
  // run sums, then the three chunks' scans interleaved: an inclusive scan in
  // the wave (Hillis-Steele over shuffles), the waves' totals through LDS --
  // block_exclusive_scan's arithmetic, one barrier pair for all three
  double x[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    double a = 0.0;
#pragma unroll
    for (int m = 0; m < kRun; ++m) a += (double)vals[kChunkTiles * c + m / kCdfPerThread][m % kCdfPerThread];
    x[c] = a;
  }
#pragma unroll
  for (int c = 1; c < kChunks; ++c)
#pragma unroll
    for (int m = 0; m < kRun; ++m) s_park[c - 1][m][tid] = vals[kChunkTiles * c + m / kCdfPerThread][m % kCdfPerThread];
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1)
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const double y = __shfl_up(x[c], o, kWave);
      if (lane >= o) x[c] += y;
    }
  __syncthreads();
  if (lane == kWave - 1)
#pragma unroll
    for (int c = 0; c < kChunks; ++c) s_wave[wid][c] = x[c];
  __syncthreads();
  double base[kChunks], carry = 0.0;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    double wave_prefix = 0.0, all = 0.0;
    for (int w = 0; w < kAcceptThreads / kWave; ++w) {
      if (w < wid) wave_prefix += s_wave[w][c];
      all += s_wave[w][c];
    }
    double excl = __shfl_up(x[c], 1, kWave);
    if (lane == 0) excl = 0.0;
    base[c] = carry + (wave_prefix + excl);
    carry += all;
  }
  // the prefix of the row's last element (zeros pad the last chunk)
  if (tid == kAcceptThreads - 1) {
    double acc = base[0];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (c != nchunks - 1) continue;
      acc = base[c];
#pragma unroll
      for (int m = 0; m < kRun; ++m) acc += (double)elem(c, m);
    }
    s_total = acc;
  }
  __syncthreads();
  const float target = u * (float)s_total;
  int count = 0;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    if (c >= nchunks) break;
    double acc = base[c];
#pragma unroll
    for (int m = 0; m < kRun; ++m) {
      acc += (double)elem(c, m);
      const int64_t idx = (int64_t)c * kChunk + kRun * tid + m;
      if (idx < vocab && (float)acc <= target) ++count;
    }
  }
  const int64_t idx = (int64_t)block_sum((double)count, scratch);
  return idx > vocab - 1 ? vocab - 1 : idx;
}

// Leading-accept count and zero-q flag of batch entry b computed by wave 0:
// lane t tests draft position t (and t+64, ...); a ballot finds the first
// rejection.  Same test as accept_stage.
template <typename T>
__device__ __forceinline__ void accept_stage_wave(const T *p, const T *q, int64_t p_bs, int64_t p_rs, int64_t q_bs,
                                                  int64_t q_rs, const int64_t *draft, const T *u_accept, int64_t b,
                                                  int64_t k, int64_t vocab, int64_t *n_out, int64_t *bad_out) {
  const int lane = threadIdx.x & (kWave - 1);
  int64_t first = k;
  bool bad = false;
  for (int64_t t0 = 0; t0 < k; t0 += kWave) {
    const int64_t t = t0 + lane;
    bool rej = false, zero = false;
    if (t < k) {
      const int64_t x = draft[b * k + t];
      if (x < 0 || x >= vocab) {
        rej = zero = true;
      } else {
        const T px = p[b * p_bs + t * p_rs + x];
        const T qx = q[b * q_bs + t * q_rs + x];
        zero = !(qx > T(0));
        rej = !(u_accept[b * k + t] * qx < px);  // u < p/q as a product
      }
    }
    const unsigned long long mr = __ballot(rej), mz = __ballot(zero);
    if (first == k && mr) first = t0 + __ffsll((long long)mr) - 1;
    bad = bad || mz != 0;
  }
  *n_out = first;
  *bad_out = bad ? 1 : 0;
}

// fp32 accept-reject with the residual row held in registers (vocab <= 49152).
template <bool VEC4>
__global__ __launch_bounds__(kAcceptThreads) void accept_reject_regs_kernel(
    const float *__restrict__ p, const float *__restrict__ q, int64_t p_bs, int64_t p_rs, int64_t q_bs,
    int64_t q_rs, const int64_t *__restrict__ draft, const float *__restrict__ u_accept,
    const float *__restrict__ u_residual, int64_t batch, int64_t k, int64_t vocab, int64_t *__restrict__ out) {
  __shared__ double scratch[kAcceptThreads / kWave + 1];
  __shared__ int64_t s_n;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid < kWave) {
    int64_t n, bad;
    accept_stage_wave(p, q, p_bs, p_rs, q_bs, q_rs, draft, u_accept, b, k, vocab, &n, &bad);
    if (tid == 0) {
      s_n = n;
      out[b] = n;
      out[2 * batch + b] = bad;
    }
  }
  __syncthreads();
  const int64_t n = s_n;
  const float *pr = p + b * p_bs + n * p_rs;
  // the q row, or (bonus position, n == k) a zero row: then p's own row is
  // read and its values are not used
  const bool has_q = n < k;
  const float *qr = has_q ? q + b * q_bs + n * q_rs : pr;
  // Every load of both rows goes out before the first is used, with no
  // branch between them (elements past the vocab read as 0 through the
  // buffer descriptors): one memory round trip for the row pair instead of
  // one per element.
  const __amdgpu_buffer_rsrc_t pb = row_buffer(pr, (unsigned)vocab), qb = row_buffer(qr, (unsigned)vocab);
  float vals[kRegTiles][kCdfPerThread], qv[kRegTiles][kCdfPerThread];
#pragma unroll
  for (int j = 0; j < kRegTiles; ++j) {
    load_run<VEC4>(pb, j, tid, vals[j]);
    load_run<VEC4>(qb, j, tid, qv[j]);
  }
  double local = 0.0;
#pragma unroll
  for (int j = 0; j < kRegTiles; ++j)
#pragma unroll
    for (int e = 0; e < kCdfPerThread; ++e) {
      float r = has_q ? vals[j][e] - qv[j][e] : vals[j][e];
      r = r > 0.0f ? r : 0.0f;
      vals[j][e] = r;
      local += (double)r;
    }
  const float total = (float)block_sum(local, scratch);
  const float denom = total > FLT_MIN ? total : FLT_MIN;
  const bool use_residual = total > 0.0f;
#pragma unroll
  for (int j = 0; j < kRegTiles; ++j)
#pragma unroll
    for (int e = 0; e < kCdfPerThread; ++e) {
      const int64_t i = run_elem(j, tid, e);
      if (use_residual) vals[j][e] = vals[j][e] / denom;
      else vals[j][e] = i < vocab ? pr[i] : 0.0f;  // p == q: fall back to p (rare: reloaded)
    }
  const int64_t idx = inverse_cdf_regs(vals, vocab, u_residual[b], scratch);
  if (tid == 0) out[batch + b] = idx;
}

template <bool VEC4>
__global__ __launch_bounds__(kAcceptThreads) void sample_inverse_cdf_regs_kernel(const float *__restrict__ probs,
                                                                                 int64_t vocab, int64_t row_stride,
                                                                                 const float *__restrict__ u,
                                                                                 int64_t *__restrict__ out) {
  __shared__ double scratch[kAcceptThreads / kWave + 1];
  const int64_t b = blockIdx.x;
  const float *row = probs + b * row_stride;
  float vals[kRegTiles][kCdfPerThread];
  const __amdgpu_buffer_rsrc_t rb = row_buffer(row, (unsigned)vocab);  // zeros past the vocab
#pragma unroll
  for (int j = 0; j < kRegTiles; ++j) load_run<VEC4>(rb, j, threadIdx.x, vals[j]);
  const int64_t idx = inverse_cdf_regs(vals, vocab, u[b], scratch);
  if (threadIdx.x == 0) out[b] = idx;
}

template <typename T>
__global__ __launch_bounds__(kAcceptThreads) void accept_reject_kernel(
    const T *__restrict__ p, const T *__restrict__ q, int64_t p_bs, int64_t p_rs, int64_t q_bs,
    int64_t q_rs, const int64_t *__restrict__ draft, const T *__restrict__ u_accept,
    const T *__restrict__ u_residual, int64_t batch, int64_t k, int64_t vocab,
    int64_t *__restrict__ out) {
  __shared__ double scratch[kAcceptThreads / kWave + 1];
  __shared__ double carry[kMaxTiles];
  __shared__ int64_t s_n;
  const int64_t b = blockIdx.x;
  if (threadIdx.x == 0) {
    int64_t n, bad;
    accept_stage(p, q, p_bs, p_rs, q_bs, q_rs, draft, u_accept, b, k, vocab, &n, &bad);
    s_n = n;
    out[b] = n;
    out[2 * batch + b] = bad;
  }
  __syncthreads();
  const int64_t n = s_n;
  const T *pr = p + b * p_bs + n * p_rs;
  const T *qr = (n < k) ? q + b * q_bs + n * q_rs : nullptr;  // zero row at n == k

  // total = sum(max(0, p - q)), accumulated in fp64 and rounded once
  double local = 0.0;
  for (int64_t i = threadIdx.x; i < vocab; i += blockDim.x) {
    T r = qr ? pr[i] - qr[i] : pr[i];
    local += (double)(r > T(0) ? r : T(0));
  }
  const double tot64 = block_sum(local, scratch);
  const T total = round_to(tot64, T());
  const T denom = total > Tiny<T>::v ? total : Tiny<T>::v;
  const bool use_residual = total > T(0);
  __syncthreads();

  auto elem = [=](int64_t i) -> T {
    if (!use_residual) return pr[i];
    T r = qr ? pr[i] - qr[i] : pr[i];
    r = r > T(0) ? r : T(0);
    return r / denom;
  };
  const int64_t idx = inverse_cdf_row<T>(elem, vocab, u_residual[b], scratch, carry);
  if (threadIdx.x == 0) out[batch + b] = idx;
}

template <typename T>
__global__ void accept_count_kernel(const T *__restrict__ p, const T *__restrict__ q, int64_t p_bs,
                                    int64_t p_rs, int64_t q_bs, int64_t q_rs,
                                    const int64_t *__restrict__ draft,
                                    const T *__restrict__ u_accept, int64_t batch, int64_t k,
                                    int64_t vocab, int64_t *__restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  int64_t n, bad;
  accept_stage(p, q, p_bs, p_rs, q_bs, q_rs, draft, u_accept, b, k, vocab, &n, &bad);
  out[b] = n;
  out[batch + b] = bad;
}

template <typename T>
__global__ __launch_bounds__(kAcceptThreads) void sample_inverse_cdf_kernel(
    const T *__restrict__ probs, int64_t vocab, int64_t row_stride, const T *__restrict__ u,
    int64_t *__restrict__ out) {
  __shared__ double scratch[kAcceptThreads / kWave + 1];
  __shared__ double carry[kMaxTiles];
  const int64_t b = blockIdx.x;
  const T *row = probs + b * row_stride;
  auto elem = [=](int64_t i) -> T { return row[i]; };
  const int64_t idx = inverse_cdf_row<T>(elem, vocab, u[b], scratch, carry);
  if (threadIdx.x == 0) out[b] = idx;
}

// ----------------------------------------- accept-reject over many CUs ----
// fp32 accept-reject with each batch row spread over G workgroups of 256
// threads -- chunk g of the row, E consecutive elements per thread -- in
// one launch, in two forms:
//   probabilities: p [B, k+1, V] and q [B, k, V] as given;
//   logits: the target and draft logits of those shapes and a temperature
//     T.  p = softmax(l / T) (the one-hot of the lowest-index argmax at
//     T = 0) is formed on the fly from row statistics; no probability row
//     is written or read back.
// The workgroups of a row meet up to three times, each meeting exchanging
// one value set per chunk:
//   A (logits form): for every logit row, the chunk's max m of y = l / T
//     and its sum of 2^((y - m) log2 e) (at T = 0 the max of l and the
//     lowest index holding it).  Every workgroup folds them in chunk order
//     into the row's (M, S), so it knows p(x) and q(x) of every drafted
//     token and the accept count n;
//   B: the fp64 sum of the chunk's residual r = max(0, p[n] - q[n]) (q[k]
//     is the zero row: the bonus samples p[k]);
//   C: once the chunk sums are added in chunk order (the residual total,
//     rounded to fp32) and the chunk's elements divided by it (or p's row
//     taken when it is 0), L_g, the fp64 inclusive prefix at the chunk's
//     last element.
// Then C_j = L_0 + ... + L_{j-1} in chunk order and the target u * fp32(C_G);
// the one workgroup whose chunk holds the first prefix above the target --
// fp32(C_g) <= target < fp32(C_{g+1}) -- counts its prefixes that do not
// exceed it.  An element's prefix is C_g + its chunk-local inclusive prefix
// (fp64, the thread's run after a fixed-order workgroup scan), so a chunk's
// last prefix is C_{g+1} exactly and the chunk test agrees with the count.
// Accumulation in fp64 with a rounding per prefix is the CPU cumsum's rule;
// only the order of the fp64 additions differs from a sequential sum.
//
// Meeting words carry the call's tag: word = (tag << 32) | 32-bit payload
// (an fp64 value takes two words).  The tag is the workspace's epoch plus
// one, read by every workgroup when it starts; the last workgroup to arrive
// at the end advances the epoch, so words left by earlier calls never carry
// the current tag, and nothing is ever cleared (the workspace is zeroed
// once, when it is allocated).  A reader reads the words it needs, then
// again at most `spin` times while some are missing (never, for spin < 0).
// A chunk whose words are still missing then is computed by the reader
// itself, with the code its own workgroup runs -- the same loads, the same
// operations in the same order, so the same bits -- and the call finishes
// whether or not the workgroups of a row are resident together.
constexpr int kMwThreads = 256;
constexpr int kMwMaxG = 64;                 // chunks per row
constexpr int kMwMaxK = 16;                 // draft positions (logits form)
constexpr int kMwMaxR = 2 * kMwMaxK + 1;    // logit rows per batch entry
constexpr int64_t kMwHead = 16;             // words before the rows: arrival counters [2], the epoch
// a row's words: B (2 per chunk), C (2 per chunk), A (2 per logit row and chunk)
constexpr int64_t kMwB = 0, kMwC = 2 * kMwMaxG, kMwA = 4 * kMwMaxG;
constexpr int64_t kMwRowWords = kMwA + 2 * (int64_t)kMwMaxR * kMwMaxG;
constexpr int kMwUnroll = 8;  // drafted positions whose scalar loads go out together
constexpr float kMwLog2e = 1.4426950408889634f;

struct MwArgs {
  const float *p, *q;  // probabilities, or the target and draft logits
  int64_t p_bs, p_rs, q_bs, q_rs;
  const int64_t *draft;
  const float *u_accept, *u_residual;
  int64_t batch, k, vocab;
  int G;
  float temperature;  // logits form
  int spin;
  int64_t *out;
  uint64_t *ws;
};

// the E elements of one thread from a row buffer (zeros past the row)
template <int E, bool VEC4>
__device__ __forceinline__ void load_elems(__amdgpu_buffer_rsrc_t rb, unsigned first, float (&v)[E]) {
  if constexpr (VEC4) {
#pragma unroll
    for (int j = 0; j < E / 4; ++j) {
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rb, (first + 4u * j) * 4u, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * j + e] = __builtin_bit_cast(float, (unsigned)w[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e)
      v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, (first + e) * 4u, 0, 0));
  }
}

__device__ __forceinline__ void put_word(uint64_t *slot, uint64_t w) {
  __hip_atomic_store(slot, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_word(const uint64_t *slot) {
  return __hip_atomic_load(const_cast<uint64_t *>(slot), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tagged(uint32_t tag, uint32_t payload) {
  return ((uint64_t)tag << 32) | payload;
}
__device__ __forceinline__ uint32_t hi32(double v) { return (uint32_t)(__builtin_bit_cast(uint64_t, v) >> 32); }
__device__ __forceinline__ uint32_t lo32(double v) { return (uint32_t)__builtin_bit_cast(uint64_t, v); }
__device__ __forceinline__ double from_words(uint32_t hi, uint32_t lo) {
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Arrival: the count only decides who advances the epoch -- the last
// workgroup of the launch to arrive, when every workgroup has read it (a
// workgroup's count goes to the counter of its epoch's parity, so its epoch
// read has completed before it counts).  The fetch-add is issued before the
// workgroup's first publish and its result used only at the end
// (mw_advance), so its round trip overlaps the work; the next call, which
// reads the new epoch, starts only after this one ends.
__device__ __forceinline__ uint64_t mw_arrive(uint64_t *ws, uint64_t epoch) {
  if (threadIdx.x != 0) return 0;
  // The counter's address passes through a VGPR the compiler cannot see
  // into: for a uniform address it would rewrite the add as a wave-combined
  // atomic whose result is spread to the lanes at once, waiting for the
  // round trip here instead of where the count is first used.  The pointer
  // is a global one: a generic pointer would make the add a flat atomic,
  // which the compiler's wait counting treats as unordered with every load.
  __attribute__((address_space(1))) uint64_t *counter = (__attribute__((address_space(1))) uint64_t *)(ws + (epoch & 1));
  __asm__ volatile("" : "+v"(counter));
  return __hip_atomic_fetch_add(counter, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void mw_advance(uint64_t *ws, uint64_t epoch, uint64_t before) {
  if (threadIdx.x == 0 && before == (uint64_t)gridDim.x - 1) {  // ready the next call's counter and tag
    __hip_atomic_store(ws + ((epoch + 1) & 1), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ws + 2, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// One meeting: chunk c's `per` words lie at slots[c * per ..]; this
// workgroup's own chunk `own` is not read (its payloads are set by the
// caller).  Payloads of the words seen with the call's tag land in
// pay[c * per + i]; miss[c] = 1 for a chunk with a word still missing after
// the first read and `spin` more rounds (every word is missing for
// spin < 0).  A thread reads up to kMwPoll words per pass, all issued
// before any is checked; more words than kMwPoll * 256 take more passes.
// Returns whether any chunk is missing (the same in every thread); ends
// with a barrier.
constexpr int kMwPoll = 4;
__device__ bool gather_meeting(const uint64_t *slots, int G, int per, int own, uint32_t tag, int spin,
                               uint32_t *pay, int *miss) {
  const int tid = threadIdx.x, n = G * per;
  bool late = false;
  for (int c = tid; c < G; c += kMwThreads) miss[c] = 0;
  if (spin < 0) __syncthreads();  // otherwise the rounds' barriers order the zeroing before any mark
  for (int i0 = 0; i0 < n; i0 += kMwPoll * kMwThreads) {
    unsigned pending = 0;  // bit j: word i0 + tid + j * kMwThreads not seen yet
#pragma unroll
    for (int j = 0; j < kMwPoll; ++j) {
      const int i = i0 + tid + j * kMwThreads;
      if (i < n && i / per != own) pending |= 1u << j;
    }
    if (spin >= 0) {
      for (int round = 0;; ++round) {
        uint64_t w[kMwPoll];
#pragma unroll
        for (int j = 0; j < kMwPoll; ++j)
          w[j] = (pending >> j & 1u) ? get_word(slots + i0 + tid + j * kMwThreads) : 0;
#pragma unroll
        for (int j = 0; j < kMwPoll; ++j) {
          if ((pending >> j & 1u) && (uint32_t)(w[j] >> 32) == tag) {
            pay[i0 + tid + j * kMwThreads] = (uint32_t)w[j];
            pending &= ~(1u << j);
          }
        }
        if (!__syncthreads_or(pending != 0u) || round >= spin) break;
        __builtin_amdgcn_s_sleep(1);
      }
    }
#pragma unroll
    for (int j = 0; j < kMwPoll; ++j)
      if (pending >> j & 1u) miss[(i0 + tid + j * kMwThreads) / per] = 1;
    late |= pending != 0u;
  }
  return __syncthreads_or(late);
}

// ---- statistics of the logits form (meeting A) ----
// Row r of the logits form: the target's rows 0..k, then the draft's 0..k-1.
// The bases are SSA values chosen by a select (selecting between two fields
// of the argument struct would make the compiler index the struct in
// scratch memory).
__device__ __forceinline__ const float *logit_row(const float *t_b, const float *d_b, int64_t t_rs, int64_t d_rs,
                                                  int64_t k, int r) {
  return r <= k ? t_b + (int64_t)r * t_rs : d_b + (int64_t)(r - k - 1) * d_rs;
}

// Logit rows a thread loads at once in chunk_stats.  E = 8 and 16 run one
// workgroup per compute unit and take the nine rows of k = 4 together; E =
// 12 and 24 run two per compute unit, which needs the kernel within 256
// VGPRs: 72 or 48 elements in flight per thread (nine rows at E = 16 take
// 256 VGPRs and 163 AGPRs).
constexpr int mw_rows_per_batch(int E) { return E == 8 || E == 16 ? 9 : E == 12 ? 6 : E >= 48 ? 1 : 48 / E; }

// Meeting A payloads of chunk gc, every logit row: pay[2r] = the max bits,
// pay[2r + 1] = the sum bits (T > 0) or the index (T = 0).  RB rows are
// loaded together.  T > 0 takes two reductions per row, each in a fixed
// order: the chunk's max M of y = l / T (wave_max_dpp, then the four
// waves), then the sum of 2^((y - M) log2 e) over the chunk (each thread
// its elements in order, wave_sum_dpp, then the waves in order).
// Uses s_red; ends with a barrier.  `issued` runs once, right after the
// first batch's loads go out (loads that depend on a value requested before
// them are issued there, waiting only for that value).
// The batch entry's rows are given as values (t_b, d_b: its first target
// and draft rows), not through the argument struct, which would be copied
// to scratch memory for the select between its fields.
template <int E, bool VEC4, typename F>
__device__ __forceinline__ void chunk_stats(const float *t_b, const float *d_b, int64_t t_rs, int64_t d_rs, int64_t k,
                                            int64_t vocab, float T, int gc, int R, uint32_t *pay,
                                            float (*s_red)[4][2], F &&issued) {
#pragma clang fp contract(off)
  constexpr int RB = mw_rows_per_batch(E);  // rows whose loads are in flight together
  constexpr int nw = kMwThreads / kWave;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const unsigned first = (unsigned)gc * (kMwThreads * E) + (unsigned)tid * E;
  // every load unconditional (rows past R load row R - 1 again, unused):
  // a row filled with zeros on one path and loaded on another made the
  // compiler wait for each row's loads before the next row's went out
  auto load = [&](int r0, float (&v)[RB][E]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      load_elems<E, VEC4>(row_buffer(logit_row(t_b, d_b, t_rs, d_rs, k, min(r0 + rb, R - 1)), (unsigned)vocab), first,
                          v[rb]);
  };
  auto reduce = [&](int r0, float (&v)[RB][E]) {
    if (T == 0.0f) {  // the max and its lowest index
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float m = -INFINITY;
        int idx = INT32_MAX;
#pragma unroll
        for (int e = 0; e < E; ++e)
          if (first + e < (unsigned)vocab) argmax_merge(m, idx, v[rb][e], (int)(first + e));
        wave_argmax_dpp(m, idx);
        if (lane == 0) {
          s_red[rb][wave][0] = m;
          s_red[rb][wave][1] = __int_as_float(idx);
        }
      }
      __syncthreads();
      if (tid < RB && r0 + tid < R) {
        float m = s_red[tid][0][0];
        int idx = __float_as_int(s_red[tid][0][1]);
        for (int w = 1; w < nw; ++w) argmax_merge(m, idx, s_red[tid][w][0], __float_as_int(s_red[tid][w][1]));
        pay[2 * (r0 + tid)] = __float_as_uint(m);
        pay[2 * (r0 + tid) + 1] = (uint32_t)idx;
      }
      __syncthreads();
      return;
    }
    // y = l / T (x / 1 is x exactly: no division at T = 1); -inf past the row
    if (T != 1.0f) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int e = 0; e < E; ++e) v[rb][e] = v[rb][e] / T;
    }
    float mt[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      mt[rb] = -INFINITY;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if (!(first + e < (unsigned)vocab)) v[rb][e] = -INFINITY;
        mt[rb] = fmaxf(mt[rb], v[rb][e]);
      }
      mt[rb] = wave_max_dpp(mt[rb]);
      if (lane == 0) s_red[rb][wave][0] = mt[rb];
    }
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float m = s_red[rb][0][0];
      for (int w = 1; w < nw; ++w) m = fmaxf(m, s_red[rb][w][0]);
      float sum = 0.0f;
      if (m != -INFINITY) {
#pragma unroll
        for (int e = 0; e < E; ++e) sum += __builtin_amdgcn_exp2f((v[rb][e] - m) * kMwLog2e);
      }
      sum = wave_sum_dpp(sum);
      if (lane == 0) s_red[rb][wave][1] = sum;
    }
    __syncthreads();
    if (tid < RB && r0 + tid < R) {
      float sum = s_red[tid][0][1];
      for (int w = 1; w < nw; ++w) sum += s_red[tid][w][1];
      float m = s_red[tid][0][0];
      for (int w = 1; w < nw; ++w) m = fmaxf(m, s_red[tid][w][0]);
      pay[2 * (r0 + tid)] = __float_as_uint(m);
      pay[2 * (r0 + tid) + 1] = __float_as_uint(sum);
    }
    __syncthreads();
  };
  // the first batch outside the loop: its loads follow the caller's
  // straight-line code (no loop header in between, where every load still
  // in flight would be waited for)
  float v[RB][E];
  load(0, v);
  issued();
  reduce(0, v);
  for (int r0 = RB; r0 < R; r0 += RB) {
    load(r0, v);
    reduce(r0, v);
  }
}

// p (or q) of one element from its logit and its row's statistics: the
// softmax 2^((y - M) log2 e) / S, rounded as exp2 times the rounded 1 / S;
// at T = 0 the one-hot of the row's argmax index.
__device__ __forceinline__ float prob_of(float l, int64_t i, float T, float M, float inv_or_idx) {
#pragma clang fp contract(off)
  if (T == 0.0f) return i == (int64_t)__float_as_int(inv_or_idx) ? 1.0f : 0.0f;
  const float y = T == 1.0f ? l : l / T;
  return __builtin_amdgcn_exp2f((y - M) * kMwLog2e) * inv_or_idx;
}

// This thread's elements of chunk gc of the residual row: x = max(0, p - q)
// and p itself (both 0 past the row).  s_fin[r] holds logit row r's
// (M, 1 / S) -- or (max, index) -- in the logits form.
template <int E, bool VEC4, bool LOGITS>
__device__ __forceinline__ void residual_elems(const MwArgs &a, int64_t b, int64_t n, int gc,
                                               const float (*s_fin)[2], float (&x)[E], float (&pv)[E]) {
#pragma clang fp contract(off)
  const unsigned first = (unsigned)gc * (kMwThreads * E) + (unsigned)threadIdx.x * E;
  float pr[E], qr[E];
  if constexpr (LOGITS) {
    load_elems<E, VEC4>(row_buffer(a.p + b * a.p_bs + n * a.p_rs, (unsigned)a.vocab), first, pr);
    if (n < a.k) load_elems<E, VEC4>(row_buffer(a.q + b * a.q_bs + n * a.q_rs, (unsigned)a.vocab), first, qr);
    const float Mp = s_fin[n][0], Ip = s_fin[n][1];
    const float Mq = n < a.k ? s_fin[a.k + 1 + n][0] : 0.0f, Iq = n < a.k ? s_fin[a.k + 1 + n][1] : 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const bool in = first + e < (unsigned)a.vocab;
      pr[e] = in ? prob_of(pr[e], first + e, a.temperature, Mp, Ip) : 0.0f;
      qr[e] = in && n < a.k ? prob_of(qr[e], first + e, a.temperature, Mq, Iq) : 0.0f;
    }
  } else {
    load_elems<E, VEC4>(row_buffer(a.p + b * a.p_bs + n * a.p_rs, (unsigned)a.vocab), first, pr);
    if (n < a.k) load_elems<E, VEC4>(row_buffer(a.q + b * a.q_bs + n * a.q_rs, (unsigned)a.vocab), first, qr);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) qr[e] = 0.0f;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float r = pr[e] - qr[e];
    x[e] = r > 0.0f ? r : 0.0f;
    pv[e] = pr[e];
  }
}

// The chunk's residual sum (meeting B's value).
template <int E>
__device__ __forceinline__ double chunk_residual_sum(const float (&x)[E], double *scratch) {
  double run = 0.0;
#pragma unroll
  for (int e = 0; e < E; ++e) run += (double)x[e];
  return block_sum(run, scratch);
}

// The chunk's elements divided by the residual total (p where it is 0) in
// place, and L_g (meeting C's value); *excl receives the thread's exclusive
// prefix within the chunk.
template <int E>
__device__ __forceinline__ double chunk_prefix(float (&x)[E], const float (&pv)[E], bool use_residual, float denom,
                                               double *scratch, double *s_last, double *excl) {
#pragma clang fp contract(off)
  double run = 0.0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    x[e] = use_residual ? x[e] / denom : pv[e];
    run += (double)x[e];
  }
  double unused;
  *excl = block_exclusive_scan(run, scratch, &unused);
  if (threadIdx.x == kMwThreads - 1) {
    double acc = *excl;
#pragma unroll
    for (int e = 0; e < E; ++e) acc += (double)x[e];
    *s_last = acc;
  }
  __syncthreads();
  const double last = *s_last;
  __syncthreads();
  return last;
}

// Sequential fp64 sum, in chunk order, of the values held as (hi, lo)
// payload pairs pay[2i], pay[2i + 1]; also the running sum before and after
// chunk j.
struct Chain {
  double total, before, after;
};
__device__ __forceinline__ Chain chain_sum(const uint32_t *pay, int n, int j) {
  Chain r{0.0, 0.0, 0.0};
  double acc = 0.0;
  for (int i0 = 0; i0 < n; i0 += 16) {
    double v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = min(i0 + i, n - 1);
      v[i] = from_words(pay[2 * c], pay[2 * c + 1]);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const double next = i0 + i < n ? acc + v[i] : acc;
      if (i0 + i == j) r.before = acc, r.after = next;
      acc = next;
    }
  }
  r.total = acc;
  return r;
}

template <int E, bool VEC4, bool LOGITS>
__global__ __launch_bounds__(kMwThreads) void accept_reject_mw_kernel(MwArgs a) {
  __shared__ double scratch[kMwThreads / kWave + 1];
  __shared__ uint32_t s_pay[2 * kMwMaxR * kMwMaxG];  // one meeting's payloads
  __shared__ int s_miss[kMwMaxG];
  __shared__ float s_fin[LOGITS ? kMwMaxR : 1][2];   // per logit row: (M, 1 / S) or (max, index)
  __shared__ float s_terms[LOGITS ? kMwMaxR * kMwMaxG : 1];  // the fold's per-chunk terms
  __shared__ float s_red[LOGITS ? mw_rows_per_batch(E) : 1][4][2];
  __shared__ int s_flag[LOGITS ? kMwMaxK : 1];        // bit 0: rejected, bit 1: bad draft
  __shared__ double s_last;
  const int G = a.G;
  const int64_t b = blockIdx.x / G, k = a.k, vocab = a.vocab;
  const int g = (int)(blockIdx.x % G);
  const int tid = threadIdx.x;
  constexpr int kChunk = kMwThreads * E;
  uint64_t *row_ws = a.ws + kMwHead + b * kMwRowWords;
  // the call's tag: the epoch before anyone arrives (mw_arrive), plus one
  // (never 0).  Read once at the start: the epoch changes only between
  // launches (the last arrival of the previous call wrote it), and a launch
  // sees what the launches before it on the stream wrote.
  typedef const __attribute__((address_space(4))) uint64_t const_u64;
  typedef const __attribute__((address_space(4))) float const_f32;
  typedef const __attribute__((address_space(4))) int64_t const_i64;
  uint64_t epoch;
  float ur;
  float lt = 0.0f, ld = 0.0f, uacc = 0.0f;  // logits form: position tid's inputs
  int64_t xid = -1;
  if constexpr (LOGITS) {
    // The epoch, the residual's uniform and, one thread per position, the
    // drafted id and its uniform are requested before the chunk's rows, as
    // vector loads (atomic, so they are neither turned into scalar loads
    // nor moved to their uses): they complete ahead of the rows, in order,
    // so no round trip of their own comes before the rows' loads go out.
    // The drafted ids' two logits follow the first batch of rows.  The
    // addresses pass through VGPRs the compiler cannot see into, so the
    // values stay in VGPRs: copying a uniform value to a scalar register
    // would wait for it at once.
    typedef const __attribute__((address_space(1))) uint64_t global_u64;
    typedef const __attribute__((address_space(1))) uint32_t global_u32;
    global_u64 *ep = (global_u64 *)(a.ws + 2);
    global_u32 *up = (global_u32 *)a.u_residual + b;
    __asm__ volatile("" : "+v"(ep), "+v"(up));
    epoch = __hip_atomic_load(ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ur = __uint_as_float(__hip_atomic_load(up, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if (tid < k) {
      xid = __hip_atomic_load(a.draft + b * k + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      uacc = __uint_as_float(__hip_atomic_load((const uint32_t *)a.u_accept + b * k + tid, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT));
    }
  } else {
    // scalar loads through the constant address space, which wait on their
    // own counter, not behind the vector loads; both in one round trip now,
    // not after the chunk's work
    epoch = ((const_u64 *)a.ws)[2];
    ur = ((const_f32 *)a.u_residual)[b];
    __asm__ volatile("" ::"s"(ur), "s"(epoch));
  }
  const uint32_t tag = (uint32_t)(epoch % 0xFFFFFFFFull) + 1u;

  uint64_t arrived = 0;  // thread 0: the arrival count before this workgroup's
  int64_t n = k, bad = 0;
  if constexpr (LOGITS) {
    const int R = (int)(2 * k + 1);
    // A: this chunk's statistics, published; the other chunks', gathered
    uint32_t *pay = s_pay;
    const float *t_b = a.p + b * a.p_bs, *d_b = a.q + b * a.q_bs;
    chunk_stats<E, VEC4>(t_b, d_b, a.p_rs, a.q_rs, k, vocab, a.temperature, g, R, pay + 2 * R * g, s_red, [&] {
      // issued by every thread (a valid element where tid >= k or the id is
      // out of range; those values go unused): loads under a branch would
      // make the compiler wait for every load in flight where the paths
      // join, the chunk's rows included
      const bool mine = tid < k && xid >= 0 && xid < vocab;
      const int64_t t = mine ? tid : 0, col = mine ? xid : 0;
      const float *d_rows = k > 0 ? d_b : t_b;
      const int64_t d_rs = k > 0 ? a.q_rs : a.p_rs;
      lt = __uint_as_float(__hip_atomic_load((const uint32_t *)t_b + t * a.p_rs + col, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
      ld = __uint_as_float(__hip_atomic_load((const uint32_t *)d_rows + t * d_rs + col, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
    });
    arrived = mw_arrive(a.ws, epoch);
    uint64_t *slots = row_ws + kMwA;
    for (int i = tid; i < 2 * R; i += kMwThreads) put_word(slots + 2 * R * g + i, tagged(tag, pay[2 * R * g + i]));
    if (gather_meeting(slots, G, 2 * R, g, tag, a.spin, pay, s_miss))
      for (int c = 0; c < G; ++c)
        if (s_miss[c])
          chunk_stats<E, VEC4>(t_b, d_b, a.p_rs, a.q_rs, k, vocab, a.temperature, c, R, pay + 2 * R * c, s_red,
                               [] {});
    // every row's (M, 1 / S) -- or (max, index) -- folded over the chunks:
    // M = the chunks' max (one wave per row, lane c holding chunk c: a max,
    // or a (max, lowest index) merge, has the same result in any order);
    // S = the sum over chunks, in chunk order, of S_c 2^((M_c - M) log2 e),
    // the terms computed one per thread
    {
      const int lane = tid & (kWave - 1);
      for (int r = tid / kWave; r < R; r += kMwThreads / kWave) {
        float m = lane < G ? __uint_as_float(pay[2 * R * lane + 2 * r]) : -INFINITY;
        int idx = lane < G ? (int)pay[2 * R * lane + 2 * r + 1] : INT32_MAX;
        if (a.temperature == 0.0f) wave_argmax_dpp(m, idx);
        else m = wave_max_dpp(m);
        if (lane == 0) {
          s_fin[r][0] = m;
          s_fin[r][1] = __int_as_float(idx);
        }
      }
    }
    __syncthreads();
    if (a.temperature != 0.0f) {
#pragma clang fp contract(off)
      for (int i = tid; i < R * G; i += kMwThreads) {
        const int r = i / G, c = i - r * G;
        const float mc = __uint_as_float(pay[2 * R * c + 2 * r]), sc = __uint_as_float(pay[2 * R * c + 2 * r + 1]);
        s_terms[i] = mc == -INFINITY ? 0.0f : sc * __builtin_amdgcn_exp2f((mc - s_fin[r][0]) * kMwLog2e);
      }
      __syncthreads();
      if (tid < R) {
        float sum = 0.0f;
        for (int c0 = 0; c0 < G; c0 += 16) {  // each 16 terms read together, added in order
          float t[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) t[i] = s_terms[tid * G + min(c0 + i, G - 1)];
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (c0 + i < G) sum += t[i];
        }
        s_fin[tid][1] = 1.0f / sum;
      }
      __syncthreads();
    }
    // the accept test of every position: u * q(x) < p(x)
    if (tid < k) {
      int f = 0;
      if (xid < 0 || xid >= vocab) {
        f = 3;
      } else {
        const float px = prob_of(lt, xid, a.temperature, s_fin[tid][0], s_fin[tid][1]);
        const float qx = prob_of(ld, xid, a.temperature, s_fin[k + 1 + tid][0], s_fin[k + 1 + tid][1]);
        f = (uacc * qx < px ? 0 : 1) | (qx > 0.0f ? 0 : 2);
      }
      s_flag[tid] = f;
    }
    __syncthreads();
    for (int64_t t = 0; t < k; ++t) {
      const int f = s_flag[t];
      if (f & 2) bad = 1;
      if (n == k && (f & 1)) n = t;
    }
  } else {
    // the accept count n and the bad-draft flag, the same in every thread
    // (accept_stage's test, u * q(x) < p(x) as a product; an id outside the
    // vocabulary is never read through)
    const_f32 *p_b = (const_f32 *)(a.p + b * a.p_bs), *q_b = (const_f32 *)(a.q + b * a.q_bs);
    const_i64 *dr = (const_i64 *)(a.draft + b * k);
    const_f32 *ua = (const_f32 *)(a.u_accept + b * k);
    for (int64_t t0 = 0; t0 < k; t0 += kMwUnroll) {
      int64_t xs[kMwUnroll];
      float pxs[kMwUnroll], qxs[kMwUnroll], us[kMwUnroll];
#pragma unroll
      for (int j = 0; j < kMwUnroll; ++j) {
        xs[j] = -1;
        if (t0 + j < k) xs[j] = dr[t0 + j];
      }
#pragma unroll
      for (int j = 0; j < kMwUnroll; ++j) {
        const int64_t t = t0 + j, x = xs[j];
        pxs[j] = qxs[j] = us[j] = 0.0f;
        if (t < k) us[j] = ua[t];
        if (t < k && x >= 0 && x < vocab) {
          pxs[j] = p_b[t * a.p_rs + x];
          qxs[j] = q_b[t * a.q_rs + x];
        }
      }
#pragma unroll
      for (int j = 0; j < kMwUnroll; ++j) {
        const int64_t t = t0 + j, x = xs[j];
        if (t >= k) break;
        if (x < 0 || x >= vocab) {
          bad = 1;
          if (n == k) n = t;
          continue;
        }
        if (!(qxs[j] > 0.0f)) bad = 1;
        if (n == k && !(us[j] * qxs[j] < pxs[j])) n = t;
      }
    }
  }
  if (g == 0 && tid == 0) {
    a.out[b] = n;
    a.out[2 * a.batch + b] = bad;
  }

  // B: the chunk's residual sum
  float x[E], pv[E];  // this thread's residual elements and p, then the quotients
  residual_elems<E, VEC4, LOGITS>(a, b, n, g, s_fin, x, pv);

  {
    const double sum = chunk_residual_sum(x, scratch);
    if constexpr (!LOGITS) arrived = mw_arrive(a.ws, epoch);
    if (tid == 0) {
      s_pay[2 * g] = hi32(sum);
      s_pay[2 * g + 1] = lo32(sum);
      put_word(row_ws + kMwB + 2 * g, tagged(tag, hi32(sum)));
      put_word(row_ws + kMwB + 2 * g + 1, tagged(tag, lo32(sum)));
    }
  }
  const bool late_b = gather_meeting(row_ws + kMwB, G, 2, g, tag, a.spin, s_pay, s_miss);
  for (int c = 0; late_b && c < G; ++c) {
    if (!s_miss[c]) continue;
    float xc[E], pc[E];
    residual_elems<E, VEC4, LOGITS>(a, b, n, c, s_fin, xc, pc);
    const double sum = chunk_residual_sum(xc, scratch);
    if (tid == 0) {
      s_pay[2 * c] = hi32(sum);
      s_pay[2 * c + 1] = lo32(sum);
    }
    __syncthreads();
  }

  // C: the total in chunk order, the quotients, L_g
  const float total = (float)chain_sum(s_pay, G, -1).total;
  const float denom = total > FLT_MIN ? total : FLT_MIN;
  const bool use_residual = total > 0.0f;
  __syncthreads();  // every thread has read meeting B's payloads
  double excl;
  {
    const double L = chunk_prefix(x, pv, use_residual, denom, scratch, &s_last, &excl);
    if (tid == 0) {
      s_pay[2 * g] = hi32(L);
      s_pay[2 * g + 1] = lo32(L);
      put_word(row_ws + kMwC + 2 * g, tagged(tag, hi32(L)));
      put_word(row_ws + kMwC + 2 * g + 1, tagged(tag, lo32(L)));
    }
  }
  const bool late_c = gather_meeting(row_ws + kMwC, G, 2, g, tag, a.spin, s_pay, s_miss);
  for (int c = 0; late_c && c < G; ++c) {
    if (!s_miss[c]) continue;
    float xc[E], pc[E];
    residual_elems<E, VEC4, LOGITS>(a, b, n, c, s_fin, xc, pc);
    double unused;
    const double L = chunk_prefix(xc, pc, use_residual, denom, scratch, &s_last, &unused);
    if (tid == 0) {
      s_pay[2 * c] = hi32(L);
      s_pay[2 * c + 1] = lo32(L);
    }
    __syncthreads();
  }

  // D: chunk bases, the target, the count in the chunk that holds it
  const Chain chain = chain_sum(s_pay, G, g);
  const double c_lo = chain.before, c_hi = chain.after, c = chain.total;
  const float target = ur * (float)c;
  if ((float)c_lo <= target && target < (float)c_hi) {
    int cnt_le = 0;
    double acc = excl;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      acc += (double)x[e];
      if ((float)(c_lo + acc) <= target) ++cnt_le;
    }
    const int64_t idx = (int64_t)g * kChunk + (int64_t)block_sum((double)cnt_le, scratch);
    if (tid == 0) a.out[a.batch + b] = idx < vocab - 1 ? idx : vocab - 1;
  } else if (g == G - 1 && !(target < (float)c)) {
    if (tid == 0) a.out[a.batch + b] = vocab - 1;  // no prefix exceeds the target
  }
  mw_advance(a.ws, epoch, arrived);
}

__global__ void one_hot_kernel(const int64_t *__restrict__ ids, int64_t n, int64_t vocab,
                               float *__restrict__ out) {
  const int64_t total = n * vocab;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / vocab, c = i - r * vocab;
    out[i] = (ids[r] == c) ? 1.0f : 0.0f;
  }
}

}  // namespace specdec

using namespace specdec;

SPECDEC_API int specdec_abi_version(void) { return 15; }

SPECDEC_API int specdec_probabilities(const void *logits, int dtype, int64_t rows, int64_t vocab,
                                      int64_t row_stride, float temperature, float *out,
                                      int64_t out_stride, int64_t *index_out, int64_t index_stride,
                                      void *stream) {
  if (rows < 0 || vocab <= 0 || vocab > INT32_MAX || temperature < 0.0f) return SPECDEC_EINVAL;
  if (rows == 0) return SPECDEC_OK;
  if (!logits || !out) return SPECDEC_EINVAL;
  dim3 grid((unsigned)rows), block(kSoftmaxThreads);
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case SPECDEC_F32: {
      // 16-byte vectors when every row starts 16-byte aligned, in and out
      const bool vec = vocab % 4 == 0 && row_stride % 4 == 0 && out_stride % 4 == 0 &&
                       ((uintptr_t)logits & 15) == 0 && ((uintptr_t)out & 15) == 0;
      const float *lg = (const float *)logits;
      if (temperature == 1.0f && vec)
        probabilities_kernel<float, true, true><<<grid, block, 0, s>>>(lg, row_stride, vocab, temperature, out,
                                                                       out_stride, index_out, index_stride);
      else if (temperature == 1.0f)
        probabilities_kernel<float, true><<<grid, block, 0, s>>>(lg, row_stride, vocab, temperature, out,
                                                                out_stride, index_out, index_stride);
      else if (vec)
        probabilities_kernel<float, false, true><<<grid, block, 0, s>>>(lg, row_stride, vocab, temperature, out,
                                                                        out_stride, index_out, index_stride);
      else
        probabilities_kernel<float><<<grid, block, 0, s>>>(lg, row_stride, vocab, temperature, out, out_stride,
                                                          index_out, index_stride);
      break;
    }
    case SPECDEC_F64:
      probabilities_kernel<double><<<grid, block, 0, s>>>((const double *)logits, row_stride, vocab,
                                                         temperature, out, out_stride, index_out, index_stride);
      break;
    case SPECDEC_BF16:
      probabilities_kernel<__hip_bfloat16><<<grid, block, 0, s>>>((const __hip_bfloat16 *)logits, row_stride,
                                                                 vocab, temperature, out, out_stride, index_out,
                                                                 index_stride);
      break;
    default: return SPECDEC_EINVAL;
  }
  return launch_status();
}

// Grid of the many-CU accept-reject: E elements per thread, taken from
// `choices` in order, the first whose G chunks per row keep the grid within
// `per_cu` workgroups per compute unit; false when none fits.  The
// probabilities form prefers 16 (12 chunks of a 49152 vocabulary, the
// fastest measured at batch 1 and 8).  The logits form reads 2k+1 rows per
// chunk: up to 21 rows of a 49152 vocabulary it takes one workgroup per
// compute unit (E = 8, then 16), beyond that two, with narrower loads
// (E = 12, then 24: up to 64 rows on 256 compute units), so that a compute
// unit's second workgroup loads while the first reduces (batch 32, k = 8:
// 53.3 -> 44.6 us; batch 64: 85 -> 66 us).  Every workgroup of a grid is
// resident at once when the GPU is otherwise idle; when it is not, the
// meetings' fallback finishes the call with the same bits.
struct MwPlan {
  int E = 0, G = 0;
};

static bool plan_mw(int64_t batch, int64_t vocab, std::initializer_list<int> choices, MwPlan &pl, int per_cu = 1) {
  const int cus = cu_count();
  if (cus <= 0) return false;
  for (int E : choices) {
    const int64_t G = (vocab + (int64_t)kMwThreads * E - 1) / ((int64_t)kMwThreads * E);
    if (G > kMwMaxG || batch * G > (int64_t)per_cu * cus) continue;
    pl.E = E;
    pl.G = (int)G;
    return true;
  }
  return false;
}

template <int E, bool LOGITS>
static void launch_mw_e(bool vec4, const MwArgs &a, hipStream_t s) {
  dim3 grid((unsigned)(a.batch * a.G)), block(kMwThreads);
  if (vec4) accept_reject_mw_kernel<E, true, LOGITS><<<grid, block, 0, s>>>(a);
  else if constexpr (!LOGITS) accept_reject_mw_kernel<E, false, LOGITS><<<grid, block, 0, s>>>(a);
}

static int64_t mw_workspace_bytes(int64_t batch) { return (kMwHead + batch * kMwRowWords) * (int64_t)sizeof(uint64_t); }

// 16-byte vectors when every row of p (and q) starts 16-byte aligned
static bool mw_vec4(const void *p, const void *q, int64_t pb, int64_t pr, int64_t qb, int64_t qr, int64_t k,
                    int64_t vocab) {
  return vocab % 4 == 0 && pb % 4 == 0 && pr % 4 == 0 &&
         (k == 0 || (qb % 4 == 0 && qr % 4 == 0 && ((uintptr_t)q & 15) == 0)) && ((uintptr_t)p & 15) == 0;
}

SPECDEC_API int specdec_accept_workspace(int64_t batch, int64_t *bytes) {
  if (batch < 0 || !bytes) return SPECDEC_EINVAL;
  *bytes = mw_workspace_bytes(batch);
  return SPECDEC_OK;
}

SPECDEC_API int specdec_accept_reject(const void *p, const void *q, int dtype,
                                      int64_t p_batch_stride, int64_t p_row_stride,
                                      int64_t q_batch_stride, int64_t q_row_stride,
                                      const int64_t *draft, const void *u_accept,
                                      const void *u_residual, int64_t batch, int64_t k,
                                      int64_t vocab, int64_t *out, void *workspace,
                                      int64_t workspace_bytes, int32_t spin, void *stream) {
  if (batch < 0 || k < 0 || vocab <= 0) return SPECDEC_EINVAL;
  if (vocab > (int64_t)kMaxTiles * kCdfPerThread * kAcceptThreads) return SPECDEC_EUNSUPPORTED;
  if (batch == 0) return SPECDEC_OK;
  if (!p || !out || !u_residual || (k > 0 && (!q || !draft || !u_accept))) return SPECDEC_EINVAL;
  dim3 grid((unsigned)batch), block(kAcceptThreads);
  hipStream_t s = as_stream(stream);
  MwPlan pl;
  if (workspace && dtype == SPECDEC_F32 && plan_mw(batch, vocab, {16, 24, 32, 48}, pl)) {
    if (workspace_bytes < mw_workspace_bytes(batch) || ((uintptr_t)workspace & 7) != 0) return SPECDEC_EINVAL;
    MwArgs a{};
    a.p = (const float *)p;
    a.q = (const float *)q;
    a.p_bs = p_batch_stride, a.p_rs = p_row_stride, a.q_bs = q_batch_stride, a.q_rs = q_row_stride;
    a.draft = draft;
    a.u_accept = (const float *)u_accept;
    a.u_residual = (const float *)u_residual;
    a.batch = batch, a.k = k, a.vocab = vocab, a.G = pl.G;
    a.temperature = 1.0f;
    a.spin = spin;
    a.out = out;
    a.ws = (uint64_t *)workspace;
    const bool vec4 = mw_vec4(p, q, p_batch_stride, p_row_stride, q_batch_stride, q_row_stride, k, vocab);
    switch (pl.E) {
      case 16: launch_mw_e<16, false>(vec4, a, s); break;
      case 24: launch_mw_e<24, false>(vec4, a, s); break;
      case 32: launch_mw_e<32, false>(vec4, a, s); break;
      default: launch_mw_e<48, false>(vec4, a, s); break;
    }
    return launch_status();
  }
  if (dtype == SPECDEC_F32 && vocab <= (int64_t)kRegTiles * kCdfPerThread * kAcceptThreads) {
    if (vocab % 4 == 0)
      accept_reject_regs_kernel<true><<<grid, block, 0, s>>>((const float *)p, (const float *)q, p_batch_stride,
                                                             p_row_stride, q_batch_stride, q_row_stride, draft,
                                                             (const float *)u_accept, (const float *)u_residual,
                                                             batch, k, vocab, out);
    else
      accept_reject_regs_kernel<false><<<grid, block, 0, s>>>((const float *)p, (const float *)q, p_batch_stride,
                                                              p_row_stride, q_batch_stride, q_row_stride, draft,
                                                              (const float *)u_accept, (const float *)u_residual,
                                                              batch, k, vocab, out);
  } else if (dtype == SPECDEC_F32) {
    accept_reject_kernel<float><<<grid, block, 0, s>>>(
        (const float *)p, (const float *)q, p_batch_stride, p_row_stride, q_batch_stride,
        q_row_stride, draft, (const float *)u_accept, (const float *)u_residual, batch, k, vocab,
        out);
  } else if (dtype == SPECDEC_F64) {
    accept_reject_kernel<double><<<grid, block, 0, s>>>(
        (const double *)p, (const double *)q, p_batch_stride, p_row_stride, q_batch_stride,
        q_row_stride, draft, (const double *)u_accept, (const double *)u_residual, batch, k,
        vocab, out);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}

SPECDEC_API int specdec_accept_reject_logits(const void *target_logits, const void *draft_logits, int dtype,
                                             int64_t t_batch_stride, int64_t t_row_stride,
                                             int64_t d_batch_stride, int64_t d_row_stride, float temperature,
                                             const int64_t *draft, const void *u_accept,
                                             const void *u_residual, int64_t batch, int64_t k, int64_t vocab,
                                             int64_t *out, void *workspace, int64_t workspace_bytes,
                                             int32_t spin, void *stream) {
  if (batch < 0 || k < 0 || vocab <= 0 || !(temperature >= 0.0f)) return SPECDEC_EINVAL;
  if (batch == 0) return SPECDEC_OK;
  if (!target_logits || !out || !u_residual || !workspace ||
      (k > 0 && (!draft_logits || !draft || !u_accept)))
    return SPECDEC_EINVAL;
  if (dtype != SPECDEC_F32) return SPECDEC_EUNSUPPORTED;
  if (workspace_bytes < mw_workspace_bytes(batch) || ((uintptr_t)workspace & 7) != 0) return SPECDEC_EINVAL;
  if (k > kMwMaxK || vocab > INT32_MAX / 2 ||
      !mw_vec4(target_logits, draft_logits, t_batch_stride, t_row_stride, d_batch_stride, d_row_stride, k, vocab))
    return SPECDEC_EUNSUPPORTED;
  MwPlan pl;
  if (!plan_mw(batch, vocab, {8, 16}, pl) && !plan_mw(batch, vocab, {12, 24}, pl, 2))
    return SPECDEC_EUNSUPPORTED;
  MwArgs a{};
  a.p = (const float *)target_logits;
  a.q = (const float *)draft_logits;
  a.p_bs = t_batch_stride, a.p_rs = t_row_stride, a.q_bs = d_batch_stride, a.q_rs = d_row_stride;
  a.draft = draft;
  a.u_accept = (const float *)u_accept;
  a.u_residual = (const float *)u_residual;
  a.batch = batch, a.k = k, a.vocab = vocab, a.G = pl.G;
  a.temperature = temperature;
  a.spin = spin;
  a.out = out;
  a.ws = (uint64_t *)workspace;
  hipStream_t s = as_stream(stream);
  switch (pl.E) {
    case 8: launch_mw_e<8, true>(true, a, s); break;
    case 12: launch_mw_e<12, true>(true, a, s); break;
    case 16: launch_mw_e<16, true>(true, a, s); break;
    default: launch_mw_e<24, true>(true, a, s); break;
  }
  return launch_status();
}

SPECDEC_API int specdec_accept_count(const void *p, const void *q, int dtype,
                                     int64_t p_batch_stride, int64_t p_row_stride,
                                     int64_t q_batch_stride, int64_t q_row_stride,
                                     const int64_t *draft, const void *u_accept, int64_t batch,
                                     int64_t k, int64_t vocab, int64_t *out, void *stream) {
  if (batch < 0 || k < 0 || vocab <= 0) return SPECDEC_EINVAL;
  if (batch == 0) return SPECDEC_OK;
  if (!p || !out || (k > 0 && (!q || !draft || !u_accept))) return SPECDEC_EINVAL;
  // a draft id outside [0, vocab) is never read through: it sets the flag
  // (out[batch + b]) and counts as the first rejection
  dim3 block(64), grid((unsigned)((batch + 63) / 64));
  hipStream_t s = as_stream(stream);
  if (dtype == SPECDEC_F32) {
    accept_count_kernel<float><<<grid, block, 0, s>>>(
        (const float *)p, (const float *)q, p_batch_stride, p_row_stride, q_batch_stride,
        q_row_stride, draft, (const float *)u_accept, batch, k, vocab, out);
  } else if (dtype == SPECDEC_F64) {
    accept_count_kernel<double><<<grid, block, 0, s>>>(
        (const double *)p, (const double *)q, p_batch_stride, p_row_stride, q_batch_stride,
        q_row_stride, draft, (const double *)u_accept, batch, k, vocab, out);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}

SPECDEC_API int specdec_sample_inverse_cdf(const void *probs, int dtype, int64_t batch,
                                           int64_t vocab, int64_t row_stride, const void *u,
                                           int64_t *out, void *stream) {
  if (batch < 0 || vocab <= 0) return SPECDEC_EINVAL;
  if (vocab > (int64_t)kMaxTiles * kCdfPerThread * kAcceptThreads) return SPECDEC_EUNSUPPORTED;
  if (batch == 0) return SPECDEC_OK;
  if (!probs || !u || !out) return SPECDEC_EINVAL;
  dim3 grid((unsigned)batch), block(kAcceptThreads);
  hipStream_t s = as_stream(stream);
  if (dtype == SPECDEC_F32 && vocab <= (int64_t)kRegTiles * kCdfPerThread * kAcceptThreads) {
    if (vocab % 4 == 0)
      sample_inverse_cdf_regs_kernel<true><<<grid, block, 0, s>>>((const float *)probs, vocab, row_stride,
                                                                  (const float *)u, out);
    else
      sample_inverse_cdf_regs_kernel<false><<<grid, block, 0, s>>>((const float *)probs, vocab, row_stride,
                                                                   (const float *)u, out);
  } else if (dtype == SPECDEC_F32) {
    sample_inverse_cdf_kernel<float><<<grid, block, 0, s>>>((const float *)probs, vocab,
                                                           row_stride, (const float *)u, out);
  } else if (dtype == SPECDEC_F64) {
    sample_inverse_cdf_kernel<double><<<grid, block, 0, s>>>((const double *)probs, vocab,
                                                            row_stride, (const double *)u, out);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}

SPECDEC_API int specdec_one_hot(const int64_t *ids, int64_t n, int64_t vocab, float *out,
                                void *stream) {
  if (n < 0 || vocab <= 0) return SPECDEC_EINVAL;
  if (n == 0) return SPECDEC_OK;
  if (!ids || !out) return SPECDEC_EINVAL;
  const int64_t total = n * vocab;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  one_hot_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_stream(stream)>>>(ids, n, vocab, out);
  return launch_status();
}
