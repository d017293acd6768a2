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
// one launch whose workgroups meet twice per row:
//   0. each workgroup finds the accept count n itself with scalar loads (the
//      drafted ids, then p(x) and q(x)) and loads its chunk of p[n] and q[n]
//      (q[k] is the zero row: the bonus samples p[k]);
//   1. it publishes the fp64 sum of its chunk of the residual
//      r = max(0, p[n] - q[n]);
//   2. once every chunk sum of its row is published, each adds them in chunk
//      order (the residual total, rounded to fp32), divides its elements by
//      it (or takes p's row when the total is 0) and publishes L_g, the fp64
//      inclusive prefix sum of its chunk at the chunk's last element;
//   3. once every L_g is published, each forms C_j = L_0 + ... + L_{j-1} in
//      chunk order and the target u * fp32(C_G); the one workgroup whose
//      chunk holds the first prefix above the target -- fp32(C_g) <= target
//      < fp32(C_{g+1}) -- counts its prefixes that do not exceed it.
// An element's prefix is C_g + its chunk-local inclusive prefix (fp64, the
// thread's run after a fixed-order workgroup scan), so a chunk's last
// prefix is C_{g+1} exactly and the chunk test agrees with the count.
// Accumulation in fp64 with a rounding per prefix is the CPU cumsum's rule;
// only the order of the fp64 additions differs from a sequential sum.
//
// Meetings: a value is published with a device-scope atomic store, encoded
// as the complement of the fp64 bits, so that it is never 0; a reader polls
// the slots it needs until none reads 0 (bounded: a timeout flags the row
// with 2 in out[2B + b]).  Slots go back to 0 without a counter: a
// workgroup clears its L slot first thing (the clear is acknowledged before
// its first publish, so no reader can pass the first meeting and still see
// the last call's L), and clears its chunk-sum slot once every L is
// published (every reader of the chunk sums has then finished with them).
// The workspace needs zeroing once, not per call.  The grid never exceeds
// one workgroup per compute unit, so every workgroup of a row is resident
// together.  At B = 1 and 8 twelve chunks of 16 elements per thread
// measured fastest (8.7 us against 9.7 with 24 chunks, 10.9 with 48, and
// 13.1 for a variant loading every candidate row before n was known).
constexpr int kMwThreads = 256;
constexpr int kMwMaxG = 64;     // chunks per row
constexpr int kMwSpin = 1 << 20;
// per-row workspace, in uint64 words: chunk sums [G], then L [G]
constexpr int64_t kMwL = kMwMaxG;
constexpr int64_t kMwRowWords = 2 * kMwMaxG;
constexpr int kMwUnroll = 8;  // drafted positions whose scalar loads go out together

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

__device__ __forceinline__ void publish(uint64_t *slot, uint64_t encoded) {
  __hip_atomic_store(slot, encoded, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t enc64(double v) { return ~__builtin_bit_cast(uint64_t, v); }
__device__ __forceinline__ double dec64(uint64_t w) { return __builtin_bit_cast(double, ~w); }

// Poll slots[0..n) (this workgroup's threads share them) until each is
// published; their raw words land in dst.  False on timeout.
__device__ bool await_slots(uint64_t *slots, int n, uint64_t *dst) {
  __shared__ int s_late;
  if (threadIdx.x == 0) s_late = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    uint64_t w = 0;
    for (int spin = 0; spin < kMwSpin; ++spin) {
      w = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (w != 0) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (w == 0) s_late = 1;
    dst[i] = w;
  }
  __syncthreads();
  return s_late == 0;
}

// Sequential fp64 sum of the decoded words w[0..n) (n >= 1), in index
// order, with the reads issued 16 at a time so their latencies overlap;
// also the running sum before and after element j (when 0 <= j < n).
struct Chain {
  double total, before, after;
};
__device__ __forceinline__ Chain chain_sum(const uint64_t *w, int n, int j) {
  Chain r{0.0, 0.0, 0.0};
  double acc = 0.0;
  for (int i0 = 0; i0 < n; i0 += 16) {
    double v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = dec64(w[min(i0 + i, n - 1)]);
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

template <int E, bool VEC4>
__global__ __launch_bounds__(kMwThreads) void accept_reject_mw_kernel(
    const float *__restrict__ p, const float *__restrict__ q, int64_t p_bs, int64_t p_rs, int64_t q_bs,
    int64_t q_rs, const int64_t *__restrict__ draft, const float *__restrict__ u_accept,
    const float *__restrict__ u_residual, int64_t batch, int64_t k, int64_t vocab, int G,
    int64_t *__restrict__ out, uint64_t *__restrict__ ws) {
  __shared__ double scratch[kMwThreads / kWave + 1];
  __shared__ uint64_t s_words[kMwMaxG];
  __shared__ double s_last;
  const int64_t b = blockIdx.x / G;
  const int g = (int)(blockIdx.x % G);
  const int tid = threadIdx.x;
  constexpr int kChunk = kMwThreads * E;
  const unsigned first = (unsigned)g * kChunk + (unsigned)tid * E;  // this thread's first element
  uint64_t *row_ws = ws + b * kMwRowWords;
  const float *p_b = p + b * p_bs;
  const float *q_b = q + b * q_bs;
  auto flag_late = [&]() {
    if (tid == 0) __hip_atomic_store(reinterpret_cast<uint64_t *>(out + 2 * batch + b), 2ull, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
  };
  // the last call's L of this chunk goes back to 0 before anything is published
  if (tid == 0) publish(row_ws + kMwL + g, 0);
  const float ur = u_residual[b];
  __asm__ volatile("" ::"s"(ur));  // loaded now, not after a meeting

  // 0. the accept count n and the bad-draft flag, the same in every thread
  // (accept_stage's test, u * q(x) < p(x) as a product; an id outside the
  // vocabulary is never read through)
  int64_t n = k, bad = 0;
  for (int64_t t0 = 0; t0 < k; t0 += kMwUnroll) {
    int64_t xs[kMwUnroll];
    float pxs[kMwUnroll], qxs[kMwUnroll], us[kMwUnroll];
#pragma unroll
    for (int j = 0; j < kMwUnroll; ++j) {
      xs[j] = -1;
      if (t0 + j < k) xs[j] = draft[b * k + t0 + j];
    }
#pragma unroll
    for (int j = 0; j < kMwUnroll; ++j) {
      const int64_t t = t0 + j, x = xs[j];
      pxs[j] = qxs[j] = us[j] = 0.0f;
      if (t < k) us[j] = u_accept[b * k + t];
      if (t < k && x >= 0 && x < vocab) {
        pxs[j] = p_b[t * p_rs + x];
        qxs[j] = q_b[t * q_rs + x];
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
  if (g == 0 && tid == 0) {
    out[b] = n;
    out[2 * batch + b] = bad;
  }
  float pr[E], qr[E];  // this thread's elements of p[n] and q[n]
  load_elems<E, VEC4>(row_buffer(p_b + n * p_rs, (unsigned)vocab), first, pr);
  if (n < k) load_elems<E, VEC4>(row_buffer(q_b + n * q_rs, (unsigned)vocab), first, qr);
  else
#pragma unroll
    for (int e = 0; e < E; ++e) qr[e] = 0.0f;

  // 1. the chunk's residual sum
  float x[E];
  double run = 0.0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float r = pr[e] - qr[e];
    x[e] = r > 0.0f ? r : 0.0f;
    run += (double)x[e];
  }
  const double chunk_sum = block_sum(run, scratch);
  if (tid == 0) {
    __builtin_amdgcn_s_waitcnt(0);  // the L clear is acknowledged before any publish
    publish(row_ws + g, enc64(chunk_sum));
  }
  if (!await_slots(row_ws, G, s_words)) {
    flag_late();
    return;
  }

  // 2. the total in chunk order, the quotients, L_g
  const float total = (float)chain_sum(s_words, G, -1).total;
  const float denom = total > FLT_MIN ? total : FLT_MIN;
  const bool use_residual = total > 0.0f;
  run = 0.0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    x[e] = use_residual ? x[e] / denom : pr[e];  // p == q: p itself
    run += (double)x[e];
  }
  double unused;
  const double excl = block_exclusive_scan(run, scratch, &unused);
  if (tid == kMwThreads - 1) {
    double acc = excl;
#pragma unroll
    for (int e = 0; e < E; ++e) acc += (double)x[e];
    s_last = acc;
  }
  __syncthreads();
  if (tid == 0) publish(row_ws + kMwL + g, enc64(s_last));
  if (!await_slots(row_ws + kMwL, G, s_words)) {
    flag_late();
    return;
  }
  // every reader of the chunk sums is past them: clear this chunk's
  if (tid == 0) publish(row_ws + g, 0);

  // 3. chunk bases, the target, the count in the chunk that holds it
  const Chain chain = chain_sum(s_words, G, g);
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
    if (tid == 0) out[batch + b] = idx < vocab - 1 ? idx : vocab - 1;
  } else if (g == G - 1 && !(target < (float)c)) {
    if (tid == 0) out[batch + b] = vocab - 1;  // no prefix exceeds the target
  }
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

SPECDEC_API int specdec_abi_version(void) { return 14; }

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

// Grid of the many-CU accept-reject: E elements per thread, preferring 16
// (12 chunks of a 49152 vocabulary, the fastest measured), then the next E
// whose G chunks per row keep the grid within one workgroup per compute
// unit; false when none fits (then one workgroup runs each row).
struct MwPlan {
  int E = 0, G = 0;
};

static bool plan_mw(int64_t batch, int64_t vocab, MwPlan &pl) {
  const int cus = cu_count();
  if (cus <= 0) return false;
  for (int E : {16, 24, 32, 48}) {
    const int64_t G = (vocab + (int64_t)kMwThreads * E - 1) / ((int64_t)kMwThreads * E);
    if (G > kMwMaxG || batch * G > cus) continue;
    pl.E = E;
    pl.G = (int)G;
    return true;
  }
  return false;
}

template <int E>
static void launch_mw_e(bool vec4, int64_t batch, int G, hipStream_t s, const float *p, const float *q, int64_t p_bs,
                        int64_t p_rs, int64_t q_bs, int64_t q_rs, const int64_t *draft, const float *ua,
                        const float *ur, int64_t k, int64_t vocab, int64_t *out, uint64_t *ws) {
  dim3 grid((unsigned)(batch * G)), block(kMwThreads);
  if (vec4)
    accept_reject_mw_kernel<E, true><<<grid, block, 0, s>>>(p, q, p_bs, p_rs, q_bs, q_rs, draft, ua, ur, batch, k,
                                                             vocab, G, out, ws);
  else
    accept_reject_mw_kernel<E, false><<<grid, block, 0, s>>>(p, q, p_bs, p_rs, q_bs, q_rs, draft, ua, ur, batch, k,
                                                              vocab, G, out, ws);
}

SPECDEC_API int specdec_accept_workspace(int64_t batch, int64_t *bytes) {
  if (batch < 0 || !bytes) return SPECDEC_EINVAL;
  *bytes = batch * kMwRowWords * (int64_t)sizeof(uint64_t);
  return SPECDEC_OK;
}

SPECDEC_API int specdec_accept_reject(const void *p, const void *q, int dtype,
                                      int64_t p_batch_stride, int64_t p_row_stride,
                                      int64_t q_batch_stride, int64_t q_row_stride,
                                      const int64_t *draft, const void *u_accept,
                                      const void *u_residual, int64_t batch, int64_t k,
                                      int64_t vocab, int64_t *out, void *workspace,
                                      int64_t workspace_bytes, void *stream) {
  if (batch < 0 || k < 0 || vocab <= 0) return SPECDEC_EINVAL;
  if (vocab > (int64_t)kMaxTiles * kCdfPerThread * kAcceptThreads) return SPECDEC_EUNSUPPORTED;
  if (batch == 0) return SPECDEC_OK;
  if (!p || !out || !u_residual || (k > 0 && (!q || !draft || !u_accept))) return SPECDEC_EINVAL;
  dim3 grid((unsigned)batch), block(kAcceptThreads);
  hipStream_t s = as_stream(stream);
  MwPlan pl;
  if (workspace && dtype == SPECDEC_F32 && plan_mw(batch, vocab, pl)) {
    if (workspace_bytes < batch * kMwRowWords * (int64_t)sizeof(uint64_t) || ((uintptr_t)workspace & 7) != 0)
      return SPECDEC_EINVAL;
    const bool vec4 = vocab % 4 == 0 && p_batch_stride % 4 == 0 && p_row_stride % 4 == 0 &&
                      (k == 0 || (q_batch_stride % 4 == 0 && q_row_stride % 4 == 0 && ((uintptr_t)q & 15) == 0)) &&
                      ((uintptr_t)p & 15) == 0;
    const float *fp = (const float *)p, *fq = (const float *)q;
    const float *ua = (const float *)u_accept, *ur = (const float *)u_residual;
    uint64_t *ws = (uint64_t *)workspace;
    const int64_t pb = p_batch_stride, pr = p_row_stride, qb = q_batch_stride, qr = q_row_stride;
    switch (pl.E) {
      case 16: launch_mw_e<16>(vec4, batch, pl.G, s, fp, fq, pb, pr, qb, qr, draft, ua, ur, k, vocab, out, ws); break;
      case 24: launch_mw_e<24>(vec4, batch, pl.G, s, fp, fq, pb, pr, qb, qr, draft, ua, ur, k, vocab, out, ws); break;
      case 32: launch_mw_e<32>(vec4, batch, pl.G, s, fp, fq, pb, pr, qb, qr, draft, ua, ur, k, vocab, out, ws); break;
      default: launch_mw_e<48>(vec4, batch, pl.G, s, fp, fq, pb, pr, qb, qr, draft, ua, ur, k, vocab, out, ws); break;
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
