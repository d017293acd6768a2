// Output head on gfx950 MFMA, with the temperature softmax / argmax of the
// logits fused into the same launch.
//
// Reference semantics: lm/forward.py:71-84 (the final hidden rows times the
// output head, accumulated and returned in fp32) followed by
// lm/sampling.py:13-18 (probabilities: one-hot of the argmax at T = 0 --
// ties to the lowest id -- else softmax(logits / T)).
//
// Layout.  The head W [V, H] bf16 is split into 16-row vocab tiles; a
// workgroup owns a slice of consecutive tiles (at most 16) and each of its
// waves one tile.  A tile's logits for 16 hidden rows are
//   D[vocab row, hidden row] = sum over k of W[row, k] * x[hidden row, k]
// on v_mfma_f32_16x16x32_bf16: A = the tile's W rows (lane 16g + c loads
// the 16 bytes of row c at k = 32s + 8g, the MFMA's own operand layout),
// B = the hidden rows staged in LDS, accumulated over k-steps s in order.
// Each output element goes through the same MFMA sequence whatever the
// number of hidden rows in the call, the other rows of its tile or the
// workgroup that computes it, so a row's logits have the same bits alone or
// among others (a token verified among k+1 and decoded alone see the same
// logits, and argmax, bit for bit).
//
// Fused softmax (at most 16 hidden rows).  The workgroups meet once:
//   1. each finds its slice's statistics per hidden row from the logits it
//      keeps in LDS -- the slice maximum of l/T and the sum of
//      2^((l/T - max) log2 e) (T > 0), or the slice's maximum and its lowest
//      index (T = 0) -- and publishes them as tagged 64-bit words into
//      each of 16 copies of the slot region (a workgroup polls one copy, so
//      few poll the same memory lines);
//   2. it reads its copy until every slice's words are there, folds them
//      in slice order with a fixed lane pattern (so every workgroup gets the
//      same bits), and writes its slice of p from the logits still in LDS:
//      2^((l/T - M) log2 e) * (1 / S), or the one-hot row;
//   3. it adds 1 to the call's arrival counter (one of two, by the parity of
//      the call epoch); the workgroup that arrives last clears the other
//      counter for the next call and advances the epoch.
// A word carries the call's tag (the epoch read at the start, plus one) in
// its upper half, so words of earlier calls never pass for this call's and
// the slots need no clearing.  The wait is bounded: a workgroup that gives
// up (or finds a word missing) computes the missing slices' statistics
// itself with the same code and the same bits, so every launch ends with
// the right result whether or not its workgroups are resident together (the
// grid is at most one workgroup per compute unit, so they normally are).
#include "common.h"

#include <float.h>
#include <math.h>

#include <algorithm>

namespace specdec {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

constexpr int kHT = 16;                     // vocab rows per tile, hidden rows per column tile
constexpr int kHMaxTpw = 16;                // tiles (and waves) per workgroup
constexpr int kHSlice = kHMaxTpw * kHT;     // vocab rows per workgroup, at most
constexpr int kHXPad = 8;                   // bf16 padding per staged hidden row (LDS banks)
constexpr int kHXElems = kHT * (2048 + kHXPad);  // staged hidden elements (bf16)
constexpr int kHMaxGrid = 256;              // workgroups of a fused call, at most
constexpr int kHFusedRows = 16;             // hidden rows of a fused call, at most
// workspace words: two arrival counters, the call epoch, then kHCopies
// regions, each holding every slice's words, [slice][row][2] packed by the
// call's row count.  Workgroup j reads region j % kHCopies: a writer stores
// its words kHCopies times, and a line is polled by grid / kHCopies readers
// (256 readers of one copy queued for the same lines; a copy per reader
// multiplied the stores by 256)
constexpr int kHCopies = 16;
constexpr int64_t kHWsHead = 3;
constexpr int64_t kHWsRegion = (int64_t)kHMaxGrid * kHFusedRows * 2;
constexpr int64_t kHWsWords = kHWsHead + kHCopies * kHWsRegion;
constexpr int kHLoadsInFlight = 8;  // region words a thread reads per round

enum HeadMode { kLogits = 0, kSoftmax = 1, kArgmax = 2 };

struct HeadArgs {
  const uint16_t *x;  // [M, H] bf16
  int64_t x_stride;
  const uint16_t *w;  // [V, H] bf16
  int64_t w_stride;
  int M, H, V;
  int steps;  // H / 32
  int kc;     // k-steps per staged chunk of the hidden rows
  int tiles;  // vocab tiles
  int tpw;    // tiles per workgroup
  int mode;
  float temperature;
  float *out;  // probabilities [M, V] (kSoftmax, kArgmax)
  int64_t out_stride;
  int64_t *index_out;  // argmax [M] (kArgmax, optional)
  int64_t index_stride;
  float *logits;  // [M, V] (kLogits; optional otherwise)
  int64_t logits_stride;
  uint64_t *ws;
  int spin;
  int vec_out, vec_logits;  // 16-byte row stores allowed
};

// ---- the logits of one vocab tile --------------------------------------
// Stage hidden rows r0 .. r0 + 16*NCT - 1 (zeros past M), k-steps
// [k0, k0 + kn), into s_x with row stride xs elements; the steps up to the
// next multiple of KB are staged as zeros.  A thread's loads of a round go
// out together, then its LDS stores.
template <int NCT, int KB>
__device__ __forceinline__ void stage_x(const HeadArgs &a, uint16_t *s_x, int xs, int r0, int k0, int kn) {
  constexpr int kU = 8;  // 16-byte units per thread per round
  const int per_row = (kn + KB - 1) / KB * KB * 4;
  const int valid = kn * 4;
  const int total = kHT * NCT * per_row;
  for (int u0 = 0; u0 < total; u0 += kU * (int)blockDim.x) {
    u32x4 v[kU];
#pragma unroll
    for (int i = 0; i < kU; ++i) {
      const int u = u0 + i * (int)blockDim.x + (int)threadIdx.x;
      const int r = u / per_row, j = u - r * per_row;
      v[i] = u32x4{0u, 0u, 0u, 0u};
      if (u < total && r0 + r < a.M && j < valid)
        v[i] = *reinterpret_cast<const u32x4 *>(a.x + (int64_t)(r0 + r) * a.x_stride + (int64_t)k0 * 32 + 8 * j);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kU; ++i) {
      const int u = u0 + i * (int)blockDim.x + (int)threadIdx.x;
      const int r = u / per_row, j = u - r * per_row;
      if (u < total) *reinterpret_cast<u32x4 *>(s_x + r * xs + 8 * j) = v[i];
    }
  }
}

// The logits of the tiles of slice j for hidden rows r0 .. r0 + 16*NCT - 1:
// wave w computes tile j*tpw + w, accumulating acc[ct] over the k-steps in
// order, the hidden rows staged chunk by chunk (barriers inside, so every
// thread of the workgroup calls it).
// Per chunk the W rows stream in batches of KB k-steps, the next batch's
// loads in flight while one is multiplied; the chunk's first batch is
// issued before its hidden rows are staged.  The loop body issues its loads
// without conditions (the last one or two batches are peeled), so the
// compiler's wait counts stay exact; the steps of a partial last batch
// re-read step kn - 1 and meet staged zeros, adding exact zeros.  The
// scheduling barriers keep each batch's loads ahead of the previous batch's
// multiplies, where the compiler would otherwise sink them.
template <int NCT, int KB>
__device__ __forceinline__ void slice_logits(const HeadArgs &a, uint16_t *s_x, int j, int r0, f32x4 (&acc)[NCT]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c = lane & 15, g = lane >> 4;
  const int tile = j * a.tpw + wave;
  const bool mine = wave < a.tpw && tile < a.tiles;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int xs = a.kc * 32 + kHXPad;  // kc is a multiple of KB
  const __amdgpu_buffer_rsrc_t wb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.w), 0, (int)((int64_t)a.V * a.w_stride * 2), 0x00020000);
  const int row = min(tile * kHT + c, a.V - 1);  // rows past the vocab read the last row; never stored
  const unsigned rowbase = (unsigned)(((int64_t)row * a.w_stride + 8 * g) * 2);
  const uint16_t *xp = s_x + c * xs + 8 * g;
  u32x4 A0[KB], A1[KB];
  auto issue = [&](u32x4 (&A)[KB], int k0, int kn, int b) {
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) {
      const int s = min(b * KB + jj, kn - 1);
      A[jj] = __builtin_amdgcn_raw_buffer_load_b128(wb, rowbase + (unsigned)(k0 + s) * 64u, 0, 0);
    }
  };
  auto consume = [&](const u32x4 (&A)[KB], int b) {
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) {
      const int s = b * KB + jj;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const u32x4 xb = *reinterpret_cast<const u32x4 *>(xp + ct * kHT * xs + s * 32);
        acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, A[jj]),
                                                          __builtin_bit_cast(bf16x8, xb), acc[ct], 0, 0, 0);
      }
    }
  };
  for (int k0 = 0; k0 < a.steps; k0 += a.kc) {
    const int kn = min(a.kc, a.steps - k0);
    const int nb = (kn + KB - 1) / KB;
    if (mine) issue(A0, k0, kn, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (k0 > 0) __syncthreads();
    stage_x<NCT, KB>(a, s_x, xs, r0, k0, kn);
    __syncthreads();
    if (mine) {
      int b = 0;
      for (; b + 2 < nb; b += 2) {
        issue(A1, k0, kn, b + 1);
        __builtin_amdgcn_sched_barrier(0);
        consume(A0, b);
        __builtin_amdgcn_sched_barrier(0);
        issue(A0, k0, kn, b + 2);
        __builtin_amdgcn_sched_barrier(0);
        consume(A1, b + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (b + 1 < nb) {  // the last two batches
        issue(A1, k0, kn, b + 1);
        __builtin_amdgcn_sched_barrier(0);
        consume(A0, b);
        __builtin_amdgcn_sched_barrier(0);
        consume(A1, b + 1);
      } else {  // the last batch
        consume(A0, b);
      }
    }
  }
}

// ---- statistics of a slice ----------------------------------------------
// Slice logits in LDS as s_l[row][i] (i < kHSlice); n valid entries.  One
// wave per hidden row, lane taking entries lane, lane + 64, ...; every
// reduction has a fixed order, so the owner and any workgroup recomputing
// the slice get the same bits.
__device__ __forceinline__ float scaled(const HeadArgs &a, float l) {
  return a.temperature == 1.0f ? l : l / a.temperature;  // x / 1 is x
}

constexpr float kHLog2e = 1.4426950408889634f;

// stat[r * rs + e * es], e = 0, 1: (max, sum) for kSoftmax, (max, index
// bits) for kArgmax
__device__ void slice_stats(const HeadArgs &a, const float (*s_l)[kHSlice], int n, int base, uint32_t *stat, int rs,
                            int es) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int r = wave; r < a.M; r += nw) {
    if (a.mode == kArgmax) {
      float best = -INFINITY;
      int best_i = INT32_MAX;
      for (int i = lane; i < n; i += 64) argmax_keep(best, best_i, s_l[r][i], base + i);
      wave_argmax_dpp(best, best_i);
      if (lane == 0) {
        stat[r * rs] = __float_as_uint(best);
        stat[r * rs + es] = (uint32_t)best_i;
      }
    } else {
      float m = -INFINITY;
      for (int i = lane; i < n; i += 64) m = fmaxf(m, scaled(a, s_l[r][i]));
      m = wave_max_dpp(m);
      float s = 0.0f;
      if (m != -INFINITY)
        for (int i = lane; i < n; i += 64) s += __builtin_amdgcn_exp2f((scaled(a, s_l[r][i]) - m) * kHLog2e);
      s = wave_sum_dpp(s);
      if (lane == 0) {
        stat[r * rs] = __float_as_uint(m);
        stat[r * rs + es] = __float_as_uint(s);
      }
    }
  }
}

// Lane layout of an accumulator: lane 16g + c holds vocab rows 4g .. 4g+3
// of the tile for hidden row c.
__device__ __forceinline__ void store_logits4(float *row_ptr, int v0, int V, const f32x4 &v, bool vec) {
  if (vec && v0 + 3 < V) {
    *reinterpret_cast<f32x4 *>(row_ptr + v0) = v;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (v0 + i < V) row_ptr[v0 + i] = v[i];
  }
}

// ---- kernels --------------------------------------------------------------
// Logits only: grid (slices, passes of 16*NCT hidden rows).
template <int NCT, int KB>
__global__ __launch_bounds__(1024) void head_logits_kernel(HeadArgs a) {
  __shared__ __align__(16) uint16_t s_x[kHXElems];
  const int r0 = blockIdx.y * kHT * NCT;
  f32x4 acc[NCT];
  slice_logits<NCT, KB>(a, s_x, blockIdx.x, r0, acc);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int tile = blockIdx.x * a.tpw + wave;
  if (wave >= a.tpw || tile >= a.tiles) return;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int r = r0 + ct * kHT + c;
    if (r < a.M) store_logits4(a.logits + (int64_t)r * a.logits_stride, tile * kHT + 4 * g, a.V, acc[ct], a.vec_logits);
  }
}

// Logits + softmax / one-hot argmax, at most 16 hidden rows; one workgroup
// per slice, every workgroup resident at once in the normal case.
template <int KB>
__global__ __launch_bounds__(1024) void head_softmax_kernel(HeadArgs a) {
  __shared__ __align__(16) uint16_t s_x[kHXElems];
  __shared__ __align__(16) float s_l[2][kHFusedRows][kHSlice];  // own slice, a recomputed slice
  __shared__ uint32_t s_ex[kHFusedRows * 2][kHMaxGrid];         // every slice's statistics, [row, e][slice]
  __shared__ uint32_t s_own[kHFusedRows][2];
  __shared__ float s_fin[kHFusedRows][2];  // (M, 1/S) or (-, index bits)
  __shared__ int s_missing[kHMaxGrid];
  __shared__ uint8_t s_seen[kHMaxGrid * kHFusedRows * 2];
  __shared__ int s_any;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int j0 = blockIdx.x, grid = gridDim.x;
  const int nw2 = a.M * 2;  // words per slice
  uint64_t *counters = a.ws, *epoch_w = a.ws + 2, *regions = a.ws + kHWsHead;
  // the call's tag: the epoch before anyone arrives, plus one (never 0)
  const uint64_t epoch = __hip_atomic_load(epoch_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t tag = (uint32_t)(epoch % 0xFFFFFFFFull) + 1u;
  uint64_t *arrivals = counters + (epoch & 1);

  auto slice_n = [&](int j) { return max(0, min(a.V - j * a.tpw * kHT, a.tpw * kHT)); };
  // logits of slice j into s_l[buf][row][..]
  auto compute_slice = [&](int j, int buf) {
    f32x4 acc[1];
    slice_logits<1, KB>(a, s_x, j, 0, acc);
    if (wave < a.tpw && c < a.M) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s_l[buf][c][wave * kHT + 4 * g + i] = acc[0][i];
    }
    __syncthreads();
  };

  // 1. own slice: logits and statistics
  compute_slice(j0, 0);
  const int n_own = slice_n(j0), base_own = j0 * a.tpw * kHT;
  slice_stats(a, s_l[0], n_own, base_own, &s_own[0][0], 2, 1);
  for (int j = tid; j < grid; j += blockDim.x) s_missing[j] = 0;
  for (int u = tid; u < grid * nw2; u += blockDim.x) s_seen[u] = 0;
  if (tid == 0) s_any = 0;
  __syncthreads();
  // 2. this workgroup's region, every other slice's words, kHLoadsInFlight
  // per thread per pass; a word seen with the call's tag is kept (s_ex) and
  // not read again.  The first pass is issued before this workgroup
  // publishes, so waiting for it does not wait for the publishing stores.
  const uint64_t *mine = regions + (int64_t)(j0 % kHCopies) * kHWsRegion;
  const int nwords = grid * nw2;
  const int per_pass = kHLoadsInFlight * (int)blockDim.x;
  uint64_t w[kHLoadsInFlight];
  auto issue = [&](int u0, bool all) {
#pragma unroll
    for (int i = 0; i < kHLoadsInFlight; ++i) {
      const int u = min(u0 + i * (int)blockDim.x + tid, nwords - 1);
      w[i] = 0;
      if (all || !s_seen[u]) w[i] = __hip_atomic_load(mine + u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  auto take = [&](int u0, bool all) {
#pragma unroll
    for (int i = 0; i < kHLoadsInFlight; ++i) {
      const int u = u0 + i * (int)blockDim.x + tid;
      if (u >= nwords || (!all && s_seen[u])) continue;
      const int j = u / nw2, re = u - j * nw2;
      if (j == j0 || (uint32_t)(w[i] >> 32) == tag) {
        if (j != j0) s_ex[re][j] = (uint32_t)w[i];
        s_seen[u] = 1;
      } else {
        s_any = 1;
      }
    }
  };
  issue(0, true);
  __builtin_amdgcn_sched_barrier(0);
  // 3. publish: this slice's words into every reader's region (8-byte
  // stores, contiguous per region)
  for (int u = tid; u < kHCopies * nw2; u += blockDim.x) {
    const int reader = u / nw2, re = u - reader * nw2;
    const uint64_t word = ((uint64_t)tag << 32) | s_own[re >> 1][re & 1];
    __hip_atomic_store(regions + reader * kHWsRegion + (int64_t)j0 * nw2 + re, word, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  if (a.logits) {
    const int nq = a.tpw * kHT / 4;
    for (int u = tid; u < a.M * nq; u += blockDim.x) {
      const int r = u / nq, q = u - r * nq;
      if (4 * q < n_own) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(&s_l[0][r][4 * q]);
        store_logits4(a.logits + (int64_t)r * a.logits_stride, base_own + 4 * q, a.V, v, a.vec_logits);
      }
    }
  }
  take(0, true);
  for (int u0 = per_pass; u0 < nwords; u0 += per_pass) {
    issue(u0, true);
    take(u0, true);
  }
  __syncthreads();
  // 4. the words not seen yet, again, at most `spin` more times; slices
  // still missing then are recomputed below
  for (int round = 0; s_any && round < a.spin; ++round) {
    __syncthreads();
    if (tid == 0) {
      s_any = 0;
      __builtin_amdgcn_s_sleep(2);
    }
    __syncthreads();
    for (int u0 = 0; u0 < nwords; u0 += per_pass) {
      issue(u0, false);
      take(u0, false);
    }
    __syncthreads();
  }
  if (tid < nw2) s_ex[tid][j0] = s_own[tid >> 1][tid & 1];
  __syncthreads();
  if (s_any) {
    for (int u = tid; u < nwords; u += blockDim.x)
      if (!s_seen[u]) s_missing[u / nw2] = 1;
    __syncthreads();
    for (int j = 0; j < grid; ++j) {
      if (!s_missing[j]) continue;
      compute_slice(j, 1);
      slice_stats(a, s_l[1], slice_n(j), j * a.tpw * kHT, &s_ex[0][j], 2 * kHMaxGrid, kHMaxGrid);
      __syncthreads();
    }
  }
  // 4. fold the slices in order, the same lane pattern in every workgroup
  for (int r = wave; r < a.M; r += nw) {
    const uint32_t *st0 = s_ex[2 * r], *st1 = s_ex[2 * r + 1];
    if (a.mode == kArgmax) {
      float best = -INFINITY;
      int best_i = INT32_MAX;
      for (int j = lane; j < grid; j += 64) argmax_keep(best, best_i, __uint_as_float(st0[j]), (int)st1[j]);
      wave_argmax_dpp(best, best_i);
      if (lane == 0) s_fin[r][1] = __int_as_float(best_i);
    } else {
      float m = -INFINITY;
      for (int j = lane; j < grid; j += 64) m = fmaxf(m, __uint_as_float(st0[j]));
      m = wave_max_dpp(m);
      float s = 0.0f;
      for (int j = lane; j < grid; j += 64) {
        const float mj = __uint_as_float(st0[j]);
        if (mj != -INFINITY) s += __uint_as_float(st1[j]) * __builtin_amdgcn_exp2f((mj - m) * kHLog2e);
      }
      s = wave_sum_dpp(s);
      if (lane == 0) {
        s_fin[r][0] = m;
        s_fin[r][1] = 1.0f / s;
      }
    }
  }
  __syncthreads();
  // 5. this slice of p
  const int nq = a.tpw * kHT / 4;
  for (int u = tid; u < a.M * nq; u += blockDim.x) {
    const int r = u / nq, q = u - r * nq;
    if (4 * q >= n_own) continue;
    const int v0 = base_own + 4 * q;
    f32x4 p;
    if (a.mode == kArgmax) {
      const int hot = __float_as_int(s_fin[r][1]);
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = (v0 + i == hot) ? 1.0f : 0.0f;
    } else {
      const float m = s_fin[r][0], inv = s_fin[r][1];
      const f32x4 l = *reinterpret_cast<const f32x4 *>(&s_l[0][r][4 * q]);
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f((scaled(a, l[i]) - m) * kHLog2e) * inv;
    }
    store_logits4(a.out + (int64_t)r * a.out_stride, v0, a.V, p, a.vec_out);
  }
  if (a.mode == kArgmax && a.index_out && j0 == 0 && tid < a.M)
    a.index_out[(int64_t)tid * a.index_stride] = (int64_t)__float_as_int(s_fin[tid][1]);
  // 5. arrive: the count only decides who advances the epoch -- the last to
  // arrive, once every workgroup has read it -- and stays off the path above
  if (tid == 0) {
    const uint64_t before = __hip_atomic_fetch_add(arrivals, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (before == (uint64_t)grid - 1) {  // ready the next call's counter and tag
      __hip_atomic_store(counters + ((epoch + 1) & 1), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(epoch_w, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---- host side ------------------------------------------------------------
struct HeadPlan {
  int tpw = 0, grid = 0;
};

// Tiles per workgroup: the vocab spread over every compute unit (at most 16
// tiles each).  `fused` calls need the grid within one workgroup per CU.
static bool plan_head(int64_t V, bool fused, HeadPlan &pl) {
  const int cus = cu_count();
  if (cus <= 0) return false;
  const int64_t tiles = (V + kHT - 1) / kHT;
  int64_t tpw = (tiles + cus - 1) / cus;
  if (tpw < 1) tpw = 1;
  if (tpw > kHMaxTpw) {
    if (fused) return false;
    tpw = kHMaxTpw;
  }
  const int64_t grid = (tiles + tpw - 1) / tpw;
  if (grid > (fused ? std::min(cus, kHMaxGrid) : 65535)) return false;
  pl.tpw = (int)tpw;
  pl.grid = (int)grid;
  return true;
}

static int head_args(const void *x, int64_t x_stride, const void *w, int64_t w_stride, int64_t M, int64_t H,
                     int64_t V, HeadArgs &a) {
  if (M < 0 || H <= 0 || V <= 0 || V > INT32_MAX / 2 || M > INT32_MAX / 2) return SPECDEC_EINVAL;
  if (H % 32 != 0 || H > 2048) return SPECDEC_EUNSUPPORTED;
  if (V * w_stride * 2 > INT32_MAX) return SPECDEC_EUNSUPPORTED;  // one buffer resource addresses W
  if (!x || !w || x_stride < H || w_stride < H || x_stride % 8 || w_stride % 8) return SPECDEC_EINVAL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15)) return SPECDEC_EINVAL;
  a = HeadArgs{};
  a.x = (const uint16_t *)x;
  a.x_stride = x_stride;
  a.w = (const uint16_t *)w;
  a.w_stride = w_stride;
  a.M = (int)M;
  a.H = (int)H;
  a.V = (int)V;
  a.steps = (int)(H / 32);
  a.tiles = (int)((V + kHT - 1) / kHT);
  return SPECDEC_OK;
}

// k-steps per W load batch: 9 for an 18-step (576-wide) head, whose two
// batches then go out together with no step re-read, else 8
static int batch_steps(int steps) { return steps == 18 ? 9 : 8; }

// k-steps per staged chunk: the hidden rows of a pass (16 * NCT of them)
// in at most kHXElems elements, a multiple of kb steps (the last chunk may
// be shorter; it is padded with zeros up to the next multiple)
static int chunk_steps(int steps, int nct, int kb) {
  const int row = kHXElems / (kHT * nct);  // elements per staged row
  const int kc = (row - kHXPad) / 32 / kb * kb;
  return std::min((steps + kb - 1) / kb * kb, kc);
}

}  // namespace specdec

using namespace specdec;

SPECDEC_API int specdec_head_workspace(int64_t *bytes) {
  if (!bytes) return SPECDEC_EINVAL;
  *bytes = kHWsWords * (int64_t)sizeof(uint64_t);
  return SPECDEC_OK;
}

SPECDEC_API int specdec_head_logits(const void *x, int64_t x_stride, const void *w, int64_t w_stride, int64_t rows,
                                    int64_t hidden, int64_t vocab, float *logits, int64_t logits_stride,
                                    void *stream) {
  HeadArgs a;
  const int st = head_args(x, x_stride, w, w_stride, rows, hidden, vocab, a);
  if (st != SPECDEC_OK) return st;
  if (rows == 0) return SPECDEC_OK;
  if (!logits || logits_stride < vocab) return SPECDEC_EINVAL;
  HeadPlan pl;
  if (!plan_head(vocab, false, pl)) return SPECDEC_EUNSUPPORTED;
  a.tpw = pl.tpw;
  a.mode = kLogits;
  a.logits = logits;
  a.logits_stride = logits_stride;
  a.vec_logits = logits_stride % 4 == 0 && ((uintptr_t)logits & 15) == 0;
  const int nct = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
  const int kb = batch_steps(a.steps);
  a.kc = chunk_steps(a.steps, nct, kb);
  const int64_t passes = (rows + kHT * nct - 1) / (kHT * nct);
  if (passes > 65535) return SPECDEC_EUNSUPPORTED;
  dim3 grid((unsigned)pl.grid, (unsigned)passes), block((unsigned)(64 * pl.tpw));
  hipStream_t s = as_stream(stream);
  if (kb == 9) {
    if (nct == 1) head_logits_kernel<1, 9><<<grid, block, 0, s>>>(a);
    else if (nct == 2) head_logits_kernel<2, 9><<<grid, block, 0, s>>>(a);
    else head_logits_kernel<4, 9><<<grid, block, 0, s>>>(a);
  } else {
    if (nct == 1) head_logits_kernel<1, 8><<<grid, block, 0, s>>>(a);
    else if (nct == 2) head_logits_kernel<2, 8><<<grid, block, 0, s>>>(a);
    else head_logits_kernel<4, 8><<<grid, block, 0, s>>>(a);
  }
  return launch_status();
}

SPECDEC_API int specdec_head_probabilities(const void *x, int64_t x_stride, const void *w, int64_t w_stride,
                                           int64_t rows, int64_t hidden, int64_t vocab, float temperature,
                                           float *out, int64_t out_stride, int64_t *index_out, int64_t index_stride,
                                           float *logits, int64_t logits_stride, void *workspace,
                                           int64_t workspace_bytes, int32_t spin, void *stream) {
  HeadArgs a;
  const int st = head_args(x, x_stride, w, w_stride, rows, hidden, vocab, a);
  if (st != SPECDEC_OK) return st;
  if (!(temperature >= 0.0f) || spin < 0) return SPECDEC_EINVAL;
  if (rows == 0) return SPECDEC_OK;
  if (rows > kHFusedRows) return SPECDEC_EUNSUPPORTED;
  if (!out || out_stride < vocab || (logits && logits_stride < vocab)) return SPECDEC_EINVAL;
  if (!workspace || workspace_bytes < kHWsWords * (int64_t)sizeof(uint64_t) || ((uintptr_t)workspace & 7))
    return SPECDEC_EINVAL;
  HeadPlan pl;
  if (!plan_head(vocab, true, pl)) return SPECDEC_EUNSUPPORTED;
  a.tpw = pl.tpw;
  a.mode = temperature == 0.0f ? kArgmax : kSoftmax;
  a.temperature = temperature;
  a.out = out;
  a.out_stride = out_stride;
  a.index_out = index_out;
  a.index_stride = index_stride;
  a.logits = logits;
  a.logits_stride = logits_stride;
  a.ws = (uint64_t *)workspace;
  a.spin = spin;
  a.vec_out = out_stride % 4 == 0 && ((uintptr_t)out & 15) == 0;
  a.vec_logits = logits && logits_stride % 4 == 0 && ((uintptr_t)logits & 15) == 0;
  const int kb = batch_steps(a.steps);
  a.kc = chunk_steps(a.steps, 1, kb);
  dim3 grid((unsigned)pl.grid), block((unsigned)(64 * pl.tpw));
  if (kb == 9) head_softmax_kernel<9><<<grid, block, 0, as_stream(stream)>>>(a);
  else head_softmax_kernel<8><<<grid, block, 0, as_stream(stream)>>>(a);
  return launch_status();
}
