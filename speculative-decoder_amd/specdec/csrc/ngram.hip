// Prompt-lookup n-gram match (reference: spec/ngram.py:32-45).
//
// For a history ctx of length L and an n-gram size n, a match at start s
// means ctx[s : s+n] == ctx[L-n : L] with s <= L-n-1.  Writing e = s+n-1 for
// the position aligned with the last token, the reference takes the largest
// n with any match and, for it, the largest s (most recent).  So every
// position e in [0, L-2] needs only its backward agreement length
//     l(e) = max j <= max_n with ctx[e-i] == ctx[L-1-i] for all i < j,
// and best(n) = max{e : l(e) >= n, e >= n-1}.  One workgroup per row scans e
// from the end of the history in tiles, keeping best(n) for every n; once
// the longest admissible n has matched, nothing earlier can change the
// answer and the scan stops.
#include "common.h"

namespace specdec {

constexpr int kNgramThreads = 256;
constexpr int kNgramPerThread = 4;  // positions per thread per tile
constexpr int kMaxN = 8;

__global__ __launch_bounds__(kNgramThreads) void ngram_lookup_kernel(
    const int32_t *__restrict__ history, int64_t row_stride, const int32_t *__restrict__ lengths,
    int32_t k, int32_t max_n, int64_t *__restrict__ draft, int32_t *__restrict__ match) {
  __shared__ int s_best[kNgramThreads / kWave][kMaxN + 1];
  __shared__ int s_tail[kMaxN];
  __shared__ int s_done;
  const int64_t b = blockIdx.x;
  const int32_t *ctx = history + b * row_stride;
  const int L = lengths[b];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const int nmax = min(max_n, L - 1);  // may be <= 0: no n-gram to match

  if (tid < kMaxN) s_tail[tid] = (tid < nmax) ? ctx[L - 1 - tid] : 0;
  if (tid == 0) s_done = 0;
  __syncthreads();

  int best[kMaxN + 1];
#pragma unroll
  for (int n = 0; n <= kMaxN; ++n) best[n] = -1;

  constexpr int tile = kNgramThreads * kNgramPerThread;
  for (int hi = L - 2; hi >= 0 && nmax > 0; hi -= tile) {
#pragma unroll
    for (int j = 0; j < kNgramPerThread; ++j) {
      const int e = hi - (j * kNgramThreads + tid);
      if (e < 0) continue;
      int len = 0;
      const int cap = min(nmax, e + 1);
      while (len < cap && ctx[e - len] == s_tail[len]) ++len;
#pragma unroll
      for (int n = 1; n <= kMaxN; ++n)
        if (n <= len && e > best[n]) best[n] = e;
    }
    // publish whether the longest n has matched anywhere in this tile
    int hit = 0;
#pragma unroll
    for (int n = 1; n <= kMaxN; ++n)
      if (n == nmax) hit = best[n] >= 0;  // constant index keeps best[] in registers
    for (int o = kWave / 2; o > 0; o >>= 1) hit |= __shfl_xor(hit, o, kWave);
    if (lane == 0 && hit) s_done = 1;
    __syncthreads();
    const int done = s_done;
    __syncthreads();
    if (done) break;
  }

  // reduce best(n) over the workgroup: wave max, then waves
#pragma unroll
  for (int n = 1; n <= kMaxN; ++n) {
    int v = best[n];
    for (int o = kWave / 2; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, kWave));
    if (lane == 0) s_best[wid][n] = v;
  }
  __syncthreads();
  if (tid != 0) return;
  int chosen_n = 0, chosen_e = -1;
  for (int n = nmax; n >= 1; --n) {
    int e = -1;
    for (int w = 0; w < kNgramThreads / kWave; ++w) e = max(e, s_best[w][n]);
    if (e >= 0) { chosen_n = n; chosen_e = e; break; }
  }
  int64_t *out = draft + b * k;
  if (chosen_n == 0) {
    const int last = ctx[L - 1];
    for (int i = 0; i < k; ++i) out[i] = last;
    match[2 * b] = -1;
    match[2 * b + 1] = 0;
    return;
  }
  // source = ctx[e+1 : L]; the copy wraps onto its own output past the end
  const int src = chosen_e + 1, src_len = L - src;
  for (int i = 0; i < k; ++i) out[i] = ctx[src + (i % src_len)];
  match[2 * b] = chosen_e - chosen_n + 1;
  match[2 * b + 1] = chosen_n;
}

}  // namespace specdec

using namespace specdec;

SPECDEC_API int specdec_ngram_lookup(const int32_t *history, int64_t row_stride,
                                     const int32_t *lengths, int64_t batch, int32_t k,
                                     int32_t max_n, int64_t *draft, int32_t *match,
                                     void *stream) {
  if (batch < 0 || k < 0 || max_n < 0) return SPECDEC_EINVAL;
  if (max_n > kMaxN) return SPECDEC_EUNSUPPORTED;
  if (batch == 0) return SPECDEC_OK;
  if (!history || !lengths || !match || (k > 0 && !draft)) return SPECDEC_EINVAL;
  ngram_lookup_kernel<<<dim3((unsigned)batch), dim3(kNgramThreads), 0, as_stream(stream)>>>(
      history, row_stride, lengths, k, max_n, draft, match);
  return launch_status();
}
