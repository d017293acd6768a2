// Prompt-lookup n-gram match (reference: spec/ngram.py:32-45).
//
// For a history ctx of length L and an n-gram size n, a match at start s
// means ctx[s : s+n] == ctx[L-n : L] with s <= L-n-1.  Writing e = s+n-1 for
// the position aligned with the last token, the reference takes the largest
// n with any match and, for it, the largest s (most recent).  So every
// position e in [0, L-2] needs only its backward agreement length
//     l(e) = max j <= max_n with ctx[e-i] == ctx[L-1-i] for all i < j,
// and best(n) = max{e : l(e) >= n, e >= n-1}.  One 1024-thread workgroup
// per row stages the history into LDS a tile of 8192 positions at a time,
// from the end, every thread's loads issued together (one memory round trip
// per tile, and a whole tile for histories up to 8193 tokens), then matches
// from LDS, keeping best(n) for every n.  Once the longest admissible n has
// matched in a tile, nothing earlier can change the answer and the scan
// stops.
#include "common.h"

namespace specdec {

constexpr int kNgramThreads = 1024;
constexpr int kNgramTile = 8192;  // positions e per tile
constexpr int kMaxN = 8;
constexpr int kNgramLoads = (kNgramTile + kMaxN - 1 + kNgramThreads - 1) / kNgramThreads;

__global__ __launch_bounds__(kNgramThreads) void ngram_lookup_kernel(
    const int32_t *__restrict__ history, int64_t row_stride, const int32_t *__restrict__ lengths,
    int32_t k, int32_t max_n, int64_t *__restrict__ draft, int32_t *__restrict__ match) {
  // ctx[base .. hi] of the current tile, base = max(lo - (kMaxN - 1), 0)
  __shared__ int32_t s_ctx[kNgramTile + kMaxN - 1];
  __shared__ int s_best[kNgramThreads / kWave][kMaxN + 1];
  __shared__ int s_tail[kMaxN];
  __shared__ int s_hit[kNgramThreads / kWave];
  __shared__ int32_t s_last;  // ctx[L - 1]
  const int64_t b = blockIdx.x;
  const int32_t *ctx = history + b * row_stride;
  const int L = lengths[b];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const int nmax = min(max_n, L - 1);  // may be <= 0: no n-gram to match
  if (L <= 0) {  // no last token to fall back on (callers reject empty histories)
    for (int i = tid; i < k; i += kNgramThreads) draft[b * k + i] = 0;
    if (tid == 0) {
      match[2 * b] = -1;
      match[2 * b + 1] = 0;
    }
    return;
  }

  if (tid < kMaxN) s_tail[tid] = (tid < nmax) ? ctx[L - 1 - tid] : 0;
  if (tid == 0) s_last = ctx[L - 1];
  int tile_base = 0, tile_hi = -1;  // ctx[tile_base .. tile_hi] is in s_ctx

  int best[kMaxN + 1];
#pragma unroll
  for (int n = 0; n <= kMaxN; ++n) best[n] = -1;

  for (int hi = L - 2; hi >= 0 && nmax > 0; hi -= kNgramTile) {
    const int lo = max(hi - kNgramTile + 1, 0);  // positions e in [lo, hi]
    const int base = max(lo - (kMaxN - 1), 0);
    const int cnt = hi - base + 1;
    int32_t v[kNgramLoads];
#pragma unroll
    for (int u = 0; u < kNgramLoads; ++u) {
      const int i = tid + u * kNgramThreads;
      v[u] = i < cnt ? ctx[base + i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kNgramLoads; ++u) {
      const int i = tid + u * kNgramThreads;
      if (i < cnt) s_ctx[i] = v[u];
    }
    __syncthreads();  // the tile (and, the first time, s_tail) is in LDS
    tile_base = base;
    tile_hi = hi;
#pragma unroll
    for (int j = 0; j < kNgramTile / kNgramThreads; ++j) {
      const int e = hi - (j * kNgramThreads + tid);
      if (e < lo) continue;
      int len = 0;
      const int cap = min(nmax, e + 1);
      while (len < cap && s_ctx[e - len - base] == s_tail[len]) ++len;
#pragma unroll
      for (int n = 1; n <= kMaxN; ++n)
        if (n <= len && e > best[n]) best[n] = e;
    }
    // has the longest n matched anywhere in this tile?
    int hit = 0;
#pragma unroll
    for (int n = 1; n <= kMaxN; ++n)
      if (n == nmax) hit = best[n] >= 0;  // constant index keeps best[] in registers
    for (int o = kWave / 2; o > 0; o >>= 1) hit |= __shfl_xor(hit, o, kWave);
    if (lane == 0) s_hit[wid] = hit;
    __syncthreads();  // also: every read of this tile's s_ctx is done
    int done = 0;
#pragma unroll
    for (int w = 0; w < kNgramThreads / kWave; ++w) done |= s_hit[w];
    if (done) break;
  }

  // reduce best(n) over the workgroup: wave max, then waves
#pragma unroll
  for (int n = 1; n <= kMaxN; ++n) {
    int x = best[n];
    for (int o = kWave / 2; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o, kWave));
    if (lane == 0) s_best[wid][n] = x;
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
    for (int i = 0; i < k; ++i) out[i] = s_last;
    match[2 * b] = -1;
    match[2 * b + 1] = 0;
    return;
  }
  // source = ctx[e+1 : L]; the copy wraps onto its own output past the end.
  // Its tokens come from the tile still in LDS (it holds e), or are ctx[L-1];
  // only a source reaching into a tile scanned before is read from memory.
  const int src = chosen_e + 1, src_len = L - src;
  for (int i = 0; i < k; ++i) {
    const int pos = src + (i % src_len);
    out[i] = pos == L - 1 ? s_last : (pos <= tile_hi ? s_ctx[pos - tile_base] : ctx[pos]);
  }
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
