// Prompt-lookup n-gram match (reference: spec/ngram.py:32-45).
//
// For a history ctx of length L and an n-gram size n, a match at start s
// means ctx[s : s+n] == ctx[L-n : L] with s <= L-n-1.  Writing e = s+n-1 for
// the position aligned with the last token, every position e in [0, L-2]
// has a backward agreement length
//     l(e) = max j <= min(max_n, L-1, e+1) with ctx[e-i] == ctx[L-1-i], i < j,
// and a match of size n ends at e iff l(e) >= n.  The reference takes the
// largest n with any match and, for it, the most recent start: that is
// n* = max_e l(e) and e* = max{e : l(e) = n*}, the largest (l(e), e) in
// lexicographic order -- one 64-bit max over positions, for any max_n.
// One 1024-thread workgroup per row stages the history into LDS a tile of
// 8192 positions at a time, from the end (every thread's loads issued
// together, with the last tokens), then compares from LDS; agreements that
// run past the staged overlap or the staged tail read ctx from memory.
// Once some position of a tile agrees over the longest admissible n,
// nothing earlier can win and the scan stops.  The first
// kNgramTile + kNgramOverlap positions of the row are requested before the
// row's length is known (a buffer whose extent is the row stride, so
// positions past it read 0): a history of up to that many tokens is then
// one tile from position 0 whose loads overlap the length's round trip, and
// its last tokens are read from the staged tile.
#include "common.h"

namespace specdec {

constexpr int kNgramThreads = 1024;
constexpr int kNgramTile = 8192;  // positions e per tile
constexpr int kNgramOverlap = 64;  // positions staged before a tile
constexpr int kNgramTail = 64;     // last tokens staged
constexpr int kNgramLoads = (kNgramTile + kNgramOverlap + kNgramThreads - 1) / kNgramThreads;

__device__ __forceinline__ long long lex_max(long long a, long long b) { return a > b ? a : b; }

__global__ __launch_bounds__(kNgramThreads) void ngram_lookup_kernel(
    const int32_t *__restrict__ history, int64_t row_stride, const int32_t *__restrict__ lengths,
    int32_t k, int32_t max_n, int64_t *__restrict__ draft, int32_t *__restrict__ match) {
  // ctx[base .. hi] of the current tile, base = max(lo - kNgramOverlap, 0)
  __shared__ int32_t s_ctx[kNgramTile + kNgramOverlap];
  __shared__ int32_t s_tail[kNgramTail];  // ctx[L - 1 - i]
  __shared__ long long s_key[kNgramThreads / kWave];
  const int64_t b = blockIdx.x;
  const int32_t *ctx = history + b * row_stride;
  const __amdgpu_buffer_rsrc_t row = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t *>(ctx), 0, (int)min(row_stride * 4, (int64_t)0x7FFFFFFC), 0x00020000);
  int32_t head[kNgramLoads];  // positions tid + u * kNgramThreads
#pragma unroll
  for (int u = 0; u < kNgramLoads; ++u)
    head[u] = __builtin_amdgcn_raw_buffer_load_b32(row, (unsigned)(threadIdx.x + u * kNgramThreads) * 4u, 0, 0);
  // a length past the row's stride is taken as the stride: no read leaves the row
  const int L = (int)min((int64_t)lengths[b], row_stride);
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

  // the whole history (last token included) is in the first tile
  const bool one_tile = L <= kNgramTile + kNgramOverlap;
  // (l, e) packed as l << 32 | e; -1: no match yet
  long long key = -1;
  int tile_base = 0, tile_hi = -1;  // ctx[tile_base .. tile_hi] is in s_ctx
  for (int hi = L - 2; hi >= 0 && nmax > 0; hi -= kNgramTile) {
    const int lo = max(hi - kNgramTile + 1, 0);  // positions e in [lo, hi]
    const int base = max(lo - kNgramOverlap, 0);
    const int cnt = hi - base + 1;
    if (tile_hi >= 0) __syncthreads();  // every read of the previous tile is done
    if (one_tile) {  // base = 0: the tile is the requested head, last token included
#pragma unroll
      for (int u = 0; u < kNgramLoads; ++u) {
        const int i = tid + u * kNgramThreads;
        if (i < kNgramTile + kNgramOverlap) s_ctx[i] = head[u];
      }
    } else {
      int32_t v[kNgramLoads];
#pragma unroll
      for (int u = 0; u < kNgramLoads; ++u) {
        const int i = tid + u * kNgramThreads;
        v[u] = i < cnt ? ctx[base + i] : 0;
      }
      int32_t tv = 0;
      if (tile_hi < 0 && tid < kNgramTail && tid < nmax) tv = ctx[L - 1 - tid];
#pragma unroll
      for (int u = 0; u < kNgramLoads; ++u) {
        const int i = tid + u * kNgramThreads;
        if (i < cnt) s_ctx[i] = v[u];
      }
      if (tile_hi < 0 && tid < kNgramTail) s_tail[tid] = tv;
    }
    __syncthreads();  // the tile (and, the first time, the tail) is in LDS
    tile_base = base;
    tile_hi = hi;
#pragma unroll
    for (int j = 0; j < kNgramTile / kNgramThreads; ++j) {
      const int e = hi - (j * kNgramThreads + tid);
      if (e < lo) continue;
      const int cap = min(nmax, e + 1);
      int len = 0;
      while (len < cap) {
        const int p = e - len;
        const int32_t x = p >= base ? s_ctx[p - base] : ctx[p];
        const int32_t y = one_tile ? s_ctx[L - 1 - len] : len < kNgramTail ? s_tail[len] : ctx[L - 1 - len];
        if (x != y) break;
        ++len;
      }
      if (len > 0) key = lex_max(key, ((long long)len << 32) | (long long)e);
    }
    if (lo == 0) break;  // the last tile: nothing earlier to skip
    // has a position of this tile agreed over the longest admissible n?
    int hit = (int)(key >> 32) == nmax;
    for (int o = kWave / 2; o > 0; o >>= 1) hit |= __shfl_xor(hit, o, kWave);
    if (lane == 0) s_key[wid] = hit;
    __syncthreads();
    int done = 0;
#pragma unroll
    for (int w = 0; w < kNgramThreads / kWave; ++w) done |= (int)s_key[w];
    if (done) break;
  }

  // the largest key over the workgroup: wave max, then waves
  for (int o = kWave / 2; o > 0; o >>= 1) key = lex_max(key, __shfl_xor(key, o, kWave));
  __syncthreads();  // s_key's hit flags are read
  if (lane == 0) s_key[wid] = key;
  __syncthreads();
  if (wid != 0) return;
  // wave 0: every lane takes the workgroup's key; lane i writes proposal i
  key = -1;
#pragma unroll
  for (int w = 0; w < kNgramThreads / kWave; ++w) key = lex_max(key, s_key[w]);
  // (staged only when a tile was scanned: none for a one-token history or max_n 0)
  const int32_t last = one_tile && tile_hi >= 0 ? s_ctx[L - 1] : ctx[L - 1];
  int64_t *out = draft + b * k;
  if (key < 0) {
    for (int i = lane; i < k; i += kWave) out[i] = last;
    if (lane == 0) {
      match[2 * b] = -1;
      match[2 * b + 1] = 0;
    }
    return;
  }
  const int chosen_n = (int)(key >> 32), chosen_e = (int)(key & 0xFFFFFFFF);
  // source = ctx[e+1 : L]; the copy wraps onto its own output past the end.
  // Its tokens come from the tile still in LDS (it holds e), or are ctx[L-1];
  // only a source reaching into a tile scanned before is read from memory.
  const int src = chosen_e + 1, src_len = L - src;
  for (int i = lane; i < k; i += kWave) {
    const int pos = src + (i % src_len);
    out[i] = pos == L - 1 ? last : (pos <= tile_hi ? s_ctx[pos - tile_base] : ctx[pos]);
  }
  if (lane == 0) {
    match[2 * b] = chosen_e - chosen_n + 1;
    match[2 * b + 1] = chosen_n;
  }
}

}  // namespace specdec

using namespace specdec;

SPECDEC_API int specdec_ngram_lookup(const int32_t *history, int64_t row_stride,
                                     const int32_t *lengths, int64_t batch, int32_t k,
                                     int32_t max_n, int64_t *draft, int32_t *match,
                                     void *stream) {
  if (batch < 0 || k < 0 || max_n < 0) return SPECDEC_EINVAL;
  if (batch == 0) return SPECDEC_OK;
  if (!history || !lengths || !match || (k > 0 && !draft)) return SPECDEC_EINVAL;
  ngram_lookup_kernel<<<dim3((unsigned)batch), dim3(kNgramThreads), 0, as_stream(stream)>>>(
      history, row_stride, lengths, k, max_n, draft, match);
  return launch_status();
}
