// Causal paged verify attention on gfx950 MFMA.
//
// Reference semantics: lm/forward.py:44-49 (positions and the mask
// "key j visible to query t iff j <= past+t and j < total") and :62-63
// (gather of every cached K/V, then scaled_dot_product_attention).  Here the
// blocks are read in place through the block table.
//
// Work split: grid.x = (batch, kv head, 16-row query tile), grid.y = KV
// split of `split` tokens; 4 waves per workgroup, each wave walking its
// quarter of the split in 32-token chunks (two 16-token groups).
//
// Per chunk and wave, with lane = 16*g + c (g = lane/16, c = lane%16):
//   S^T[token, query] = K . Q^T      A = K rows (token c, dims 32kk+8g..+7)
//                                    B = Q^T    (query c, same dims)
//   D layout: lane holds S^T[4g+i, c], i = 0..3, i.e. 4 tokens of query c
//   online softmax per query column (fp32), p = exp(s - m)
//   O^T[dim, query] += V^T . P^T     A = V^T rows (dim c+16t, tokens of g)
//                                    B = P^T (the lane's own 8 p values)
// The MFMA k index of lane group g is mapped to tokens {4g..4g+3} of the
// first group and {4g..4g+3} of the second, so P^T comes straight out of the
// S^T accumulators and V^T is read as two 8-byte runs from the dim-major V
// tile.  All per-query statistics live in lane column c, so the running
// rescale is lane-local.
//
// Splits write (O / l, lse) partials to a workspace; a second small kernel
// (attention_combine_kernel), launched right after on the same stream,
// folds them per (batch, head, tile).  With 2 to 4 splits one 16-wave
// workgroup per tile runs all of them and folds them in LDS with the same
// arithmetic, so short contexts (decode, the draft) need one launch.  So
// does a tiled call (5 to 12 splits, a tile for every CU): one 16-wave
// workgroup per tile whose four wave groups take its splits in rounds,
// every wave keeping each split's softmax state in LDS with no barrier
// until the last; the fold then follows the split kernel's and the combine
// kernel's arithmetic.
// Every query's reduction order depends only on the absolute key positions,
// never on how many queries share the call, so a token verified among k+1
// gets the same bits as the same token decoded alone.
#include "common.h"

#include <math.h>

#include <mutex>

namespace specdec {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

constexpr int kD = 64;            // head dim
constexpr int kAttnThreads = 256;  // 4 waves
constexpr int kRows = 16;          // query rows per tile
constexpr int kDefaultSplit = 512;
constexpr int kPart = kRows * (kD + 1);  // floats per split partial: O/l [16][64], lse [16]
constexpr int kStage = 16;  // appended tokens per workgroup taken from LDS
// Tiled calls (one 16-wave workgroup per tile, wave groups taking splits in
// rounds): splits and live query rows whose per-wave softmax states fit LDS
constexpr int kTSplits = 12, kTRows = 8;

struct AttnArgs {
  const void *q;
  int64_t q_stride;
  // fused RoPE + append (rope != 0): q points at qkv; q heads are rotated in
  // registers and the new tokens' k (rotated) and v are written to k/v
  int rope;
  const float *cos_t;
  const float *sin_t;
  // input RMSNorm finished here (rope calls only; null: q/k/v are already
  // normalised): hidden [batch, width, hdim] bf16 is the residual stream the
  // q/k/v projection read, its norm weight folded into the projection
  const void *hidden;
  int hdim;
  float eps;
  const void *k;
  const void *v;
  const int32_t *tables;
  int64_t table_stride;
  const int32_t *meta;
  int batch, width, H, Hkv, bs;
  float scale;
  int split, max_splits, n_qtiles;
  int max_kv;  // the call's max_kv_len: no row may hold more keys
  // split partial slots per unit in the workspace (1 when no combine runs)
  int parts;
  // 16-wave launches only: one split over every key, wave w taking the
  // 64-token steps w, w+16, ... (results need not match other calls)
  int flat;
  // 16-wave launches only: every split of the tile, wave group grp taking
  // splits grp, grp + 4, ... (at most kTSplits splits, kTRows live rows)
  int tiled;
  float *ws;
  void *out;
  int64_t out_stride;
};

struct TileInfo {
  int b, h, qt, group, row, past, nnew, nrows, kv_len, nsplit, unit;
  bool overflow;  // the tile's keys pass the call's max_kv_len
};

// A unit's coordinates from the grid alone (no memory read): query tile,
// kv head, batch entry, query heads per kv head.
__device__ __forceinline__ void tile_coords(const AttnArgs &a, int unit, TileInfo &ti) {
  ti.unit = unit;
  ti.qt = unit % a.n_qtiles;
  const int bh = unit / a.n_qtiles;
  ti.h = bh % a.Hkv;
  ti.b = bh / a.Hkv;
  ti.group = a.H / a.Hkv;
}

// The row metadata of a unit whose coordinates are set; false when the
// tile holds no live query row (or its keys pass max_kv_len: ti.overflow).
// The three words are read through the constant address space (the host
// writes them before the launch), as one scalar round trip that vector
// loads issued earlier do not hold up.
__device__ __forceinline__ bool tile_meta(const AttnArgs &a, TileInfo &ti, bool any_split) {
  typedef const __attribute__((address_space(4))) int32_t const_i32;
  const_i32 *meta = (const_i32 *)a.meta;
  ti.row = meta[ti.b];
  ti.past = meta[a.batch + ti.b];
  ti.nnew = meta[2 * a.batch + ti.b];
  // the empty asm uses all three here, so none of the loads is sunk past
  // the early exits below into a round trip of its own
  __asm__ volatile("" ::"s"(ti.row), "s"(ti.past), "s"(ti.nnew));
  ti.nrows = ti.nnew * ti.group;
  ti.overflow = false;
  const int r0 = ti.qt * kRows;
  if (r0 >= ti.nrows) return false;
  const int t_hi = min(r0 + kRows - 1, ti.nrows - 1) / ti.group;
  ti.kv_len = ti.past + t_hi + 1;
  ti.nsplit = (ti.kv_len + a.split - 1) / a.split;
  ti.overflow = ti.kv_len > a.max_kv || ti.nsplit > a.max_splits;
  if (ti.overflow) return false;
  if (!any_split && (int)blockIdx.y >= ti.nsplit) return false;
  return true;
}

__device__ __forceinline__ bool tile_info_at(const AttnArgs &a, int unit, TileInfo &ti, bool any_split) {
  tile_coords(a, unit, ti);
  return tile_meta(a, ti, any_split);
}

__device__ __forceinline__ bool tile_info(const AttnArgs &a, TileInfo &ti, bool any_split = false) {
  return tile_info_at(a, blockIdx.x, ti, any_split);
}

__device__ __forceinline__ int64_t block_of(const AttnArgs &a, const TileInfo &ti, int pos) {
  return a.tables[(int64_t)ti.row * a.table_stride + pos / a.bs];
}

// Fused append: this workgroup writes kv head h of every new token whose
// position lies in [lo, hi) -- its own split -- rotated k and plain v, into
// the paged pools, before it reads any key.  Workgroups whose ranges
// overlap write identical values.
template <typename T>
__device__ void append_new_kv(const AttnArgs &a, const TileInfo &ti, int lo, int hi) {
  const int p0 = max(lo, ti.past), p1 = min(hi, ti.past + ti.nnew);
  if (p0 >= p1) return;
  const int half = kD / 2;
  const T *qkv = reinterpret_cast<const T *>(a.q);
  T *kp = reinterpret_cast<T *>(const_cast<void *>(a.k));
  T *vp = reinterpret_cast<T *>(const_cast<void *>(a.v));
  const int n = (p1 - p0) * half;
  for (int task = threadIdx.x; task < n; task += blockDim.x) {
    const int pos = p0 + task / half, i = task % half;
    const int t = pos - ti.past;
    const T *x = qkv + ((int64_t)ti.b * a.width + t) * a.q_stride;
    const T *kx = x + (int64_t)(a.H + ti.h) * kD;
    const T *vx = x + (int64_t)(a.H + a.Hkv + ti.h) * kD;
    float y1, y2;
    rope_pair(to_f32(kx[i]), to_f32(kx[i + half]), a.cos_t[(int64_t)pos * half + i], a.sin_t[(int64_t)pos * half + i],
              y1, y2);
    const int64_t blk = a.tables[(int64_t)ti.row * a.table_stride + pos / a.bs];
    const int off = pos % a.bs;
    T *kd = kp + ((blk * a.Hkv + ti.h) * a.bs + off) * kD;
    kd[i] = from_f32<T>(y1);
    kd[i + half] = from_f32<T>(y2);
    T *vd = vp + (blk * a.Hkv + ti.h) * (int64_t)kD * a.bs + off;
    vd[(int64_t)i * a.bs] = vx[i];
    vd[(int64_t)(i + half) * a.bs] = vx[i + half];
  }
}

// Statistics are in the log2 domain: a wave's (m, l, o) mean
// o / l = sum_j 2^(t_j - m) v_j / sum_j 2^(t_j - m), with t_j the score times
// scale * log2(e).  Waves hand them over in LDS as s_m/s_l [wave][query] and
// s_o [wave][query][dim].

// Fold of waves w0 .. w0+n-1 (n = N unless given) for query row qq, dims
// d0 .. d0+3 (R rows per wave in LDS).  A wave that saw no key holds
// (-inf, 0, 0) and adds nothing: leaving it out of n changes no bit.
template <int N = 4, int R = kRows>
__device__ __forceinline__ void fold_waves(const float (*s_m)[R], const float (*s_l)[R],
                                           const float (*s_o)[R][kD + 4], int w0, int qq, int d0, float &M,
                                           float &L, float (&O)[4], int n = N) {
  M = s_m[w0][qq];
  for (int w = 1; w < n; ++w) M = fmaxf(M, s_m[w0 + w][qq]);
  L = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) O[i] = 0.0f;
  for (int w = 0; w < n; ++w) {
    const float mw = s_m[w0 + w][qq];
    const float f = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
    L = __builtin_fmaf(f, s_l[w0 + w][qq], L);
#pragma unroll
    for (int i = 0; i < 4; ++i) O[i] = __builtin_fmaf(f, s_o[w0 + w][qq][d0 + i], O[i]);
  }
}

template <typename T>
__device__ __forceinline__ void store_row4(const AttnArgs &a, const TileInfo &ti, int qq, int d0, const float (&v)[4]) {
  const int r = ti.qt * kRows + qq;
  const int t = r / ti.group, hq = ti.h * ti.group + r % ti.group;
  T *dst = reinterpret_cast<T *>(a.out) + ((int64_t)ti.b * a.width + t) * a.out_stride + (int64_t)hq * kD + d0;
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = from_f32<T>(v[i]);
}

// A row whose cached length exceeds the call's max_kv_len (a caller broke
// the contract): its tile's output rows are set to NaN by the tile's first
// workgroup, so the error shows instead of stale output.
template <typename T>
__device__ void poison_tile(const AttnArgs &a, const TileInfo &ti) {
  if (!ti.overflow || blockIdx.y != 0 || threadIdx.x >= 256) return;
  const int qq = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 4;
  if (ti.qt * kRows + qq >= ti.nrows) return;
  const float nan4[4] = {NAN, NAN, NAN, NAN};
  store_row4<T>(a, ti, qq, d0, nan4);
}

// Fold of the 4 waves of a 256-thread workgroup through LDS: thread
// (qq = tid / 16, d0 = 4 * (tid % 16)) receives (M, L, O) of query row qq,
// dims d0 .. d0+3.  Ends with a barrier, so the LDS can be reused.
__device__ __forceinline__ void fold_wg4(float m, float l, const f32x4 (&o)[4], float &M, float &L, float (&O)[4]) {
  __shared__ float s_m[4][kRows], s_l[4][kRows];
  __shared__ float s_o[4][kRows][kD + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  if (g == 0) {
    s_m[wave][c] = m;
    s_l[wave][c] = l;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_o[wave][c][16 * t + 4 * g + i] = o[t][i];
  __syncthreads();
  fold_waves(s_m, s_l, s_o, 0, tid >> 4, (tid & 15) * 4, M, L, O);
  __syncthreads();
}

// A split's folded (M, L, O) for one thread's row and dims: the output when
// the tile has one split, else the split partial (O / l, lse = m + log2 l)
// in workspace slot `slot` for the combine kernel.
template <typename T>
__device__ __forceinline__ void write_split(const AttnArgs &a, const TileInfo &ti, int slot, int qq, int d0, float M,
                                            float L, const float (&O)[4]) {
  if (ti.nsplit == 1) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = O[i] / L;
    store_row4<T>(a, ti, qq, d0, v);
    return;
  }
  float *ws = a.ws + ((int64_t)ti.unit * a.parts + slot) * kPart;
  const bool any = L > 0.0f;
  f32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = any ? O[i] / L : 0.0f;
  *reinterpret_cast<f32x4 *>(ws + qq * kD + d0) = v;
  if (d0 == 0) ws[kRows * kD + qq] = any ? M + __builtin_amdgcn_logf(L) : -INFINITY;
}

// Combine the 4 waves of a one-split workgroup (grid.y = split).
template <typename T>
__device__ void finish(const AttnArgs &a, const TileInfo &ti, float m, float l, const f32x4 (&o)[4]) {
  float M, L, O[4];
  fold_wg4(m, l, o, M, L, O);
  const int qq = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 4;
  if (qq < min(kRows, ti.nrows - ti.qt * kRows)) write_split<T>(a, ti, blockIdx.y, qq, d0, M, L, O);
}

// Folds the split partials s0 .. s0+G-1 that lie below ns into the running
// (Mx, den, num): the group's largest lse rescales what is accumulated, then
// each split adds w = 2^(lse - Mx) times its O / l row, in split order.
// The combine kernel (G = 4 per group, then G = 8 over groups) and the
// single-workgroup path below (G = 4, at most 4 splits) use it; splits past ns take no part, so for a
// query with at most 4 splits both run the same operations in the same
// order and the result does not depend on which of them ran.
template <int G>
__device__ __forceinline__ void fold_splits(int s0, int ns, const float (&lse)[G], const f32x4 (&ov)[G], float &Mx,
                                            float &den, float (&num)[4]) {
  float Mg = Mx;
#pragma unroll
  for (int u = 0; u < G; ++u)
    if (s0 + u < ns) Mg = fmaxf(Mg, lse[u]);
  if (Mg > Mx) {  // rescale what is accumulated to the new maximum
    const float r = (Mx == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(Mx - Mg);
    den *= r;
#pragma unroll
    for (int i = 0; i < 4; ++i) num[i] *= r;
    Mx = Mg;
  }
#pragma unroll
  for (int u = 0; u < G; ++u) {
    if (s0 + u < ns && lse[u] != -INFINITY) {
      const float w = __builtin_amdgcn_exp2f(lse[u] - Mx);
      den += w;
#pragma unroll
      for (int i = 0; i < 4; ++i) num[i] = __builtin_fmaf(w, ov[u][i], num[i]);
    }
  }
}

// First level of the fold tree: up to four consecutive split partials
// folded into the group's (O / l, lse).
__device__ __forceinline__ void group_partial(int n, const float (&lse)[4], const f32x4 (&ov)[4], float &glse,
                                              f32x4 &gov) {
  float m4 = -INFINITY, d4 = 0.0f, n4[4] = {0.f, 0.f, 0.f, 0.f};
  fold_splits(0, n, lse, ov, m4, d4, n4);
  const bool any = d4 > 0.0f;
  glse = any ? m4 + __builtin_amdgcn_logf(d4) : -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) gov[i] = any ? n4[i] / d4 : 0.0f;
}

// Final combine of the split partials, one workgroup per (row, head, tile)
// with more than one split.  The fold tree depends only on the key
// positions: splits are folded in groups of four (4 consecutive splits,
// fold_splits<4>), each group becomes (O / l, lse) like a split, and
// the groups are folded in order, eight per step (fold_splits<8>).  A tile
// with at most four splits is run by one 16-wave workgroup that folds its
// single group the same way, so a query gets the same bits on either path;
// splits or groups holding none of a query's keys take no part.  Thread
// (q, 4 dims) does the folding.  The first NG groups' loads (4 * NG splits,
// NG = min(8, groups of the longest tile)) are issued before the row
// metadata arrives, since their addresses depend only on the workgroup;
// groups NG .. 7 of the first step lie past every tile's last split and are
// skipped by the fold as they would be with all eight loaded.
template <int NG>
__global__ __launch_bounds__(kAttnThreads) void attention_combine_kernel(AttnArgs a, int dtype) {
  constexpr int NL = 4 * NG;
  const int tid = threadIdx.x;
  const int qq = tid >> 4, d0 = (tid & 15) * 4;
  // rows past width * (H / Hkv) exist in no batch entry: nothing to load
  if ((int)(blockIdx.x % a.n_qtiles) * kRows + qq >= a.width * (a.H / a.Hkv)) return;
  const float *ws0 = a.ws + (int64_t)blockIdx.x * a.parts * kPart;
  float lse[32];
  f32x4 ov[32];
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const float *p = ws0 + (int64_t)min(u, a.parts - 1) * kPart;
    lse[u] = p[kRows * kD + qq];
    ov[u] = *reinterpret_cast<const f32x4 *>(p + qq * kD + d0);
  }
  TileInfo ti;
  if (!tile_info(a, ti, /*any_split=*/true) || ti.nsplit == 1) return;
  const int nq = min(kRows, ti.nrows - ti.qt * kRows);
  if (qq >= nq) return;
  const int ns = ti.nsplit, ngroups = (ns + 3) / 4;
  float Mx = -INFINITY, den = 0.0f, num[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < ns; s0 += 32) {
    if (s0 > 0) {  // only when NG == 8
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        const float *p = ws0 + (int64_t)min(s0 + u, ns - 1) * kPart;
        lse[u] = p[kRows * kD + qq];
        ov[u] = *reinterpret_cast<const f32x4 *>(p + qq * kD + d0);
      }
    }
    float gl[8];
    f32x4 gv[8];
#pragma unroll
    for (int y = 0; y < 8; ++y) {
      if (y >= NG) {  // past ngroups: fold_splits skips it
        gl[y] = -INFINITY;
        gv[y] = f32x4{0.f, 0.f, 0.f, 0.f};
        continue;
      }
      const int n_y = min(max(ns - (s0 + 4 * y), 0), 4);
      float l4[4];
      f32x4 v4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        l4[u] = lse[4 * y + u];
        v4[u] = ov[4 * y + u];
      }
      group_partial(n_y, l4, v4, gl[y], gv[y]);
    }
    fold_splits(s0 / 4, ngroups, gl, gv, Mx, den, num);
  }
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = num[i] / den;
  if (dtype == SPECDEC_BF16) store_row4<__hip_bfloat16>(a, ti, qq, d0, v);
  else store_row4<float>(a, ti, qq, d0, v);
}

// finish() of a 16-wave bf16 workgroup running every split of its tile (at
// most four): each group of four waves folds into its split partial exactly
// as finish() does, the partials meet in LDS and group 0 folds them with
// fold_splits<4> -- the first level of the combine kernel's fold tree, whose
// result for a single group is the same bits.  With a.flat (one split over
// every key, results that need not match other calls) all 16 waves fold
// straight into the output.
// LDS floats of finish_grouped, carved from the kernel's pool.
constexpr int kGroupedFloats = 32 * kRows + 16 * kRows * (kD + 4) + 4 * kRows * kD + 4 * kRows;
template <typename T>
__device__ void finish_grouped(const AttnArgs &a, const TileInfo &ti, float m, float l, const f32x4 (&o)[4],
                               float *pool) {
  float(*s_m)[kRows] = reinterpret_cast<float(*)[kRows]>(pool);
  float(*s_l)[kRows] = reinterpret_cast<float(*)[kRows]>(pool + 16 * kRows);
  float(*s_o)[kRows][kD + 4] = reinterpret_cast<float(*)[kRows][kD + 4]>(pool + 32 * kRows);
  float *pv0 = pool + 32 * kRows + 16 * kRows * (kD + 4);
  float(*s_pv)[kRows][kD] = reinterpret_cast<float(*)[kRows][kD]>(pv0);
  float(*s_pl)[kRows] = reinterpret_cast<float(*)[kRows]>(pv0 + 4 * kRows * kD);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  if (g == 0) {
    s_m[wave][c] = m;
    s_l[wave][c] = l;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_o[wave][c][16 * t + 4 * g + i] = o[t][i];
  __syncthreads();

  const int grp = wave >> 2, w0 = 4 * grp;
  const int qq = (tid & 255) >> 4, d0 = (tid & 15) * 4;
  const int nq = min(kRows, ti.nrows - ti.qt * kRows);
  float M, L, O[4];
  if (a.flat) {
    if (grp == 0 && qq < nq) {
      // wave w's first step starts at key 64 w: the waves past the tile's
      // keys saw none
      fold_waves<16>(s_m, s_l, s_o, 0, qq, d0, M, L, O, max(1, min(16, (ti.kv_len + 63) / 64)));
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = O[i] / L;
      store_row4<T>(a, ti, qq, d0, v);
    }
    return;
  }
  fold_waves(s_m, s_l, s_o, w0, qq, d0, M, L, O);
  if (ti.nsplit == 1) {  // uniform: the direct path of finish()
    if (grp == 0 && qq < nq) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = O[i] / L;
      store_row4<T>(a, ti, qq, d0, v);
    }
    return;
  }
  if (grp < ti.nsplit) {
    const bool any = L > 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s_pv[grp][qq][d0 + i] = any ? O[i] / L : 0.0f;
    if (d0 == 0) s_pl[grp][qq] = any ? M + __builtin_amdgcn_logf(L) : -INFINITY;
  }
  __syncthreads();
  if (grp == 0 && qq < nq) {
    float lse[4];
    f32x4 ov[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int sp = min(u, ti.nsplit - 1);
      lse[u] = s_pl[sp][qq];
      ov[u] = *reinterpret_cast<const f32x4 *>(&s_pv[sp][qq][d0]);
    }
    float Mx = -INFINITY, den = 0.0f, num[4] = {0.f, 0.f, 0.f, 0.f};
    fold_splits(0, ti.nsplit, lse, ov, Mx, den, num);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = num[i] / den;
    store_row4<T>(a, ti, qq, d0, v);
  }
}

// Tiled calls: each wave's (m, l, O) of one split, rows < kTRows, kept in
// LDS slot 4 * split + (wave & 3) until every wave is done -- no barrier
// between splits, so the tile's waves run free.
constexpr int kTiledFloats = kTSplits * 4 * kTRows * (2 + kD + 4);
__device__ __forceinline__ void keep_wave_state(float *pool, int split, float m, float l, const f32x4 (&o)[4]) {
  float(*st_m)[kTRows] = reinterpret_cast<float(*)[kTRows]>(pool);
  float(*st_l)[kTRows] = reinterpret_cast<float(*)[kTRows]>(pool + kTSplits * 4 * kTRows);
  float(*st_o)[kTRows][kD + 4] = reinterpret_cast<float(*)[kTRows][kD + 4]>(pool + 2 * kTSplits * 4 * kTRows);
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int slot = 4 * split + ((threadIdx.x >> 6) & 3);
  if (c < kTRows) {
    if (g == 0) {
      st_m[slot][c] = m;
      st_l[slot][c] = l;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) st_o[slot][c][16 * t + 4 * g + i] = o[t][i];
  }
}

// After the last split of a tiled call: each split's four wave states are
// folded as fold_wg4 folds them, turned into the partial write_split would
// write, and the partials folded with the combine kernel's tree, so a query
// gets the bits it gets from the split kernel and the combine.
template <typename T>
__device__ void fold_tiled(const AttnArgs &a, const TileInfo &ti, const float *pool) {
  const float(*st_m)[kTRows] = reinterpret_cast<const float(*)[kTRows]>(pool);
  const float(*st_l)[kTRows] = reinterpret_cast<const float(*)[kTRows]>(pool + kTSplits * 4 * kTRows);
  const float(*st_o)[kTRows][kD + 4] =
      reinterpret_cast<const float(*)[kTRows][kD + 4]>(pool + 2 * kTSplits * 4 * kTRows);
  __syncthreads();
  const int tid = threadIdx.x;
  const int qq = tid >> 4, d0 = (tid & 15) * 4;
  const int nq = min(kRows, ti.nrows - ti.qt * kRows);
  if (tid >= 256 || qq >= nq) return;
  const int ns = ti.nsplit, ngroups = (ns + 3) / 4;
  float gl[8];
  f32x4 gv[8];
#pragma unroll
  for (int y = 0; y < 8; ++y) {
    const int n_y = min(max(ns - 4 * y, 0), 4);
    gl[y] = -INFINITY;
    gv[y] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (4 * y >= kTSplits || n_y == 0) continue;
    float l4[4];
    f32x4 v4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int sp = min(4 * y + u, ns - 1);
      float M, L, O[4];
      fold_waves<4, kTRows>(st_m + 4 * sp, st_l + 4 * sp, st_o + 4 * sp, 0, qq, d0, M, L, O);
      const bool any = L > 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) v4[u][i] = any ? O[i] / L : 0.0f;
      l4[u] = any ? M + __builtin_amdgcn_logf(L) : -INFINITY;
    }
    group_partial(n_y, l4, v4, gl[y], gv[y]);
  }
  float Mx = -INFINITY, den = 0.0f, num[4] = {0.f, 0.f, 0.f, 0.f};
  fold_splits(0, ngroups, gl, gv, Mx, den, num);
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = num[i] / den;
  store_row4<T>(a, ti, qq, d0, v);
}

// Online-softmax update over N scores per lane (t = score * scale * log2 e,
// -inf where not visible), replaced by their weights 2^(t - m).
template <int N>
__device__ __forceinline__ void online_update(float (&sv)[N], float &m, float &l, f32x4 (&o)[4]) {
  float cm = sv[0];
#pragma unroll
  for (int j = 1; j < N; ++j) cm = fmaxf(cm, sv[j]);
  cm = fmaxf(cm, __shfl_xor(cm, 16, 64));
  cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
  const float m_new = fmaxf(m, cm);
  const float alpha = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - m_new);
  const float mu = (m_new == -INFINITY) ? 0.0f : m_new;
  float ps = 0.0f;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    sv[j] = __builtin_amdgcn_exp2f(sv[j] - mu);
    ps += sv[j];
  }
  ps += __shfl_xor(ps, 16, 64);
  ps += __shfl_xor(ps, 32, 64);
  l = l * alpha + ps;
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] *= alpha;
  m = m_new;
}

// ---------------------------------------------------------------- bf16 ----
// MODE 1: block_size == 16 (constant arithmetic); MODE 2: block_size % 16 == 0;
// MODE 0: any block size (per-token addressing).
//
// Within a 32-token chunk starting at cs, MFMA half hf (0, 1) gives lane c
// the K row of token cs + 8*(c/4) + 4*hf + c%4.  The S^T accumulator row
// 4g+i of half hf is then token cs + 8g + 4hf + i, so lane group g holds the
// scores of the 8 consecutive tokens cs+8g .. cs+8g+7 and reads their V^T
// as one 16-byte run per dim.
// Four waves per SIMD (<= 128 VGPRs): enough resident waves to keep HBM
// busy at batch 8 and beyond.
//
// NW = 4: one split per workgroup (grid.y = split), partials folded by the
// combine kernel.  NW = 16: one workgroup runs all (at most four) splits of
// its tile, four waves each, and folds them in LDS (finish_grouped) -- no
// combine launch, same bits; or, with a.flat, one split over every key with
// all 16 waves striding it; or, TILED, all of a tile's 5 to 12 splits in
// rounds of four (keep_wave_state, fold_tiled), same bits again.
// PF (4 waves, 512-token splits, few workgroups): two waves per SIMD, so a
// wave holds both of its steps' K/V at once -- their loads go out together
// and the steps are computed in the same order (same bits, one memory
// round trip fewer).
template <int MODE, int NW, bool TILED = false, bool PF = false>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(PF ? 2 : 4, PF ? 2 : 4))) void
attention_bf16_kernel(
    AttnArgs a) {
  typedef unsigned short u16;
  constexpr int kThreads = NW * kWave;
  constexpr int kKT = (kStage * (kD / 2) + kThreads - 1) / kThreads;  // k pairs per thread
  constexpr int kVT = (kStage * kD + kThreads - 1) / kThreads;        // v elements per thread
  TileInfo ti;
  tile_coords(a, blockIdx.x, ti);
  // ---- loads that need the grid coordinates only, in flight while the
  // row metadata is read: the q rows of the call's tokens (rows past a
  // row's new tokens are dropped below), and with 16 waves (one workgroup
  // takes every new token of its rows) the new tokens' hidden rows for the
  // norm and their k / v values for the append
  const int tid0 = threadIdx.x, lane0 = tid0 & 63;
  const int r_call = ti.qt * kRows + (lane0 & 15);
  const bool r_in = r_call < a.width * ti.group;
  u32x4 qraw[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  if (r_in) {
    const u16 *qr = reinterpret_cast<const u16 *>(a.q) +
                    ((int64_t)ti.b * a.width + r_call / ti.group) * a.q_stride +
                    (int64_t)(ti.h * ti.group + r_call % ti.group) * kD + 8 * (lane0 >> 4);
    qraw[0] = *reinterpret_cast<const u32x4 *>(qr);
    qraw[1] = *reinterpret_cast<const u32x4 *>(qr + 32);
  }
  const bool pre_norm = NW == 16 && MODE != 0 && a.hidden && a.hdim <= 4 * kWave * 8;
  const int pre_tok = tid0 >> 6;
  u32x4 hv_pre[4];
  if (pre_norm && pre_tok < min(a.width, kStage)) {
    const int nvec = a.hdim / 8;
    const u32x4 *hr = reinterpret_cast<const u32x4 *>(a.hidden) + ((int64_t)ti.b * a.width + pre_tok) * nvec;
#pragma unroll
    for (int k = 0; k < 4; ++k) hv_pre[k] = hr[min(lane0 + kWave * k, nvec - 1)];
  }
  const bool pre_kv = NW == 16 && MODE != 0 && a.rope && a.width <= kStage;
  u16 sk1[kKT], sk2[kKT], svv[kVT];
  if (pre_kv) {
    const u16 *qkv16 = reinterpret_cast<const u16 *>(a.q);
#pragma unroll
    for (int u = 0; u < kKT; ++u) {
      const int task = tid0 + u * kThreads;
      if (task < a.width * (kD / 2)) {
        const int tk = task / (kD / 2), i = task % (kD / 2);
        const u16 *kx = qkv16 + ((int64_t)ti.b * a.width + tk) * a.q_stride + (int64_t)(a.H + ti.h) * kD;
        sk1[u] = kx[i];
        sk2[u] = kx[i + kD / 2];
      }
    }
    // v token-fastest (task -> token task % width, dim task / width), the
    // order its dim-major pool tile is stored in below
#pragma unroll
    for (int u = 0; u < kVT; ++u) {
      const int task = tid0 + u * kThreads;
      if (task < a.width * kD) {
        const int tk = task % a.width, dd = task / a.width;
        svv[u] = qkv16[((int64_t)ti.b * a.width + tk) * a.q_stride + (int64_t)(a.H + a.Hkv + ti.h) * kD + dd];
      }
    }
  }
  if (!tile_meta(a, ti, /*any_split=*/NW == 16)) {
    poison_tile<__hip_bfloat16>(a, ti);
    return;
  }
  const bool flat = NW == 16 && a.flat;
  const int tid = threadIdx.x, lane = tid & 63, wave = flat ? (tid >> 6) : ((tid >> 6) & 3);
  int split_idx = (NW == 16) ? (flat ? 0 : (tid >> 8)) : (int)blockIdx.y;
  const int wstride = flat ? 16 * 64 : 4 * 64;  // tokens between a wave's steps
  const int g = lane >> 4, c = lane & 15;
  const int r = ti.qt * kRows + c;
  const bool row_ok = r < ti.nrows;
  const int t = row_ok ? r / ti.group : 0;
  const int hq = ti.h * ti.group + (row_ok ? r % ti.group : 0);
  const int qpos = ti.past + t;

  const u16 *kp = reinterpret_cast<const u16 *>(a.k);
  const u16 *vp = reinterpret_cast<const u16 *>(a.v);

  const int Hkv = a.Hkv;
  const float c2 = a.scale * 1.4426950408889634f;  // scores in log2 units
  const int bs = (MODE == 1) ? 16 : a.bs;
  const int64_t tile_elems = (int64_t)bs * kD;  // one (block, head) tile
  const int32_t *trow = a.tables + (int64_t)ti.row * a.table_stride;
  const int kv_len = ti.kv_len;
  const int last_blk = (kv_len - 1) / bs;
  // wave w takes the 64-token steps w, w+4, w+8, ... of its split (none
  // when the split lies past this tile's keys); flat: w, w+16, ...
  int s_lo = split_idx * a.split;
  int s_hi = min(s_lo + a.split, kv_len);
  int c_first = s_lo + 64 * wave;

  // Fused append.  The new tokens of this workgroup's key range [lo, hi)
  // are rotated once into LDS (and written to the pools for later calls);
  // the key loop takes them from LDS instead of the pool, so no pool store
  // has to complete before the first key load.  More than kStage of them
  // (a long prefill) take the plain path: append, fence, then read.
  const int lo = (NW == 16) ? 0 : split_idx * a.split;
  const int hi = (NW == 16) ? ti.nsplit * a.split : lo + a.split;
  const int p0 = max(lo, ti.past), p1 = min(hi, ti.past + ti.nnew);
  const int n_in = max(p1 - p0, 0);
  const bool staged = MODE != 0 && a.rope && n_in <= kStage;
  // tokens per dim in the staged v tasks' token-fastest order: the row's
  // width when the values were loaded before the metadata (then p0 = past)
  const int vw = pre_kv ? a.width : max(n_in, 1);
  __shared__ __align__(16) u16 s_nk[kStage][kD];
  __shared__ __align__(16) u16 s_nv[kStage][kD];
  // 16 waves: the LDS of finish_grouped, or of a tiled call's wave states
  constexpr int kPool = NW != 16 ? 4 : TILED ? kTiledFloats : kGroupedFloats;
  __shared__ __align__(16) float s_pool[kPool];

  // ---- prologue: every load here depends on the row metadata only, so
  // all of them are in flight together
  // this wave's first-step block ids: lane j (j = lane & 3) holds the block
  // of tokens c0 + 16j .. c0 + 16j + 15
  int bj = 0, bj1 = 0;  // bj1: the second step's (PF)
  if (MODE != 0 && c_first < s_hi) bj = trow[min((c_first + 16 * (lane & 3)) / bs, last_blk)];
  if (PF && c_first + wstride < s_hi) bj1 = trow[min((c_first + wstride + 16 * (lane & 3)) / bs, last_blk)];
  // k halves kept as raw bf16 bits until the rotation, so no wait for them
  // comes before the q and cos/sin loads below are issued (with 16 waves
  // they are in flight already: pos - past of a task is its token index)
  float scs[kKT], ssn[kKT];
  int skb[kKT], svb[kVT];
  const u16 *qkv16 = reinterpret_cast<const u16 *>(a.q);
  auto new_row = [&](int pos) { return qkv16 + ((int64_t)ti.b * a.width + (pos - ti.past)) * a.q_stride; };
  if (staged) {
#pragma unroll
    for (int u = 0; u < kKT; ++u) {
      const int task = tid + u * kThreads;
      if (task < n_in * (kD / 2)) {
        const int pos = p0 + task / (kD / 2), i = task % (kD / 2);
        if (!pre_kv) {
          const u16 *kx = new_row(pos) + (int64_t)(a.H + ti.h) * kD;
          sk1[u] = kx[i];
          sk2[u] = kx[i + kD / 2];
        }
        scs[u] = a.cos_t[(int64_t)pos * (kD / 2) + i];
        ssn[u] = a.sin_t[(int64_t)pos * (kD / 2) + i];
        skb[u] = trow[pos / bs];
      }
    }
#pragma unroll
    for (int u = 0; u < kVT; ++u) {
      const int task = tid + u * kThreads;
      const int t = task % vw, dd = task / vw;  // token-fastest
      if (task < vw * kD && t < n_in) {
        const int pos = p0 + t;
        if (!pre_kv) svv[u] = new_row(pos)[(int64_t)(a.H + Hkv + ti.h) * kD + dd];
        svb[u] = trow[pos / bs];
      }
    }
  }

  // Q operand: lane (query c, group g) holds dims 8g..8g+7 (kk = 0) and
  // 32+8g..32+8g+7 (kk = 1) -- the two halves of 8 RoPE pairs
  // (loaded above for the call's rows; zeros for rows past the row's new
  // tokens, as those lanes never load)
  bf16x8 qop[2];
  {
    const u32x4 zero = {0u, 0u, 0u, 0u};
    qop[0] = __builtin_bit_cast(bf16x8, row_ok ? qraw[0] : zero);
    qop[1] = __builtin_bit_cast(bf16x8, row_ok ? qraw[1] : zero);
  }
  // the rotation's cos/sin, loaded before the norm's barrier below
  float qcs[8], qsn[8];
  if (a.rope && row_ok) {
    const float *cs = a.cos_t + (int64_t)qpos * (kD / 2) + 8 * g;
    const float *sn = a.sin_t + (int64_t)qpos * (kD / 2) + 8 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) qcs[j] = cs[j], qsn[j] = sn[j];
  }

  // Input RMSNorm finished here (a.hidden): q, k and v come from a
  // projection of the unnormalised residual stream, so each new token's
  // values are scaled by s = rsqrt(mean(hidden^2) + eps) of its row, rounded
  // to bf16 as a projection's output is, before RoPE.  Wave w reduces tokens
  // w, w + NW, ... (the host allows at most kStage new tokens): lane l adds
  // the row's 16-byte vectors l, l+64, ... in order, then wave_sum_dpp -- one
  // fixed order, so every workgroup of every call gets the same s for a
  // token, and the same s the MLP's norm kernel computes for a row.
  __shared__ float s_tok[kStage];
  const bool norm_in = MODE != 0 && a.hidden;  // the host sends no other
  if (norm_in) {
    const int nvec = a.hdim / 8;
    const int ntok = min(min(ti.nnew, a.width), kStage);
    for (int tk = tid >> 6; tk < ntok; tk += NW) {
      const u32x4 *hr = reinterpret_cast<const u32x4 *>(a.hidden) + ((int64_t)ti.b * a.width + tk) * nvec;
      float ss = 0.0f;
      for (int base = 0; base < nvec; base += 4 * kWave) {
        u32x4 hv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          hv[k] = (pre_norm && base == 0) ? hv_pre[k] : hr[min(base + lane + kWave * k, nvec - 1)];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const bool in = base + lane + kWave * k < nvec;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const unsigned w = hv[k][e >> 1];
            const float x = __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
            ss += in ? x * x : 0.0f;
          }
        }
      }
      ss = wave_sum_dpp(ss);
      if (lane == 0) s_tok[tk] = rsqrtf(ss / (float)a.hdim + a.eps);
    }
    __syncthreads();
  }
  // v * s rounded to bf16 (raw bits in and out)
  auto scaled_bits = [&](u16 bits, float sc) -> u16 {
    return __builtin_bit_cast(u16, from_f32<__hip_bfloat16>(sc * to_f32(__builtin_bit_cast(__hip_bfloat16, bits))));
  };

  if (a.rope && row_ok) {
    const float sq = norm_in ? s_tok[t] : 1.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float x1 = (float)qop[0][j], x2 = (float)qop[1][j], y1, y2;
      if (norm_in) x1 = (float)(__bf16)(sq * x1), x2 = (float)(__bf16)(sq * x2);
      rope_pair(x1, x2, qcs[j], qsn[j], y1, y2);
      qop[0][j] = (__bf16)y1;
      qop[1][j] = (__bf16)y2;
    }
  }

  if (staged) {
    u16 *kpw = const_cast<u16 *>(kp);
#pragma unroll
    for (int u = 0; u < kKT; ++u) {
      const int task = tid + u * kThreads;
      if (task < n_in * (kD / 2)) {
        const int pos = p0 + task / (kD / 2), i = task % (kD / 2);
        if (norm_in) {
          const float st = s_tok[pos - ti.past];
          sk1[u] = scaled_bits(sk1[u], st);
          sk2[u] = scaled_bits(sk2[u], st);
        }
        float y1, y2;
        rope_pair(to_f32(__builtin_bit_cast(__hip_bfloat16, sk1[u])), to_f32(__builtin_bit_cast(__hip_bfloat16, sk2[u])),
                  scs[u], ssn[u], y1, y2);
        const u16 b1 = __builtin_bit_cast(u16, from_f32<__hip_bfloat16>(y1));
        const u16 b2 = __builtin_bit_cast(u16, from_f32<__hip_bfloat16>(y2));
        s_nk[pos - p0][i] = b1;
        s_nk[pos - p0][i + kD / 2] = b2;
        u16 *kd = kpw + ((int64_t)skb[u] * Hkv + ti.h) * tile_elems + (int64_t)(pos % bs) * kD;
        kd[i] = b1;
        kd[i + kD / 2] = b2;
      }
    }
    // V token-fastest: its pool tile is dim-major (a 32-byte row of 16
    // slots per dim), so the lanes of one dim store consecutive slots of
    // its row, not one token's dims 32 bytes apart in separate lanes
    u16 *vpw = const_cast<u16 *>(vp);
#pragma unroll
    for (int u = 0; u < kVT; ++u) {
      const int task = tid + u * kThreads;
      const int t = task % vw, dd = task / vw;
      if (task < vw * kD && t < n_in) {
        const int pos = p0 + t;
        if (norm_in) svv[u] = scaled_bits(svv[u], s_tok[pos - ti.past]);
        s_nv[t][dd] = svv[u];
        vpw[((int64_t)svb[u] * Hkv + ti.h) * tile_elems + (int64_t)dd * bs + pos % bs] = svv[u];
      }
    }
  }
  if (a.rope) {
    if (!staged) {
      append_new_kv<__hip_bfloat16>(a, ti, lo, hi);
      __threadfence_block();
    }
    __syncthreads();
  }

  // element offset of the (block, head) tile holding token pos
  auto tile_of = [&](int pos) -> int64_t { return ((int64_t)trow[pos / bs] * Hkv + ti.h) * tile_elems; };
  f32x4 o[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) o[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  // K/V operands of one 64-token step
  struct StepRegs {
    u32x4 k[2][2][2];  // [chunk][half][kk]
    u32x4 v[2][4];     // [chunk][dim tile]
  };
  // this lane's block ids for the step at c0 (lane j & 3: tokens c0 + 16j ..)
  auto step_blocks = [&](int c0) -> int { return trow[min((c0 + 16 * (lane & 3)) / bs, last_blk)]; };
  // issue every K/V load of the step at c0; bjv holds its block ids
  auto issue = [&](int c0, int bjv, StepRegs &r) {
    // tile offsets of the step's four 16-token groups (MODE != 0), uniform
    // across the wave; a lane picks between two of them with a select (a
    // dynamically indexed array would be placed in memory)
    int64_t tofs0 = 0, tofs1 = 0, tofs2 = 0, tofs3 = 0;
    if (MODE != 0) {
      tofs0 = ((int64_t)__builtin_amdgcn_readlane(bjv, 0) * Hkv + ti.h) * tile_elems;
      tofs1 = ((int64_t)__builtin_amdgcn_readlane(bjv, 1) * Hkv + ti.h) * tile_elems;
      tofs2 = ((int64_t)__builtin_amdgcn_readlane(bjv, 2) * Hkv + ti.h) * tile_elems;
      tofs3 = ((int64_t)__builtin_amdgcn_readlane(bjv, 3) * Hkv + ti.h) * tile_elems;
    }
    auto group_tile = [&](int ch, bool upper) -> int64_t {
      return ch == 0 ? (upper ? tofs1 : tofs0) : (upper ? tofs3 : tofs2);
    };
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      const int cs = c0 + 32 * ch;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int tok = cs + 8 * (c >> 2) + 4 * hf + (c & 3);
        const bool ok = (MODE == 0) ? tok < kv_len : (tok / bs) * bs < kv_len;
        const bool fresh = staged && tok >= p0 && tok < p1;  // appended by this call: from LDS
        r.k[ch][hf][0] = r.k[ch][hf][1] = u32x4{0u, 0u, 0u, 0u};
        if (ok && !fresh) {
          const int64_t to = (MODE != 0) ? group_tile(ch, (c >> 3) != 0) : tile_of(tok);
          const u16 *kb = kp + to + (int64_t)(tok % bs) * kD + 8 * g;
          r.k[ch][hf][0] = *reinterpret_cast<const u32x4 *>(kb);
          r.k[ch][hf][1] = *reinterpret_cast<const u32x4 *>(kb + 32);
        }
      }
      const int vt = cs + 8 * g;  // first of this lane group's 8 tokens
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) r.v[ch][tt] = u32x4{0u, 0u, 0u, 0u};
      if (MODE != 0) {
        if ((vt / bs) * bs < kv_len) {
          const u16 *vb = vp + group_tile(ch, (g >> 1) != 0) + vt % bs;
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            r.v[ch][tt] = *reinterpret_cast<const u32x4 *>(vb + (int64_t)(16 * tt + c) * bs);
        }
      } else {
        unsigned int w[4][4] = {};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int pos = vt + i;
          if (pos >= kv_len) continue;
          const u16 *vb = vp + tile_of(pos) + pos % bs;
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            w[tt][i >> 1] |= (unsigned)vb[(int64_t)(16 * tt + c) * bs] << (16 * (i & 1));
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) r.v[ch][tt] = u32x4{w[tt][0], w[tt][1], w[tt][2], w[tt][3]};
      }
    }
  };
  // keys appended by this call: K rows and V elements from LDS, then the
  // step's scores, online softmax and P V
  auto compute = [&](int c0, StepRegs &r) {
    if (staged && c0 + 64 > p0 && c0 < p1) {
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        const int cs = c0 + 32 * ch;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int tok = cs + 8 * (c >> 2) + 4 * hf + (c & 3);
          if (tok >= p0 && tok < p1) {
            r.k[ch][hf][0] = *reinterpret_cast<const u32x4 *>(&s_nk[tok - p0][8 * g]);
            r.k[ch][hf][1] = *reinterpret_cast<const u32x4 *>(&s_nk[tok - p0][32 + 8 * g]);
          }
        }
        const int vt = cs + 8 * g;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int pos = vt + i;
          if (pos >= p0 && pos < p1) {
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
              const unsigned sh = 16 * (i & 1);
              const unsigned wd = r.v[ch][tt][i >> 1];
              r.v[ch][tt][i >> 1] = (wd & ~(0xFFFFu << sh)) | ((unsigned)s_nv[pos - p0][16 * tt + c] << sh);
            }
          }
        }
      }
    }
    // scores of both chunks (S^T = K Q^T), in log2 units
    float sv[16];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[ch][hf][0]), qop[0], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[ch][hf][1]), qop[1], sc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[8 * ch + 4 * hf + i] = sc[i] * c2;
      }
    }
    // keys past a query's position (or past kv_len) only occur in chunks
    // reaching beyond `past`; elsewhere every score is visible
    if (c0 + 64 > ti.past) {
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int pos = c0 + 32 * ch + 8 * g + j;
          if (!(row_ok && pos <= qpos && pos < kv_len)) sv[8 * ch + j] = -INFINITY;
        }
    }
    online_update<16>(sv, m, l, o);
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      bf16x8 pop;
#pragma unroll
      for (int j = 0; j < 8; ++j) pop[j] = (__bf16)sv[8 * ch + j];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.v[ch][tt]), pop, o[tt], 0, 0, 0);
    }
  };

  // tiled: wave group grp runs splits grp, grp + 4, ... one after another,
  // keeping each split's state in LDS without waiting for the other waves
  constexpr bool tiled = NW == 16 && TILED;
  const int rounds = tiled ? (ti.nsplit + 3) / 4 : 1;
  for (int round = 0;; ++round) {
    if constexpr (PF) {  // at most two steps per wave
      if (c_first < s_hi) {
        const bool two = c_first + wstride < s_hi;
        StepRegs r0, r1;
        issue(c_first, bj, r0);
        if (two) issue(c_first + wstride, bj1, r1);
        compute(c_first, r0);
        if (two) compute(c_first + wstride, r1);
      }
    } else {
      for (int c0 = c_first; c0 < s_hi; c0 += wstride) {
        StepRegs r;
        issue(c0, bj, r);
        // next step's block ids, in flight during this step's arithmetic
        if (MODE != 0 && c0 + wstride < s_hi) bj = step_blocks(c0 + wstride);
        compute(c0, r);
      }
    }
    if (!tiled) break;
    keep_wave_state(s_pool, split_idx, m, l, o);
    if (round + 1 >= rounds) break;
    split_idx += 4;
    s_lo = split_idx * a.split;
    s_hi = min(s_lo + a.split, kv_len);
    c_first = s_lo + 64 * wave;
    if (MODE != 0 && c_first < s_hi) bj = step_blocks(c_first);
    m = -INFINITY;
    l = 0.0f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) o[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if constexpr (NW != 16) finish<__hip_bfloat16>(a, ti, m, l, o);
  else if constexpr (tiled) fold_tiled<__hip_bfloat16>(a, ti, s_pool);
  else finish_grouped<__hip_bfloat16>(a, ti, m, l, o, s_pool);
}

// ------------------------------------------------------------- decode -----
// Latency decode steps of one new token per row (the draft model's steps,
// split_tokens < 0: results that need not match other calls), bf16, block
// size a multiple of 16, q/k/v from the fused projection, at most 16 query
// heads per kv head.  A (row, kv head)'s keys are taken by 4 waves, wave w
// taking the 64-token steps w, w+4, ... two at a time with both steps'
// loads in flight (decode_wave); the waves are either one workgroup that
// folds them in LDS (attention_decode_kernel) or four one-wave workgroups on
// four compute units that write their (m, l, O) for the output projection to
// fold (attention_decode_parts_kernel).  Compared with the 16-wave flat grid
// it takes no barrier before its fold:
//   - the loads that need only the grid coordinates (q, the new token's k
//     and v, the residual row for the input norm) go out before the row
//     metadata is read (decode_early);
//   - every wave computes the norm scale itself (the same lane order for
//     all), rotates q and the new k in registers and takes the new token's
//     K and V from registers inside its step (the pool copy is written for
//     later calls, not read back).
struct DecodeEarly {
  u32x4 qraw[2];
  u32x4 kraw0, kraw1;
  unsigned short vraw[4];
  u32x4 hv[4];
  const u32x4 *hr;
};

__device__ __forceinline__ void decode_early(const AttnArgs &a, const TileInfo &ti, int lane, DecodeEarly &e) {
  typedef unsigned short u16;
  const int g = lane >> 4, c = lane & 15;
  const u16 *xrow = reinterpret_cast<const u16 *>(a.q) + (int64_t)ti.b * a.width * a.q_stride;
  e.qraw[0] = e.qraw[1] = u32x4{0u, 0u, 0u, 0u};
  if (c < ti.group) {
    const u16 *qr = xrow + (int64_t)(ti.h * ti.group + c) * kD + 8 * g;
    e.qraw[0] = *reinterpret_cast<const u32x4 *>(qr);
    e.qraw[1] = *reinterpret_cast<const u32x4 *>(qr + 32);
  }
  const u16 *kx = xrow + (int64_t)(a.H + ti.h) * kD + 8 * g;
  e.kraw0 = *reinterpret_cast<const u32x4 *>(kx);
  e.kraw1 = *reinterpret_cast<const u32x4 *>(kx + 32);
  const u16 *vx = xrow + (int64_t)(a.H + a.Hkv + ti.h) * kD + c;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) e.vraw[tt] = vx[16 * tt];
  const int nvh = a.hdim / 8;
  e.hr = a.hidden ? reinterpret_cast<const u32x4 *>(a.hidden) + (int64_t)ti.b * a.width * nvh : nullptr;
  if (a.hidden) row_pass_loads<4>(e.hr, 0, nvh, lane, e.hv);
}

// Wave w (of nwaves) of kv head ti.h, row metadata read: its (m, l, O)
// over the 64-token steps w, w + nwaves, ...  `writer`: this wave writes the
// new token's K and V to the pools (one wave per (row, kv head) of the
// launch).
template <int MODE>
__device__ __forceinline__ void decode_wave(const AttnArgs &a, const TileInfo &ti, int wave, int nwaves, bool writer,
                                            const DecodeEarly &e, float &m, float &l, f32x4 (&o)[4]) {
  typedef unsigned short u16;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  const bool row_in = c < ti.group;  // this lane's query row exists (one token per row)
  const bool norm_in = a.hidden != nullptr;
  const int p = ti.past;  // the new token's position, and the query's
  const int kv_len = ti.kv_len;
  const int bs = (MODE == 1) ? 16 : a.bs;
  const int Hkv = a.Hkv;
  const int64_t tile_elems = (int64_t)bs * kD;
  const int32_t *trow = a.tables + (int64_t)ti.row * a.table_stride;
  const int last_blk = (kv_len - 1) / bs;
  const u16 *kp = reinterpret_cast<const u16 *>(a.k);
  const u16 *vp = reinterpret_cast<const u16 *>(a.v);
  // the first two steps' block ids (lane j & 3: tokens c0 + 16j ..), RoPE tables at p
  const int kPair = 64 * nwaves;  // tokens from a wave's first step to its second
  const int c_first = 64 * wave;
  auto step_blocks = [&](int c0) -> int { return trow[min((c0 + 16 * (lane & 3)) / bs, last_blk)]; };
  int bj0 = 0, bj1 = 0;
  if (c_first < kv_len) bj0 = step_blocks(c_first);
  if (c_first + kPair < kv_len) bj1 = step_blocks(c_first + kPair);
  float cs8[8], sn8[8];
  {
    const float *cs = a.cos_t + (int64_t)p * (kD / 2) + 8 * g;
    const float *sn = a.sin_t + (int64_t)p * (kD / 2) + 8 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) cs8[j] = cs[j], sn8[j] = sn[j];
  }
  // ---- the input norm's scale, RoPE of q and of the new k (registers)
  const float sc = norm_in ? row_rms_scale_bf16_from<4>(e.hr, e.hv, a.hdim / 8, a.hdim, a.eps, lane) : 1.0f;
  auto scaled = [&](unsigned short bits) -> float {
    const float x = __uint_as_float((unsigned)bits << 16);
    return norm_in ? to_f32(from_f32<__hip_bfloat16>(sc * x)) : x;
  };
  auto half_of = [](const u32x4 &v, int j) -> unsigned short {
    return (unsigned short)((j & 1) ? (v[j >> 1] >> 16) : (v[j >> 1] & 0xFFFFu));
  };
  bf16x8 qop[2], knew[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float y1, y2;
    rope_pair(scaled(half_of(e.qraw[0], j)), scaled(half_of(e.qraw[1], j)), cs8[j], sn8[j], y1, y2);
    qop[0][j] = row_in ? (__bf16)y1 : (__bf16)0.0f;
    qop[1][j] = row_in ? (__bf16)y2 : (__bf16)0.0f;
    rope_pair(scaled(half_of(e.kraw0, j)), scaled(half_of(e.kraw1, j)), cs8[j], sn8[j], y1, y2);
    knew[0][j] = (__bf16)y1;
    knew[1][j] = (__bf16)y2;
  }
  u16 vnew[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
    vnew[tt] = norm_in ? __builtin_bit_cast(u16, from_f32<__hip_bfloat16>(sc * __uint_as_float((unsigned)e.vraw[tt] << 16)))
                       : e.vraw[tt];
  // the pool copy of the new token, for later calls
  const int64_t pblk = trow[p / bs];
  if (writer) {
    const int64_t ptile = (pblk * Hkv + ti.h) * tile_elems;
    if (c == 0) {
      u16 *kd = const_cast<u16 *>(kp) + ptile + (int64_t)(p % bs) * kD + 8 * g;
      *reinterpret_cast<u32x4 *>(kd) = __builtin_bit_cast(u32x4, knew[0]);
      *reinterpret_cast<u32x4 *>(kd + 32) = __builtin_bit_cast(u32x4, knew[1]);
    }
    if (g == 0) {
      u16 *vd = const_cast<u16 *>(vp) + ptile + p % bs;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) vd[(int64_t)(16 * tt + c) * bs] = vnew[tt];
    }
  }
  struct StepRegs {
    u32x4 k[2][2][2];  // [chunk][half][kk]
    u32x4 v[2][4];     // [chunk][dim tile]
  };
  auto issue = [&](int c0, int bjv, StepRegs &r) {
    const int64_t t0 = ((int64_t)__builtin_amdgcn_readlane(bjv, 0) * Hkv + ti.h) * tile_elems;
    const int64_t t1 = ((int64_t)__builtin_amdgcn_readlane(bjv, 1) * Hkv + ti.h) * tile_elems;
    const int64_t t2 = ((int64_t)__builtin_amdgcn_readlane(bjv, 2) * Hkv + ti.h) * tile_elems;
    const int64_t t3 = ((int64_t)__builtin_amdgcn_readlane(bjv, 3) * Hkv + ti.h) * tile_elems;
    auto group_tile = [&](int ch, bool upper) -> int64_t { return ch == 0 ? (upper ? t1 : t0) : (upper ? t3 : t2); };
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      const int cs = c0 + 32 * ch;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int tok = cs + 8 * (c >> 2) + 4 * hf + (c & 3);
        r.k[ch][hf][0] = r.k[ch][hf][1] = u32x4{0u, 0u, 0u, 0u};
        if ((tok / bs) * bs < kv_len) {
          const u16 *kb = kp + group_tile(ch, (c >> 3) != 0) + (int64_t)(tok % bs) * kD + 8 * g;
          r.k[ch][hf][0] = *reinterpret_cast<const u32x4 *>(kb);
          r.k[ch][hf][1] = *reinterpret_cast<const u32x4 *>(kb + 32);
        }
      }
      const int vt = cs + 8 * g;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) r.v[ch][tt] = u32x4{0u, 0u, 0u, 0u};
      if ((vt / bs) * bs < kv_len) {
        const u16 *vb = vp + group_tile(ch, (g >> 1) != 0) + vt % bs;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) r.v[ch][tt] = *reinterpret_cast<const u32x4 *>(vb + (int64_t)(16 * tt + c) * bs);
      }
    }
  };
  const float c2 = a.scale * 1.4426950408889634f;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) o[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  m = -INFINITY;
  l = 0.0f;
  auto compute = [&](int c0, StepRegs &r) {
    if (c0 + 64 > p) {  // the step holding the new token: its K and V from registers
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        const int cs = c0 + 32 * ch;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int tok = cs + 8 * (c >> 2) + 4 * hf + (c & 3);
          if (tok == p) {
            r.k[ch][hf][0] = __builtin_bit_cast(u32x4, knew[0]);
            r.k[ch][hf][1] = __builtin_bit_cast(u32x4, knew[1]);
          }
        }
        const int i = p - (cs + 8 * g);
        if (i >= 0 && i < 8) {
          const unsigned sh = 16 * (i & 1);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
            for (int w = 0; w < 4; ++w)
              if (w == (i >> 1)) r.v[ch][tt][w] = (r.v[ch][tt][w] & ~(0xFFFFu << sh)) | ((unsigned)vnew[tt] << sh);
          }
        }
      }
    }
    float sv[16];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[ch][hf][0]), qop[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[ch][hf][1]), qop[1], acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[8 * ch + 4 * hf + i] = acc[i] * c2;
      }
    }
    if (c0 + 64 > p) {  // keys past the query (the new token is the last key)
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (!(row_in && c0 + 32 * ch + 8 * g + j <= p)) sv[8 * ch + j] = -INFINITY;
    } else if (!row_in) {
#pragma unroll
      for (int j = 0; j < 16; ++j) sv[j] = -INFINITY;
    }
    online_update<16>(sv, m, l, o);
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      bf16x8 pop;
#pragma unroll
      for (int j = 0; j < 8; ++j) pop[j] = (__bf16)sv[8 * ch + j];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.v[ch][tt]), pop, o[tt], 0, 0, 0);
    }
  };
  // two steps at a time (c0 and c0 + kPair), both steps' loads in flight
  for (int c0 = c_first; c0 < kv_len; c0 += 2 * kPair) {
    const bool two = c0 + kPair < kv_len;
    StepRegs r0, r1;
    issue(c0, bj0, r0);
    if (two) issue(c0 + kPair, bj1, r1);
    if (c0 + 2 * kPair < kv_len) bj0 = step_blocks(c0 + 2 * kPair);
    if (c0 + 3 * kPair < kv_len) bj1 = step_blocks(c0 + 3 * kPair);
    compute(c0, r0);
    if (two) compute(c0 + kPair, r1);
  }
}

// One 4-wave workgroup per (row, kv head): the waves fold in LDS.
template <int MODE>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_decode_kernel(
    AttnArgs a) {
  TileInfo ti;
  tile_coords(a, blockIdx.x, ti);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  DecodeEarly e;
  decode_early(a, ti, lane, e);
  if (!tile_meta(a, ti, /*any_split=*/true)) {
    poison_tile<__hip_bfloat16>(a, ti);
    return;
  }
  float m, l;
  f32x4 o[4];
  decode_wave<MODE>(a, ti, wave, kDecWaves, /*writer=*/wave == 0, e, m, l, o);
  float M, L, O[4];
  fold_wg4(m, l, o, M, L, O);
  const int qq = tid >> 4, d0 = (tid & 15) * 4;
  if (qq < ti.group) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = O[i] / L;
    store_row4<__hip_bfloat16>(a, ti, qq, d0, v);
  }
}

// NP (4, 8 or 16) one-wave workgroups per (row, kv head), on as many
// compute units (one CU issuing all of a head's K/V loads is what bounds the
// 4-wave kernel; with a part per 64-token step no wave waits for a second
// step): workgroup w runs wave w of decode_wave and writes its (m, l, O), O
// not divided by l, for the rows of its kv head to parts [batch, H, NP,
// kDecPart] floats (m, l, two unused, then O's 64 dims).  Folding a row's parts in
// order with fold_waves' arithmetic and rounding O / L to bf16
// (linear_parts_kernel's prologue) gives, for kDecWaves parts, the bits of
// attention_decode_kernel's output.  A row past max_kv_len gets a partial
// that folds to NaN; a row without a new token gets none.
template <int MODE, int NP>
__global__ __launch_bounds__(kWave) void attention_decode_parts_kernel(AttnArgs a, float *parts) {
  TileInfo ti;
  const int wave = blockIdx.x % NP;
  tile_coords(a, blockIdx.x / NP, ti);
  const int lane = threadIdx.x, g = lane >> 4, c = lane & 15;
  DecodeEarly e;
  decode_early(a, ti, lane, e);
  float m = -INFINITY, l = 0.0f;
  f32x4 o[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) o[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (tile_meta(a, ti, /*any_split=*/true)) {
    decode_wave<MODE>(a, ti, wave, NP, /*writer=*/wave == 0, e, m, l, o);
  } else {
    if (!ti.overflow) return;
    m = 0.0f;
    l = NAN;
  }
  if (c < ti.group) {
    float *dst = parts + (((int64_t)ti.b * a.H + ti.h * ti.group + c) * NP + wave) * kDecPart;
    if (g == 0) {
      dst[0] = m;
      dst[1] = l;
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) *reinterpret_cast<f32x4 *>(dst + 4 + 16 * tt + 4 * g) = o[tt];
  }
}

// ------------------------------------------------------------- prefill ----
// Wide bf16 calls (more than kStage new tokens per row: a prompt), with the
// new K/V already in the pools (rope_append ran first, or the caller wrote
// them).  One 8-wave workgroup per (row, kv head, eight consecutive 16-row
// query tiles); each wave owns one tile.  The workgroup walks its keys in
// 128-token stages: each stage's K and V tiles (8 pool tiles of 16 tokens,
// 32 KB) are staged into LDS once, with coalesced 16-byte loads issued two
// stages ahead (three LDS buffers: a stage's loads have two stages' compute
// to arrive in), two 64-token steps per stage; every wave reads its MFMA
// operands from LDS, and a wave whose queries end before a step skips it.  Online softmax in registers, then O / l.  No split partials,
// no cross-wave fold.  Per step and wave the arithmetic is the decode
// kernel's (K rows permuted so P^T comes out of the S^T accumulators); the
// fold order differs from the split kernels', so prefill rows need not equal
// the bits a decode step of the same token would get (nothing compares
// them: every path prefills with this kernel).
constexpr int kPrefillTiles = 8;                     // query tiles (waves) per workgroup
constexpr int kPrefillThreads = kPrefillTiles * kWave;
constexpr int kPKStride = kD + 8;                    // bf16 per staged K row (token): 144 bytes
constexpr int kPVStride = 16 + 8;                    // bf16 per staged V row (dim of a 16-token group): 48 bytes
constexpr int kPStage = 128;                         // tokens per staged stage
constexpr int kPGroups = kPStage / 16;               // 16-token groups per stage
constexpr int kPKElems = kPStage * kPKStride;        // one stage's K
constexpr int kPVElems = kPGroups * kD * kPVStride;  // one stage's V: [group][dim][token]
constexpr int kPUnits = 2 * kPGroups * 128 / kPrefillThreads;  // 16-byte staging units per thread

template <int MODE>
__global__ __launch_bounds__(kPrefillThreads) void attention_prefill_kernel(AttnArgs a) {
  __shared__ __align__(16) unsigned short s_k[3][kPKElems];
  __shared__ __align__(16) unsigned short s_v[3][kPVElems];
  typedef unsigned short u16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int nqb = (a.n_qtiles + kPrefillTiles - 1) / kPrefillTiles;
  const int qb = blockIdx.x % nqb, bh = blockIdx.x / nqb;
  const int qt = qb * kPrefillTiles + wave;
  // this wave's tile; a wave without one (past the tiles, or rows past the
  // row's new tokens) still stages and meets the barriers
  TileInfo ti;
  const bool live = qt < a.n_qtiles && tile_info_at(a, bh * a.n_qtiles + qt, ti, /*any_split=*/true);
  if (!live && qt < a.n_qtiles && ti.overflow && ti.qt * kRows + c < ti.nrows) {
    // beyond max_kv_len: NaN rows, as the other kernels
    const int rr = ti.qt * kRows + c, tr = rr / ti.group, hr = ti.h * ti.group + rr % ti.group;
    __hip_bfloat16 *dst =
        reinterpret_cast<__hip_bfloat16 *>(a.out) + ((int64_t)ti.b * a.width + tr) * a.out_stride + (int64_t)hr * kD;
#pragma unroll
    for (int i = 0; i < 16; ++i) dst[16 * g + i] = from_f32<__hip_bfloat16>(NAN);
  }
  // the workgroup's key range: up to its first wave's tile's row metadata
  // and the last live tile's last query
  TileInfo t0;
  if (!tile_info_at(a, bh * a.n_qtiles + qb * kPrefillTiles, t0, /*any_split=*/true)) return;  // no live tile
  // (tiles whose keys would pass max_kv_len took the NaN branch above)
  const int last_qt = min(qb * kPrefillTiles + kPrefillTiles - 1, (t0.nrows - 1) / kRows);
  const int t_last = min(min(last_qt * kRows + kRows - 1, t0.nrows - 1) / t0.group,
                         a.max_kv - 1 - t0.past);
  const int wg_kv = t0.past + t_last + 1;
  const int bs = (MODE == 1) ? 16 : a.bs;
  const int Hkv = a.Hkv;
  const int32_t *trow = a.tables + (int64_t)t0.row * a.table_stride;
  const int last_blk = (wg_kv - 1) / bs;
  const u16 *kp = reinterpret_cast<const u16 *>(a.k);
  const u16 *vp = reinterpret_cast<const u16 *>(a.v);
  const int64_t tile_elems = (int64_t)bs * kD;

  // staging: thread tid takes 16-byte units tid + 512 i of the stage's
  // 2048 (units 0..1023: K, 8 groups x 16 tokens x 8; 1024..2047: V, 8
  // groups x 64 dims x 2): groups tid / 128 and tid / 128 + 4, the same for
  // a whole wave, so their block ids are scalar loads (counted apart from
  // the vector loads: waiting for an id never waits for staged data)
  u32x4 stg_a[kPUnits], stg_b[kPUnits];
  const int grp_lo = __builtin_amdgcn_readfirstlane(tid >> 7);
  // the table is not written while the kernel runs: read through the
  // constant address space, so a uniform index becomes a scalar load
  typedef const __attribute__((address_space(4))) int32_t const_i32;
  const_i32 *trow_c = (const_i32 *)trow;
  auto blocks_of_stage = [&](int c0, int (&bid)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      bid[h] = trow_c[__builtin_amdgcn_readfirstlane(min((c0 + 16 * (grp_lo + 4 * h)) / bs, last_blk))];
  };
  auto unit_of = [&](int i, int &isv, int &grp, int &x) {
    const int u = tid + i * kPrefillThreads;
    isv = u >> 10;
    const int w = u & 1023;
    grp = w >> 7;
    x = w & 127;
  };
  // Loads are unconditional (a group past the workgroup's keys reads its
  // clamped block, which is the row's own), so the compiler counts them in
  // straight-line code and a store waits only for its own stage's loads;
  // such groups are zeroed when stored.
  auto stage_load = [&](u32x4 (&stg)[kPUnits], int c0, const int (&bid)[2]) {
#pragma unroll
    for (int i = 0; i < kPUnits; ++i) {
      int isv, grp, x;
      unit_of(i, isv, grp, x);
      const int tok0 = c0 + 16 * grp;
      const int64_t tile = ((int64_t)bid[grp >> 2] * Hkv + t0.h) * tile_elems;
      if (!isv) {  // K: token x / 8, dims 8 (x % 8) ..
        const int tk = x >> 3, dd = (x & 7) * 8;
        stg[i] = *reinterpret_cast<const u32x4 *>(kp + tile + (int64_t)(tok0 % bs + tk) * kD + dd);
      } else {  // V: dim x / 2, tokens 8 (x % 2) .. of the group
        const int dim = x >> 1, t8 = (x & 1) * 8;
        stg[i] = *reinterpret_cast<const u32x4 *>(vp + tile + (int64_t)dim * bs + tok0 % bs + t8);
      }
    }
  };
  auto stage_store = [&](const u32x4 (&stg)[kPUnits], int buf, int c0) {
#pragma unroll
    for (int i = 0; i < kPUnits; ++i) {
      int isv, grp, x;
      unit_of(i, isv, grp, x);
      const u32x4 v = c0 + 16 * grp < wg_kv ? stg[i] : u32x4{0u, 0u, 0u, 0u};
      if (!isv) {
        const int tk = x >> 3, dd = (x & 7) * 8;
        *reinterpret_cast<u32x4 *>(&s_k[buf][(16 * grp + tk) * kPKStride + dd]) = v;
      } else {
        const int dim = x >> 1, t8 = (x & 1) * 8;
        *reinterpret_cast<u32x4 *>(&s_v[buf][(grp * kD + dim) * kPVStride + t8]) = v;
      }
    }
  };

  // this wave's queries
  const int r = live ? ti.qt * kRows + c : 0;
  const bool row_ok = live && r < ti.nrows;
  const int t = row_ok ? r / ti.group : 0;
  const int hq = live ? ti.h * ti.group + (row_ok ? r % ti.group : 0) : 0;
  const int qpos = t0.past + t;
  const int my_kv = live ? ti.kv_len : 0;
  const float c2 = a.scale * 1.4426950408889634f;  // scores in log2 units
  bf16x8 qop[2];
  {
    u32x4 raw[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    if (row_ok) {
      const u16 *qrow =
          reinterpret_cast<const u16 *>(a.q) + ((int64_t)t0.b * a.width + t) * a.q_stride + (int64_t)hq * kD;
      raw[0] = *reinterpret_cast<const u32x4 *>(qrow + 8 * g);
      raw[1] = *reinterpret_cast<const u32x4 *>(qrow + 32 + 8 * g);
    }
    qop[0] = __builtin_bit_cast(bf16x8, raw[0]);
    qop[1] = __builtin_bit_cast(bf16x8, raw[1]);
  }
  if (a.rope && row_ok) {
    const float *cs = a.cos_t + (int64_t)qpos * (kD / 2) + 8 * g;
    const float *sn = a.sin_t + (int64_t)qpos * (kD / 2) + 8 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float y1, y2;
      rope_pair((float)qop[0][j], (float)qop[1][j], cs[j], sn[j], y1, y2);
      qop[0][j] = (__bf16)y1;
      qop[1][j] = (__bf16)y2;
    }
  }
  f32x4 o[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) o[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;
  // one 64-token step (half hs of the stage) from LDS buffer buf
  auto compute = [&](int c0, int buf, int hs) {
    float sv[16];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int tk = 64 * hs + 32 * ch + 8 * (c >> 2) + 4 * hf + (c & 3);  // token within the stage
        const u16 *kr = &s_k[buf][tk * kPKStride + 8 * g];
        const u32x4 k0 = *reinterpret_cast<const u32x4 *>(kr);
        const u32x4 k1 = *reinterpret_cast<const u32x4 *>(kr + 32);
        f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, k0), qop[0], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, k1), qop[1], sc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[8 * ch + 4 * hf + i] = sc[i] * c2;
      }
    }
    if (c0 + 64 > t0.past) {
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int pos = c0 + 32 * ch + 8 * g + j;
          if (!(row_ok && pos <= qpos && pos < my_kv)) sv[8 * ch + j] = -INFINITY;
        }
    }
    online_update<16>(sv, m, l, o);
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      bf16x8 pop;
#pragma unroll
      for (int j = 0; j < 8; ++j) pop[j] = (__bf16)sv[8 * ch + j];
      // lane group g's 8 tokens: 16-token group 2 ch + g / 2, tokens 8 (g % 2) ..
      const u16 *vr = &s_v[buf][((4 * hs + 2 * ch + (g >> 1)) * kD + c) * kPVStride + 8 * (g & 1)];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const u32x4 vv = *reinterpret_cast<const u32x4 *>(vr + 16 * tt * kPVStride);
        o[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vv), pop, o[tt], 0, 0, 0);
      }
    }
  };
  // stage s lives in LDS buffer s % 3; its loads go out during stage s - 2
  int bid[2];
  blocks_of_stage(0, bid);
  stage_load(stg_a, 0, bid);
  blocks_of_stage(kPStage, bid);
  stage_store(stg_a, 0, 0);
  stage_load(stg_a, kPStage, bid);  // stage 1, stored during stage 0
  blocks_of_stage(2 * kPStage, bid);
  __syncthreads();
  auto stage_step = [&](int c0, int buf, u32x4 (&held)[kPUnits], u32x4 (&ahead)[kPUnits]) {
    // held: stage c0 + kPStage's data, stored now; ahead: stage c0 + 2 kPStage's, loaded now
    // (every step loads and stores, also past the keys: no branch around a
    // load, so each wait is for exactly the loads it needs)
    stage_load(ahead, c0 + 2 * kPStage, bid);
    blocks_of_stage(c0 + 3 * kPStage, bid);
    if (c0 < my_kv) compute(c0, buf, 0);
    if (c0 + 64 < my_kv) compute(c0 + 64, buf, 1);
    stage_store(held, buf == 2 ? 0 : buf + 1, c0 + kPStage);
    __syncthreads();
  };
  int buf = 0;
  for (int c0 = 0; c0 < wg_kv; c0 += 2 * kPStage) {
    stage_step(c0, buf, stg_a, stg_b);
    buf = buf == 2 ? 0 : buf + 1;
    if (c0 + kPStage >= wg_kv) break;
    stage_step(c0 + kPStage, buf, stg_b, stg_a);
    buf = buf == 2 ? 0 : buf + 1;
  }
  // O^T accumulators: lane (c, g) holds dims 16 tt + 4 g + i of query row c
  if (row_ok) {
    __hip_bfloat16 *dst = reinterpret_cast<__hip_bfloat16 *>(a.out) + ((int64_t)t0.b * a.width + t) * a.out_stride +
                          (int64_t)hq * kD;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[16 * tt + 4 * g + i] = from_f32<__hip_bfloat16>(o[tt][i] / l);
  }
}

// ---------------------------------------------------------------- fp32 ----
// Same structure on v_mfma_f32_16x16x4_f32: per 16-token group the k index
// of lane group g is dim 16g+s at step s (QK^T) and token 4g+i at step i (PV).
template <bool BS16>
__global__ __launch_bounds__(kAttnThreads) void attention_f32_kernel(AttnArgs a) {
  TileInfo ti;
  if (!tile_info(a, ti)) {
    poison_tile<float>(a, ti);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int r = ti.qt * kRows + c;
  const bool row_ok = r < ti.nrows;
  const int t = row_ok ? r / ti.group : 0;
  const int hq = ti.h * ti.group + (row_ok ? r % ti.group : 0);
  const int qpos = ti.past + t;

  const float *kp = reinterpret_cast<const float *>(a.k);
  const float *vp = reinterpret_cast<const float *>(a.v);
  const float *qrow =
      reinterpret_cast<const float *>(a.q) + ((int64_t)ti.b * a.width + t) * a.q_stride + (int64_t)hq * kD;
  if (a.rope) {
    append_new_kv<float>(a, ti, blockIdx.y * a.split, (blockIdx.y + 1) * a.split);
    __threadfence_block();
    __syncthreads();
  }
  // lane group g holds dims 16g..16g+15; its RoPE partners are 32 dims away
  float qv[16];
#pragma unroll
  for (int s = 0; s < 16; ++s) qv[s] = row_ok ? qrow[16 * g + s] : 0.0f;
  if (a.rope && row_ok) {
    const int lo = (16 * g) % 32;  // index into the cos/sin half-table
    const float *cs = a.cos_t + (int64_t)qpos * (kD / 2) + lo;
    const float *sn = a.sin_t + (int64_t)qpos * (kD / 2) + lo;
    const float *partner = qrow + (16 * g + 32) % 64;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      float y1, y2;
      if (g < 2) rope_pair(qv[s], partner[s], cs[s], sn[s], y1, y2), qv[s] = y1;
      else rope_pair(partner[s], qv[s], cs[s], sn[s], y1, y2), qv[s] = y2;
    }
  }

  f32x4 o[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) o[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  const int Hkv = a.Hkv, bs = a.bs;
  const int s_lo = blockIdx.y * a.split;
  const int s_hi = min(s_lo + a.split, ti.kv_len);

  // wave w takes the 32-token chunks 2w, 2w+1, 2w+8, 2w+9, ... of this split
  for (int step = s_lo + 64 * wave; step < s_hi; step += 256)
  for (int c0 = step; c0 < min(step + 64, s_hi); c0 += 32) {
    float sv[8];
    float vv[2][4][4];  // [group][tile][token i]
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int gs = c0 + 16 * gi;
      float kv[16];
#pragma unroll
      for (int s = 0; s < 16; ++s) kv[s] = 0.0f;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) vv[gi][tt][i] = 0.0f;
      if (gs < ti.kv_len) {
        const int pos = gs + c;
        if (BS16 || pos < ti.kv_len) {
          const int64_t blk = block_of(a, ti, BS16 ? gs : pos);
          const float *kb = kp + ((blk * Hkv + ti.h) * bs + (BS16 ? gs % bs + c : pos % bs)) * kD + 16 * g;
#pragma unroll
          for (int s = 0; s < 16; ++s) kv[s] = kb[s];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int vpos = gs + 4 * g + i;
          const bool ok = BS16 || vpos < ti.kv_len;
          const int64_t blk = ok ? block_of(a, ti, vpos) : 0;
          const float *vb = vp + (blk * Hkv + ti.h) * (int64_t)kD * bs + vpos % bs;
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) vv[gi][tt][i] = ok ? vb[(int64_t)(16 * tt + c) * bs] : 0.0f;
        }
      }
      f32x4 s4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 16; ++s) s4 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[s], qv[s], s4, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = gs + 4 * g + i;
        const bool ok = row_ok && pos <= qpos && pos < ti.kv_len;
        sv[4 * gi + i] = ok ? s4[i] * (a.scale * 1.4426950408889634f) : -INFINITY;
      }
    }
    online_update(sv, m, l, o);
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[gi][tt][i], sv[4 * gi + i], o[tt], 0, 0, 0);
  }
  finish<float>(a, ti, m, l, o);
}

inline int qtiles(int width, int H, int Hkv) { return (width * (H / Hkv) + kRows - 1) / kRows; }

constexpr int kMaxSplits = 128;  // bounds the split workspace of one (row, head, tile)

inline int choose_split(int batch, int width, int H, int Hkv, int max_kv_len) {
  const int nqt = qtiles(width, H, Hkv);
  if (nqt == 1) {
    // fixed 512 up to 65536 keys, so a query's reduction order does not
    // depend on how many queries share the call (512 rather than 256: half
    // the workgroups and partials at the same batch-1 time, 7% faster at
    // batch 8 with K/V from HBM)
    const int mult = (max_kv_len + kDefaultSplit * kMaxSplits - 1) / (kDefaultSplit * kMaxSplits);
    return kDefaultSplit * (mult > 1 ? mult : 1);
  }
  // many query tiles (prefill): fewer, longer splits keep the workspace small
  const int64_t units = (int64_t)batch * Hkv * nqt;
  const int want = units >= 1024 ? 1 : (int)((2048 + units - 1) / units);
  int split = (max_kv_len + want - 1) / want;
  split = ((split + 255) / 256) * 256;  // waves take 64-token steps
  if (split < kDefaultSplit) split = kDefaultSplit;
  const int min_split = ((max_kv_len + kMaxSplits - 1) / kMaxSplits + 255) / 256 * 256;
  return split < min_split ? min_split : split;
}

// A caller-chosen split, rounded up to whole 256-token steps of the four
// waves and raised if it would need more than kMaxSplits splits.
inline int round_split(int split, int max_kv_len) {
  split = ((split + 255) / 256) * 256;
  const int min_split = ((max_kv_len + kMaxSplits - 1) / kMaxSplits + 255) / 256 * 256;
  return split < min_split ? min_split : split;
}

}  // namespace specdec

using namespace specdec;

SPECDEC_API int specdec_attention_split(int32_t batch, int32_t width, int32_t n_heads,
                                        int32_t n_kv_heads, int32_t max_kv_len) {
  if (batch <= 0 || width <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads) return -1;
  return choose_split(batch, width, n_heads, n_kv_heads, max_kv_len);
}

SPECDEC_API int specdec_attention_workspace(int32_t batch, int32_t width, int32_t n_heads,
                                            int32_t n_kv_heads, int32_t head_dim,
                                            int32_t max_kv_len, int32_t split_tokens,
                                            int64_t *floats) {
  if (!floats || batch < 0 || width < 0 || n_kv_heads <= 0 || n_heads <= 0 ||
      n_heads % n_kv_heads || max_kv_len < 0)
    return SPECDEC_EINVAL;
  if (head_dim != kD) return SPECDEC_EUNSUPPORTED;
  // split_tokens < 0 (one flat split) needs no partials; sizing it as the
  // default also covers the fp32 kernels, which take the default instead
  split_tokens = split_tokens > 0 ? round_split(split_tokens, max_kv_len)
                                  : choose_split(batch > 0 ? batch : 1, width > 0 ? width : 1, n_heads,
                                                 n_kv_heads, max_kv_len);
  const int64_t units = (int64_t)batch * n_kv_heads * qtiles(width, n_heads, n_kv_heads);
  const int64_t splits = (max_kv_len + split_tokens - 1) / split_tokens;
  *floats = units * splits * kPart;
  return SPECDEC_OK;
}

// Grid of one call: the split, the kernel family and how many split
// partials per unit the workspace must hold.
struct AttnPlan {
  int64_t units = 0;       // (row, kv head, query tile) workgroups
  int64_t need_floats = 0; // workspace floats this call reads and writes
  bool single = false;     // one 16-wave workgroup per unit, no combine
  bool prefill = false;    // wide bf16 call: attention_prefill_kernel (after rope_append)
  bool decode = false;     // latency decode step: attention_decode_kernel
  bool nothing = false;    // no work: the call returns at once
};

static int plan_attention(AttnArgs &a, AttnPlan &plan, int dtype, int32_t batch, int32_t width, int32_t n_heads,
                          int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t max_kv_len,
                          int32_t split_tokens) {
  if (batch < 0 || width < 0 || n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads ||
      block_size <= 0 || max_kv_len < 0)
    return SPECDEC_EINVAL;
  if (head_dim != kD) return SPECDEC_EUNSUPPORTED;
  if (a.hidden) {
    // the scales are computed in the staged prologue: bf16, whole 16-token
    // block groups, every new token of a row staged in LDS
    if (dtype != SPECDEC_BF16 || block_size % 16 != 0 || width > kStage) return SPECDEC_EUNSUPPORTED;
    if (a.hdim <= 0 || a.hdim % 8 != 0 || ((uintptr_t)a.hidden & 15) != 0) return SPECDEC_EINVAL;
  }
  if (dtype != SPECDEC_BF16 && dtype != SPECDEC_F32) return SPECDEC_EINVAL;
  if (batch == 0 || width == 0 || max_kv_len == 0) {
    plan.nothing = true;
    return SPECDEC_OK;
  }
  if (!a.q || !a.k || !a.v || !a.tables || !a.meta || !a.out) return SPECDEC_EINVAL;
  // a token's row of q (of qkv, with rope) and of out holds all of its
  // heads, so the rows of a call never overlap
  const int64_t q_row = (int64_t)(a.rope ? n_heads + 2 * n_kv_heads : n_heads) * head_dim;
  if (a.q_stride < q_row || a.out_stride < (int64_t)n_heads * head_dim) return SPECDEC_EINVAL;
  a.batch = batch;
  a.width = width;
  a.H = n_heads;
  a.Hkv = n_kv_heads;
  a.bs = block_size;
  a.flat = split_tokens < 0 && dtype == SPECDEC_BF16;
  if (a.flat) a.split = (max_kv_len + 63) / 64 * 64;
  else
    a.split = split_tokens > 0 ? round_split(split_tokens, max_kv_len)
                               : choose_split(batch, width, n_heads, n_kv_heads, max_kv_len);
  a.max_splits = (max_kv_len + a.split - 1) / a.split;
  a.max_kv = max_kv_len;
  a.n_qtiles = qtiles(width, n_heads, n_kv_heads);
  const int64_t units = (int64_t)batch * n_kv_heads * a.n_qtiles;
  // bf16 tiles with more than four splits (at most kTSplits), when every CU
  // gets a tile and a tile's live rows fit kTRows, run tiled: one 16-wave
  // workgroup per tile takes all of its splits, no partials, no combine
  a.tiled = dtype == SPECDEC_BF16 && !a.flat && block_size % 16 == 0 && a.max_splits > 4 &&
            a.max_splits <= kTSplits && a.n_qtiles == 1 && width * (n_heads / n_kv_heads) <= kTRows &&
            cu_count() > 0 && units >= cu_count();
  // bf16 tiles with at most four splits (or one flat split, or tiled) run
  // in one 16-wave workgroup; otherwise one 4-wave workgroup per split +
  // combine
  plan.single = dtype == SPECDEC_BF16 && (a.flat || a.tiled || a.max_splits <= 4);
  // more than kStage new tokens per row (a prompt): one pass per query tile
  plan.prefill = dtype == SPECDEC_BF16 && !a.flat && width > kStage && block_size % 16 == 0;
  if (plan.prefill) {
    a.tiled = 0;
    plan.single = true;
  }
  // one new token per row, latency split, fused RoPE (+ norm), a kv head's
  // queries in one tile, contexts up to 2048 (at most two rounds of two
  // steps per wave): the 4-wave decode kernel
  plan.decode = a.flat && a.rope && width == 1 && block_size % 16 == 0 && max_kv_len <= 2048 &&
                n_heads / n_kv_heads <= kRows && (!a.hidden || a.hdim <= 4 * kWave * 8);
  if (plan.decode) a.tiled = 0;
  a.parts = plan.single ? 1 : a.max_splits;
  if (units > INT32_MAX || a.max_splits > 65535) return SPECDEC_EUNSUPPORTED;
  plan.units = units;
  plan.need_floats = a.parts > 1 ? units * a.parts * kPart : 0;
  return SPECDEC_OK;
}

static int run_attention(AttnArgs &a, const AttnPlan &plan, int dtype, int32_t block_size, void *stream) {
  hipStream_t s = as_stream(stream);
  const bool bs16 = (block_size % 16) == 0;
  const int64_t units = plan.units;
  dim3 grid((unsigned)units, (unsigned)a.parts);
  if (plan.prefill) {
    if (a.rope) {  // the new tokens' rotated K and V into the pools, once; q is rotated in registers
      int st = launch_rope_append_groups(const_cast<void *>(a.q), a.q_stride, a.H, a.Hkv, a.cos_t, a.sin_t, a.meta,
                                         a.batch, a.width, a.tables, a.table_stride, block_size,
                                         const_cast<void *>(a.k), const_cast<void *>(a.v), s);
      if (st == SPECDEC_EUNSUPPORTED)  // unaligned operands: the per-element kernel
        st = launch_rope_append(const_cast<void *>(a.q), SPECDEC_BF16, a.q_stride, a.H, a.Hkv, kD, a.cos_t, a.sin_t,
                                a.meta, a.batch, a.width, a.tables, a.table_stride, block_size,
                                const_cast<void *>(a.k), const_cast<void *>(a.v), /*kv_only=*/true, s);
      if (st != SPECDEC_OK) return st;
    }
    const int64_t blocks = (int64_t)a.batch * a.Hkv * ((a.n_qtiles + kPrefillTiles - 1) / kPrefillTiles);
    if (blocks > INT32_MAX) return SPECDEC_EUNSUPPORTED;
    dim3 pgrid((unsigned)blocks), pblock(kPrefillThreads);
    if (block_size == 16) attention_prefill_kernel<1><<<pgrid, pblock, 0, s>>>(a);
    else attention_prefill_kernel<2><<<pgrid, pblock, 0, s>>>(a);
    return launch_status();
  }
  if (plan.decode) {
    dim3 block(kAttnThreads);
    if (block_size == 16) attention_decode_kernel<1><<<grid, block, 0, s>>>(a);
    else attention_decode_kernel<2><<<grid, block, 0, s>>>(a);
    return launch_status();
  }
  if (a.tiled) {
    dim3 block(16 * kWave);
    if (block_size == 16) attention_bf16_kernel<1, 16, true><<<grid, block, 0, s>>>(a);
    else attention_bf16_kernel<2, 16, true><<<grid, block, 0, s>>>(a);
  } else if (plan.single) {
    dim3 block(16 * kWave);
    if (block_size == 16) attention_bf16_kernel<1, 16><<<grid, block, 0, s>>>(a);
    else if (bs16) attention_bf16_kernel<2, 16><<<grid, block, 0, s>>>(a);
    else attention_bf16_kernel<0, 16><<<grid, block, 0, s>>>(a);
  } else if (dtype == SPECDEC_BF16 && block_size % 16 == 0 && a.split == kDefaultSplit &&
             units * a.parts <= 2 * (int64_t)cu_count()) {
    // few workgroups (batch 1 at long contexts): two waves per SIMD is all
    // the grid fills, so each wave takes both of its steps' loads at once
    dim3 block(kAttnThreads);
    if (block_size == 16) attention_bf16_kernel<1, 4, false, true><<<grid, block, 0, s>>>(a);
    else attention_bf16_kernel<2, 4, false, true><<<grid, block, 0, s>>>(a);
  } else if (dtype == SPECDEC_BF16) {
    dim3 block(kAttnThreads);
    if (block_size == 16) attention_bf16_kernel<1, 4><<<grid, block, 0, s>>>(a);
    else if (bs16) attention_bf16_kernel<2, 4><<<grid, block, 0, s>>>(a);
    else attention_bf16_kernel<0, 4><<<grid, block, 0, s>>>(a);
  } else {
    dim3 block(kAttnThreads);
    if (bs16) attention_f32_kernel<true><<<grid, block, 0, s>>>(a);
    else attention_f32_kernel<false><<<grid, block, 0, s>>>(a);
  }
  if (a.parts > 1) {
    dim3 cg((unsigned)units), cb(kAttnThreads);
    switch (min((a.parts + 3) / 4, 8)) {
      case 1: attention_combine_kernel<1><<<cg, cb, 0, s>>>(a, dtype); break;
      case 2: attention_combine_kernel<2><<<cg, cb, 0, s>>>(a, dtype); break;
      case 3: attention_combine_kernel<3><<<cg, cb, 0, s>>>(a, dtype); break;
      case 4: attention_combine_kernel<4><<<cg, cb, 0, s>>>(a, dtype); break;
      case 5: attention_combine_kernel<5><<<cg, cb, 0, s>>>(a, dtype); break;
      case 6: attention_combine_kernel<6><<<cg, cb, 0, s>>>(a, dtype); break;
      case 7: attention_combine_kernel<7><<<cg, cb, 0, s>>>(a, dtype); break;
      default: attention_combine_kernel<8><<<cg, cb, 0, s>>>(a, dtype); break;
    }
  }
  return launch_status();
}

static int launch_attention(AttnArgs &a, int dtype, int32_t batch, int32_t width, int32_t n_heads,
                            int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t max_kv_len,
                            int32_t split_tokens, float *workspace, int64_t workspace_floats, void *stream) {
  AttnPlan plan;
  const int st = plan_attention(a, plan, dtype, batch, width, n_heads, n_kv_heads, head_dim, block_size,
                                max_kv_len, split_tokens);
  if (st != SPECDEC_OK || plan.nothing) return st;
  if (plan.need_floats > 0 && (!workspace || workspace_floats < plan.need_floats)) return SPECDEC_EINVAL;
  a.ws = workspace;
  return run_attention(a, plan, dtype, block_size, stream);
}

// ---- split partials held by the library ---------------------------------
// specdec_paged_attention_static's workspace: one array per GPU the library
// runs on (each device holds its own copy, at its own address, until the
// process ends).  In host code `static_partials` names a host-side stand-in,
// not device memory: its device address on the current device comes from
// hipGetSymbolAddress, looked up once per device and kept in
// static_partials_ptr[].  Partials need no initialisation (every slot the
// combine reads was written by the same call's split kernel), so a call
// clears nothing; calls that overlap on one GPU race for the array.
constexpr int64_t kStaticPartialFloats = SPECDEC_STATIC_PARTIAL_FLOATS;
static __device__ __align__(256) float static_partials[kStaticPartialFloats];

constexpr int kMaxDevices = 64;
static float *static_partials_ptr[kMaxDevices];
static std::mutex static_partials_lock;

// Device address of this device's static_partials (the device must be
// current), or null if HIP cannot provide it.
static float *static_partials_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> hold(static_partials_lock);
  if (!static_partials_ptr[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(static_partials)) != hipSuccess || !p) return nullptr;
    static_partials_ptr[dev] = static_cast<float *>(p);
  }
  return static_partials_ptr[dev];
}

SPECDEC_API int specdec_paged_attention(const void *q, int dtype, int64_t q_token_stride,
                                        const void *k_pool, const void *v_pool,
                                        const int32_t *tables, int64_t table_stride,
                                        const int32_t *meta, int32_t batch, int32_t width,
                                        int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                        int32_t block_size, float scale, int32_t max_kv_len,
                                        int32_t split_tokens, float *workspace,
                                        int64_t workspace_floats, void *out,
                                        int64_t out_token_stride, void *stream) {
  AttnArgs a{};
  a.q = q;
  a.q_stride = q_token_stride;
  a.rope = 0;
  a.k = k_pool;
  a.v = v_pool;
  a.tables = tables;
  a.table_stride = table_stride;
  a.meta = meta;
  a.scale = scale;
  a.out = out;
  a.out_stride = out_token_stride;
  return launch_attention(a, dtype, batch, width, n_heads, n_kv_heads, head_dim, block_size, max_kv_len,
                          split_tokens, workspace, workspace_floats, stream);
}

SPECDEC_API int specdec_rope_paged_attention(void *qkv, int dtype, int64_t token_stride,
                                             const float *cos_table, const float *sin_table,
                                             const void *hidden, int64_t hidden_dim, float eps,
                                             void *k_pool, void *v_pool, const int32_t *tables,
                                             int64_t table_stride, const int32_t *meta, int32_t batch,
                                             int32_t width, int32_t n_heads, int32_t n_kv_heads,
                                             int32_t head_dim, int32_t block_size, float scale,
                                             int32_t max_kv_len, int32_t split_tokens,
                                             float *workspace, int64_t workspace_floats, void *out,
                                             int64_t out_token_stride, void *stream) {
  if (!cos_table || !sin_table) return SPECDEC_EINVAL;
  AttnArgs a{};
  a.q = qkv;
  a.q_stride = token_stride;
  a.rope = 1;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  if (hidden && (hidden_dim <= 0 || hidden_dim > (1 << 20))) return SPECDEC_EINVAL;
  a.hidden = hidden;
  a.hdim = (int)hidden_dim;
  a.eps = eps;
  a.k = k_pool;
  a.v = v_pool;
  a.tables = tables;
  a.table_stride = table_stride;
  a.meta = meta;
  a.scale = scale;
  a.out = out;
  a.out_stride = out_token_stride;
  return launch_attention(a, dtype, batch, width, n_heads, n_kv_heads, head_dim, block_size, max_kv_len,
                          split_tokens, workspace, workspace_floats, stream);
}

SPECDEC_API int specdec_rope_paged_attention_parts(void *qkv, int64_t token_stride, const float *cos_table,
                                                   const float *sin_table, const void *hidden, int64_t hidden_dim,
                                                   float eps, void *k_pool, void *v_pool, const int32_t *tables,
                                                   int64_t table_stride, const int32_t *meta, int32_t batch,
                                                   int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                                   int32_t block_size, float scale, int32_t max_kv_len,
                                                   int32_t nparts, float *parts, void *stream) {
  if (batch < 0 || n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads || block_size <= 0 || max_kv_len < 0)
    return SPECDEC_EINVAL;
  if (batch == 0 || max_kv_len == 0) return SPECDEC_OK;
  if (!qkv || !cos_table || !sin_table || !k_pool || !v_pool || !tables || !meta || !parts) return SPECDEC_EINVAL;
  if (nparts != 4 && nparts != 8 && nparts != 16) return SPECDEC_EINVAL;
  if (((uintptr_t)parts & 15)) return SPECDEC_EINVAL;
  if (head_dim != kD || block_size % 16 != 0 || max_kv_len > 2048 || n_heads / n_kv_heads > kRows)
    return SPECDEC_EUNSUPPORTED;
  if (hidden && (hidden_dim <= 0 || hidden_dim % 8 != 0 || ((uintptr_t)hidden & 15))) return SPECDEC_EINVAL;
  if (hidden && hidden_dim > 4 * kWave * 8) return SPECDEC_EUNSUPPORTED;
  if (token_stride < (int64_t)(n_heads + 2 * n_kv_heads) * kD || token_stride % 8 || ((uintptr_t)qkv & 15))
    return SPECDEC_EINVAL;
  const int64_t wgs = (int64_t)batch * n_kv_heads * nparts;
  if (wgs > INT32_MAX) return SPECDEC_EUNSUPPORTED;
  AttnArgs a{};
  a.q = qkv;
  a.q_stride = token_stride;
  a.rope = 1;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.hidden = hidden;
  a.hdim = hidden ? (int)hidden_dim : 0;
  a.eps = eps;
  a.k = k_pool;
  a.v = v_pool;
  a.tables = tables;
  a.table_stride = table_stride;
  a.meta = meta;
  a.scale = scale;
  a.batch = batch;
  a.width = 1;
  a.H = n_heads;
  a.Hkv = n_kv_heads;
  a.bs = block_size;
  a.flat = 1;  // one split over every key
  a.split = (max_kv_len + 63) / 64 * 64;
  a.max_splits = 1;
  a.max_kv = max_kv_len;
  a.n_qtiles = 1;
  a.parts = 1;
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)wgs), block(kWave);
#define SPECDEC_PARTS(NP)                                                                  \
  do {                                                                                     \
    if (block_size == 16) attention_decode_parts_kernel<1, NP><<<grid, block, 0, s>>>(a, parts); \
    else attention_decode_parts_kernel<2, NP><<<grid, block, 0, s>>>(a, parts);           \
  } while (0)
  if (nparts == 4) SPECDEC_PARTS(4);
  else if (nparts == 8) SPECDEC_PARTS(8);
  else SPECDEC_PARTS(16);
#undef SPECDEC_PARTS
  return launch_status();
}

SPECDEC_API int specdec_paged_attention_static(const void *q, int dtype, int64_t q_token_stride,
                                               const void *k_pool, const void *v_pool,
                                               const int32_t *tables, int64_t table_stride,
                                               const int32_t *meta, int32_t batch, int32_t width,
                                               int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                               int32_t block_size, float scale, int32_t max_kv_len,
                                               int32_t split_tokens, void *out, int64_t out_token_stride,
                                               void *stream) {
  AttnArgs a{};
  a.q = q;
  a.q_stride = q_token_stride;
  a.rope = 0;
  a.k = k_pool;
  a.v = v_pool;
  a.tables = tables;
  a.table_stride = table_stride;
  a.meta = meta;
  a.scale = scale;
  a.out = out;
  a.out_stride = out_token_stride;
  AttnPlan plan;
  const int st = plan_attention(a, plan, dtype, batch, width, n_heads, n_kv_heads, head_dim, block_size,
                                max_kv_len, split_tokens);
  if (st != SPECDEC_OK || plan.nothing) return st;
  if (plan.need_floats > kStaticPartialFloats) return SPECDEC_ENOSCRATCH;
  if (plan.need_floats > 0) {
    a.ws = static_partials_on_current_device();
    if (!a.ws) return SPECDEC_EHIP;
  }
  return run_attention(a, plan, dtype, block_size, stream);
}
