// Paged KV-cache index kernels: the LIFO block allocator (push = rollback or
// release, pop = growth) applied to device block tables, slot arithmetic,
// the fused RoPE + append of new K/V, and a gather used for inspection.
//
// Reference semantics: cache/paged.py:11-76 (allocator, tables, slots),
// cache/kv.py:79-118 (append, write, gather, truncate), lm/forward.py:53,60
// (rotary embedding).
//
// Pool layout per layer: K [num_blocks, Hkv, bs, d], V [num_blocks, Hkv, d, bs].
#include "common.h"

namespace specdec {

constexpr int kPlanThreads = 256;

// entries: (row, col, count, off) x (n_push + n_pop); pushes first.
__global__ __launch_bounds__(kPlanThreads) void block_plan_kernel(
    int32_t *__restrict__ tables, int64_t table_stride, int32_t *__restrict__ stack,
    uint8_t *__restrict__ used, int32_t top, const int32_t *__restrict__ entries, int32_t n_push,
    int32_t n_pop, int32_t *__restrict__ popped) {
  __shared__ int32_t s_pushed;
  if (threadIdx.x == 0) {
    int32_t total = 0;
    for (int e = 0; e < n_push; ++e) total += entries[4 * e + 2];
    s_pushed = total;
  }
  // phase 1: rollbacks/releases push their blocks in table order
  for (int e = threadIdx.x; e < n_push; e += blockDim.x) {
    const int32_t row = entries[4 * e], col = entries[4 * e + 1];
    const int32_t cnt = entries[4 * e + 2], off = entries[4 * e + 3];
    for (int j = 0; j < cnt; ++j) {
      const int32_t blk = tables[(int64_t)row * table_stride + col + j];
      stack[top + off + j] = blk;
      used[blk] = 0;
    }
  }
  __threadfence();
  __syncthreads();
  // phase 2: growth pops from the top of the stack, rows in call order
  const int32_t top2 = top + s_pushed;
  for (int e = threadIdx.x; e < n_pop; e += blockDim.x) {
    const int32_t *ent = entries + 4 * (n_push + e);
    const int32_t row = ent[0], col = ent[1], cnt = ent[2], off = ent[3];
    for (int j = 0; j < cnt; ++j) {
      const int32_t blk = stack[top2 - 1 - off - j];
      tables[(int64_t)row * table_stride + col + j] = blk;
      used[blk] = 1;
      if (popped) popped[off + j] = blk;
    }
  }
}

__global__ void block_free_checked_kernel(int32_t *__restrict__ stack, uint8_t *__restrict__ used,
                                          int32_t top, int32_t block, int32_t *__restrict__ status) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  if (!used[block]) {
    status[0] = 1;
    return;
  }
  used[block] = 0;
  stack[top] = block;
  status[0] = 0;
}

__global__ void block_slots_kernel(const int32_t *__restrict__ row, int64_t start, int64_t n,
                                   int32_t bs, int64_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t pos = start + i;
  out[i] = (int64_t)row[pos / bs] * bs + pos % bs;
}

__device__ __forceinline__ int64_t slot_of(const int32_t *tables, int64_t table_stride, int32_t row,
                                           int64_t pos, int32_t bs) {
  return (int64_t)tables[(int64_t)row * table_stride + pos / bs] * bs + pos % bs;
}

__global__ void slot_map_kernel(const int32_t *__restrict__ tables, int64_t table_stride,
                                const int32_t *__restrict__ meta, int32_t batch, int32_t bs,
                                int32_t width, int32_t read_width,
                                const int32_t *__restrict__ write_offsets,
                                int64_t *__restrict__ write, int64_t *__restrict__ write_index,
                                int64_t *__restrict__ read) {
  const int b = blockIdx.y;
  const int32_t row = meta[b], past = meta[batch + b], n = meta[2 * batch + b];
  const int32_t total = past + n;
  for (int pos = blockIdx.x * blockDim.x + threadIdx.x; pos < read_width;
       pos += gridDim.x * blockDim.x) {
    read[(int64_t)b * read_width + pos] = pos < total ? slot_of(tables, table_stride, row, pos, bs) : 0;
    if (pos < n) {
      const int64_t o = write_offsets[b] + pos;
      write[o] = slot_of(tables, table_stride, row, past + pos, bs);
      write_index[o] = (int64_t)b * width + pos;
    }
  }
}

// One thread per (token, q or k head, rotation pair), then one thread per
// (row, v head, dim, token).  Heads [0, H) are queries, [H, H+Hkv) keys,
// [H+Hkv, H+2Hkv) values (copied, not rotated).  Heads below head0 are
// skipped (head0 = H: k and v only, q left as it is).  V's pool tile is
// dim-major ([dim][slot], one 32-byte row of 16 slots per dim at block size
// 16), so the value threads run token-fastest: the lanes of one dim write
// consecutive slots of its row -- one run per (dim, block) -- instead of a
// token's 64 dims landing 32 bytes apart in 64 separate lanes.
template <typename T>
__global__ void rope_append_kernel(T *__restrict__ qkv, int64_t token_stride, int32_t H,
                                   int32_t Hkv, int32_t d, const float *__restrict__ cos_t,
                                   const float *__restrict__ sin_t, const int32_t *__restrict__ meta,
                                   int32_t batch, int32_t width, const int32_t *__restrict__ tables,
                                   int64_t table_stride, int32_t bs, T *__restrict__ kpool,
                                   T *__restrict__ vpool, int32_t head0) {
  const int half = d / 2;
  const int heads = H + Hkv - head0;  // rotated heads
  const int64_t n_qk = (int64_t)batch * width * heads * half;
  const int64_t total = n_qk + (int64_t)batch * Hkv * d * width;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    if (idx >= n_qk) {  // a value element: (row, v head, dim, token), token fastest
      const int64_t j = idx - n_qk;
      const int t = (int)(j % width);
      const int c = (int)((j / width) % d);
      const int h = (int)((j / ((int64_t)width * d)) % Hkv);
      const int b = (int)(j / ((int64_t)width * d * Hkv));
      const int32_t row = meta[b], past = meta[batch + b], n = meta[2 * batch + b];
      if (t >= n) continue;  // right padding
      const int64_t pos = past + t;
      const int64_t blk = tables[(int64_t)row * table_stride + pos / bs];
      vpool[((blk * Hkv + h) * d + c) * bs + pos % bs] =
          qkv[((int64_t)b * width + t) * token_stride + (int64_t)(H + Hkv + h) * d + c];
      continue;
    }
    const int i = (int)(idx % half);
    const int head = head0 + (int)((idx / half) % heads);
    const int64_t tok = idx / ((int64_t)half * heads);
    const int b = (int)(tok / width), t = (int)(tok % width);
    const int32_t row = meta[b], past = meta[batch + b], n = meta[2 * batch + b];
    if (t >= n) continue;  // right padding
    const int64_t pos = past + t;
    T *x = qkv + tok * token_stride + (int64_t)head * d;
    // q*cos + rotate_half(q)*sin, each product and the sum rounded
    // separately (rope_pair), cos/sin in fp32
    float y1, y2;
    rope_pair(to_f32(x[i]), to_f32(x[i + half]), cos_t[pos * half + i], sin_t[pos * half + i], y1, y2);
    const T v1 = from_f32<T>(y1), v2 = from_f32<T>(y2);
    x[i] = v1;  // q rotated in place; the rotated key is kept in qkv as well
    x[i + half] = v2;
    if (head >= H) {
      const int64_t blk = tables[(int64_t)row * table_stride + pos / bs];
      T *dst = kpool + ((blk * Hkv + (head - H)) * bs + pos % bs) * d;
      dst[i] = v1;
      dst[i + half] = v2;
    }
  }
}

template <typename T>
__global__ void kv_write_kernel(const T *__restrict__ k, const T *__restrict__ v, int32_t Hkv,
                                int32_t d, const int32_t *__restrict__ meta, int32_t batch,
                                int32_t width, const int32_t *__restrict__ tables,
                                int64_t table_stride, int32_t bs, T *__restrict__ kpool,
                                T *__restrict__ vpool) {
  const int64_t total = (int64_t)batch * Hkv * width * d;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % d);
    const int t = (int)((idx / d) % width);
    const int h = (int)((idx / ((int64_t)d * width)) % Hkv);
    const int b = (int)(idx / ((int64_t)d * width * Hkv));
    const int32_t row = meta[b], past = meta[batch + b], n = meta[2 * batch + b];
    if (t >= n) continue;
    const int64_t pos = past + t;
    const int64_t blk = tables[(int64_t)row * table_stride + pos / bs];
    const int off = (int)(pos % bs);
    kpool[((blk * Hkv + h) * bs + off) * d + c] = k[idx];
    vpool[((blk * Hkv + h) * d + c) * bs + off] = v[idx];
  }
}

template <typename T>
__global__ void kv_gather_kernel(const T *__restrict__ kpool, const T *__restrict__ vpool,
                                 int32_t Hkv, int32_t d, const int32_t *__restrict__ meta,
                                 int32_t batch, const int32_t *__restrict__ tables,
                                 int64_t table_stride, int32_t bs, int32_t read_width,
                                 T *__restrict__ k_out, T *__restrict__ v_out) {
  const int64_t total = (int64_t)batch * Hkv * read_width * d;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % d);
    const int pos = (int)((idx / d) % read_width);
    const int h = (int)((idx / ((int64_t)d * read_width)) % Hkv);
    const int b = (int)(idx / ((int64_t)d * read_width * Hkv));
    const int32_t row = meta[b], total_b = meta[batch + b] + meta[2 * batch + b];
    if (pos >= total_b) {
      k_out[idx] = from_f32<T>(0.0f);
      v_out[idx] = from_f32<T>(0.0f);
      continue;
    }
    const int64_t blk = tables[(int64_t)row * table_stride + pos / bs];
    const int off = pos % bs;
    k_out[idx] = kpool[((blk * Hkv + h) * bs + off) * d + c];
    v_out[idx] = vpool[((blk * Hkv + h) * d + c) * bs + off];
  }
}

// The new tokens' K (rotated) and V of a prompt-sized bf16 call, head_dim
// 64, block_size % 16 == 0: one workgroup per (batch entry, kv head,
// 16-position group aligned to 16), so the group's tokens share one block
// and its V is written as 8-byte runs of four tokens per dim (the pool
// keeps V dim-major within a block, where one token's values lie bs
// elements apart).  Thread (token tid / 16, pairs 2 (tid % 16) ..) rotates
// K as rope_append_kernel does (rope_pair, then one rounding) into the pool
// (qkv is left as it is, as in the fused decode-sized calls); thread (dim
// tid / 4, tokens 4 (tid % 4) ..) copies V.  Positions outside
// [past, past + n_new) are left alone.
__global__ __launch_bounds__(256) void rope_append_groups_kernel(__hip_bfloat16 *__restrict__ qkv,
                                                                 int64_t token_stride, int32_t H, int32_t Hkv,
                                                                 const float *__restrict__ cos_t,
                                                                 const float *__restrict__ sin_t,
                                                                 const int32_t *__restrict__ meta, int32_t batch,
                                                                 int32_t width, const int32_t *__restrict__ tables,
                                                                 int64_t table_stride, int32_t bs,
                                                                 __hip_bfloat16 *__restrict__ kpool,
                                                                 __hip_bfloat16 *__restrict__ vpool) {
  constexpr int d = 64, half = 32;
  typedef unsigned short u16;
  const int b = blockIdx.x / Hkv, h = blockIdx.x % Hkv;
  const int32_t row = meta[b], past = meta[batch + b], n = meta[2 * batch + b];
  const int first = past / 16 * 16 + 16 * (int)blockIdx.y;
  if (first >= past + n) return;
  const int64_t blk = tables[(int64_t)row * table_stride + first / bs];
  const int off0 = first % bs;
  u16 *q16 = reinterpret_cast<u16 *>(qkv);
  const int tid = threadIdx.x;
  {  // K
    const int tt = tid >> 4, i = 2 * (tid & 15);
    const int pos = first + tt;
    if (pos >= past && pos < past + n) {
      const u16 *x = q16 + ((int64_t)b * width + (pos - past)) * token_stride + (int64_t)(H + h) * d;
      const uint32_t w1 = *reinterpret_cast<const uint32_t *>(x + i);
      const uint32_t w2 = *reinterpret_cast<const uint32_t *>(x + i + half);
      const float2 cs = *reinterpret_cast<const float2 *>(cos_t + (int64_t)pos * half + i);
      const float2 sn = *reinterpret_cast<const float2 *>(sin_t + (int64_t)pos * half + i);
      float y1a, y2a, y1b, y2b;
      rope_pair(__uint_as_float(w1 << 16), __uint_as_float(w2 << 16), cs.x, sn.x, y1a, y2a);
      rope_pair(__uint_as_float(w1 & 0xFFFF0000u), __uint_as_float(w2 & 0xFFFF0000u), cs.y, sn.y, y1b, y2b);
      auto bits = [](float v) { return (uint32_t)__builtin_bit_cast(u16, from_f32<__hip_bfloat16>(v)); };
      const uint32_t o1 = bits(y1a) | (bits(y1b) << 16), o2 = bits(y2a) | (bits(y2b) << 16);
      u16 *dst = reinterpret_cast<u16 *>(kpool) + ((blk * Hkv + h) * bs + off0 + tt) * d;
      *reinterpret_cast<uint32_t *>(dst + i) = o1;
      *reinterpret_cast<uint32_t *>(dst + i + half) = o2;
    }
  }
  {  // V
    const int dim = tid >> 2, t4 = 4 * (tid & 3);
    u16 v[4];
    bool all = true;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = first + t4 + j;
      const bool in = pos >= past && pos < past + n;
      all = all && in;
      v[j] = in ? q16[((int64_t)b * width + (pos - past)) * token_stride + (int64_t)(H + Hkv + h) * d + dim] : 0;
    }
    u16 *dst = reinterpret_cast<u16 *>(vpool) + ((blk * Hkv + h) * d + dim) * bs + off0 + t4;
    if (all) {
      *reinterpret_cast<uint2 *>(dst) =
          make_uint2((uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pos = first + t4 + j;
        if (pos >= past && pos < past + n) dst[j] = v[j];
      }
    }
  }
}

inline unsigned grid_for(int64_t n, int threads) {
  int64_t g = (n + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > 1 << 20) g = 1 << 20;
  return (unsigned)g;
}

int launch_rope_append_groups(void *qkv, int64_t token_stride, int32_t H, int32_t Hkv, const float *cos_t,
                              const float *sin_t, const int32_t *meta, int32_t batch, int32_t width,
                              const int32_t *tables, int64_t table_stride, int32_t bs, void *k_pool, void *v_pool,
                              hipStream_t s) {
  // 4- and 8-byte accesses: even token stride, 8-byte aligned bases
  const uintptr_t bases = (uintptr_t)qkv | (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)cos_t | (uintptr_t)sin_t;
  if (bs % 16 != 0 || token_stride % 2 != 0 || (bases & 7)) return SPECDEC_EUNSUPPORTED;
  // a row's new positions [past, past + n) meet at most (15 + width + 15) / 16
  // aligned groups (past % 16 <= 15 positions before the first new one)
  dim3 grid((unsigned)((int64_t)batch * Hkv), (unsigned)((width + 30) / 16)), block(256);
  rope_append_groups_kernel<<<grid, block, 0, s>>>((__hip_bfloat16 *)qkv, token_stride, H, Hkv, cos_t, sin_t, meta,
                                                   batch, width, tables, table_stride, bs,
                                                   (__hip_bfloat16 *)k_pool, (__hip_bfloat16 *)v_pool);
  return launch_status();
}

int launch_rope_append(void *qkv, int dtype, int64_t token_stride, int32_t H, int32_t Hkv, int32_t d,
                       const float *cos_t, const float *sin_t, const int32_t *meta, int32_t batch, int32_t width,
                       const int32_t *tables, int64_t table_stride, int32_t bs, void *k_pool, void *v_pool,
                       bool kv_only, hipStream_t s) {
  const int32_t head0 = kv_only ? H : 0;
  const int64_t n = (int64_t)batch * width * ((H + Hkv - head0) * (d / 2) + Hkv * d);
  dim3 grid(grid_for(n, 256)), block(256);
  if (dtype == SPECDEC_BF16) {
    rope_append_kernel<__hip_bfloat16><<<grid, block, 0, s>>>((__hip_bfloat16 *)qkv, token_stride, H, Hkv, d, cos_t,
                                                              sin_t, meta, batch, width, tables, table_stride, bs,
                                                              (__hip_bfloat16 *)k_pool, (__hip_bfloat16 *)v_pool,
                                                              head0);
  } else if (dtype == SPECDEC_F32) {
    rope_append_kernel<float><<<grid, block, 0, s>>>((float *)qkv, token_stride, H, Hkv, d, cos_t, sin_t, meta, batch,
                                                     width, tables, table_stride, bs, (float *)k_pool,
                                                     (float *)v_pool, head0);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}

}  // namespace specdec

using namespace specdec;

SPECDEC_API int specdec_block_plan(int32_t *tables, int64_t table_stride, int32_t *free_stack,
                                   uint8_t *used, int64_t num_blocks, int32_t top,
                                   const int32_t *entries, int32_t n_push, int32_t n_pop,
                                   int32_t *popped, void *stream) {
  if (n_push < 0 || n_pop < 0 || top < 0 || top > num_blocks) return SPECDEC_EINVAL;
  if (n_push + n_pop == 0) return SPECDEC_OK;
  if (!tables || !free_stack || !used || !entries) return SPECDEC_EINVAL;
  block_plan_kernel<<<dim3(1), dim3(kPlanThreads), 0, as_stream(stream)>>>(
      tables, table_stride, free_stack, used, top, entries, n_push, n_pop, popped);
  return launch_status();
}

SPECDEC_API int specdec_block_free_checked(int32_t *free_stack, uint8_t *used, int64_t num_blocks,
                                           int32_t top, int32_t block, int32_t *status,
                                           void *stream) {
  if (block < 0 || block >= num_blocks || top < 0 || top >= num_blocks) return SPECDEC_EINVAL;
  if (!free_stack || !used || !status) return SPECDEC_EINVAL;
  block_free_checked_kernel<<<dim3(1), dim3(64), 0, as_stream(stream)>>>(free_stack, used, top,
                                                                         block, status);
  return launch_status();
}

SPECDEC_API int specdec_block_slots(const int32_t *table_row, int64_t start, int64_t stop,
                                    int32_t block_size, int64_t *out, void *stream) {
  if (start < 0 || stop < start || block_size <= 0) return SPECDEC_EINVAL;
  const int64_t n = stop - start;
  if (n == 0) return SPECDEC_OK;
  if (!table_row || !out) return SPECDEC_EINVAL;
  block_slots_kernel<<<dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream)>>>(
      table_row, start, n, block_size, out);
  return launch_status();
}

SPECDEC_API int specdec_slot_map(const int32_t *tables, int64_t table_stride, const int32_t *meta,
                                 int32_t batch, int32_t block_size, int32_t width,
                                 int32_t read_width, const int32_t *write_offsets, int64_t *write,
                                 int64_t *write_index, int64_t *read, void *stream) {
  if (batch < 0 || block_size <= 0 || width < 0 || read_width < 0) return SPECDEC_EINVAL;
  if (batch == 0 || read_width == 0) return SPECDEC_OK;
  if (!tables || !meta || !write_offsets || !read) return SPECDEC_EINVAL;
  dim3 grid(grid_for(read_width, 256) > 64 ? 64 : grid_for(read_width, 256), (unsigned)batch);
  slot_map_kernel<<<grid, dim3(256), 0, as_stream(stream)>>>(tables, table_stride, meta, batch,
                                                             block_size, width, read_width,
                                                             write_offsets, write, write_index,
                                                             read);
  return launch_status();
}

SPECDEC_API int specdec_rope_append(void *qkv, int dtype, int64_t token_stride, int32_t n_heads,
                                    int32_t n_kv_heads, int32_t head_dim, const float *cos_table,
                                    const float *sin_table, int64_t max_positions,
                                    const int32_t *meta, int32_t batch, int32_t width,
                                    const int32_t *tables, int64_t table_stride,
                                    int32_t block_size, void *k_pool, void *v_pool,
                                    void *stream) {
  (void)max_positions;  // positions are range-checked by the caller against the table size
  if (batch < 0 || width < 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 ||
      head_dim % 2 || block_size <= 0)
    return SPECDEC_EINVAL;
  if (batch == 0 || width == 0) return SPECDEC_OK;
  if (!qkv || !cos_table || !sin_table || !meta || !tables || !k_pool || !v_pool)
    return SPECDEC_EINVAL;
  return launch_rope_append(qkv, dtype, token_stride, n_heads, n_kv_heads, head_dim, cos_table, sin_table, meta,
                            batch, width, tables, table_stride, block_size, k_pool, v_pool, false,
                            as_stream(stream));
}

SPECDEC_API int specdec_kv_write(const void *k, const void *v, int dtype, int32_t n_kv_heads,
                                 int32_t head_dim, const int32_t *meta, int32_t batch,
                                 int32_t width, const int32_t *tables, int64_t table_stride,
                                 int32_t block_size, void *k_pool, void *v_pool, void *stream) {
  if (batch < 0 || width < 0 || n_kv_heads <= 0 || head_dim <= 0 || block_size <= 0)
    return SPECDEC_EINVAL;
  if (batch == 0 || width == 0) return SPECDEC_OK;
  if (!k || !v || !meta || !tables || !k_pool || !v_pool) return SPECDEC_EINVAL;
  const int64_t n = (int64_t)batch * n_kv_heads * width * head_dim;
  dim3 grid(grid_for(n, 256)), block(256);
  hipStream_t s = as_stream(stream);
  if (dtype == SPECDEC_BF16) {
    kv_write_kernel<__hip_bfloat16><<<grid, block, 0, s>>>(
        (const __hip_bfloat16 *)k, (const __hip_bfloat16 *)v, n_kv_heads, head_dim, meta, batch,
        width, tables, table_stride, block_size, (__hip_bfloat16 *)k_pool,
        (__hip_bfloat16 *)v_pool);
  } else if (dtype == SPECDEC_F32) {
    kv_write_kernel<float><<<grid, block, 0, s>>>((const float *)k, (const float *)v, n_kv_heads,
                                                 head_dim, meta, batch, width, tables,
                                                 table_stride, block_size, (float *)k_pool,
                                                 (float *)v_pool);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}

SPECDEC_API int specdec_kv_gather(const void *k_pool, const void *v_pool, int dtype,
                                  int32_t n_kv_heads, int32_t head_dim, const int32_t *meta,
                                  int32_t batch, const int32_t *tables, int64_t table_stride,
                                  int32_t block_size, int32_t read_width, void *k_out,
                                  void *v_out, void *stream) {
  if (batch < 0 || read_width < 0 || n_kv_heads <= 0 || head_dim <= 0 || block_size <= 0)
    return SPECDEC_EINVAL;
  if (batch == 0 || read_width == 0) return SPECDEC_OK;
  if (!k_pool || !v_pool || !meta || !tables || !k_out || !v_out) return SPECDEC_EINVAL;
  const int64_t n = (int64_t)batch * n_kv_heads * read_width * head_dim;
  dim3 grid(grid_for(n, 256)), block(256);
  hipStream_t s = as_stream(stream);
  if (dtype == SPECDEC_BF16) {
    kv_gather_kernel<__hip_bfloat16><<<grid, block, 0, s>>>(
        (const __hip_bfloat16 *)k_pool, (const __hip_bfloat16 *)v_pool, n_kv_heads, head_dim,
        meta, batch, tables, table_stride, block_size, read_width, (__hip_bfloat16 *)k_out,
        (__hip_bfloat16 *)v_out);
  } else if (dtype == SPECDEC_F32) {
    kv_gather_kernel<float><<<grid, block, 0, s>>>(
        (const float *)k_pool, (const float *)v_pool, n_kv_heads, head_dim, meta, batch, tables,
        table_stride, block_size, read_width, (float *)k_out, (float *)v_out);
  } else {
    return SPECDEC_EINVAL;
  }
  return launch_status();
}
