// Linear layers of few rows (decode, draft and verify steps) on gfx950 MFMA.
//
// Reference semantics: the q/k/v, o, gate/up and down projections of
// lm/forward.py:56-58,63-64 (transformers' nn.Linear without bias, bf16),
// here with the projections fused as the model stores them (one q|k|v
// weight, one gate|up weight) and, for the residual adds of :63-64, the
// add folded into the same rounding: out = bf16(x W^T + out).
//
// At decode sizes a projection reads a few MB of weights for one to 64
// rows, so its time is the latency of one pass over the weight with every
// load in flight.  Layout: the weight W [N, K] bf16 is split into 16-row
// feature tiles, one workgroup per tile; the K/32 k-steps of the tile are
// split between the workgroup's waves (up to 8), each wave streaming its
// steps' W rows and x rows in batches of 8 k-steps with the next batch's
// loads in flight while one is multiplied on v_mfma_f32_16x16x32_bf16:
//   D[feature 4g+i, row c] += W[feature c'][k 8g..] . x[row c][k 8g..]
// (A = the tile's W rows, lane 16g + c loading the 16 bytes of row c at
// k = 32s + 8g; B = x rows, the same layout, rows past M reading zeros
// through the buffer bound).  The waves' partial sums meet in LDS and are
// added in wave order; lane (c, g) then holds row c's features 4g .. 4g+3.
// More than 16 rows: up to four 16-row column tiles per wave, each W load
// feeding one MFMA per column tile.
// Each output element goes through the same operations whatever M is, so
// a row's result does not depend on the other rows of the call: a token
// verified among k+1 and decoded alone get the same bits.
#include "common.h"

#include <algorithm>

namespace specdec {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;

constexpr int kLinRows = 64;        // rows of a call, at most (four 16-row column tiles)
constexpr int kLinMaxWaves = 8;     // waves per workgroup (k-step split)
constexpr int kLinMaxSteps = 256;   // K / 32, at most (K <= 8192)

struct LinArgs {
  const uint16_t *x;  // [M, K] bf16
  int64_t x_stride;
  const uint16_t *w;  // [N, K] bf16
  int64_t w_stride;
  uint16_t *out;  // [M, N] bf16
  int64_t out_stride;
  int M, K, N;
  int steps;     // K / 32
  int per_wave;  // k-steps per wave (the last waves may take fewer or none)
  int accumulate;
  int w_tiled;  // W in the tiled layout (w_lane below), w_stride = K
};

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// The byte offset in W of lane (c = lane % 16, g = lane / 16)'s 16 bytes at
// k-step 0 of feature row `row` (row c of feature tile `tile`), and the
// bytes from one k-step to the next.  Row-major W [N, w_stride]: row `row`,
// k 8g .. 8g+7.  Tiled W (N % 16 == 0): the 16 x 32 block of each (tile,
// k-step) is 1 KB contiguous in lane order, block (t, s) at (t * K/32 + s) KB,
// lane (c, g) holding row 16t + c, k 32s + 8g .. 32s + 8g + 7 -- every
// load instruction of a wave reads one contiguous KB instead of 64 bytes
// from each of 16 rows.
__device__ __forceinline__ void w_lane(const LinArgs &a, int tile, int row, int lane, unsigned &base,
                                       unsigned &step) {
  if (a.w_tiled) {
    base = (unsigned)(((int64_t)tile * a.steps * 64 + lane) * 16);
    step = 1024u;
  } else {
    base = (unsigned)(((int64_t)row * a.w_stride + 8 * (lane >> 4)) * 2);
    step = 64u;
  }
}

// NCT 16-row column tiles of x per wave (each W load feeds NCT MFMAs),
// KB k-steps per load batch (8 / NCT: the same registers for every NCT).
template <int NCT, int KB>
__global__ __launch_bounds__(kLinMaxWaves * 64) void linear_kernel(LinArgs a) {
  __shared__ f32x4 s_acc[kLinMaxWaves][NCT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int s_lo = wave * a.per_wave;
  const int cnt = max(min(a.per_wave, a.steps - s_lo), 0);
  // W rows past N read the last row (never stored); x rows past M read zeros
  const __amdgpu_buffer_rsrc_t wb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.w), 0, (int)((int64_t)a.N * a.w_stride * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t xb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.x), 0, (int)(((int64_t)(a.M - 1) * a.x_stride + a.K) * 2), 0x00020000);
  const int row = min(n0 + c, a.N - 1);
  unsigned wbase, wstep;
  w_lane(a, blockIdx.x, row, lane, wbase, wstep);
  const unsigned xbase = (unsigned)(((int64_t)c * a.x_stride + 8 * g) * 2);
  const unsigned xtile = (unsigned)(16 * a.x_stride * 2);  // bytes between column tiles
  // accumulate: the values added before the rounding, loaded now for the
  // first column tile this wave stores (wave w stores tiles w, w + nw, ...),
  // so their round trip overlaps the weight's
  // (through a buffer resource, by every wave and call, with no branch --
  // a branch would make the compiler convert, and so wait for, the values
  // right there: rows past M read zeros, features past N are read but never
  // stored, and waves past NCT read tile NCT - 1's and do not use them)
  const int f0 = n0 + 4 * g;
  uint16_t pre[4];
  {
    // (without accumulate the resource is empty: every read is out of range,
    // returns zero and touches no memory)
    const int obytes = a.accumulate ? (int)(((int64_t)(a.M - 1) * a.out_stride + a.N) * 2) : 0;
    const __amdgpu_buffer_rsrc_t ob = __builtin_amdgcn_make_buffer_rsrc(a.out, 0, obytes, 0x00020000);
    const unsigned obase = (unsigned)(((int64_t)(min(wave, NCT - 1) * 16 + c) * a.out_stride + f0) * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) pre[i] = __builtin_amdgcn_raw_buffer_load_b16(ob, obase + 2u * i, 0, 0);
  }
  f32x4 acc[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 A0[KB], A1[KB], B0[KB][NCT], B1[KB][NCT];
  // batch b's loads: steps s_lo + KB b .. (past the wave's last step, its
  // last step again; those are not multiplied)
  auto issue = [&](u32x4 (&A)[KB], u32x4 (&B)[KB][NCT], int b) {
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const unsigned s = (unsigned)(s_lo + min(b * KB + j, cnt - 1));
      A[j] = __builtin_amdgcn_raw_buffer_load_b128(wb, wbase + s * wstep, 0, 0);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        B[j][ct] = __builtin_amdgcn_raw_buffer_load_b128(xb, xbase + ct * xtile + s * 64u, 0, 0);
    }
  };
  auto consume = [&](const u32x4 (&A)[KB], const u32x4 (&B)[KB][NCT], int b) {
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (b * KB + j < cnt) {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, A[j]),
                                                            __builtin_bit_cast(bf16x8, B[j][ct]), acc[ct], 0, 0, 0);
      }
  };
  if (cnt > 0) {
    const int nb = (cnt + KB - 1) / KB;
    issue(A0, B0, 0);
    __builtin_amdgcn_sched_barrier(0);
    int b = 0;
    for (; b + 2 < nb; b += 2) {
      issue(A1, B1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
      consume(A0, B0, b);
      __builtin_amdgcn_sched_barrier(0);
      issue(A0, B0, b + 2);
      __builtin_amdgcn_sched_barrier(0);
      consume(A1, B1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (b + 1 < nb) {  // the last two batches
      issue(A1, B1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
      consume(A0, B0, b);
      __builtin_amdgcn_sched_barrier(0);
      consume(A1, B1, b + 1);
    } else {  // the last batch
      consume(A0, B0, b);
    }
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) s_acc[wave][ct][lane] = acc[ct];
  __syncthreads();
  // the sums of the waves, in wave order: wave w stores column tiles w,
  // w + nw, ...
  for (int ct = wave; ct < NCT; ct += nw) {
    const int r = ct * 16 + c;
    if (r >= a.M) continue;
    f32x4 t = s_acc[0][ct][lane];
    for (int w = 1; w < nw; ++w) t += s_acc[w][ct][lane];
    uint16_t *dst = a.out + (int64_t)r * a.out_stride + f0;
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = t[i];
      if (a.accumulate && f0 + i < a.N) v += bf16_bits_to_f32(ct == wave ? pre[i] : dst[i]);
      o[i] = __builtin_bit_cast(uint16_t, __float2bfloat16(v));  // round to nearest even
    }
    if (f0 + 3 < a.N && ((uintptr_t)dst & 7) == 0) {
      *reinterpret_cast<u32x2 *>(dst) =
          u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (f0 + i < a.N) dst[i] = o[i];
    }
  }
}

// linear_kernel<1, KB> of the attention rows a draft decode step left as
// split partials (attention_decode_parts_kernel: `nparts` per row and query
// head): each workgroup first folds them into its LDS copy of the rows --
// per (row, head, 4 dims) the max of the partials' m, then L and O summed
// in part order with the same exp2 and fma steps as the attention kernel's
// own fold, O / L rounded to bf16 (with kDecWaves parts, that kernel's
// bits) -- while the weight's first load batch is in flight, then projects
// them with the plain projection's k-split (x read from LDS instead of
// memory): the bits of those rows followed by specdec_linear.  Workgroup 0
// also writes the rows to attn_out when that is given.
template <int KB, int NP>
__global__ __launch_bounds__(kLinMaxWaves * 64) void linear_parts_kernel(LinArgs a, const float *parts, int heads,
                                                                          uint16_t *attn_out) {
  extern __shared__ __align__(16) uint16_t s_x[];  // [M][K] bf16
  __shared__ f32x4 s_acc[kLinMaxWaves][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int s_lo = wave * a.per_wave;
  const int cnt = max(min(a.per_wave, a.steps - s_lo), 0);
  const __amdgpu_buffer_rsrc_t wb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.w), 0, (int)((int64_t)a.N * a.w_stride * 2), 0x00020000);
  const int row = min(n0 + c, a.N - 1);
  unsigned wbase, wstep;
  w_lane(a, blockIdx.x, row, lane, wbase, wstep);
  const int f0 = n0 + 4 * g;
  uint16_t pre[4];
  {
    const int obytes = a.accumulate ? (int)(((int64_t)(a.M - 1) * a.out_stride + a.N) * 2) : 0;
    const __amdgpu_buffer_rsrc_t ob = __builtin_amdgcn_make_buffer_rsrc(a.out, 0, obytes, 0x00020000);
    const unsigned obase = (unsigned)(((int64_t)c * a.out_stride + f0) * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) pre[i] = __builtin_amdgcn_raw_buffer_load_b16(ob, obase + 2u * i, 0, 0);
  }
  u32x4 A0[KB], A1[KB];
  auto issue = [&](u32x4 (&A)[KB], int b) {
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const unsigned s = (unsigned)(s_lo + min(b * KB + j, cnt - 1));
      A[j] = __builtin_amdgcn_raw_buffer_load_b128(wb, wbase + s * wstep, 0, 0);
    }
  };
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  const int xrow = c * a.K;  // this lane's row of x in LDS (rows past M are zero)
  // the batch's x operands are read from LDS first, then its MFMAs run back
  // to back (reading each operand just before its MFMA waited out one LDS
  // round trip per k-step)
  auto consume = [&](const u32x4 (&A)[KB], int b) {
    u32x4 bv[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      bv[j] = u32x4{0u, 0u, 0u, 0u};
      if (c < a.M && b * KB + j < cnt)
        bv[j] = *reinterpret_cast<const u32x4 *>(&s_x[xrow + 32 * (s_lo + b * KB + j) + 8 * g]);
    }
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (b * KB + j < cnt)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, A[j]),
                                                      __builtin_bit_cast(bf16x8, bv[j]), acc, 0, 0, 0);
  };
  if (cnt > 0) issue(A0, 0);
  // ---- the fold: item (row r, head hq, dims d0 .. d0+3)
  const int items = a.M * heads * 16;
  for (int it = tid; it < items; it += blockDim.x) {
    const int r = it / (heads * 16), hq = (it / 16) % heads, d0 = (it % 16) * 4;
    const float *pp = parts + ((int64_t)r * heads + hq) * NP * kDecPart;
    // every part's values first, in one round trip
    float mw[NP], lw[NP];
    f32x4 ow[NP];
#pragma unroll
    for (int w = 0; w < NP; ++w) {
      const f32x2 ml = *reinterpret_cast<const f32x2 *>(pp + w * kDecPart);
      mw[w] = ml[0];
      lw[w] = ml[1];
      ow[w] = *reinterpret_cast<const f32x4 *>(pp + w * kDecPart + 4 + d0);
    }
    float M = mw[0];
#pragma unroll
    for (int w = 1; w < NP; ++w) M = fmaxf(M, mw[w]);
    float L = 0.0f, O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < NP; ++w) {
      const float f = (mw[w] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - M);
      L = __builtin_fmaf(f, lw[w], L);
#pragma unroll
      for (int i = 0; i < 4; ++i) O[i] = __builtin_fmaf(f, ow[w][i], O[i]);
    }
    uint16_t ob[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ob[i] = __builtin_bit_cast(uint16_t, from_f32<__hip_bfloat16>(O[i] / L));
    const u32x2 packed = u32x2{(uint32_t)ob[0] | ((uint32_t)ob[1] << 16), (uint32_t)ob[2] | ((uint32_t)ob[3] << 16)};
    *reinterpret_cast<u32x2 *>(&s_x[r * a.K + hq * 64 + d0]) = packed;
    if (attn_out && blockIdx.x == 0)
      *reinterpret_cast<u32x2 *>(attn_out + (int64_t)r * a.K + hq * 64 + d0) = packed;
  }
  __syncthreads();
  if (cnt > 0) {
    const int nb = (cnt + KB - 1) / KB;
    int b = 0;
    for (; b + 2 < nb; b += 2) {
      issue(A1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
      consume(A0, b);
      __builtin_amdgcn_sched_barrier(0);
      issue(A0, b + 2);
      __builtin_amdgcn_sched_barrier(0);
      consume(A1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (b + 1 < nb) {
      issue(A1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
      consume(A0, b);
      __builtin_amdgcn_sched_barrier(0);
      consume(A1, b + 1);
    } else {
      consume(A0, b);
    }
  }
  s_acc[wave][lane] = acc;
  __syncthreads();
  // the sums of the waves, in wave order (wave 0 stores), then the value
  // added before the rounding
  if (wave == 0 && c < a.M) {
    f32x4 t = s_acc[0][lane];
    for (int w = 1; w < nw; ++w) t += s_acc[w][lane];
    uint16_t *dst = a.out + (int64_t)c * a.out_stride + f0;
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = t[i];
      if (a.accumulate && f0 + i < a.N) v += bf16_bits_to_f32(pre[i]);
      o[i] = __builtin_bit_cast(uint16_t, __float2bfloat16(v));
    }
    if (f0 + 3 < a.N && ((uintptr_t)dst & 7) == 0) {
      *reinterpret_cast<u32x2 *>(dst) =
          u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (f0 + i < a.N) dst[i] = o[i];
    }
  }
}

// The gate/up projection with the MLP's activation in its epilogue: a
// workgroup computes feature tile t of the gate half (W rows 16 t ..) and
// of the up half (W rows inter + 16 t ..) of the fused [2 inter, K] weight
// with the k-split the plain projection of that weight takes, so each of
// its sums has the plain projection's bits; the sums are rounded to bf16
// (the projection's output) and turned into act = SiLU(bf16(s g)) *
// bf16(s u) with the row's post-attention norm scale s computed here from
// the residual row (row_rms_scale_bf16, the MLP norm kernel's arithmetic).
// So act has the bits of the projection followed by rms_silu_mul, in one
// launch, and the [rows, 2 inter] intermediate is never written.
template <int NCT, int KB, int NVH>
__global__ __launch_bounds__(kLinMaxWaves * 64) void linear_silu_kernel(LinArgs a, const uint16_t *hid,
                                                                         int64_t hid_stride, int hdim, float eps,
                                                                         int inter) {
  __shared__ f32x4 s_acc[kLinMaxWaves][2][NCT][64];
  __shared__ float s_scale[kLinRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int s_lo = wave * a.per_wave;
  const int cnt = max(min(a.per_wave, a.steps - s_lo), 0);
  const __amdgpu_buffer_rsrc_t wb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.w), 0, (int)((int64_t)a.N * a.w_stride * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t xb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.x), 0, (int)(((int64_t)(a.M - 1) * a.x_stride + a.K) * 2), 0x00020000);
  const int rg = min(n0 + c, inter - 1);  // past the gate half: its last row, never stored
  unsigned gbase, ubase, wstep;
  w_lane(a, blockIdx.x, rg, lane, gbase, wstep);
  w_lane(a, inter / 16 + blockIdx.x, inter + rg, lane, ubase, wstep);
  const unsigned xbase = (unsigned)(((int64_t)c * a.x_stride + 8 * g) * 2);
  const unsigned xtile = (unsigned)(16 * a.x_stride * 2);
  // the first pass over this wave's first residual row (row `wave`), loaded
  // now so its round trip overlaps the weight's (rows past M: not used)
  // (and of its second row, wave + nw, when the call has more rows than waves)
  const int nvh = hdim / 8;
  const u32x4 *h0 = reinterpret_cast<const u32x4 *>(hid + (int64_t)min(wave, a.M - 1) * hid_stride);
  const u32x4 *h1 = reinterpret_cast<const u32x4 *>(hid + (int64_t)min(wave + nw, a.M - 1) * hid_stride);
  u32x4 hv0[NVH], hv1[NVH];
  row_pass_loads<NVH>(h0, 0, nvh, lane, hv0);
  row_pass_loads<NVH>(h1, 0, nvh, lane, hv1);
  f32x4 accg[NCT], accu[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) accg[ct] = accu[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 G0[KB], G1[KB], U0[KB], U1[KB], B0[KB][NCT], B1[KB][NCT];
  auto issue = [&](u32x4 (&G)[KB], u32x4 (&U)[KB], u32x4 (&B)[KB][NCT], int b) {
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const unsigned s = (unsigned)(s_lo + min(b * KB + j, cnt - 1));
      G[j] = __builtin_amdgcn_raw_buffer_load_b128(wb, gbase + s * wstep, 0, 0);
      U[j] = __builtin_amdgcn_raw_buffer_load_b128(wb, ubase + s * wstep, 0, 0);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        B[j][ct] = __builtin_amdgcn_raw_buffer_load_b128(xb, xbase + ct * xtile + s * 64u, 0, 0);
    }
  };
  auto consume = [&](const u32x4 (&G)[KB], const u32x4 (&U)[KB], const u32x4 (&B)[KB][NCT], int b) {
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (b * KB + j < cnt) {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
          accg[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, G[j]),
                                                             __builtin_bit_cast(bf16x8, B[j][ct]), accg[ct], 0, 0, 0);
          accu[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, U[j]),
                                                             __builtin_bit_cast(bf16x8, B[j][ct]), accu[ct], 0, 0, 0);
        }
      }
  };
  if (cnt > 0) {
    const int nb = (cnt + KB - 1) / KB;
    issue(G0, U0, B0, 0);
    __builtin_amdgcn_sched_barrier(0);
    int b = 0;
    for (; b + 2 < nb; b += 2) {
      issue(G1, U1, B1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
      consume(G0, U0, B0, b);
      __builtin_amdgcn_sched_barrier(0);
      issue(G0, U0, B0, b + 2);
      __builtin_amdgcn_sched_barrier(0);
      consume(G1, U1, B1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (b + 1 < nb) {
      issue(G1, U1, B1, b + 1);
      __builtin_amdgcn_sched_barrier(0);
      consume(G0, U0, B0, b);
      __builtin_amdgcn_sched_barrier(0);
      consume(G1, U1, B1, b + 1);
    } else {
      consume(G0, U0, B0, b);
    }
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    s_acc[wave][0][ct][lane] = accg[ct];
    s_acc[wave][1][ct][lane] = accu[ct];
  }
  // the rows' norm scales, wave w taking rows w, w + nw, ...
  for (int r = wave; r < a.M; r += nw) {
    const u32x4 *hr = reinterpret_cast<const u32x4 *>(hid + (int64_t)r * hid_stride);
    const float sc = r == wave        ? row_rms_scale_bf16_from<NVH>(hr, hv0, nvh, hdim, eps, lane)
                     : r == wave + nw ? row_rms_scale_bf16_from<NVH>(hr, hv1, nvh, hdim, eps, lane)
                                      : row_rms_scale_bf16<NVH>(hr, nvh, hdim, eps, lane);
    if (lane == 0) s_scale[r] = sc;
  }
  __syncthreads();
  const int f0 = n0 + 4 * g;
  for (int ct = wave; ct < NCT; ct += nw) {
    const int r = ct * 16 + c;
    if (r >= a.M) continue;
    f32x4 tg = s_acc[0][0][ct][lane], tu = s_acc[0][1][ct][lane];
    for (int w = 1; w < nw; ++w) {
      tg += s_acc[w][0][ct][lane];
      tu += s_acc[w][1][ct][lane];
    }
    const float sc = s_scale[r];
    uint16_t *dst = a.out + (int64_t)r * a.out_stride + f0;
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // the projection's bf16 outputs, then the activation
      const float gv = to_f32(from_f32<__hip_bfloat16>(tg[i]));
      const float uv = to_f32(from_f32<__hip_bfloat16>(tu[i]));
      o[i] = silu_mul_scaled_bf16(gv, uv, sc);
    }
    if (f0 + 3 < inter && ((uintptr_t)dst & 7) == 0) {
      *reinterpret_cast<u32x2 *>(dst) =
          u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (f0 + i < inter) dst[i] = o[i];
    }
  }
}

// The k-split of a [N, K] weight: waves per workgroup and k-steps per wave.
static void linear_split(LinArgs &a, int64_t tiles, int &waves) {
  // The k-split depends on the weight's shape only (never on the rows), so
  // a row's sums are the same in every call.  Up to 8 k-steps per wave
  // (one load batch) while that takes at most 8 waves; with a feature tile
  // for every compute unit, 4 waves of up to 16 steps (more workgroups
  // resident at once, the whole weight requested in one pass); the steps of
  // wider weights spread evenly over 8 waves.
  const int max_waves = tiles >= cu_count() ? 4 : kLinMaxWaves;
  waves = std::min(max_waves, (a.steps + 7) / 8);
  a.per_wave = (a.steps + waves - 1) / waves;
}

}  // namespace specdec

using namespace specdec;

SPECDEC_API int specdec_linear(const void *x, int64_t x_stride, const void *w, int64_t w_stride, int32_t w_layout,
                               int64_t rows, int64_t in_features, int64_t out_features, void *out,
                               int64_t out_stride, int32_t accumulate, void *stream) {
  if (rows < 0 || in_features <= 0 || out_features <= 0) return SPECDEC_EINVAL;
  if (w_layout != SPECDEC_W_ROWS && w_layout != SPECDEC_W_TILED) return SPECDEC_EINVAL;
  if (w_layout == SPECDEC_W_TILED) {
    if (out_features % 16 != 0) return SPECDEC_EINVAL;
    w_stride = in_features;
  }
  if (rows == 0) return SPECDEC_OK;
  if (rows > kLinRows || in_features % 32 != 0 || in_features / 32 > kLinMaxSteps) return SPECDEC_EUNSUPPORTED;
  // one buffer resource addresses W, another the rows of x (32-bit offsets)
  if (out_features * w_stride * 2 > INT32_MAX || out_features > INT32_MAX / 2) return SPECDEC_EUNSUPPORTED;
  if ((int64_t)kLinRows * std::max(x_stride, out_stride) * 2 > INT32_MAX) return SPECDEC_EUNSUPPORTED;
  if (!x || !w || !out || x_stride < in_features || w_stride < in_features || out_stride < out_features)
    return SPECDEC_EINVAL;
  if (x_stride % 8 || w_stride % 8 || ((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)out & 1))
    return SPECDEC_EINVAL;
  LinArgs a{};
  a.x = (const uint16_t *)x;
  a.x_stride = x_stride;
  a.w = (const uint16_t *)w;
  a.w_stride = w_stride;
  a.out = (uint16_t *)out;
  a.out_stride = out_stride;
  a.M = (int)rows;
  a.K = (int)in_features;
  a.N = (int)out_features;
  a.steps = (int)(in_features / 32);
  a.accumulate = accumulate != 0;
  a.w_tiled = w_layout == SPECDEC_W_TILED;
  const int64_t tiles = (out_features + 15) / 16;
  if (tiles > INT32_MAX) return SPECDEC_EUNSUPPORTED;
  int waves = 0;
  linear_split(a, tiles, waves);
  const dim3 grid((unsigned)tiles), block((unsigned)(64 * waves));
  hipStream_t s = as_stream(stream);
  if (rows <= 16) linear_kernel<1, 8><<<grid, block, 0, s>>>(a);
  else if (rows <= 32) linear_kernel<2, 4><<<grid, block, 0, s>>>(a);
  else linear_kernel<4, 2><<<grid, block, 0, s>>>(a);
  return launch_status();
}

SPECDEC_API int specdec_linear_attn_parts(const float *parts, int64_t rows, int64_t n_heads, int32_t nparts,
                                         const void *w, int64_t w_stride, int32_t w_layout, int64_t out_features,
                                         void *out, int64_t out_stride, int32_t accumulate, void *attn_out,
                                         void *stream) {
  if (rows < 0 || n_heads <= 0 || out_features <= 0) return SPECDEC_EINVAL;
  if (nparts != 4 && nparts != 8 && nparts != 16) return SPECDEC_EINVAL;
  if (((uintptr_t)parts & 15) || (attn_out && ((uintptr_t)attn_out & 7))) return SPECDEC_EINVAL;
  if (w_layout != SPECDEC_W_ROWS && w_layout != SPECDEC_W_TILED) return SPECDEC_EINVAL;
  if (rows == 0) return SPECDEC_OK;
  const int64_t k = n_heads * 64;
  if (w_layout == SPECDEC_W_TILED) {
    if (out_features % 16 != 0) return SPECDEC_EINVAL;
    w_stride = k;
  }
  if (rows > 16 || k > 2048) return SPECDEC_EUNSUPPORTED;
  if (out_features * w_stride * 2 > INT32_MAX || out_features > INT32_MAX / 2) return SPECDEC_EUNSUPPORTED;
  if (16 * out_stride * 2 > INT32_MAX) return SPECDEC_EUNSUPPORTED;
  if (!parts || !w || !out || w_stride < k || out_stride < out_features) return SPECDEC_EINVAL;
  if (w_stride % 8 || ((uintptr_t)w & 15) || ((uintptr_t)out & 1)) return SPECDEC_EINVAL;
  LinArgs a{};
  a.w = (const uint16_t *)w;
  a.w_stride = w_stride;
  a.out = (uint16_t *)out;
  a.out_stride = out_stride;
  a.M = (int)rows;
  a.K = (int)k;
  a.N = (int)out_features;
  a.steps = (int)(k / 32);
  a.accumulate = accumulate != 0;
  a.w_tiled = w_layout == SPECDEC_W_TILED;
  const int64_t tiles = (out_features + 15) / 16;
  if (tiles > INT32_MAX) return SPECDEC_EUNSUPPORTED;
  int waves = 0;
  linear_split(a, tiles, waves);  // the plain projection's k-split
  const dim3 grid((unsigned)tiles), block((unsigned)(64 * waves));
  const size_t lds = (size_t)rows * k * 2;
  hipStream_t s = as_stream(stream);
  uint16_t *ao = (uint16_t *)attn_out;
  if (nparts == 4) linear_parts_kernel<8, 4><<<grid, block, lds, s>>>(a, parts, (int)n_heads, ao);
  else if (nparts == 8) linear_parts_kernel<8, 8><<<grid, block, lds, s>>>(a, parts, (int)n_heads, ao);
  else linear_parts_kernel<8, 16><<<grid, block, lds, s>>>(a, parts, (int)n_heads, ao);
  return launch_status();
}

SPECDEC_API int specdec_linear_silu(const void *x, int64_t x_stride, const void *w, int64_t w_stride,
                                    int32_t w_layout, int64_t rows, int64_t in_features, int64_t inter,
                                    const void *hidden, int64_t hidden_stride, int64_t hidden_dim, float eps,
                                    void *out, int64_t out_stride, void *stream) {
  if (rows < 0 || in_features <= 0 || inter <= 0 || hidden_dim <= 0) return SPECDEC_EINVAL;
  if (w_layout != SPECDEC_W_ROWS && w_layout != SPECDEC_W_TILED) return SPECDEC_EINVAL;
  if (w_layout == SPECDEC_W_TILED) {
    if (inter % 16 != 0) return SPECDEC_EINVAL;
    w_stride = in_features;
  }
  if (rows == 0) return SPECDEC_OK;
  if (rows > kLinRows || in_features % 32 != 0 || in_features / 32 > kLinMaxSteps) return SPECDEC_EUNSUPPORTED;
  if (hidden_dim % 8 != 0 || hidden_dim > 8 * 64 * 8) return SPECDEC_EUNSUPPORTED;
  const int64_t n = 2 * inter;
  if (n * w_stride * 2 > INT32_MAX || n > INT32_MAX / 2) return SPECDEC_EUNSUPPORTED;
  if ((int64_t)kLinRows * x_stride * 2 > INT32_MAX) return SPECDEC_EUNSUPPORTED;
  if (!x || !w || !out || !hidden || x_stride < in_features || w_stride < in_features || out_stride < inter ||
      hidden_stride < hidden_dim)
    return SPECDEC_EINVAL;
  if (x_stride % 8 || w_stride % 8 || hidden_stride % 8 || ((uintptr_t)x & 15) || ((uintptr_t)w & 15) ||
      ((uintptr_t)hidden & 15) || ((uintptr_t)out & 1))
    return SPECDEC_EINVAL;
  LinArgs a{};
  a.x = (const uint16_t *)x;
  a.x_stride = x_stride;
  a.w = (const uint16_t *)w;
  a.w_stride = w_stride;
  a.out = (uint16_t *)out;
  a.out_stride = out_stride;
  a.M = (int)rows;
  a.K = (int)in_features;
  a.N = (int)n;
  a.steps = (int)(in_features / 32);
  a.w_tiled = w_layout == SPECDEC_W_TILED;
  // the plain projection's k-split for this [2 inter, K] weight
  int waves = 0;
  linear_split(a, (n + 15) / 16, waves);
  const dim3 grid((unsigned)((inter + 15) / 16)), block((unsigned)(64 * waves));
  const uint16_t *h = (const uint16_t *)hidden;
  const int hd = (int)hidden_dim, nvec = hd / 8;
  hipStream_t s = as_stream(stream);
#define SPECDEC_LINEAR_SILU(NCT, KB)                                                                          \
  do {                                                                                                    \
    if (nvec <= 2 * 64) linear_silu_kernel<NCT, KB, 2><<<grid, block, 0, s>>>(a, h, hidden_stride, hd, eps, (int)inter); \
    else if (nvec <= 4 * 64) linear_silu_kernel<NCT, KB, 4><<<grid, block, 0, s>>>(a, h, hidden_stride, hd, eps, (int)inter); \
    else linear_silu_kernel<NCT, KB, 8><<<grid, block, 0, s>>>(a, h, hidden_stride, hd, eps, (int)inter); \
  } while (0)
  if (rows <= 16) SPECDEC_LINEAR_SILU(1, 4);
  else if (rows <= 32) SPECDEC_LINEAR_SILU(2, 2);
  else SPECDEC_LINEAR_SILU(4, 1);
#undef SPECDEC_LINEAR_SILU
  return launch_status();
}
