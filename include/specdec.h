/*
 * specdec.h - C ABI of libspecdec.so, the gfx950 (MI355X) kernels behind the
 * speculative-decoding hot path of beriltatli/speculative-decoder.
 *
 * Every entry point takes plain device pointers, element counts and strides
 * (in elements, not bytes) and a HIP stream passed as `void *` (0 = the null
 * stream).  Nothing here allocates device memory: buffers are owned by the
 * caller.  Every call returns an `int` status:
 *
 *   SPECDEC_OK           0  launched
 *   SPECDEC_EINVAL       1  a size, stride or pointer argument is out of range
 *   SPECDEC_EHIP         2  the HIP launch failed (hipGetLastError)
 *   SPECDEC_EUNSUPPORTED 3  a shape the kernels do not implement (e.g. head_dim != 64)
 *   SPECDEC_ENOSCRATCH   4  the call needs more scratch than the library's static
 *                           buffer holds (specdec_paged_attention_static only)
 *
 * Data-dependent conditions that the reference raises on (a drafted token
 * with zero draft probability, a double free) are reported through status
 * words written by the kernel into caller memory, so the host decides which
 * exception to raise after it reads them.
 *
 * Element types are selected with SPECDEC_F32 / SPECDEC_F64 / SPECDEC_BF16.
 *
 * Per-call batch metadata ("meta") is one int32 array of 3*batch entries:
 *   meta[0*batch + b] = table row of batch entry b (row in `tables`)
 *   meta[1*batch + b] = cached length before this call (past)
 *   meta[2*batch + b] = tokens appended by this call (n_new, <= width)
 * Block tables are int32 [rows, table_stride]; entry [r, j] is the physical
 * block holding positions j*block_size .. j*block_size+block_size-1 of row r.
 *
 * KV pool layout, per layer:
 *   K: [num_blocks, n_kv_heads, block_size, head_dim]   (token-major tile)
 *   V: [num_blocks, n_kv_heads, head_dim, block_size]   (dim-major tile)
 * so that one (block, head) tile of K or V is contiguous in HBM.
 */
#ifndef SPECDEC_H
#define SPECDEC_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPECDEC_OK 0
#define SPECDEC_EINVAL 1
#define SPECDEC_EHIP 2
#define SPECDEC_EUNSUPPORTED 3
#define SPECDEC_ENOSCRATCH 4

#define SPECDEC_F32 0
#define SPECDEC_F64 1
#define SPECDEC_BF16 2

/* Layouts of a projection weight W [N, K] bf16 (w_layout of the linear
 * entries):
 *   SPECDEC_W_ROWS   row-major, row n at w + n * w_stride;
 *   SPECDEC_W_TILED  N % 16 == 0 and K % 32 == 0, element (n, k) at
 *                    ((n / 16 * (K / 32) + k / 32) * 64 + (k % 32) / 8 * 16
 *                     + n % 16) * 8 + k % 8
 *                    -- each 16 x 32 block 1 KB contiguous, in the order a
 *                    wave's lanes load it (w_stride is ignored).  The same
 *                    arithmetic as SPECDEC_W_ROWS, so the same bits; the
 *                    loads are contiguous, 1.2-1.4x the throughput at
 *                    decode sizes. */
#define SPECDEC_W_ROWS 0
#define SPECDEC_W_TILED 1

/* ABI version; bumped whenever a signature or the meaning of an argument
 * below changes (currently 15). */
int specdec_abi_version(void);

/* ---------------------------------------------------------------- accept --- */

/* Temperature softmax, or one-hot argmax at temperature 0 (ties -> lowest id).
 * logits [rows, vocab] (row_stride apart, dtype F32/F64/BF16) -> out fp32
 * (out_stride apart).  At temperature 0 a non-NULL index_out also receives
 * each row's argmax (index_out[row * index_stride]): the token an
 * inverse-CDF draw from that one-hot row returns for any u in [0, 1).
 * Replaces lm/sampling.py:13-18 `probabilities`. */
int specdec_probabilities(const void *logits, int dtype, int64_t rows, int64_t vocab,
                          int64_t row_stride, float temperature, float *out,
                          int64_t out_stride, int64_t *index_out, int64_t index_stride,
                          void *stream);

/* Bytes of the workspace specdec_accept_reject and
 * specdec_accept_reject_logits use for `batch` rows (arrival counters, the
 * call epoch, and each row's meeting words).  It must be zeroed once, when
 * it is allocated; calls never need it cleared again.  Calls sharing a
 * workspace must be ordered (one stream). */
int specdec_accept_workspace(int64_t batch, int64_t *bytes);

/* Fused accept-reject for a batch: gather p(x), q(x) of the drafted tokens,
 * test u*q(x) < p(x), count the leading accepts n, build the residual
 * norm(max(0, p[n] - q[n])) (q[k] is the implicit zero row, so n == k is the
 * bonus token sampled from p[k]) and sample it by inverse CDF with u_residual.
 * p [batch, k+1, vocab], q [batch, k, vocab] (dtype F32 or F64, strides in
 * elements), draft int64 [batch, k], u_accept [batch, k] and u_residual [batch]
 * of the same dtype as p.  out int64 [3, batch]: n_accepted, next_token, and
 * a flag that is 1 when a drafted token had q(x) <= 0 or an id outside
 * [0, vocab).
 * With a workspace (fp32, and batch * chunks within one workgroup per
 * compute unit) each row is spread over many workgroups of one launch that
 * exchange chunk values twice.  A workgroup reads the values it waits for
 * at most `spin` more times after its first read (not at all for spin < 0)
 * and then computes the missing chunks' values itself, with the same bits,
 * so every call completes whether or not a row's workgroups are resident
 * together.  Without a workspace one workgroup runs each row.
 * Replaces spec/accept.py:44-79 `accept_reject` with the default residual
 * (spec/accept.py:18-26) and spec/accept.py:29-35 `sample_inverse_cdf`. */
int specdec_accept_reject(const void *p, const void *q, int dtype,
                          int64_t p_batch_stride, int64_t p_row_stride,
                          int64_t q_batch_stride, int64_t q_row_stride,
                          const int64_t *draft, const void *u_accept,
                          const void *u_residual, int64_t batch, int64_t k,
                          int64_t vocab, int64_t *out, void *workspace,
                          int64_t workspace_bytes, int32_t spin, void *stream);

/* Accept-reject from logits in one launch: p = probabilities(target_logits,
 * temperature) and q = probabilities(draft_logits, temperature) -- the
 * softmax of logits / T, or the one-hot of the lowest-index argmax at
 * T = 0 -- are formed inside the launch from row statistics the row's
 * workgroups exchange, and the accept test, residual and inverse-CDF sample
 * follow as in specdec_accept_reject.  Every logit is read from memory once
 * (the residual row's chunk a second time); no probability row is written.
 * target_logits [batch, k+1, vocab] and draft_logits [batch, k, vocab] fp32
 * (16-byte aligned rows: vocab and the strides multiples of 4), k <= 16;
 * draft, u_accept, u_residual, out, workspace and spin as above (the
 * workspace is required).  SPECDEC_EUNSUPPORTED when the shapes do not fit
 * (more rows than two workgroups per compute unit hold: 64 rows of a 49152
 * vocabulary on 256 compute units), and then probabilities + accept_reject
 * give the same decisions.
 * Replaces lm/sampling.py:13-18 `probabilities` of the target and draft
 * rows followed by spec/accept.py:44-79 `accept_reject`. */
int specdec_accept_reject_logits(const void *target_logits, const void *draft_logits, int dtype,
                                 int64_t t_batch_stride, int64_t t_row_stride,
                                 int64_t d_batch_stride, int64_t d_row_stride, float temperature,
                                 const int64_t *draft, const void *u_accept,
                                 const void *u_residual, int64_t batch, int64_t k, int64_t vocab,
                                 int64_t *out, void *workspace, int64_t workspace_bytes,
                                 int32_t spin, void *stream);

/* First stage of accept-reject alone (for a caller-supplied residual):
 * out int64 [2, batch]: n_accepted and a flag that is 1 when a drafted token
 * had q(x) <= 0 or an id outside [0, vocab) (such an id is never read
 * through; it counts as the first rejection).
 * Replaces spec/accept.py:65-71. */
int specdec_accept_count(const void *p, const void *q, int dtype,
                         int64_t p_batch_stride, int64_t p_row_stride,
                         int64_t q_batch_stride, int64_t q_row_stride,
                         const int64_t *draft, const void *u_accept, int64_t batch,
                         int64_t k, int64_t vocab, int64_t *out, void *stream);

/* Inverse-CDF sampling: token i is chosen iff u*total lies in
 * [cdf[i-1], cdf[i]) with the prefix sums accumulated in fp64 and rounded to
 * the element type (searchsorted right, clamped to vocab-1).
 * probs [batch, vocab] (row_stride apart), u [batch] of the same dtype, out int64 [batch].
 * Replaces spec/accept.py:29-35 `sample_inverse_cdf`. */
int specdec_sample_inverse_cdf(const void *probs, int dtype, int64_t batch,
                               int64_t vocab, int64_t row_stride, const void *u,
                               int64_t *out, void *stream);

/* out fp32 [n, vocab] = one_hot(ids[n], vocab).  Replaces the
 * `one_hot(...).float()` of spec/ngram.py:23 and lm/sampling.py:17. */
int specdec_one_hot(const int64_t *ids, int64_t n, int64_t vocab, float *out,
                    void *stream);

/* ----------------------------------------------------------------- n-gram --- */

/* Prompt lookup for a batch of token histories.  history int32 [batch,
 * row_stride], lengths int32 [batch] (>= 1).  For n = min(max_n, len-1) down
 * to 1 the most recent earlier occurrence of the last n tokens is found; the
 * k tokens that followed it are proposed, the copy reading its own output
 * once it passes the end of the history.  Without a match the last token is
 * repeated k times.  draft int64 [batch, k]; match int32 [batch, 2] = (start
 * of the matched n-gram, n), or (-1, 0) when nothing matched.  A length
 * beyond row_stride is taken as row_stride (no read leaves a row).
 * Replaces spec/ngram.py:32-45 `lookup` (and the per-row loop of :19-23). */
int specdec_ngram_lookup(const int32_t *history, int64_t row_stride,
                         const int32_t *lengths, int64_t batch, int32_t k,
                         int32_t max_n, int64_t *draft, int32_t *match,
                         void *stream);

/* ------------------------------------------------------------------ cache --- */

/* One batched pass of the LIFO block allocator.  free_stack int32
 * [num_blocks] holds the free ids, top of stack at index top-1; used uint8
 * [num_blocks] marks allocated blocks.  entries int32 [(n_push+n_pop), 4]
 * rows of (table row, first column, count, stack offset):
 *   push e (rollback / release, in order): for j < count
 *       free_stack[top + off + j] = tables[row, col + j]; used[...] = 0
 *   pop e (growth, after every push):      for j < count
 *       tables[row, col + j] = free_stack[top + n_pushed - 1 - off - j]
 * `popped` (optional, int32 [total popped]) receives the popped ids in order.
 * Replaces cache/paged.py:28-40 (allocate/free) as driven by
 * cache/paged.py:54-71 (grow_to/shrink_to) and cache/kv.py:79-87,114-118. */
int specdec_block_plan(int32_t *tables, int64_t table_stride, int32_t *free_stack,
                       uint8_t *used, int64_t num_blocks, int32_t top,
                       const int32_t *entries, int32_t n_push, int32_t n_pop,
                       int32_t *popped, void *stream);

/* Single checked free: if used[block] is 0, status[0] = 1 and nothing changes
 * (double free); otherwise the block is pushed at free_stack[top] and
 * status[0] = 0.  Replaces cache/paged.py:36-40. */
int specdec_block_free_checked(int32_t *free_stack, uint8_t *used,
                               int64_t num_blocks, int32_t top, int32_t block,
                               int32_t *status, void *stream);

/* Slot ids of positions [start, stop) through one table row:
 * out[i] = row[p / bs] * bs + p % bs.  Replaces cache/paged.py:73-76. */
int specdec_block_slots(const int32_t *table_row, int64_t start, int64_t stop,
                        int32_t block_size, int64_t *out, void *stream);

/* The reference's slot map for one append (cache/kv.py:88-99): write int64
 * [sum n_new] slots of the new tokens, write_index int64 [sum n_new] =
 * b*width + j, read int64 [batch, read_width] (slot of every cached position,
 * 0 past the row's total).  write_offsets int32 [batch] = exclusive scan of
 * n_new. */
int specdec_slot_map(const int32_t *tables, int64_t table_stride,
                     const int32_t *meta, int32_t batch, int32_t block_size,
                     int32_t width, int32_t read_width,
                     const int32_t *write_offsets, int64_t *write,
                     int64_t *write_index, int64_t *read, void *stream);

/* Fused RoPE + cache append for one layer.  qkv [batch, width, (H + 2*Hkv) *
 * head_dim] (token_stride elements between tokens; q heads, then k heads,
 * then v heads).  For every real token (t < n_new[b]) at position
 * past[b] + t: q and k are rotated in place (HF rotate_half convention, cos
 * and sin fp32 tables [max_positions, head_dim/2]) and k, v are written into
 * the layer's paged pools at the slot given by the block table.
 * Replaces lm/forward.py:53,60 (rotary) + cache/kv.py:101-106 (write). */
int specdec_rope_append(void *qkv, int dtype, int64_t token_stride, int32_t n_heads,
                        int32_t n_kv_heads, int32_t head_dim, const float *cos_table,
                        const float *sin_table, int64_t max_positions,
                        const int32_t *meta, int32_t batch, int32_t width,
                        const int32_t *tables, int64_t table_stride,
                        int32_t block_size, void *k_pool, void *v_pool, void *stream);

/* Cache append without rotation: k, v [batch, Hkv, width, head_dim]
 * contiguous (the reference's write() argument layout).
 * Replaces cache/kv.py:101-106. */
int specdec_kv_write(const void *k, const void *v, int dtype, int32_t n_kv_heads,
                     int32_t head_dim, const int32_t *meta, int32_t batch,
                     int32_t width, const int32_t *tables, int64_t table_stride,
                     int32_t block_size, void *k_pool, void *v_pool, void *stream);

/* Copy of every cached position, k_out/v_out [batch, Hkv, read_width,
 * head_dim] (zeros past each row's total).  Diagnostic counterpart of
 * cache/kv.py:108-112; the attention kernel reads blocks in place instead. */
int specdec_kv_gather(const void *k_pool, const void *v_pool, int dtype,
                      int32_t n_kv_heads, int32_t head_dim, const int32_t *meta,
                      int32_t batch, const int32_t *tables, int64_t table_stride,
                      int32_t block_size, int32_t read_width, void *k_out,
                      void *v_out, void *stream);

/* ------------------------------------------------------------ layer glue --- */

/* Residual add + RMSNorm over rows of `dim` <= 8192 (BF16 or F32).  If delta is not
 * null, hidden <- hidden + delta (rounded to the element type) first; then
 * out <- weight * round(hidden * rsqrt(mean(hidden^2) + eps)).  The norm and
 * the add follow transformers' LlamaRMSNorm and the residual adds of the
 * decoder layer that lm/forward.py:56,64-66 runs. */
int specdec_add_rmsnorm(void *hidden, const void *delta, const void *weight, void *out, int dtype,
                        int64_t rows, int64_t dim, float eps, void *stream);

/* out [rows, inter] = round(silu(gate)) * up, with gate_up [rows, 2*inter]
 * holding gate then up per row (the Llama MLP activation, lm/forward.py:65). */
int specdec_silu_mul(const void *gate_up, void *out, int dtype, int64_t rows, int64_t inter,
                     void *stream);

/* The post-attention RMSNorm and the MLP activation around a gate/up
 * projection of the unnormalised residual stream (lm/forward.py:64-65, with
 * transformers' LlamaRMSNorm and LlamaMLP).  gate_up [rows, 2*inter] holds
 * hidden @ (W diag(norm weight))^T; per row, s = rsqrt(mean(hidden^2) + eps)
 * over hidden [rows, dim], then gate = round(s * gate), up = round(s * up) and
 * out [rows, inter] = round(round(silu(gate)) * up).  Algebraically the same
 * as normalising before the projection; the rounding points differ.  The row
 * sum of squares is reduced in one fixed order, so a row's result does not
 * depend on the other rows of the call. */
int specdec_rms_silu_mul(const void *gate_up, const void *hidden, void *out, int dtype, int64_t rows,
                         int64_t inter, int64_t dim, float eps, void *stream);

/* -------------------------------------------------------------- attention --- */

/* Workspace needed by specdec_paged_attention for a call shape: `floats`
 * fp32 elements of split partials (no initialisation needed). */
int specdec_attention_workspace(int32_t batch, int32_t width, int32_t n_heads,
                                int32_t n_kv_heads, int32_t head_dim,
                                int32_t max_kv_len, int32_t split_tokens,
                                int64_t *floats);

/* Split-KV size the attention kernel uses by default for a call shape
 * (tokens per workgroup; a fixed 512 whenever all queries of a kv head fit
 * one 16-row tile and the context is at most 65536, so that a query's
 * reduction order does not depend on how many tokens are verified with it). */
int specdec_attention_split(int32_t batch, int32_t width, int32_t n_heads,
                            int32_t n_kv_heads, int32_t max_kv_len);

/* Causal paged attention of `width` new query tokens per row over the paged
 * cache (keys 0 .. past+t for query t, read through the block table in
 * place).  q token (b, t), head h at q + (b*width + t)*q_token_stride +
 * h*head_dim; out likewise with out_token_stride.  Softmax in fp32 with
 * `scale`; QK^T and PV on MFMA (bf16) or fp32 MFMA (F32).  Query rows with
 * t >= n_new[b] are not written.  head_dim must be 64.  split_tokens = 0
 * selects the fixed split of specdec_attention_split (a query's bits then
 * do not depend on the other queries of the call); a positive value is
 * rounded up to a multiple of 256; a negative value asks for one workgroup
 * per (row, kv head, query tile) over every key, for latency when the bits
 * need not match other calls (the draft; bf16 only, fp32 takes the default).
 * When a row needs more than four splits, a second kernel combining the
 * split partials is launched on the same stream (2 to 4 splits are folded
 * inside one workgroup with the same arithmetic, and so are 5 to 12 splits
 * when the call has a (row, kv head) tile for every compute unit and at
 * most 8 query rows per kv head: the workspace is then not used); calls
 * sharing a workspace must be ordered.  max_kv_len must bound every row's
 * cached length after the call (past + n_new): the grid is sized from it,
 * and a query tile whose keys pass it (16 query rows of a kv head) gets NaN
 * in its output rows (and, in the fused-append entry point, nothing
 * appended) instead of a silent skip; no key past it is read.  q_token_stride
 * and out_token_stride must cover a token's n_heads * head_dim elements (for
 * the fused-append entry point, the qkv row's (n_heads + 2 n_kv_heads) *
 * head_dim), else SPECDEC_EINVAL.
 * Replaces lm/forward.py:44-49,62-63 (mask, gather copy, SDPA) and
 * cache/kv.py:108-112. */
int specdec_paged_attention(const void *q, int dtype, int64_t q_token_stride,
                            const void *k_pool, const void *v_pool,
                            const int32_t *tables, int64_t table_stride,
                            const int32_t *meta, int32_t batch, int32_t width,
                            int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                            int32_t block_size, float scale, int32_t max_kv_len,
                            int32_t split_tokens, float *workspace,
                            int64_t workspace_floats, void *out,
                            int64_t out_token_stride, void *stream);

/* specdec_paged_attention fused with specdec_rope_append: qkv [batch,
 * width, (H + 2*Hkv) * head_dim] holds the projections before RoPE.  The q
 * heads are rotated in registers, and each workgroup first writes the new
 * tokens' rotated k and their v for its kv head and split into the paged
 * pools (identical values where workgroups overlap), so one launch per layer
 * replaces two.  Same rounding as the two separate kernels; qkv itself is
 * not modified.  bf16 calls of more than 16 new tokens per row (a prompt)
 * append the new tokens' k and v in a launch of their own first (one
 * workgroup per 16 positions and kv head), then run one workgroup per
 * eight query tiles over its causal keys.
 * With `hidden` not null, the layer's input RMSNorm is finished here too:
 * qkv is then a projection of hidden [batch, width, hidden_dim] bf16 (the
 * unnormalised residual stream) with the norm weight folded into the
 * projection, and every new token's q, k and v are multiplied by
 * s = rsqrt(mean(hidden^2) + eps) of its row and rounded to bf16 before
 * RoPE.  Needs bf16, block_size % 16 == 0 and width <= 16 (else
 * SPECDEC_EUNSUPPORTED); hidden_dim % 8 == 0 and hidden 16-byte aligned.
 * Replaces lm/forward.py:53,60-63 + cache/kv.py:101-112 (and the decoder
 * layer's input_layernorm). */
int specdec_rope_paged_attention(void *qkv, int dtype, int64_t token_stride,
                                 const float *cos_table, const float *sin_table,
                                 const void *hidden, int64_t hidden_dim, float eps,
                                 void *k_pool, void *v_pool, const int32_t *tables,
                                 int64_t table_stride, const int32_t *meta, int32_t batch,
                                 int32_t width, int32_t n_heads, int32_t n_kv_heads,
                                 int32_t head_dim, int32_t block_size, float scale,
                                 int32_t max_kv_len, int32_t split_tokens,
                                 float *workspace, int64_t workspace_floats, void *out,
                                 int64_t out_token_stride, void *stream);

/* A latency decode step (specdec_rope_paged_attention with width 1,
 * split_tokens < 0: the same norm, RoPE and append) whose attention is left
 * as split partials for the output projection to fold: nparts (4, 8 or 16)
 * one-wave workgroups per (row, kv head), on as many compute units,
 * workgroup w taking the 64-token steps w, w + nparts, ... of the keys and
 * writing its (m, l, O) -- the running max in log2 units, the sum of
 * 2^(s - m) and O = sum 2^(s - m) v, not divided -- for each query head of
 * the kv head to parts [batch, n_heads, nparts, 68] fp32 (m, l, two unused,
 * then O's 64 dims; 16-byte aligned).  Folding a row's partials in order (specdec_linear_attn_parts)
 * gives, with nparts = 4, the bits specdec_rope_paged_attention writes
 * (with more parts, the same attention folded in another order).  A row whose cached length exceeds
 * max_kv_len gets partials that fold to NaN.  Needs head_dim 64, block_size
 * % 16 == 0, max_kv_len <= 2048, n_heads / n_kv_heads <= 16 and hidden_dim
 * <= 2048 (else SPECDEC_EUNSUPPORTED); qkv and hidden 16-byte aligned.
 * Replaces lm/forward.py:40-49,53,60-63 for one new token per row (the
 * draft model's steps) + cache/kv.py:101-112. */
int specdec_rope_paged_attention_parts(void *qkv, int64_t token_stride, const float *cos_table,
                                       const float *sin_table, const void *hidden, int64_t hidden_dim,
                                       float eps, void *k_pool, void *v_pool, const int32_t *tables,
                                       int64_t table_stride, const int32_t *meta, int32_t batch,
                                       int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                       int32_t block_size, float scale, int32_t max_kv_len,
                                       int32_t nparts, float *parts, void *stream);

/* ---------------------------------------------------------------- linear --- */

/* out [rows, out_features] bf16 (out_stride apart) = x [rows, in_features]
 * bf16 (x_stride apart) times w [out_features, in_features] bf16 (rows
 * w_stride apart, or tiled: w_layout, SPECDEC_W_TILED needs out_features %
 * 16 == 0) transposed, products accumulated in fp32 and rounded once to bf16
 * (round to nearest even); with `accumulate`, the existing out is added
 * before that rounding (a residual add).  At most 64 rows, in_features a
 * multiple of 32 up to 8192, w within 2 GiB (else SPECDEC_EUNSUPPORTED); x
 * and w 16-byte aligned with strides % 8 == 0.  A row's result does not
 * depend on the other rows of the call or their number.
 * Replaces the bias-free projections of lm/forward.py:56-58,63-64
 * (transformers' q/k/v_proj, o_proj, gate/up/down_proj) at decode sizes. */
int specdec_linear(const void *x, int64_t x_stride, const void *w, int64_t w_stride, int32_t w_layout,
                   int64_t rows, int64_t in_features, int64_t out_features, void *out,
                   int64_t out_stride, int32_t accumulate, void *stream);

/* specdec_linear of the attention rows a specdec_rope_paged_attention_parts
 * call left as partials: out [rows, out_features] (+)= attn w^T, with attn
 * [rows, n_heads * 64] folded from parts [rows, n_heads, nparts, 68] by
 * each workgroup in its prologue (the attention kernel's own fold order, so
 * with 4 parts attn has specdec_rope_paged_attention's bits) and w
 * [out_features, n_heads * 64] bf16 (w_layout as for specdec_linear).  With
 * attn_out not null the folded rows are written there too (bf16 [rows,
 * n_heads * 64], 8-byte aligned).  The k-split is specdec_linear's for that weight, so out has the
 * bits of specdec_rope_paged_attention followed by specdec_linear.
 * rows <= 16, n_heads * 64 <= 2048 (else SPECDEC_EUNSUPPORTED).  Replaces
 * lm/forward.py:60-63 (o_proj and the residual add) for the draft's steps. */
int specdec_linear_attn_parts(const float *parts, int64_t rows, int64_t n_heads, int32_t nparts,
                              const void *w, int64_t w_stride, int32_t w_layout, int64_t out_features,
                              void *out, int64_t out_stride, int32_t accumulate, void *attn_out,
                              void *stream);

/* specdec_linear of x and the fused gate/up weight w [2*inter, in_features]
 * followed by specdec_rms_silu_mul, in one launch: out [rows, inter] bf16 =
 * SiLU(bf16(s * g)) * bf16(s * u), where g and u are the bf16 projections
 * of the gate half (w rows 0 .. inter-1) and the up half, with the bits
 * specdec_linear gives them, and s = rsqrt(mean(hidden_row^2) + eps) of the
 * row's residual `hidden` [rows, hidden_dim] bf16 (hidden_stride apart) as
 * specdec_rms_silu_mul computes it -- the same bits as the two calls, and
 * the [rows, 2*inter] intermediate is never written.  Limits as
 * specdec_linear; hidden_dim % 8 == 0 and at most 4096, hidden 16-byte
 * aligned with hidden_stride % 8 == 0.
 * Replaces lm/forward.py:64 (post_attention_layernorm, gate/up projection
 * and act_fn(gate) * up of transformers' LlamaMLP) at decode sizes. */
int specdec_linear_silu(const void *x, int64_t x_stride, const void *w, int64_t w_stride,
                        int32_t w_layout, int64_t rows, int64_t in_features, int64_t inter, const void *hidden,
                        int64_t hidden_stride, int64_t hidden_dim, float eps, void *out,
                        int64_t out_stride, void *stream);

/* ------------------------------------------------------------------ head --- */

/* Output head: logits [rows, vocab] fp32 (logits_stride apart) = x [rows,
 * hidden] bf16 (x_stride apart) times w [vocab, hidden] bf16 (w_stride
 * apart) transposed, bf16 products accumulated in fp32 on MFMA in a fixed
 * k order, so a row's logits do not depend on the other rows of the call or
 * their number.  hidden % 32 == 0, hidden <= 2048 and w within 2 GiB, else
 * SPECDEC_EUNSUPPORTED; x and w 16-byte aligned with strides % 8 == 0.
 * Replaces lm/forward.py:71-84 (the fp32 output projection). */
int specdec_head_logits(const void *x, int64_t x_stride, const void *w, int64_t w_stride,
                        int64_t rows, int64_t hidden, int64_t vocab, float *logits,
                        int64_t logits_stride, void *stream);

/* Bytes of the workspace of specdec_head_probabilities: zeroed once by the
 * caller, then never cleared (its words carry a per-call tag). */
int specdec_head_workspace(int64_t *bytes);

/* The output head and probabilities in one launch, for at most 16 rows:
 * out [rows, vocab] fp32 (out_stride apart) = one-hot of each row's argmax
 * (lowest id among ties) at temperature 0, else softmax(logits /
 * temperature), with the logits of specdec_head_logits (same bits, also
 * written to `logits` when non-NULL).  At temperature 0 a non-NULL
 * index_out receives each row's argmax.  The workgroups exchange per-slice
 * statistics through `workspace` (specdec_head_workspace bytes, zeroed
 * before its first call; calls sharing it must be ordered on one stream);
 * a workgroup that has polled `spin` times without seeing every slice
 * computes the missing statistics itself, with the same bits.  Shapes the
 * launch does not take (more than 16 rows, a vocab needing more than one
 * workgroup of 16 tiles per compute unit) return SPECDEC_EUNSUPPORTED.
 * Replaces lm/forward.py:71-84 followed by lm/sampling.py:13-18. */
int specdec_head_probabilities(const void *x, int64_t x_stride, const void *w, int64_t w_stride,
                               int64_t rows, int64_t hidden, int64_t vocab, float temperature,
                               float *out, int64_t out_stride, int64_t *index_out,
                               int64_t index_stride, float *logits, int64_t logits_stride,
                               void *workspace, int64_t workspace_bytes, int32_t spin,
                               void *stream);

/* fp32 split partials the library holds per GPU for
 * specdec_paged_attention_static (8 MiB). */
#define SPECDEC_STATIC_PARTIAL_FLOATS (2 * 1024 * 1024)

/* specdec_paged_attention without a workspace argument: the split partials
 * of calls that need them live in a file-scope device array of the library
 * (SPECDEC_STATIC_PARTIAL_FLOATS floats, one copy per GPU, held until the
 * process ends), so the call allocates nothing and takes no buffer beyond
 * its inputs and outputs.  A call whose partials would not fit returns
 * SPECDEC_ENOSCRATCH before anything is launched (specdec_attention_workspace
 * bounds the need from above; calls answered by one workgroup per tile, as
 * at most four 512-token splits, or the tiled grid, need none).  Every call
 * on a GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams, two threads) race, so order them.  The array needs no clearing:
 * each call writes every partial it reads.  The first call on a device
 * looks the array's address up (hipGetSymbolAddress) with that device
 * current.
 * No counterpart in the reference (whose attention is
 * lm/forward.py:44-49,62-63 on torch): it is for callers that cannot
 * allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation. */
int specdec_paged_attention_static(const void *q, int dtype, int64_t q_token_stride,
                                   const void *k_pool, const void *v_pool,
                                   const int32_t *tables, int64_t table_stride,
                                   const int32_t *meta, int32_t batch, int32_t width,
                                   int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                   int32_t block_size, float scale, int32_t max_kv_len,
                                   int32_t split_tokens, void *out,
                                   int64_t out_token_stride, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SPECDEC_H */
