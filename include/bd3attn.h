/*
 * bd3attn.h - C ABI of the MI355X (gfx950) BD3-LM attention library
 * (libbd3attn.so).
 *
 * Scope: the attention hot path of block-diffusion language models.
 *   - training attention forward/backward over cat(x_t, x_0) (length 2n)
 *     under the BD3-LM block-diffusion mask;
 *   - block-sparse decode attention of the last q_len positions over a
 *     KV cache of kv_len positions (block-causal);
 *   - split-KV decode attention (partials + LSE merge).
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are DEVICE pointers to bf16 data (uint16 bit
 *     patterns of bfloat16) unless the type says float. Row-major 4-D
 *     tensors (batch, heads, seq, head_dim) with the last stride 1;
 *     `strides` passes the other three element strides (batch, head, seq)
 *     of each tensor, in the order the entry point lists.
 *   - The library never allocates device memory and never synchronises.
 *     Work is enqueued on `stream` (a hipStream_t; NULL = default stream).
 *     Workspaces are caller-allocated; *_workspace_bytes() sizes them.
 *   - Every entry point returns 0 on success, BD3_EINVAL when an argument
 *     violates a precondition (nothing is launched), or BD3_EHIP when the
 *     HIP runtime reports an error. bd3_last_error() returns a thread-local
 *     message describing the last failure on the calling thread.
 *   - head_dim must be 64 (the reference's only configuration: d_model
 *     768 / 12 heads).
 *   - The attention entry points take the softmax scale (the reference
 *     passes 1 / sqrt(head_dim)); it must be finite and > 0. Scores are
 *     the exact fp32 dot products of the bf16 rows, scaled in fp32.
 *
 * Reentrant: no mutable global state besides the thread-local error
 * message.
 */
#ifndef BD3ATTN_H
#define BD3ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BD3_OK 0
#define BD3_EINVAL 1
#define BD3_EHIP 2

/* 2: bd3_train_tile_census writes 8 values (out[1] and out[6], out[7] are
 * the executed pairs of each kernel), the second workspace plane of the
 * backward holds -L / scale, and bd3_attn_bwd_delta / bd3_attn_bwd_main
 * split the backward into its Delta pass and one main launch. */
#define BD3_ABI_VERSION 2

/* Version of this ABI (BD3_ABI_VERSION). No reference counterpart. */
int bd3_abi_version(void);

/* Thread-local message for the last non-zero status on this thread. */
const char* bd3_last_error(void);

/*
 * Training attention forward:
 *   O = softmax(Q K^T * scale + M) V,  lse = logsumexp(Q K^T * scale + M)
 * over the 2n-long sequence cat(x_t, x_0), M the BD3-LM block-diffusion
 * mask (model/bd3lm.py:10-52). lse is natural-log, fp32, contiguous
 * (batch, heads, 2n).
 * strides: 12 int64 = (b, h, s) element strides of q, k, v, o.
 * Preconditions: n % 128 == 0, block_size >= 1, head_dim == 64.
 *
 * Replaces the launch of block_sparse_attention_fwd_kern in
 * BlockSparseFlashAttention.forward
 * (kernels/BlockSparseFlashAttention.py:466-506, kernel :75-172).
 */
int bd3_attn_fwd(const void* q, const void* k, const void* v, void* o,
                 float* lse, int32_t batch, int32_t heads, int32_t n,
                 int32_t head_dim, int32_t block_size, const int64_t* strides,
                 float scale, void* stream);

/*
 * Bytes of workspace bd3_attn_bwd needs: two fp32 (batch, heads, 2n)
 * planes, Delta = rowsum(dO * O) and -L / scale. No reference counterpart
 * (the reference allocates Delta with a torch op,
 * kernels/BlockSparseFlashAttention.py:525).
 */
size_t bd3_attn_bwd_workspace_bytes(int32_t batch, int32_t heads, int32_t n,
                                    int32_t head_dim);

/*
 * Training attention backward: dQ, dK, dV of the forward above, given
 * dO and the forward's O and lse: bd3_attn_bwd_delta (Delta and -L / scale
 * into the workspace) then bd3_attn_bwd_main (every dQ and dK/dV work item
 * in one launch).
 * strides: 24 int64 = (b, h, s) element strides of
 *          q, k, v, o, dout, dq, dk, dv.
 * Preconditions: as the forward, plus n % block_size == 0 (the reference
 * asserts it, :522) and workspace_bytes >= bd3_attn_bwd_workspace_bytes().
 * Every precondition of both stages is checked before the first launch.
 *
 * Replaces BlockSparseFlashAttention.backward's device work
 * (kernels/BlockSparseFlashAttention.py:508-562).
 */
int bd3_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                 const void* dout, const float* lse, void* dq, void* dk,
                 void* dv, void* workspace, size_t workspace_bytes,
                 int32_t batch, int32_t heads, int32_t n, int32_t head_dim,
                 int32_t block_size, const int64_t* strides, float scale,
                 void* stream);

/*
 * Backward, Delta pass: Delta = rowsum(dO * O) and minus the forward's L
 * over scale, written to `delta`: fp32, contiguous (2, batch, heads, 2n),
 * plane 0 Delta, plane 1 -L / scale (the first bd3_attn_bwd_workspace_bytes()
 * bytes of the backward workspace).
 * strides: 6 int64 = (b, h, s) element strides of o, dout.
 * Preconditions: as bd3_attn_bwd.
 *
 * Replaces the Delta torch op (kernels/BlockSparseFlashAttention.py:525).
 */
int bd3_attn_bwd_delta(const void* o, const void* dout, const float* lse,
                       float* delta, int32_t batch, int32_t heads, int32_t n,
                       int32_t head_dim, int32_t block_size,
                       const int64_t* strides, float scale, void* stream);

/*
 * Backward, main launch: dQ = scale * dS K, dV = P^T dO and dK = scale *
 * dS^T Q from the planes bd3_attn_bwd_delta wrote to `delta`; `lse` is
 * checked but not read (the kernel uses the plane). One launch holds every
 * query-stationary dQ item and key-stationary dK/dV item, longest first;
 * with a block size dividing 32 the noisy key tiles' dK and dV (their
 * diagonal blocks) come from the dQ items of the same rows.
 * strides: 21 int64 = (b, h, s) element strides of q, k, v, dout, dq, dk, dv.
 * Preconditions: as bd3_attn_bwd.
 *
 * Replaces block_sparse_attention_bwd_dq_kern and
 * block_sparse_attention_dk_dv_bwd_kern with their launches
 * (kernels/BlockSparseFlashAttention.py:212-452, :532-560).
 */
int bd3_attn_bwd_main(const void* q, const void* k, const void* v,
                      const void* dout, const float* lse, const float* delta,
                      void* dq, void* dk, void* dv, int32_t batch,
                      int32_t heads, int32_t n, int32_t head_dim,
                      int32_t block_size, const int64_t* strides, float scale,
                      void* stream);

/*
 * bd3_attn_bwd without a workspace argument: the same kernels and results
 * (bit for bit), with the Delta and -L / scale planes kept in a fixed
 * device array inside the library (8 MiB per GPU, held from the library's
 * first call of this function on that GPU until the process ends).
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc). Makes no allocation of any kind.
 * Limit: batch * heads * 2n <= BD3_NOALLOC_MAX_ROWS (e.g. B=8, H=12,
 * 2n=8192); larger calls return BD3_EINVAL. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams or
 * threads, no ordering between them) race and must not be made. The calling
 * thread's current device must be the device of `stream`. Under HIP graph
 * capture: make one eager call on the device first (it looks up the array's
 * device address); later calls only enqueue the kernels and can be captured
 * and replayed (the planes are fully rewritten by every call).
 */
#define BD3_NOALLOC_MAX_ROWS (1 << 20)
int bd3_attn_bwd_noalloc(const void* q, const void* k, const void* v,
                         const void* o, const void* dout, const float* lse,
                         void* dq, void* dk, void* dv, int32_t batch,
                         int32_t heads, int32_t n, int32_t head_dim,
                         int32_t block_size, const int64_t* strides,
                         float scale, void* stream);

/*
 * Backward in two stages (the reference's two kernels): first stage = the
 * Delta pass (bd3_attn_bwd_delta) and the dQ items, dQ = scale * dS K with
 * dS = P o (dP - Delta); the planes go to `delta`: fp32, contiguous (2,
 * batch, heads, 2n), plane 0 Delta, plane 1 -L / scale.
 * strides: 18 int64 = (b, h, s) element strides of q, k, v, o, dout, dq.
 * Preconditions: as bd3_attn_bwd.
 *
 * Replaces the Delta torch op (kernels/BlockSparseFlashAttention.py:525)
 * and block_sparse_attention_bwd_dq_kern with its launch (:368-452, :532-543).
 */
int bd3_attn_bwd_dq(const void* q, const void* k, const void* v,
                    const void* o, const void* dout, const float* lse,
                    void* dq, float* delta, int32_t batch, int32_t heads,
                    int32_t n, int32_t head_dim, int32_t block_size,
                    const int64_t* strides, float scale, void* stream);

/*
 * Backward, second stage: the dK/dV items, dV = P^T dO and dK = scale *
 * dS^T Q, given the two planes (Delta, -L / scale) the first stage wrote to
 * `delta`; `lse` is checked but not read (the kernel uses the plane).
 * bd3_attn_bwd runs both stages' items in one launch instead.
 * strides: 18 int64 = (b, h, s) element strides of q, k, v, dout, dk, dv.
 * Preconditions: as bd3_attn_bwd.
 *
 * Replaces block_sparse_attention_dk_dv_bwd_kern and its launch
 * (kernels/BlockSparseFlashAttention.py:212-328, :545-560).
 */
int bd3_attn_bwd_dkdv(const void* q, const void* k, const void* v,
                      const void* dout, const float* lse, const float* delta,
                      void* dk, void* dv, int32_t batch, int32_t heads,
                      int32_t n, int32_t head_dim, int32_t block_size,
                      const int64_t* strides, float scale, void* stream);

/*
 * Block-sparse decode attention: queries are the LAST q_len of kv_len
 * positions; row i (position p = kv_len - q_len + i) sees key j iff
 * j / block_size <= p / block_size (block-causal), j < kv_len.
 * n_splits = 0 lets the library choose a key split that fills the GPU
 * (a workspace of bd3_decode_workspace_bytes(..., 0, ...) is then needed;
 * pass NULL/0 when that size is 0).
 * q_len > 64 (a long query block or a whole-sequence prefill) runs a
 * kernel with 128-row query tiles sharing each K / V tile.
 * strides: 12 int64 = (b, h, s) element strides of q, k, v, o.
 * Preconditions: 1 <= q_len <= kv_len, head_dim == 64, block_size >= 1;
 * for q_len > 64 the k and v sequence strides are below 2^24 elements
 * (32-bit per-lane tile load offsets).
 *
 * Replaces block_sparse_decode_kern and its launch in
 * block_sparse_decode_attention
 * (kernels/BlockSparseDecodeAttention.py:40-110, :118-148).
 */
int bd3_decode(const void* q, const void* k, const void* v, void* o,
               int32_t batch, int32_t heads, int32_t q_len, int32_t kv_len,
               int32_t head_dim, int32_t block_size, const int64_t* strides,
               float scale, void* workspace, size_t workspace_bytes,
               void* stream);

/*
 * Number of key splits bd3_decode / bd3_decode_splitkv use for
 * n_splits == 0 (auto). No reference counterpart.
 */
int32_t bd3_decode_auto_splits(int32_t batch, int32_t heads, int32_t q_len,
                               int32_t kv_len);

/*
 * Workspace bytes for a split-KV decode with n_splits splits (0 = the auto
 * count bd3_decode uses):
 * fp32 partial O and LSE per (batch*head, query tile, split). 0 when a
 * single split needs no workspace. No reference counterpart (the
 * reference allocates o_part / lse with torch.empty,
 * kernels/SplitKVDecodeAttention.py:148-151).
 */
size_t bd3_decode_workspace_bytes(int32_t batch, int32_t heads, int32_t q_len,
                                  int32_t kv_len, int32_t head_dim,
                                  int32_t n_splits);

/*
 * Split-KV decode attention: the keys [0, kv_len) are cut into n_splits
 * contiguous ranges, each producing a normalised fp32 partial O and its
 * LSE, merged with LSE weights (FlashDecoding). Same result as bd3_decode.
 * The reference's default split count is ceil(kv_len / 256)
 * (kernels/SplitKVDecodeAttention.py:147); callers pass it explicitly.
 * strides: 12 int64 = (b, h, s) element strides of q, k, v, o.
 * Preconditions: 1 <= q_len <= kv_len, head_dim == 64,
 * 1 <= n_splits <= kv_len, workspace large enough; for q_len > 64 the k
 * and v sequence strides are below 2^24 elements (as bd3_decode).
 *
 * Replaces split_kv_kern + split_kv_reduce_kern and their launches in
 * split_kv_decode_attention (kernels/SplitKVDecodeAttention.py:16-171).
 */
int bd3_decode_splitkv(const void* q, const void* k, const void* v, void* o,
                       int32_t batch, int32_t heads, int32_t q_len,
                       int32_t kv_len, int32_t head_dim, int32_t block_size,
                       int32_t n_splits, const int64_t* strides, float scale,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Attention inputs of one layer in one pass: splits the fused projection
 * into heads, applies the rotary embedding to q and k, and stores q, k and v
 * to (batch, heads, seq, head_dim) destinations with arbitrary (b, h, s)
 * strides -- k_out / v_out may be the slot [len, len + seq) of a
 * preallocated KV cache, so attention reads cache and block in place.
 * Replaces the rearrange and the two RoPE calls of
 * BidirectionalMultiHeadAttention.forward (model/modules.py:395-407,
 * RoPE.forward :212-240) and, with a cache, the per-step
 * torch.cat([cache, block]) (model/modules.py:409-414).
 *   qkv: (batch, seq, 3 * heads * head_dim) bf16, last stride 1;
 *        qkv_strides = its (batch, seq) element strides. Column
 *        c*heads*head_dim + h*head_dim + j is component c (0 q, 1 k, 2 v)
 *        of head h, coordinate j (the reference's
 *        "(three n_heads d_k)" order).
 *   positions: device int64 (seq) absolute positions, or NULL for
 *        pos0 .. pos0 + seq - 1 (then pos0 + seq <= max_pos is checked).
 *        Explicit positions outside [0, max_pos) are clamped (the
 *        reference's table lookup would raise).
 *   sin_table, cos_table: device fp32 (max_pos, head_dim / 2), the RoPE
 *        module's tables (sin/cos of p * theta^(-2k/head_dim)).
 *   out_strides: 3 x 3 (b, h, s) element strides of q_out, k_out, v_out.
 * The rotation repeats the reference's eager bf16 arithmetic (tables
 * rounded to bf16, every product, difference and sum rounded to bf16), so
 * outputs are bit-identical to it. seq == 0 is a no-op.
 */
int bd3_qkv_rope(const void* qkv, const int64_t* qkv_strides, int32_t batch, int32_t seq,
                 int32_t heads, int32_t head_dim, const int64_t* positions, int32_t pos0,
                 const float* sin_table, const float* cos_table, int32_t max_pos, void* q_out,
                 void* k_out, void* v_out, const int64_t* out_strides, void* stream);

/*
 * Copies (batch, heads, seq, head_dim) bf16 k and v into k_dst / v_dst
 * (any (b, h, s) strides; typically the slot [len, len + seq) of a
 * preallocated cache). strides: 4 x 3 for k, v, k_dst, v_dst. Replaces the
 * torch.cat growth of KVCache.append (model/kv_cache.py:42-55). seq == 0 is
 * a no-op.
 */
int bd3_kv_write(const void* k, const void* v, void* k_dst, void* v_dst, int32_t batch,
                 int32_t heads, int32_t seq, int32_t head_dim, const int64_t* strides,
                 void* stream);

/*
 * One ancestral denoising step of BD3-LM sampling for `rows` token
 * positions: SUBS parameterization of the logits (zero mass on [MASK],
 * log-softmax), the categorical draw by Gumbel-max with float64 noise, and
 * the carry-over of unmasked tokens, fused; no (rows, vocab) intermediate is
 * written. Replaces subs_parameterization (model/subs.py:11-43) plus the
 * sampler's update and sample_categorical (sample/sampler.py:110-122,
 * :11-34):
 *   out[r] = xt[r]                                   if xt[r] != mask_index
 *          = argmax_i q_i / (1e-10 - log(u_i + 1e-10)) otherwise,
 *   q_i = exp(log_softmax(logits + bias))_i * (1 - keep), q_mask = keep,
 * keep = s / t of the step, with the reference's dtypes (bf16 logits: the
 * bias add and the shift by the max in bf16, exp / sum / log in fp32; q,
 * noise and ratio in float64).
 *   logits: (rows, ld) device array, bf16 (logits_fp32 = 0) or fp32 (1);
 *   xt, out: device int64 (rows); out may alias xt;
 *   u: device float64 (rows, vocab) uniforms in [0, 1) (the reference's
 *      torch.rand_like draw), or NULL to draw them with Philox4x32-10:
 *      element e = r * vocab + i takes the 64 bits of words (0, 1) (e even)
 *      or (2, 3) (e odd) of the block with counter
 *      {e/2 low, e/2 high, offset low, offset high} and key {seed low,
 *      seed high}, as (bits >> 11) * 2^-53.
 * Logits must be finite. vocab in [2, 2^31), mask_index in [0, vocab).
 */
int bd3_subs_sample(const void* logits, int64_t ld, int32_t logits_fp32, const int64_t* xt,
                    int64_t* out, int32_t rows, int32_t vocab, int32_t mask_index, double keep,
                    const double* u, uint64_t seed, uint64_t offset, void* stream);

/*
 * modulate(LN(x), shift, scale) of a DiT block's pre-norm (weight-only
 * LayerNorm, model/modules.py:243-288; modulate, :778-788; call sites in
 * DiTBlock.forward, :537-568), one pass over x:
 *   y = (weight * (x - mean)) * rsqrt(var + eps)   fp32 over the upcast row,
 *       var with correction 0, then cast back to x's dtype;
 *   out = y * (1 + scale) + shift                  1 + scale in the vectors'
 *       dtype; the product and sum in bf16 op by op if x and the vectors
 *       are bf16, else in fp32;
 * out is written in that dtype, or rounded to bf16 (out_fp32 = 0) when it is
 * fp32 (the cast autocast applies at the next matmul's input).
 *   x, out: (batch, seq, d_model); shift, scale: (batch, d_model) (the
 *   reference's (batch, 1, d_model) broadcast); weight: (d_model).
 *   *_fp32: 1 = fp32, 0 = bf16 for each operand.
 *   strides: 5 element strides: x (batch, seq), shift / scale (batch), out
 *   (batch, seq); last strides 1; bases 16-byte aligned, strides and d_model
 *   multiples of 8; d_model <= 4096.
 */
int bd3_ln_modulate(const void* x, int32_t x_fp32, const void* weight, int32_t weight_fp32,
                    const void* shift, const void* scale, int32_t mod_fp32, void* out,
                    int32_t out_fp32, int32_t batch, int32_t seq, int32_t d_model,
                    const int64_t* strides, float eps, void* stream);

/*
 * out = x + gate * y, the residual updates of DiTBlock.forward
 * (model/modules.py:560-566): gate * y in bf16 if both are bf16 (rounded)
 * else fp32, then the add in bf16 if x and that product are bf16 else fp32;
 * out has that dtype (bf16 only when x, gate and y all are). Bit-exact with
 * the eager ops; out may alias x.
 *   x, y, out: (batch, seq, d_model); gate: (batch, d_model).
 *   strides: 7 element strides: x (batch, seq), gate (batch), y (batch,
 *   seq), out (batch, seq); same alignment rules as bd3_ln_modulate.
 */
int bd3_gate_residual(const void* x, int32_t x_fp32, const void* gate, int32_t gate_fp32,
                      const void* y, int32_t y_fp32, void* out, int32_t batch, int32_t seq,
                      int32_t d_model, const int64_t* strides, void* stream);

/*
 * The two above fused, as DiTBlock.forward chains them (model/modules.py:
 * 560-566, then the next sublayer's :537-568): x_out = x + gate * y with
 * bd3_gate_residual's dtypes and roundings, then out = modulate(LN(x_out),
 * shift, scale) with bd3_ln_modulate's, x_out's dtype as the LayerNorm
 * input's. One launch and one read of the residual instead of two of each;
 * bit-exact with the two calls in sequence. x_out may alias x.
 *   x, y, x_out, out: (batch, seq, d_model); gate, shift, scale:
 *   (batch, d_model), all of dtype mod_fp32; weight: (d_model).
 *   x_out's dtype is bf16 when x, y and the vectors all are, else fp32.
 *   strides: 9 element strides: x (batch, seq), gate / shift / scale
 *   (batch), y (batch, seq), x_out (batch, seq), out (batch, seq); same
 *   alignment rules and d_model limit as bd3_ln_modulate.
 */
int bd3_gate_residual_ln_modulate(const void* x, int32_t x_fp32, const void* gate, const void* y,
                                  int32_t y_fp32, void* x_out, const void* weight,
                                  int32_t weight_fp32, const void* shift, const void* scale,
                                  int32_t mod_fp32, void* out, int32_t out_fp32, int32_t batch,
                                  int32_t seq, int32_t d_model, const int64_t* strides, float eps,
                                  void* stream);

/*
 * Writes the mask the device predicate applies, one byte per (row, key)
 * (1 = may attend), row-major:
 *   mode 0 (training): (2n, 2n) with n = rows, kv_len ignored;
 *   mode 1 (decode):   (rows = q_len, kv_len).
 * For bit-exact comparison against block_diff_mask (model/bd3lm.py:10-52)
 * and the decode slice (kernels/BlockSparseDecodeAttention.py:84-88).
 */
int bd3_mask_dump(uint8_t* out, int32_t mode, int32_t rows, int32_t kv_len,
                  int32_t block_size, void* stream);

/*
 * Measurement aid, no reference counterpart: the shader clock under a
 * matrix-core load, for pricing kernels against the clock the chip holds
 * rather than the datasheet's 2.4 GHz. Launches `workgroups` workgroups of
 * 256 threads that each run `iters` rounds of four independent bf16 MFMA
 * chains per wave (no memory reads). Workgroup i writes out[2i] = shader
 * clock ticks (s_memtime) and out[2i+1] = constant-rate real-time ticks
 * (s_memrealtime) elapsed over its loop; *wall_rate_khz receives the
 * real-time counter's rate (hipDeviceAttributeWallClockRate), so the clock
 * is out[2i] / out[2i+1] * wall_rate_khz kHz.
 * Preconditions: out holds 2 * workgroups uint64; 1 <= workgroups <= 65536;
 * iters >= 1.
 */
int bd3_clock_probe(uint64_t* out, int32_t workgroups, int32_t iters, int64_t* wall_rate_khz,
                    void* stream);

/*
 * Host-only (no GPU needed): tile census of the training-attention
 * schedules for one (batch, head). Writes out[0..7] =
 *   {useful pairs,
 *    pairs the forward kernel computes (its 32-row waves compute both 32-key
 *      halves of a 64-key tile when either half has a live pair; when
 *      32 % block_size == 0 each noisy 32-row wave computes only its
 *      diagonal 32 x 32 block of the noisy keys),
 *    full / partial / skipped 32x32 sub-blocks of that schedule,
 *    useful pairs per (b,h) closed form n^2 + n*bs,
 *    pairs the main launch's dQ items compute (the forward's schedule; when
 *      block_size % 16 == 0 every live 32 x 32 block once),
 *    pairs the dK/dV work computes (32-key waves, both 32-row halves of a
 *      64-row tile when either has a live pair; when 32 % block_size == 0
 *      only the diagonal 32 x 32 block of a noisy key tile's waves; when
 *      block_size % 16 == 0 every live 32 x 32 block once)}.
 * `out` must hold 8 values. Mirrors the reference's tile-skipping ranges
 * (kernels/BlockSparseFlashAttention.py:132-164, :274-325, :419-450) at the
 * library's own tile granularity.
 */
int bd3_train_tile_census(int32_t n, int32_t block_size, int64_t* out);

/*
 * Host-only: classification the device code uses for a 32-row query group
 * starting at q0 and a 32-key sub-block starting at k0 in training mode:
 * 0 = no live pair, 1 = every pair live, 2 = partial. For CPU tests. The
 * class is computed both from the row group's bounds and from the
 * per-tile threshold form the kernels keep in registers; -2 if they differ.
 */
int bd3_train_classify(int32_t n, int32_t block_size, int32_t q0, int32_t k0);

/*
 * Host-only: the same classification computed the way the key-stationary
 * backward kernel does it (fixed 32-key group at k0, 32-row group at q0),
 * again in both forms (-2 if they differ).
 */
int bd3_train_classify_keys(int32_t n, int32_t block_size, int32_t q0,
                            int32_t k0);

/*
 * Host-only: tile classes (0 none, 1 full, 2 partial) in the walk-index
 * interval form (walk_classes in the device headers). The forward kernel
 * keeps these intervals in scalar registers and uses the whole-tile class
 * of mode 0. mode 0: the 32-row group starting at g0, walking the key tiles
 * (64 keys) of its 128-row query tile; mode 1: the 32-key group starting at
 * g0, walking the query tiles (64 rows) of its 128-key tile. *tile receives
 * the i-th tile's index. Returns the class of the whole tile | (class of its
 * first 32 positions) << 2 | (class of its last 32) << 4; -1 on bad
 * arguments, -3 when the walk has fewer than i + 1 tiles. For CPU tests.
 */
int bd3_train_walk_class(int32_t n, int32_t block_size, int32_t g0, int32_t i, int32_t mode,
                         int32_t* tile);

/*
 * Host-only: the interval form of the training mask the kernels apply inside
 * partial blocks, for CPU tests. mode 0: the keys row `index` sees; mode 1:
 * the rows that see key `index`. Writes out[0..3] = {lo1, hi1, lo2, hi2}:
 * the set is [lo1, hi1) union [lo2, hi2). Returns 0, or -1 on bad arguments.
 */
int bd3_train_intervals(int32_t n, int32_t block_size, int32_t index,
                        int32_t mode, int32_t* out);

#ifdef __cplusplus
}
#endif

#endif /* BD3ATTN_H */
