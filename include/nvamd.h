/*
 * nvamd.h — C ABI of the MI355X (gfx950) continuous-batching attention path.
 *
 * Every entry point:
 *   - takes device pointers, scalar sizes/strides and an explicit hipStream_t;
 *   - returns 0 on success, a negative NVAMD_E* code for an argument error
 *     (nothing is launched), or a positive hipError_t if the launch failed;
 *   - allocates nothing and never synchronises the host, so every call can be
 *     captured into a hipGraph.
 *
 * Tensor conventions (bf16 = 16-bit brain float stored as uint16_t):
 *   KV cache of one layer: [num_blocks, block_size, num_kv_heads, head_dim]
 *   contiguous bf16; a "slot" is block_id * block_size + offset, i.e. the row
 *   index into the flattened [num_blocks * block_size, num_kv_heads, head_dim]
 *   view.  head_dim must be 128; block_size a power of two >= 16.
 *   Token-major activations ([T, heads, 128]) may have a row stride (elements
 *   between consecutive tokens) larger than heads * 128, so views into a fused
 *   qkv projection are accepted without a copy.
 *
 * Reference citations are relative to the nano_vllm_ascend source tree;
 * "nv/" = src/nanovllm_ascend/.
 */
#ifndef NVAMD_H
#define NVAMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NVAMD_OK 0
#define NVAMD_EINVAL (-1)      /* a size, stride or pointer is invalid        */
#define NVAMD_EUNSUPPORTED (-2) /* head_dim / GQA group / block_size not built */
#define NVAMD_EWORKSPACE (-3)  /* workspace missing or too small               */
#define NVAMD_ETOOLARGE (-4)   /* needs more than the library's static scratch  */
#define NVAMD_ECAPTURE (-5)    /* first use of the static scratch on a device   */
                               /* made while `stream` is being captured         */

/* ABI version of this header; nvamd_version() returns the version the library was built
   with, for the loader's sanity check. */
#define NVAMD_ABI_VERSION 3
int nvamd_version(void);

/* ------------------------------------------------------------------------- */
/* Index errors.  Where the reference's indexing raises -- index_copy_ with a */
/* slot outside the cache (nv/npu/paged_kv_cache.py:68-69), the RoPE cache    */
/* indexed past its end (nv/layers/rotary_embedding.py:49-50), a context     */
/* longer than its block-table row or the launch's bound, a block id outside */
/* the pool (nv/layers/npu_paged_attention.py:89-99,                         */
/* nv/layers/npu_prefill_attention.py:73-96) -- the kernels skip the write or */
/* clamp the read, so no access leaves its buffer, and set the matching bit   */
/* in a per-device error word (an atomic OR; nothing is done on the normal    */
/* path).  A slot of -1 marks a padding row: skipped without an error.      */
/* nvamd_errors_fetch enqueues a copy of the word into `host` (4 bytes;      */
/* pinned memory keeps the copy asynchronous) on `stream`, so a caller reads  */
/* it with the step's other results instead of synchronising per call;       */
/* nvamd_errors_clear enqueues a kernel that zeroes it.  Both can be         */
/* captured.  The word starts at zero when the library is loaded.            */
/* Neither has a counterpart in the reference, which raises synchronously.   */
#define NVAMD_ERR_SLOT 1u     /* slot_mapping entry < -1 or >= cache slots   */
#define NVAMD_ERR_POSITION 2u /* position < 0 or >= the RoPE table's rows    */
#define NVAMD_ERR_CONTEXT 4u  /* context < 0 or past its table row / bound   */
#define NVAMD_ERR_BLOCK 8u    /* block-table entry < 0 or >= num_blocks      */
int nvamd_errors_fetch(unsigned *host, hipStream_t stream);
int nvamd_errors_clear(hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* P4: GQA paged decode attention.                                            */
/* Replaces torch_npu._npu_paged_attention as called at                       */
/*   nv/layers/npu_paged_attention.py:89-99 (eager) and                       */
/*   nv/npu/acl_graph.py:232-243 (graph replay update), and                   */
/*   torch_npu._npu_paged_attention_get_workspace at                          */
/*   nv/layers/npu_paged_attention.py:42-52.                                  */
/* For every decode token i and query head h (kv head g = h / (Hq / Hkv)):    */
/*   out[i,h,:] = softmax(q[i,h,:] . K_g[0:ctx_i]^T * scale) V_g[0:ctx_i]     */
/* with K/V gathered through block_tables[i, :].  context_lens lives on the   */
/* DEVICE (the reference keeps it on the host, which forced a per-replay task */
/* update; here a captured graph replays with no host work).                  */
/* workspace: split-KV partial results plus per-(seq, kv head) arrival        */
/* counters.  It must be zero-filled once when allocated; every call leaves   */
/* the counters at zero again, so one workspace serves any number of calls    */
/* and graph replays.  Calls that run concurrently must not share it.         */
/* ------------------------------------------------------------------------- */
size_t nvamd_paged_decode_workspace_size(int max_batch, int num_heads,
                                         int num_kv_heads,
                                         int max_context_len);

int nvamd_paged_decode(void *out, int64_t out_stride,
                       const void *q, int64_t q_stride,
                       const void *k_cache, const void *v_cache,
                       int num_blocks, int block_size,
                       const int32_t *block_tables, int bt_stride, int bt_width,
                       const int32_t *context_lens,
                       int batch, int num_heads, int num_kv_heads, int head_dim,
                       float scale, int max_context_len,
                       void *workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* Allocation-free variant of nvamd_paged_decode.  It has no counterpart in  */
/* the reference: it is for callers that cannot allocate device memory      */
/* (code under graph capture, tight serving loops, harnesses that forbid     */
/* allocation).  Same arguments and results as nvamd_paged_decode, without  */
/* the workspace: the library's own device array of                        */
/* NVAMD_DECODE_SCRATCH_BYTES, one copy per GPU held until the process      */
/* ends, serves as the workspace.  A call that would need more returns      */
/* NVAMD_ETOOLARGE and launches nothing (the need is                        */
/* nvamd_paged_decode_workspace_size(batch, ...); 64 MiB covers e.g. 100    */
/* sequences x 16384 tokens or 32 x 32768 at 16 query / 8 KV heads).  The   */
/* first call on a device also clears the array's counters on `stream`, so */
/* it must not be made while `stream` is captured into a graph (the clear  */
/* would only be recorded): it then returns NVAMD_ECAPTURE and launches     */
/* nothing.  Once one call has run outside capture, calls may be captured.  */
/* All calls on one GPU share its array: calls that overlap on one GPU race. */
#define NVAMD_DECODE_SCRATCH_BYTES (64u * 1024u * 1024u)
int nvamd_paged_decode_noalloc(void *out, int64_t out_stride,
                               const void *q, int64_t q_stride,
                               const void *k_cache, const void *v_cache,
                               int num_blocks, int block_size,
                               const int32_t *block_tables, int bt_stride,
                               int bt_width, const int32_t *context_lens,
                               int batch, int num_heads, int num_kv_heads,
                               int head_dim, float scale,
                               int max_context_len, hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* P5 + P2 + P4 fused: one decode step of a layer's attention.                */
/* Replaces the sequence Qwen3Attention.forward runs for a decode batch       */
/* (nv/models/qwen3.py:83-96 then :105-112): q_norm/k_norm, RoPE, kv write    */
/* of post-RoPE k and raw v at slot_mapping, then paged attention.            */
/* Equivalent to nvamd_qk_norm_rope(q, k, v, ..., k_cache, v_cache,          */
/* slot_mapping) followed by nvamd_paged_decode over the normalised q, bit    */
/* for bit, provided slot_mapping[i] is the cache slot of row positions[i]   */
/* of sequence i's block table (as the block manager builds decode metadata:  */
/* position = context_lens[i] - 1).  q, k, v are the raw projection rows      */
/* [batch, *] and are NOT rewritten (only out and the cache are written).     */
/* q_weight, k_weight, cos_sin and every row stride: 16-byte aligned.         */
/* Workspace rules as for nvamd_paged_decode.                                 */
/* ------------------------------------------------------------------------- */
int nvamd_paged_decode_fused(void *out, int64_t out_stride,
                             const void *q, int64_t q_stride,
                             const void *k, int64_t k_stride,
                             const void *v, int64_t v_stride,
                             const void *q_weight, const void *k_weight,
                             const int64_t *positions,
                             const float *cos_sin, int max_positions, float eps,
                             void *k_cache, void *v_cache,
                             int num_blocks, int block_size,
                             const int64_t *slot_mapping,
                             const int32_t *block_tables, int bt_stride, int bt_width,
                             const int32_t *context_lens,
                             int batch, int num_heads, int num_kv_heads, int head_dim,
                             float scale, int max_context_len,
                             void *workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* P2: paged KV store.                                                       */
/* Replaces PagedKVCache.write (nv/npu/paged_kv_cache.py:44-69): the two      */
/* index_copy_ calls  cache_flat[slot_mapping[t]] = kv[t]  for K and V.       */
/* A negative slot skips that token (padding rows).                           */
/* ------------------------------------------------------------------------- */
int nvamd_kv_cache_write(const void *k, int64_t k_stride,
                         const void *v, int64_t v_stride,
                         void *k_cache, void *v_cache,
                         const int64_t *slot_mapping, int num_tokens,
                         int num_kv_heads, int head_dim, int64_t num_slots,
                         hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* P5 (+P2 fused): per-head RMSNorm of q and k, then rotate-half RoPE, then   */
/* (optionally) the KV store of post-RoPE k and raw v.                        */
/* Replaces q_norm / k_norm (npu_rms_norm, nv/layers/layernorm.py:12-17,      */
/* called at nv/models/qwen3.py:83-84), apply_rotary_pos_emb_tnd              */
/* (npu_rotary_mul rotary_mode="half", nv/layers/rotary_embedding.py:78-97)   */
/* and kv_cache.write (nv/models/qwen3.py:91-96).                             */
/* q and k are rewritten IN PLACE.  cos_sin is the fp32 table                 */
/* [max_positions, 128] laid out as 64 cos values then 64 sin values per      */
/* position (the reference's emb = cat(freqs, freqs) halves are identical,    */
/* so one half of each is stored).  Rounding points follow the reference:     */
/* normed value rounded to bf16, cos/sin rounded to bf16, rotation in fp32    */
/* with one final rounding.                                                   */
/* Pass k_cache = v_cache = NULL to skip the store (slot_mapping unused).     */
/* q, k, v, the weights, cos_sin and the caches: 16-byte aligned, row strides */
/* multiples of 8 elements (every access is 16 bytes).                        */
/* ------------------------------------------------------------------------- */
int nvamd_qk_norm_rope(void *q, int64_t q_stride,
                       void *k, int64_t k_stride,
                       const void *v, int64_t v_stride,
                       const void *q_weight, const void *k_weight,
                       const int64_t *positions,
                       const float *cos_sin, int max_positions,
                       void *k_cache, void *v_cache,
                       const int64_t *slot_mapping, int64_t num_slots,
                       int num_tokens, int num_heads, int num_kv_heads,
                       int head_dim, float eps,
                       hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* P3: causal varlen prefill attention (bf16 MFMA).                           */
/* Replaces torch_npu.npu_fused_infer_attention_score as called at            */
/* nv/layers/npu_prefill_attention.py:98-112 (dense route) and :66-96 (paged, */
/* prefix-hit route), TND layout, scale = head_dim^-0.5, GQA h -> h/(Hq/Hkv). */
/* cu_seqlens_q: int32 [n_seqs+1] on the device (the reference passes the     */
/* cumulative ends without the leading 0 as a host list).                     */
/* dense: k/v hold the same tokens as q; row i of a sequence sees keys 0..i.  */
/* paged: keys come from the cache through block_tables; kv_lens (device,     */
/*   per sequence -- the reference's per-layer context_lens.tolist()) gives   */
/*   each sequence's key count; query row r of a q_len-row sequence sees keys */
/*   0..kv_len-q_len+r (causal, bottom-right aligned).                        */
/* max_q_len bounds every q_len (it sizes the grid).                          */
/* ------------------------------------------------------------------------- */
int nvamd_varlen_prefill(void *out, int64_t out_stride,
                         const void *q, int64_t q_stride,
                         const void *k, int64_t k_stride,
                         const void *v, int64_t v_stride,
                         const int32_t *cu_seqlens_q, int n_seqs, int max_q_len,
                         int num_heads, int num_kv_heads, int head_dim,
                         float scale, hipStream_t stream);

int nvamd_paged_prefill(void *out, int64_t out_stride,
                        const void *q, int64_t q_stride,
                        const void *k_cache, const void *v_cache,
                        int num_blocks, int block_size,
                        const int32_t *block_tables, int bt_stride, int bt_width,
                        const int32_t *cu_seqlens_q, const int32_t *kv_lens,
                        int n_seqs, int max_q_len,
                        int num_heads, int num_kv_heads, int head_dim,
                        float scale, hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* P1: ragged-batch packing.                                                  */
/* Replaces BlockManager.get_block_tables_tensor / get_context_lens_tensor /  */
/* get_slot_mapping (nv/npu/block_manager.py:207-250; the per-token Python    */
/* slot loop and one H2D copy per table row) and the input build of           */
/* ModelRunner._prepare_prefill_inputs (nv/model_runner.py:169-197) and       */
/* ModelRunner.decode (nv/model_runner.py:245-258).                           */
/* desc: int32 [5][batch] on the device = mirror row, start position, query   */
/*   length, table length (blocks), context length of each sequence.         */
/* updates: int32 [num_updates][3] = (mirror row, column, block id) entries   */
/*   of the device block-table mirror [mirror_rows, mirror_stride] that       */
/*   changed since the last call; applied before anything is read.  At most   */
/*   one entry per (row, column).                                             */
/* Outputs (any may be NULL to skip):                                         */
/*   block_tables[i, c] = c < table_len_i ? mirror[row_i, c] : 0, c < bt_width*/
/*   context_lens[i]; cu_seqlens[0..batch] (cumulative query lengths);        */
/*   last_token_indices[i] = cu_seqlens[i+1] - 1;                             */
/*   for token k of sequence i (t = cu_seqlens[i] + k, pos = start_i + k):    */
/*     positions[t] = pos;                                                    */
/*     slot_mapping[t] = mirror[row_i, pos / bs] * bs + pos % bs (-1 if the   */
/*       table does not reach pos);                                           */
/*     input_ids[t] = token_ids[t] (int32 -> int64).                          */
/* ------------------------------------------------------------------------- */
int nvamd_pack_batch(const int32_t *desc, int batch,
                     const int32_t *updates, int num_updates,
                     const int32_t *token_ids,
                     int32_t *mirror, int mirror_stride, int mirror_rows,
                     int block_size,
                     int32_t *block_tables, int bt_stride, int bt_width,
                     int32_t *context_lens, int64_t *slot_mapping,
                     int64_t *positions, int32_t *cu_seqlens,
                     int64_t *last_token_indices, int64_t *input_ids,
                     hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* Fused elementwise kernels of the decoder around the attention path.        */
/* add_rms_norm: residual[r] += delta[r] (bf16 rounding; skipped when delta   */
/*   is NULL), then out[r] = residual[r] * rsqrt(mean(residual[r]^2) + eps)   */
/*   * weight, fp32 math, one bf16 rounding.  The decoder layer's residual    */
/*   add + RMSNorm (nv/models/qwen3.py:138-150; npu_rms_norm at               */
/*   nv/layers/layernorm.py:12-17).  hidden: any multiple of 8.              */
/* silu_mul: out[r, i] = bf16(bf16(silu(gu[r, i])) * gu[r, inter + i]) for the */
/*   fused gate/up projection (nv/models/qwen3.py:34-35).                     */
/* argmax_rows: out[r] = first index of the maximum of logits[r, 0:vocab]     */
/*   (greedy sampling, torch.argmax at nv/layers/sampler.py:13-14).           */
/* ------------------------------------------------------------------------- */
int nvamd_add_rms_norm(const void *delta, void *residual, const void *weight,
                       void *out, int rows, int hidden, float eps,
                       hipStream_t stream);

int nvamd_silu_mul(const void *gate_up, int64_t gu_stride, void *out,
                   int64_t out_stride, int rows, int inter,
                   hipStream_t stream);

int nvamd_argmax_rows(const void *logits, int64_t row_stride, int rows,
                      int vocab, int64_t *out, hipStream_t stream);

/* ------------------------------------------------------------------------- */
/* Skinny-M projections of the decode step (m <= 128 rows), a weight stream:  */
/*   acc[r, c] = sum_k a[r, k] * w[c, k] (fp32), for the decoder's qkv / o /  */
/*   gate_up / down projections and the LM head at decode batch sizes        */
/*   (F.linear at nv/models/qwen3.py:26-35, 48-51, 119 and                    */
/*   nv/layers/embed_head.py:24-39), with the residual add + RMSNorm of the   */
/*   decoder layer (nv/models/qwen3.py:138-150, nv/layers/layernorm.py:12-17) */
/*   folded into the GEMMs on either side of it.                              */
/* Tiled layout: a [R, C] bf16 matrix (R % 16 == 0, C % 32 == 0) stored as    */
/*   (R/16) x (C/32) tiles of 16 rows x 32 columns, 512 elements each, in     */
/*   row-tile-major order; element (r, c) of a tile at                        */
/*   128 * (c / 8) + 8 * r + c % 8 -- the MFMA operand order, so a wave loads */
/*   1 KB of contiguous memory per instruction.  Index of element (r, c):     */
/*   ((r/16) * (C/32) + c/32) * 512 + 128 * ((c%32)/8) + 8 * (r%16) + c%8.    */
/* w_tiled: the weight [n, k] (epilogue 1: [2n, k]) in tiled layout, no       */
/*   stride.  flags: NVAMD_GEMM_X_TILED -- x is tiled with 16 * ceil(m/16)    */
/*   rows (x_stride unused; rows past m only reach dropped outputs);          */
/*   NVAMD_GEMM_Y_TILED -- y is tiled [16 * ceil(m/16), n] (y_stride unused;  */
/*   rows past m are neither read as inputs nor written).                     */
/* Prologue: with x_ssq == NULL, a = x.  Otherwise x is the residual stream,  */
/*   x_ssq[r * (k/32) + t] holds the sum of squares of x[r, 32t..32t+31], and */
/*   a = bf16((x * rsqrt(sum_t x_ssq / k + eps)) * norm_weight); k <= 2048   */
/*   (NVAMD_EUNSUPPORTED above).                                              */
/* epilogue 0 (store): y[r, c] = bf16(acc).                                   */
/* epilogue 1 (silu_mul): w is the fused [2n, k] gate/up weight;              */
/*   y[r, c] = bf16(bf16(silu(bf16(acc_gate))) * bf16(acc_up)).               */
/* epilogue 2 (residual): y is the residual stream, updated in place:         */
/*   y[r, c] = bf16(y[r, c] + bf16(acc)); y_ssq[r * (n/32) + t] = sum of      */
/*   squares of the new y[r, 32t..32t+31] (the next prologue's x_ssq).        */
/* n % 32 == 0, k % 256 == 0; x, w_tiled, x_ssq, norm_weight 16-byte aligned, */
/* y 8-byte aligned; row strides in elements (x: multiple of 8; y: of 4).     */
/* Shapes that split K over workgroups need a zero-filled workspace of        */
/* nvamd_skinny_linear_workspace_size(n, k, epilogue) bytes (0: none); calls  */
/* leave it zero-filled and must not overlap.  m > 128: NVAMD_EUNSUPPORTED.  */
/* embed_rows: out[r] = table[ids[r]] (zeros for an id outside [0, vocab)),   */
/*   the token embedding (torch.embedding at nv/layers/embed_head.py:20-21),  */
/*   and, if ssq != NULL, ssq[r * (hidden/32) + t] = sum of squares of        */
/*   out[r, 32t..32t+31].  hidden % 1024 == 0.  out_tiled != 0: out is tiled  */
/*   (the layout above, out_stride unused).                                   */
/* ------------------------------------------------------------------------- */
size_t nvamd_skinny_linear_workspace_size(int n, int k, int epilogue);

#define NVAMD_GEMM_X_TILED 1
#define NVAMD_GEMM_Y_TILED 2

int nvamd_skinny_linear(const void *x, int64_t x_stride, const float *x_ssq,
                        const void *norm_weight, float eps,
                        const void *w_tiled, void *y, int64_t y_stride,
                        float *y_ssq, int epilogue, int flags, int m, int n,
                        int k, void *workspace, size_t workspace_bytes,
                        hipStream_t stream);

int nvamd_embed_rows(const int64_t *ids, const void *table,
                     int64_t table_stride, int vocab, void *out,
                     int64_t out_stride, int out_tiled, float *ssq, int rows,
                     int hidden, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NVAMD_H */
