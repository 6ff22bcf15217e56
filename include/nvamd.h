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

/* Library version, for the loader's sanity check. */
int nvamd_version(void);

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

/* ------------------------------------------------------------------------- */
/* P2: paged KV store.                                                        */
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

#ifdef __cplusplus
}
#endif

#endif /* NVAMD_H */
