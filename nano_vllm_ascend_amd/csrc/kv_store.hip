// Paged KV store and the fused per-head QK-RMSNorm + RoPE (+ KV store) for gfx950.
//
// kv_cache_write  replaces PagedKVCache.write (nv/npu/paged_kv_cache.py:44-69):
//   key_cache_flat.index_copy_(0, slot_mapping, key_states) and the same for V.
// qk_norm_rope    replaces q_norm/k_norm + apply_rotary_pos_emb_tnd + kv_cache.write
//   as composed in Qwen3Attention.forward (nv/models/qwen3.py:83-96).
//
// Both are pure HBM streams: every byte is read once and written once, with 16-byte
// accesses (eight lanes cover one 256-byte head row in two 128-byte halves).  A slot past the
// cache or a position past the RoPE table, where the reference's indexing raises, is skipped or
// clamped and reported in the index-error word.
#include "common.h"

namespace nvamd {
namespace {

// One thread moves one 16-byte chunk (8 dims) of K and the same chunk of V.
__global__ void __launch_bounds__(256)
kv_cache_write_kernel(const u16 *__restrict__ k, int64_t k_stride, const u16 *__restrict__ v, int64_t v_stride,
                      u16 *__restrict__ k_cache, u16 *__restrict__ v_cache, const int64_t *__restrict__ slots,
                      int num_tokens, int num_kv_heads, int64_t num_slots, u32 *err) {
  const int chunks_per_token = num_kv_heads * (kHeadDim / 8);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)num_tokens * chunks_per_token) return;
  const int t = (int)(i / chunks_per_token);
  const int ch = (int)(i % chunks_per_token);  // = head * 16 + chunk
  const int64_t slot = slots[t];
  if (slot >= num_slots || slot < -1) {  // index_copy_ would raise: skip the row, report it once per token
    if (ch == 0) flag_index_error(err, NVAMD_ERR_SLOT);
    return;
  }
  if (slot < 0) return;  // -1: a padding row
  const int64_t dst = slot * ((int64_t)num_kv_heads * kHeadDim) + (int64_t)ch * 8;
  // Nontemporal loads and stores: each byte is touched once.  Over 38k tokens, with consecutive
  // launches on different buffers (so no launch finds its bytes in the Infinity Cache), this runs
  // at the device's plain-copy rate (5.26 TB/s); plain loads measure 1.03x slower.
  const u32x4 kk = ld16_stream(k + (int64_t)t * k_stride + ch * 8);
  const u32x4 vv = ld16_stream(v + (int64_t)t * v_stride + ch * 8);
  __builtin_nontemporal_store(kk, reinterpret_cast<u32x4 *>(k_cache + dst));
  __builtin_nontemporal_store(vv, reinterpret_cast<u32x4 *>(v_cache + dst));
}

struct NormRopeArgs {
  u16 *q;
  int64_t q_stride;
  u16 *k;
  int64_t k_stride;
  const u16 *v;
  int64_t v_stride;
  const u16 *q_w;
  const u16 *k_w;
  const int64_t *positions;
  const float *cos_sin;
  u16 *k_cache;
  u16 *v_cache;
  const int64_t *slots;
  int64_t num_slots;
  int max_positions;
  int num_tokens;
  int num_heads;
  int num_kv_heads;
  float eps;
  u32 *err;  // index-error word
};

// An aligned group of 8 lanes owns one head vector of one token: lane c holds dims
// 8c..8c+7 and their rotate-half partners 64+8c..64+8c+7, so RoPE needs no lane exchange,
// every access is 16 bytes, and the norm's sum of squares is an 8-lane reduction
// (head_norm_rope, shared with the fused decode kernel, so both round identically).
// Vectors per token: num_heads q heads, num_kv_heads k heads, then (when a cache is given)
// num_kv_heads v heads that are only stored.  A 256-thread workgroup takes 32 vectors.
__global__ void __launch_bounds__(256)
qk_norm_rope_kernel(NormRopeArgs a) {
  const bool store = a.k_cache != nullptr;
  const int vecs = a.num_heads + a.num_kv_heads * (store ? 2 : 1);
  const int64_t gv = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  if (gv >= (int64_t)a.num_tokens * vecs) return;  // whole 8-lane groups leave together
  const int t = (int)(gv / vecs);
  const int vec = (int)(gv % vecs);
  const int c = threadIdx.x & 7;

  int64_t slot = -1;
  if (store) {
    slot = a.slots[t];
    if (slot >= a.num_slots || slot < -1) {  // index_copy_ would raise: skip the row, report it once per token
      if (vec == 0 && c == 0) flag_index_error(a.err, NVAMD_ERR_SLOT);
      slot = -1;
    }
  }
  const int64_t cache_row = slot * ((int64_t)a.num_kv_heads * kHeadDim);

  if (vec >= a.num_heads + a.num_kv_heads) {  // raw V -> cache
    const int h = vec - a.num_heads - a.num_kv_heads;
    if (slot < 0) return;
    const u16 *src = a.v + (int64_t)t * a.v_stride + h * kHeadDim + 8 * c;
    u16 *dst = a.v_cache + cache_row + h * kHeadDim + 8 * c;
    const u32x4 lo = ld16(src), hi = ld16(src + 64);
    __builtin_nontemporal_store(lo, reinterpret_cast<u32x4 *>(dst));
    __builtin_nontemporal_store(hi, reinterpret_cast<u32x4 *>(dst + 64));
    return;
  }

  const bool is_q = vec < a.num_heads;
  const int h = is_q ? vec : vec - a.num_heads;
  u16 *x = (is_q ? a.q + (int64_t)t * a.q_stride : a.k + (int64_t)t * a.k_stride) + h * kHeadDim + 8 * c;
  const u16 *wt = (is_q ? a.q_w : a.k_w) + 8 * c;
  u32x4 lo = ld16(x), hi = ld16(x + 64);
  const u32x4 w_lo = ld16(wt), w_hi = ld16(wt + 64);
  int64_t pos = a.positions[t];
  if (pos < 0 || pos >= a.max_positions) {  // the RoPE cache lookup would raise: clamp and report
    if (vec == 0 && c == 0) flag_index_error(a.err, NVAMD_ERR_POSITION);
    pos = pos < 0 ? 0 : a.max_positions - 1;
  }
  float cs[8], sn[8];
  rope_row8(a.cos_sin, pos, c, cs, sn);
  head_norm_rope(lo, hi, w_lo, w_hi, cs, sn, a.eps);
  st16(x, lo);
  st16(x + 64, hi);
  if (!is_q && slot >= 0) {  // post-RoPE k into the cache; not read again by this step
    u16 *dst = a.k_cache + cache_row + h * kHeadDim + 8 * c;
    __builtin_nontemporal_store(lo, reinterpret_cast<u32x4 *>(dst));
    __builtin_nontemporal_store(hi, reinterpret_cast<u32x4 *>(dst + 64));
  }
}

}  // namespace
}  // namespace nvamd

using namespace nvamd;

extern "C" int nvamd_kv_cache_write(const void *k, int64_t k_stride, const void *v, int64_t v_stride, void *k_cache,
                                    void *v_cache, const int64_t *slot_mapping, int num_tokens, int num_kv_heads,
                                    int head_dim, int64_t num_slots, hipStream_t stream) {
  if (num_tokens == 0) return NVAMD_OK;
  if (!k || !v || !k_cache || !v_cache || !slot_mapping || num_tokens < 0 || num_kv_heads <= 0 || num_slots <= 0)
    return NVAMD_EINVAL;
  if (head_dim != kHeadDim) return NVAMD_EUNSUPPORTED;
  if (!aligned16(k) || !aligned16(v) || !aligned16(k_cache) || !aligned16(v_cache) || k_stride % 8 || v_stride % 8 ||
      k_stride < (int64_t)num_kv_heads * head_dim || v_stride < (int64_t)num_kv_heads * head_dim)
    return NVAMD_EINVAL;
  const int64_t total = (int64_t)num_tokens * num_kv_heads * (kHeadDim / 8);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return NVAMD_EINVAL;
  hipLaunchKernelGGL(kv_cache_write_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const u16 *>(k), k_stride, static_cast<const u16 *>(v), v_stride,
                     static_cast<u16 *>(k_cache), static_cast<u16 *>(v_cache), slot_mapping, num_tokens, num_kv_heads,
                     num_slots, index_error_word());
  return launch_status();
}

extern "C" int nvamd_qk_norm_rope(void *q, int64_t q_stride, void *k, int64_t k_stride, const void *v,
                                  int64_t v_stride, const void *q_weight, const void *k_weight,
                                  const int64_t *positions, const float *cos_sin, int max_positions, void *k_cache,
                                  void *v_cache, const int64_t *slot_mapping, int64_t num_slots, int num_tokens,
                                  int num_heads, int num_kv_heads, int head_dim, float eps, hipStream_t stream) {
  if (num_tokens == 0) return NVAMD_OK;
  if (!q || !k || !q_weight || !k_weight || !positions || !cos_sin || num_tokens < 0 || num_heads <= 0 ||
      num_kv_heads <= 0 || max_positions <= 0)
    return NVAMD_EINVAL;
  if (head_dim != kHeadDim) return NVAMD_EUNSUPPORTED;
  const bool store = k_cache != nullptr || v_cache != nullptr;
  if (store && (!k_cache || !v_cache || !v || !slot_mapping || num_slots <= 0)) return NVAMD_EINVAL;
  // 16-byte accesses: rows, weights, the rope table and the caches 16-byte aligned
  if (!aligned16(q) || !aligned16(k) || !aligned16(q_weight) || !aligned16(k_weight) || !aligned16(cos_sin) ||
      q_stride % 8 || k_stride % 8 || q_stride < (int64_t)num_heads * head_dim ||
      k_stride < (int64_t)num_kv_heads * head_dim)
    return NVAMD_EINVAL;
  if (store && (!aligned16(v) || !aligned16(k_cache) || !aligned16(v_cache) || v_stride % 8 ||
                v_stride < (int64_t)num_kv_heads * head_dim))
    return NVAMD_EINVAL;

  NormRopeArgs a;
  a.q = static_cast<u16 *>(q);
  a.q_stride = q_stride;
  a.k = static_cast<u16 *>(k);
  a.k_stride = k_stride;
  a.v = static_cast<const u16 *>(v);
  a.v_stride = v_stride;
  a.q_w = static_cast<const u16 *>(q_weight);
  a.k_w = static_cast<const u16 *>(k_weight);
  a.positions = positions;
  a.cos_sin = cos_sin;
  a.k_cache = store ? static_cast<u16 *>(k_cache) : nullptr;
  a.v_cache = store ? static_cast<u16 *>(v_cache) : nullptr;
  a.slots = slot_mapping;
  a.num_slots = num_slots;
  a.max_positions = max_positions;
  a.num_tokens = num_tokens;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.eps = eps;
  a.err = index_error_word();
  const int vecs = num_heads + num_kv_heads * (store ? 2 : 1);
  const int64_t blocks = ((int64_t)num_tokens * vecs + 31) / 32;
  if (blocks > 0x7fffffff) return NVAMD_EINVAL;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return launch_status();
}

extern "C" int nvamd_version(void) { return NVAMD_ABI_VERSION; }
