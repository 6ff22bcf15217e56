// Paged KV store and the fused per-head QK-RMSNorm + RoPE (+ KV store) for gfx950.
//
// kv_cache_write  replaces PagedKVCache.write (nv/npu/paged_kv_cache.py:44-69):
//   key_cache_flat.index_copy_(0, slot_mapping, key_states) and the same for V.
// qk_norm_rope    replaces q_norm/k_norm + apply_rotary_pos_emb_tnd + kv_cache.write
//   as composed in Qwen3Attention.forward (nv/models/qwen3.py:83-96).
//
// Both are pure HBM streams: every byte is read once and written once, with
// 16-byte (store) / 128-byte-per-32-lanes (norm) coalesced accesses.
#include "common.h"

namespace nvamd {
namespace {

// One thread moves one 16-byte chunk (8 dims) of K and the same chunk of V.
__global__ void __launch_bounds__(256)
kv_cache_write_kernel(const u16 *__restrict__ k, int64_t k_stride, const u16 *__restrict__ v, int64_t v_stride,
                      u16 *__restrict__ k_cache, u16 *__restrict__ v_cache, const int64_t *__restrict__ slots,
                      int num_tokens, int num_kv_heads, int64_t num_slots) {
  const int chunks_per_token = num_kv_heads * (kHeadDim / 8);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)num_tokens * chunks_per_token) return;
  const int t = (int)(i / chunks_per_token);
  const int ch = (int)(i % chunks_per_token);  // = head * 16 + chunk
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t dst = slot * ((int64_t)num_kv_heads * kHeadDim) + (int64_t)ch * 8;
  // Nontemporal stores: the pages are not read again by this step, so they should not displace
  // L2 lines (1.14x faster over 38k tokens; nontemporal loads as well measure 1.11x slower).
  const u32x4 kk = ld16(k + (int64_t)t * k_stride + ch * 8);
  const u32x4 vv = ld16(v + (int64_t)t * v_stride + ch * 8);
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
};

// A half-wave (32 lanes) owns one head vector of one token.  Lane l holds dims
// (2l, 2l+1) and their rotate-half partners (64+2l, 65+2l), so RoPE needs no
// cross-lane traffic and each 32-lane load covers one 128-byte line.
// Vectors per token: num_heads q heads, num_kv_heads k heads, then (when a
// cache is given) num_kv_heads v heads that are only stored.
__global__ void __launch_bounds__(256)
qk_norm_rope_kernel(NormRopeArgs a) {
  const bool store = a.k_cache != nullptr;
  const int vecs = a.num_heads + a.num_kv_heads * (store ? 2 : 1);
  const int64_t hw = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (hw >= (int64_t)a.num_tokens * vecs) return;
  const int t = (int)(hw / vecs);
  const int vec = (int)(hw % vecs);
  const int l = threadIdx.x & 31;
  const int d0 = 2 * l;

  int64_t slot = -1;
  if (store) {
    slot = a.slots[t];
    if (slot >= a.num_slots) slot = -1;
  }
  const int64_t cache_row = slot * ((int64_t)a.num_kv_heads * kHeadDim);

  if (vec >= a.num_heads + a.num_kv_heads) {  // raw V -> cache
    const int h = vec - a.num_heads - a.num_kv_heads;
    if (slot < 0) return;
    const u16 *src = a.v + (int64_t)t * a.v_stride + h * kHeadDim;
    u16 *dst = a.v_cache + cache_row + h * kHeadDim;
    const u32 lo = *reinterpret_cast<const u32 *>(src + d0);
    const u32 hi = *reinterpret_cast<const u32 *>(src + 64 + d0);
    *reinterpret_cast<u32 *>(dst + d0) = lo;
    *reinterpret_cast<u32 *>(dst + 64 + d0) = hi;
    return;
  }

  const bool is_q = vec < a.num_heads;
  const int h = is_q ? vec : vec - a.num_heads;
  u16 *x = is_q ? a.q + (int64_t)t * a.q_stride + h * kHeadDim : a.k + (int64_t)t * a.k_stride + h * kHeadDim;
  const u16 *wt = is_q ? a.q_w : a.k_w;

  const u32 x_lo = *reinterpret_cast<const u32 *>(x + d0);       // dims d0, d0+1
  const u32 x_hi = *reinterpret_cast<const u32 *>(x + 64 + d0);  // dims 64+d0, 65+d0
  const u32 w_lo = *reinterpret_cast<const u32 *>(wt + d0);
  const u32 w_hi = *reinterpret_cast<const u32 *>(wt + 64 + d0);
  const float x0 = bf16_lo(x_lo), x1 = bf16_hi(x_lo), x2 = bf16_lo(x_hi), x3 = bf16_hi(x_hi);

  float ss = head_ssq4(x0, x1, x2, x3);
  ss = sum16(ss);
  ss += swizzle_xor16(ss);  // the 32 lanes of this half-wave: a balanced tree in lane order
  const float rstd = head_rstd(ss, a.eps);

  // RMSNorm output rounded to bf16 (the reference's norm returns bf16).
  const float y0 = head_norm(x0, rstd, bf16_lo(w_lo));
  const float y1 = head_norm(x1, rstd, bf16_hi(w_lo));
  const float y2 = head_norm(x2, rstd, bf16_lo(w_hi));
  const float y3 = head_norm(x3, rstd, bf16_hi(w_hi));

  int64_t pos = a.positions[t];
  pos = pos < 0 ? 0 : (pos >= a.max_positions ? a.max_positions - 1 : pos);
  const float *cs = a.cos_sin + pos * kHeadDim;
  const float c0 = round_bf16(cs[d0]), c1 = round_bf16(cs[d0 + 1]);
  const float s0 = round_bf16(cs[64 + d0]), s1 = round_bf16(cs[64 + d0 + 1]);

  const u32 o_lo = pack_bf16x2(rope_lo(y0, y2, c0, s0), rope_lo(y1, y3, c1, s1));
  const u32 o_hi = pack_bf16x2(rope_hi(y0, y2, c0, s0), rope_hi(y1, y3, c1, s1));
  *reinterpret_cast<u32 *>(x + d0) = o_lo;
  *reinterpret_cast<u32 *>(x + 64 + d0) = o_hi;
  if (!is_q && slot >= 0) {
    u16 *dst = a.k_cache + cache_row + h * kHeadDim;
    *reinterpret_cast<u32 *>(dst + d0) = o_lo;
    *reinterpret_cast<u32 *>(dst + 64 + d0) = o_hi;
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
                     num_slots);
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
  auto a4 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; };
  if (!a4(q) || !a4(k) || !a4(q_weight) || !a4(k_weight) || q_stride % 2 || k_stride % 2 ||
      q_stride < (int64_t)num_heads * head_dim || k_stride < (int64_t)num_kv_heads * head_dim)
    return NVAMD_EINVAL;
  if (store && (!a4(v) || !a4(k_cache) || !a4(v_cache) || v_stride % 2 || v_stride < (int64_t)num_kv_heads * head_dim))
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
  const int vecs = num_heads + num_kv_heads * (store ? 2 : 1);
  const int64_t blocks = ((int64_t)num_tokens * vecs + 7) / 8;
  if (blocks > 0x7fffffff) return NVAMD_EINVAL;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return launch_status();
}

extern "C" int nvamd_version(void) { return NVAMD_ABI_VERSION; }
