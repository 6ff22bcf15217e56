// GQA paged decode attention for gfx950 (replaces torch_npu._npu_paged_attention,
// nv/layers/npu_paged_attention.py:27-100).
//
// Work decomposition (split-KV, one kernel):
//   a workgroup of NW waves owns one (sequence b, kv head g, partition p) of
//   PART = NW * CPW * 64 consecutive context tokens, for all GQA query heads
//   that read kv head g, so every K/V byte is read from HBM once.  Each wave
//   owns CPW chunks of 64 tokens.  The grid is 1-D over the items in b, g, p
//   order with p fastest, counted over the partitions that exist for the
//   device-side context lengths: a unit's partitions run side by side, so its
//   merge overlaps other units' loads, and the slack a loose context bound adds
//   (graph capture uses max_model_len) is a run of empty workgroups at the end.
//
// Lane layout inside a wave (64 lanes): r = lane/8 picks token rows r and r+8
// of each 16-row tile, c = lane%8 picks dims 8c..8c+7 and 64+8c..64+8c+7.
// Eight lanes read one 256-byte K/V row as two whole 128-byte lines.
//
// Per 64-token chunk a wave's 32 16-byte loads (32 KB) come before any math in the
// source; at 4 waves per SIMD (<= 128 VGPRs) the compiler issues them in register-sized
// batches behind the per-tile block-table reads, so two or three batches are in flight
// at a time.  Split launches load K/V nontemporally (read once; no L2 allocation).
// Tiles past the wave's range re-read its last valid tile (a cache hit, not HBM
// traffic) so the load stream stays branch free.  Then:
//   QK:  v_dot2 over bf16 pairs for the whole chunk, 3-step DPP sum over 8 lanes;
//   softmax: each 8-lane row group keeps its own running max, so a chunk
//        needs no cross-lane max and no branch -- one rescale per chunk;
//   PV:  the two rows a lane holds are paired per dim with v_perm, P is
//        rounded to bf16 pairs, one v_dot2 adds both tokens' terms.
// GQA 2 fills 2 of 16 rows of an MFMA tile, so the contraction stays on v_dot2
// in the vector ALUs, which have ample headroom: the kernel is HBM bound.
//
// Merge: each wave folds its 8 row groups with DPP and swizzles, wave 0 folds the
// NW waves through LDS.  A multi-partition unit's wave 0 then publishes
// (max, sum, acc[128]) per head with agent-scope write-through stores, waits for
// them, and bumps a wrapping arrival counter; the last to arrive reads the partials with
// agent-scope loads, all issued before the first is used, and writes the output.  No L2
// writeback or invalidate is needed.  Launches with few items (short contexts, small
// batches) give each (sequence, kv head) one workgroup that covers the whole context
// bound: no partials and no item scan.
//
// Fused decode step (nvamd_paged_decode_fused): the same kernel also runs the per-head
// RMSNorm + RoPE of the raw query rows (each wave normalises its GQA rows while its first
// K/V loads are in flight) and of the new token's k, and stores that k and the raw v at
// slots[b] -- one launch instead of qk_norm_rope + decode, with identical results: the
// norm's partial sums are combined in the same balanced tree as the standalone kernel's.
// The wave whose chunk holds the new token's row stores it before loading its chunk.
#include <mutex>

#include "common.h"

namespace nvamd {
namespace {

constexpr int kPartFloats = 132;  // max, sum, 128 accumulators, 2 pad (16-byte rows)
// Arrival counters live in a fixed-size region at the front of the workspace so
// calls with different batch sizes or context bounds never place partial
// results where another call expects a zero counter.
constexpr int kCounterSlots = 16384;
constexpr size_t kCounterBytes = kCounterSlots * sizeof(int);
constexpr int kMinPart = 256;  // smallest partition of a split launch (sizes the workspace)

struct DecodeArgs {
  u16 *out;
  int64_t out_stride;
  const u16 *q;
  int64_t q_stride;
  const u16 *k_cache;
  const u16 *v_cache;
  const int32_t *block_tables;
  const int32_t *context_lens;
  float *partials;
  int *counters;
  int bt_stride;
  int bt_width;
  int num_blocks;
  int num_kv_heads;
  int bs_log2;
  int max_parts;
  int max_ctx;
  int batch;
  float scale_log2e;
  // Query heads of kv head g in q / out: q_group * g + q_head0 + (0 .. GQA-1).  One launch covers
  // a whole group (q_group == GQA, q_head0 == 0) unless the ratio needs several launches.
  int q_group;
  int q_head0;
  // Fused decode step only: q holds the raw projection rows; the kernel applies the per-head
  // RMSNorm and RoPE to q and to the new token's k, and stores that k and the raw v at slots[b].
  const u16 *k_new;
  int64_t k_new_stride;
  const u16 *v_new;
  int64_t v_new_stride;
  const u16 *q_w;
  const u16 *k_w;
  const int64_t *positions;
  const float *cos_sin;
  const int64_t *slots;
  int64_t num_slots;
  int max_positions;
  float eps;
  bool store_new;  // this launch stores the new token's k / v (the first of a group's launches)
  u32 *err;        // index-error word
};

struct KVTile {
  u32x4 ka0, ka1, kb0, kb1, va0, va1, vb0, vb1;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Inclusive prefix sum over the 64 lanes of a wave, in registers: a Hillis-Steele scan inside
// each 16-lane row by DPP row shifts (lanes shifted in from outside the row read 0), then each
// row adds the totals of the rows before it (lane 15 of each row, read into scalar registers).
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
  v += __builtin_amdgcn_mov_dpp(v, 0x111, 0xF, 0xF, true);  // row_shr:1
  v += __builtin_amdgcn_mov_dpp(v, 0x112, 0xF, 0xF, true);  // row_shr:2
  v += __builtin_amdgcn_mov_dpp(v, 0x114, 0xF, 0xF, true);  // row_shr:4
  v += __builtin_amdgcn_mov_dpp(v, 0x118, 0xF, 0xF, true);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
  const int r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane >> 4;
  return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// 2 * GQA consecutive floats of a partial record through an agent-coherent buffer range
// (write-through stores, loads that bypass the non-coherent caches): 8 bytes for one head,
// 16-byte pieces for two or four.
template <int GQA>
__device__ __forceinline__ void store_block(__amdgpu_buffer_rsrc_t rsrc, int byte_off, const float (&v)[2 * GQA]) {
  if constexpr (GQA == 1) {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(v[0]), __float_as_uint(v[1])}, rsrc, byte_off, 0,
                                          kCachePolicyAgent);
  } else {
#pragma unroll
    for (int h = 0; h < GQA / 2; ++h)
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4{__float_as_uint(v[4 * h]), __float_as_uint(v[4 * h + 1]), __float_as_uint(v[4 * h + 2]),
                __float_as_uint(v[4 * h + 3])},
          rsrc, byte_off + 16 * h, 0, kCachePolicyAgent);
  }
}
template <int GQA>
__device__ __forceinline__ void load_block(__amdgpu_buffer_rsrc_t rsrc, int byte_off, float (&v)[2 * GQA]) {
  if constexpr (GQA == 1) {
    const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rsrc, byte_off, 0, kCachePolicyAgent);
    v[0] = __uint_as_float(x[0]);
    v[1] = __uint_as_float(x[1]);
  } else {
#pragma unroll
    for (int h = 0; h < GQA / 2; ++h) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rsrc, byte_off + 16 * h, 0, kCachePolicyAgent);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * h + e] = __uint_as_float(x[e]);
    }
  }
}

// GQA 1, and GQA 2 with one chunk per wave, fit 128 VGPRs without spills: four waves
// per SIMD.
template <int GQA, int NW, int CPW, int TILES, bool WHOLE, bool FUSED>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu((GQA == 1 || (GQA == 2 && CPW == 1)) ? 4 : 1)))
paged_decode_kernel(DecodeArgs a) {
  constexpr int D = kHeadDim;
  constexpr int CT = 16 * TILES;  // tokens per chunk: TILES tiles of 16 rows
  constexpr int WT = CPW * CT;    // tokens per wave
  constexpr int PART = NW * WT;

  const int hkv = a.num_kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;

  // Work item of this workgroup: the blockIdx.x-th (b, g, p) in b, g, p order (p fastest)
  // over the partitions that exist for the current context lengths; a sequence with no
  // context has one item, which writes zeros.  Every wave finds it by itself: a wave-wide
  // prefix sum of the partition counts, 64 sequences at a time.
  const int ctx_cap = min(a.max_ctx, a.bt_width << a.bs_log2);
  const int item = blockIdx.x;
  int b = -1, n_parts = 0, first = 0, ctx = 0;
  int64_t nr = -1;  // fused step: the new token's position (its row in the context)
  // Index errors seen by this wave (wave-uniform, so it stays in scalar registers); reported with
  // one atomic after the K/V loop.
  u32 err_bits = 0;
  if constexpr (WHOLE) {
    // One workgroup per (b, g) covers the whole context bound: the item needs no scan, so the
    // context length, the block-table entries and q are loaded together.
    b = item / hkv;
    n_parts = 1;
    first = b;
    const int raw = a.context_lens[b];
    if (raw < 0 || raw > ctx_cap) err_bits |= NVAMD_ERR_CONTEXT;
    ctx = max(min(raw, ctx_cap), 0);
    if constexpr (FUSED) nr = a.positions[b];
  } else
  for (int b0 = 0, base = 0; b0 < a.batch; b0 += 64) {
    const int bi = b0 + lane;
    int ci = 0, np = 0;
    int64_t pi = 0;
    bool bad = false;
    if (bi < a.batch) {
      const int raw = a.context_lens[bi];
      bad = raw < 0 || raw > ctx_cap;
      ci = max(min(raw, ctx_cap), 0);
      np = max(ceil_div(ci, PART), 1);
      if constexpr (FUSED) pi = a.positions[bi];  // with the lengths: no later round trip
    }
    // every sequence is scanned by the workgroup holding its first partition, which reports a
    // context its table row or the launch's bound cannot hold
    if (__ballot(bad)) err_bits |= NVAMD_ERR_CONTEXT;
    const int incl = wave_incl_scan(np, lane);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    if (item < (base + total) * hkv) {
      const uint64_t past = __ballot((base + incl) * hkv > item);
      const int sel = __ffsll((unsigned long long)past) - 1;
      b = b0 + sel;
      // sel is wave-uniform (a ballot): read the chosen lane's values into scalar registers
      n_parts = __builtin_amdgcn_readlane(np, sel);
      first = base + __builtin_amdgcn_readlane(incl, sel) - n_parts;
      ctx = __builtin_amdgcn_readlane(ci, sel);
      if constexpr (FUSED) {
        const int lo = __builtin_amdgcn_readlane((int)(uint32_t)pi, sel);
        const int hi = __builtin_amdgcn_readlane((int)(pi >> 32), sel);
        nr = (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
      }
      break;
    }
    base += total;
  }
  if (b < 0) return;  // past the last item
  b = __builtin_amdgcn_readfirstlane(b);
  n_parts = __builtin_amdgcn_readfirstlane(n_parts);
  if constexpr (!WHOLE) {
    ctx = __builtin_amdgcn_readfirstlane(ctx);  // a scalar load already
    if constexpr (FUSED) {
      const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)nr);
      const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)nr >> 32));
      nr = (int64_t)(((uint64_t)hi << 32) | lo);
    }
  }
  const int rem = item - __builtin_amdgcn_readfirstlane(first) * hkv;
  const int g = rem / n_parts;
  const int p = rem - g * n_parts;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar address math
  const int r = lane >> 3;
  const int c = lane & 7;

  __shared__ float s_o[NW][2][GQA][D];  // per wave and half-wave: summed row groups
  __shared__ float s_l[NW][2][GQA];
  __shared__ float s_m[NW][GQA];

  const int32_t *bt_row = a.block_tables + (int64_t)b * a.bt_stride;
  const int t_begin = p * PART + w * WT;

  // Query rows of the GQA group, as bf16 pairs for v_dot2.
  u32x4 qr[GQA][2];
#pragma unroll
  for (int j = 0; j < GQA; ++j) {
    const u16 *qp = a.q + (int64_t)b * a.q_stride + (int64_t)(g * a.q_group + a.q_head0 + j) * D + 8 * c;
    qr[j][0] = ld16(qp);
    qr[j][1] = ld16(qp + 64);
  }

  float m[GQA], l[GQA], o[GQA][16];
#pragma unroll
  for (int j = 0; j < GQA; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[j][i] = 0.f;
  }

  const int t_end = min(t_begin + WT, ctx);
  const int bs_mask = (1 << a.bs_log2) - 1;
  const int64_t row_elems = (int64_t)hkv * D;  // elements between consecutive tokens
  const int64_t step8 = 8 * row_elems;

  // Fused step: the wave that will read the new token's row (its position nr, when it lies
  // inside the attended context; else wave 0 of the unit's last item) first stores the token's
  // post-RoPE k and raw v at slots[b] and waits for the stores to be acknowledged, so its own
  // K/V loads below read those values back (a wave's loads issued after its acknowledged stores
  // see them).  No other wave reads that row.  The rope row and norm weights are loaded before
  // the chunk's K/V loads and the query rows are normalised after those are issued, in the
  // same branch-free block, so the normalisation overlaps the K/V round trip.
  f32x4 rc0 = {}, rc1 = {}, rs0 = {}, rs1 = {};
  u32x4 qw0 = {}, qw1 = {};
  // The first chunk's block-table entries are read before the owner's store: after a store the
  // compiler cannot prove the table unchanged and would read it with vector loads, which then
  // queue behind the rope and K/V loads instead of completing on the scalar path.
  int first_blk[TILES] = {};
  if constexpr (FUSED) {
    if (t_begin < t_end) {
      const int last = (min(t_begin + WT, ctx) - 1) & ~15;
#pragma unroll
      for (int i = 0; i < TILES; ++i) first_blk[i] = bt_row[min(t_begin + 16 * i, last) >> a.bs_log2];
    }
  }
  auto rope_row = [&](float (&cs)[8], float (&sn)[8]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cs[e] = round_bf16(rc0[e]);
      cs[4 + e] = round_bf16(rc1[e]);
      sn[e] = round_bf16(rs0[e]);
      sn[4 + e] = round_bf16(rs1[e]);
    }
  };
  auto norm_queries = [&]() {
    float cs[8], sn[8];
    rope_row(cs, sn);
#pragma unroll
    for (int j = 0; j < GQA; ++j) head_norm_rope(qr[j][0], qr[j][1], qw0, qw1, cs, sn, a.eps);
  };
  if constexpr (FUSED) {
    const bool nr_in = nr >= 0 && nr < ctx;
    const bool owner = a.store_new && (nr_in ? (nr >= t_begin && nr < t_end) : (p == n_parts - 1 && w == 0));
    if (t_begin < t_end || owner) {
      if (owner && (nr < 0 || nr >= a.max_positions)) err_bits |= NVAMD_ERR_POSITION;
      const int64_t pc = nr < 0 ? 0 : (nr >= a.max_positions ? a.max_positions - 1 : nr);
      const float *row = a.cos_sin + pc * D + 8 * c;
      rc0 = *reinterpret_cast<const f32x4 *>(row);
      rc1 = *reinterpret_cast<const f32x4 *>(row + 4);
      rs0 = *reinterpret_cast<const f32x4 *>(row + 64);
      rs1 = *reinterpret_cast<const f32x4 *>(row + 68);
      qw0 = ld16(a.q_w + 8 * c);
      qw1 = ld16(a.q_w + 64 + 8 * c);
    }
    if (owner) {
      const u16 *kp = a.k_new + (int64_t)b * a.k_new_stride + g * D + 8 * c;
      const u16 *vp = a.v_new + (int64_t)b * a.v_new_stride + g * D + 8 * c;
      // every load of the store issued together, before any of it is used
      u32x4 k0 = ld16(kp), k1 = ld16(kp + 64);
      const u32x4 v0 = ld16(vp), v1 = ld16(vp + 64);
      const u32x4 kw0 = ld16(a.k_w + 8 * c), kw1 = ld16(a.k_w + 64 + 8 * c);
      const int64_t slot = a.slots[b];
      __builtin_amdgcn_sched_barrier(0);
      float cs[8], sn[8];
      rope_row(cs, sn);
      head_norm_rope(k0, k1, kw0, kw1, cs, sn, a.eps);
      if (slot >= a.num_slots || slot < -1) err_bits |= NVAMD_ERR_SLOT;
      if (r == 0 && slot >= 0 && slot < a.num_slots) {
        const int64_t dst = slot * row_elems + (int64_t)g * D + 8 * c;
        u16 *kc = const_cast<u16 *>(a.k_cache);
        u16 *vc = const_cast<u16 *>(a.v_cache);
        st16(kc + dst, k0);
        st16(kc + dst + 64, k1);
        st16(vc + dst, v0);
        st16(vc + dst + 64, v1);
      }
      __builtin_amdgcn_s_waitcnt(0);  // vmcnt counts stores on gfx9: they are acknowledged
    }
    if constexpr (CPW > 1) {  // several chunks per wave: normalise once, before the loop
      if (t_begin < t_end) norm_queries();
    }
  }

  if (t_begin < t_end) {
    const int last_tile = (t_end - 1) & ~15;
#pragma unroll 1
    for (int tc = t_begin; tc < t_end; tc += CT) {
      KVTile T[TILES];
      // the chunk's block-table entries first, so their scalar loads share one wait
      int blk_t[TILES];
#pragma unroll
      for (int i = 0; i < TILES; ++i)
        blk_t[i] = (FUSED && CPW == 1) ? first_blk[i] : bt_row[min(tc + 16 * i, last_tile) >> a.bs_log2];
#pragma unroll
      for (int i = 0; i < TILES; ++i) {
        const int t0 = min(tc + 16 * i, last_tile);
        int blk = blk_t[i];
        if ((unsigned)blk >= (unsigned)a.num_blocks) err_bits |= NVAMD_ERR_BLOCK;
        blk = min(max(blk, 0), a.num_blocks - 1);               // never leave the pool
        const int64_t slot = ((int64_t)blk << a.bs_log2) + (t0 & bs_mask) + r;
        const int64_t off = slot * row_elems + (int64_t)g * D + 8 * c;
        const u16 *kp = a.k_cache + off;
        const u16 *vp = a.v_cache + off;
        // K/V are read once per step.  Bandwidth-bound (split) launches use nontemporal loads,
        // which keep them from displacing other lines in the L2 (1.08x faster over a
        // 32 x U[256, 2304] step); latency-bound whole-unit launches use plain loads, whose
        // round trip is shorter (1.16x faster over a 4 x U[1, 512] step).
        auto ld = [](const u16 *ptr) { return WHOLE ? ld16(ptr) : ld16_stream(ptr); };
        T[i].ka0 = ld(kp);
        T[i].ka1 = ld(kp + 64);
        T[i].kb0 = ld(kp + step8);
        T[i].kb1 = ld(kp + step8 + 64);
        T[i].va0 = ld(vp);
        T[i].va1 = ld(vp + 64);
        T[i].vb0 = ld(vp + step8);
        T[i].vb1 = ld(vp + step8 + 64);
      }
      if constexpr (FUSED && CPW == 1) norm_queries();  // the wave's only chunk
      // QK for the chunk: s[tile][row a/b][head]
      float s[TILES][2][GQA];
#pragma unroll
      for (int i = 0; i < TILES; ++i) {
#pragma unroll
        for (int j = 0; j < GQA; ++j) {
          float sa = 0.f, sb = 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sa = dot2_bf16(qr[j][0][e], T[i].ka0[e], sa);
            sb = dot2_bf16(qr[j][0][e], T[i].kb0[e], sb);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sa = dot2_bf16(qr[j][1][e], T[i].ka1[e], sa);
            sb = dot2_bf16(qr[j][1][e], T[i].kb1[e], sb);
          }
          s[i][0][j] = sa;
          s[i][1][j] = sb;
        }
      }
      bool ok[TILES][2];
#pragma unroll
      for (int i = 0; i < TILES; ++i) {
        ok[i][0] = (tc + 16 * i + r) < t_end;
        ok[i][1] = (tc + 16 * i + 8 + r) < t_end;
#pragma unroll
        for (int j = 0; j < GQA; ++j) {
          const float sa = sum8(s[i][0][j]) * a.scale_log2e;
          const float sb = sum8(s[i][1][j]) * a.scale_log2e;
          s[i][0][j] = ok[i][0] ? sa : -INFINITY;
          s[i][1][j] = ok[i][1] ? sb : -INFINITY;
        }
      }

      // Online softmax, one step per chunk, per 8-lane row group.
      u32 pp[TILES][GQA];
#pragma unroll
      for (int j = 0; j < GQA; ++j) {
        float cm = m[j];
#pragma unroll
        for (int i = 0; i < TILES; ++i) cm = fmaxf(cm, fmaxf(s[i][0][j], s[i][1][j]));
        const float ref = cm == -INFINITY ? 0.f : cm;  // a group with no valid row yet
        const float alpha = fast_exp2(m[j] - ref);
        m[j] = cm;
        float add = 0.f;
#pragma unroll
        for (int i = 0; i < TILES; ++i) {
          pp[i][j] = pack_bf16x2(fast_exp2(s[i][0][j] - ref), fast_exp2(s[i][1][j] - ref));
          add += bf16_lo(pp[i][j]) + bf16_hi(pp[i][j]);
        }
        l[j] = l[j] * alpha + add;
#pragma unroll
        for (int e = 0; e < 16; ++e) o[j][e] *= alpha;
      }

      // Rows past the context may hold stale bits (NaN * 0 = NaN): zero their V.
      if (tc + CT > t_end) {
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < TILES; ++i) {
          if (!ok[i][0]) { T[i].va0 = z; T[i].va1 = z; }
          if (!ok[i][1]) { T[i].vb0 = z; T[i].vb1 = z; }
        }
      }
#pragma unroll
      for (int i = 0; i < TILES; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const u32 lo0 = pair_lo(T[i].va0[e], T[i].vb0[e]);
          const u32 hi0 = pair_hi(T[i].va0[e], T[i].vb0[e]);
          const u32 lo1 = pair_lo(T[i].va1[e], T[i].vb1[e]);
          const u32 hi1 = pair_hi(T[i].va1[e], T[i].vb1[e]);
#pragma unroll
          for (int j = 0; j < GQA; ++j) {
            o[j][2 * e] = dot2_bf16(pp[i][j], lo0, o[j][2 * e]);
            o[j][2 * e + 1] = dot2_bf16(pp[i][j], hi0, o[j][2 * e + 1]);
            o[j][8 + 2 * e] = dot2_bf16(pp[i][j], lo1, o[j][8 + 2 * e]);
            o[j][8 + 2 * e + 1] = dot2_bf16(pp[i][j], hi1, o[j][8 + 2 * e + 1]);
          }
        }
      }
    }
  }

  err_bits = __builtin_amdgcn_readfirstlane(err_bits);
  if (err_bits != 0 && lane == 0) flag_index_error(a.err, err_bits);

  // Wave merge: rescale the 8 row groups to the wave-wide max, then add groups r and r^1
  // (DPP row_ror:8) and r and r^2 (swizzle xor 16).  Lanes 0-31 then hold the sum over
  // groups 0-3 and lanes 32-63 the sum over groups 4-7.
  const int half = lane >> 5;
#pragma unroll
  for (int j = 0; j < GQA; ++j) {
    const float M = wave_max_from_groups8(m[j]);
    const float f = m[j] == -INFINITY ? 0.f : fast_exp2(m[j] - M);
    float lj = l[j] * f;
    lj += dpp<kDppRowRor8>(lj);
    lj += swizzle_xor16(lj);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float v = o[j][e] * f;
      v += dpp<kDppRowRor8>(v);
      v += swizzle_xor16(v);
      o[j][e] = v;
    }
    if ((lane & 31) < 8) {  // lanes 0-7 and 32-39 publish their half
      float *dst = &s_o[w][half][j][0];
      *reinterpret_cast<f32x4 *>(dst + 8 * c) = f32x4{o[j][0], o[j][1], o[j][2], o[j][3]};
      *reinterpret_cast<f32x4 *>(dst + 8 * c + 4) = f32x4{o[j][4], o[j][5], o[j][6], o[j][7]};
      *reinterpret_cast<f32x4 *>(dst + 64 + 8 * c) = f32x4{o[j][8], o[j][9], o[j][10], o[j][11]};
      *reinterpret_cast<f32x4 *>(dst + 64 + 8 * c + 4) = f32x4{o[j][12], o[j][13], o[j][14], o[j][15]};
      if (c == 0) s_l[w][half][j] = lj;
    }
    if (lane == 0) s_m[w][j] = M;
  }
  __syncthreads();
  if (w != 0) return;  // wave 0 finishes the workgroup

  // Workgroup merge: lane owns dims 2*lane, 2*lane+1 of every head.
  float acc[GQA][2], ls[GQA], mx[GQA];
#pragma unroll
  for (int j = 0; j < GQA; ++j) {
    float M = -INFINITY;
#pragma unroll
    for (int x = 0; x < NW; ++x) M = fmaxf(M, s_m[x][j]);
    acc[j][0] = acc[j][1] = ls[j] = 0.f;
#pragma unroll
    for (int x = 0; x < NW; ++x) {
      const float mv = s_m[x][j];
      const float f = mv == -INFINITY ? 0.f : fast_exp2(mv - M);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float2 ov = *reinterpret_cast<const float2 *>(&s_o[x][h][j][2 * lane]);
        acc[j][0] += f * ov.x;
        acc[j][1] += f * ov.y;
        ls[j] += f * s_l[x][h][j];
      }
    }
    mx[j] = M;
  }

  u16 *out_base = a.out + (int64_t)b * a.out_stride + (int64_t)(g * a.q_group + a.q_head0) * D + 2 * lane;
  if (n_parts <= 1) {
#pragma unroll
    for (int j = 0; j < GQA; ++j) {
      const float inv = ls[j] > 0.f ? 1.f / ls[j] : 0.f;
      *reinterpret_cast<u32 *>(out_base + j * D) = pack_bf16x2(acc[j][0] * inv, acc[j][1] * inv);
    }
    return;
  }

  // A partition's record (GQA * kPartFloats floats): the heads' (max, sum) pairs, then lane l's
  // accumulators of every head (dims 2l, 2l+1 of head j at 2j, 2j+1), 2 * GQA floats at
  // kHdr + 2 * GQA * l, so a lane publishes and reads its share of a partition in 16-byte pieces.
  constexpr int kRec = GQA * kPartFloats;
  constexpr int kHdr = GQA <= 2 ? 4 : 2 * GQA;
  static_assert(kHdr + 2 * GQA * 64 <= kRec, "partial record");
  float *part_base = a.partials + (((int64_t)b * hkv + g) * a.max_parts) * kRec;
  // Buffer range over exactly the n_parts partitions: reads past them return zeros without a
  // memory access.
  const __amdgpu_buffer_rsrc_t parts_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(part_base, 0, n_parts * kRec * (int)sizeof(float), kBufferRsrcWord3);
  // Publish with write-through stores, wait for them, then count the arrival.  The last wave 0
  // of (b, g) to arrive merges all partitions.
  {
    float blk[2 * GQA], hdr[2 * GQA];
#pragma unroll
    for (int j = 0; j < GQA; ++j) {
      blk[2 * j] = acc[j][0];
      blk[2 * j + 1] = acc[j][1];
      hdr[2 * j] = mx[j];
      hdr[2 * j + 1] = ls[j];
    }
    store_block<GQA>(parts_rsrc, (p * kRec + kHdr + 2 * GQA * lane) * (int)sizeof(float), blk);
    if (lane == 0) store_block<GQA>(parts_rsrc, p * kRec * (int)sizeof(float), hdr);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // keep the stores above the wait
  __builtin_amdgcn_s_waitcnt(0);
  // The arrival count wraps: the n_parts-th arrival reads n_parts - 1 and leaves 0 behind, so the
  // workspace is ready for the next call without a reset store at the end of the merge.
  int *counter = a.counters + (int64_t)b * hkv + g;
  int prev = 0;
  if (lane == 0)
    prev = (int)__builtin_amdgcn_atomic_inc32(reinterpret_cast<unsigned *>(counter), (unsigned)(n_parts - 1),
                                              __ATOMIC_RELAXED, "agent");
  prev = __shfl(prev, 0);
  if (prev != n_parts - 1) return;

  // Merge.  Lane x holds partition x's (max, sum) of every head; the accumulators of the
  // first MP partitions are loaded in the same round (every load issued before the first
  // use, so the merge waits for one memory round trip), later ones 8 partitions per round.
  constexpr int MP = GQA <= 2 ? 16 : 8;
  float pm[GQA], pl[GQA], v0f[GQA][MP], v1f[GQA][MP];
  {
    float hx[2 * GQA];
    load_block<GQA>(parts_rsrc, lane * kRec * (int)sizeof(float), hx);
#pragma unroll
    for (int j = 0; j < GQA; ++j) {
      pm[j] = lane < n_parts ? hx[2 * j] : -INFINITY;
      pl[j] = hx[2 * j + 1];
    }
  }
#pragma unroll
  for (int k = 0; k < MP; ++k) {
    float vk[2 * GQA];
    load_block<GQA>(parts_rsrc, (k * kRec + kHdr + 2 * GQA * lane) * (int)sizeof(float), vk);
#pragma unroll
    for (int j = 0; j < GQA; ++j) {
      v0f[j][k] = vk[2 * j];
      v1f[j][k] = vk[2 * j + 1];
    }
  }
  float fx[GQA], den[GQA], n0[GQA], n1[GQA];
#pragma unroll
  for (int j = 0; j < GQA; ++j) {
    const float M = wave_max(pm[j]);
    fx[j] = pm[j] == -INFINITY ? 0.f : fast_exp2(pm[j] - M);
    den[j] = wave_sum(fx[j] * pl[j]);
    n0[j] = n1[j] = 0.f;
#pragma unroll
    for (int k = 0; k < MP; ++k) {  // partitions past n_parts load zeros and weigh 0
      const float f = readlane(fx[j], k);
      n0[j] += f * v0f[j][k];
      n1[j] += f * v1f[j][k];
    }
  }
  for (int x0 = MP; x0 < n_parts; x0 += 8) {
    float v0[GQA][8], v1[GQA][8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float vk[2 * GQA];
      load_block<GQA>(parts_rsrc, ((x0 + k) * kRec + kHdr + 2 * GQA * lane) * (int)sizeof(float), vk);
#pragma unroll
      for (int j = 0; j < GQA; ++j) {
        v0[j][k] = vk[2 * j];
        v1[j][k] = vk[2 * j + 1];
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (x0 + k < n_parts) {
#pragma unroll
        for (int j = 0; j < GQA; ++j) {
          const float f = readlane(fx[j], x0 + k);
          n0[j] += f * v0[j][k];
          n1[j] += f * v1[j][k];
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < GQA; ++j) {
    const float inv = den[j] > 0.f ? 1.f / den[j] : 0.f;
    *reinterpret_cast<u32 *>(out_base + j * D) = pack_bf16x2(n0[j] * inv, n1[j] * inv);
  }
}

template <int GQA, int NW, int CPW, int TILES = 4, bool WHOLE = false, bool FUSED = false>
int launch(DecodeArgs a, int batch, hipStream_t stream) {
  constexpr int PART = NW * CPW * 16 * TILES;
  a.max_parts = ceil_div(a.max_ctx, PART);
  if (a.max_parts > 64) return NVAMD_EUNSUPPORTED;  // merge stage holds <= 64 partitions
  if (WHOLE && a.max_parts != 1) return NVAMD_EINVAL;
  a.batch = batch;
  // One workgroup per possible (b, g, p); the ones past the last existing item exit at once.
  dim3 grid((unsigned)((int64_t)batch * a.num_kv_heads * a.max_parts));
  hipLaunchKernelGGL((paged_decode_kernel<GQA, NW, CPW, TILES, WHOLE, FUSED>), grid, dim3(NW * 64), 0, stream, a);
  return launch_status();
}

int num_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) ==
                                                 hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

template <int GQA, bool FUSED>
int dispatch(const DecodeArgs &a, int batch, hipStream_t stream) {
  // 256-token partitions of 4 waves (measured best on MI355X for 32 x ~1.3k contexts).  A launch
  // whose context bound gives fewer than two such items per CU is latency-bound: with a bound of
  // <= 512 tokens one workgroup of bound/64 waves takes a whole (sequence, kv head), so there is
  // no cross-workgroup merge.  Beyond that one CU would stream a whole unit, and a CU alone reads
  // at most ~41-57 GB/s: bounds of 513-1024 tokens split into 256-token partitions too (whole
  // units of 16 waves measured 1.2-1.7x slower for 1-16 sequences).  The 256-token partitions
  // stay at any batch: 128- or 64-token partitions of 2 or 1 waves (more workgroups, more partials
  // to merge) measured 1.1-1.7x slower for 1-8 sequences of 2-4k tokens and for one kv head.
  const int64_t units = (int64_t)batch * a.num_kv_heads;
  const int64_t want = 2LL * num_cus();
  if (units * ceil_div(a.max_ctx, 256) < want) {
    const int nw_whole = ceil_div(a.max_ctx, 64);
    if (nw_whole <= 2) return launch<GQA, 2, 1, 4, true, FUSED>(a, batch, stream);
    if (nw_whole <= 4) return launch<GQA, 4, 1, 4, true, FUSED>(a, batch, stream);
    if (nw_whole <= 8) return launch<GQA, 8, 1, 4, true, FUSED>(a, batch, stream);
  }
  int cpw = 1;
  while (ceil_div(a.max_ctx, 256 * cpw) > 64) cpw *= 2;
  switch (cpw) {
    case 1: return launch<GQA, 4, 1, 4, false, FUSED>(a, batch, stream);
    case 2: return launch<GQA, 4, 2, 4, false, FUSED>(a, batch, stream);
    case 4: return launch<GQA, 4, 4, 4, false, FUSED>(a, batch, stream);
    case 8: return launch<GQA, 4, 8, 4, false, FUSED>(a, batch, stream);
    default: return NVAMD_EUNSUPPORTED;
  }
}

}  // namespace
}  // namespace nvamd

using namespace nvamd;

extern "C" size_t nvamd_paged_decode_workspace_size(int max_batch, int num_heads, int num_kv_heads,
                                                    int max_context_len) {
  if (max_batch <= 0 || num_kv_heads <= 0 || num_heads <= 0 || max_context_len <= 0) return 0;
  const int gqa = num_heads / num_kv_heads;
  const size_t parts = (size_t)ceil_div(max_context_len, kMinPart);
  const size_t units = (size_t)max_batch * num_kv_heads;
  return kCounterBytes + units * parts * gqa * kPartFloats * sizeof(float);
}

namespace {

// Argument checks and DecodeArgs shared by the plain and the fused entry points.
int fill_decode_args(DecodeArgs &a, void *out, int64_t out_stride, const void *q, int64_t q_stride,
                     const void *k_cache, const void *v_cache, int num_blocks, int block_size,
                     const int32_t *block_tables, int bt_stride, int bt_width, const int32_t *context_lens, int batch,
                     int num_heads, int num_kv_heads, int head_dim, float scale, int max_context_len, void *workspace,
                     size_t workspace_bytes) {
  if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens) return NVAMD_EINVAL;
  if (batch < 0 || num_blocks <= 0 || num_kv_heads <= 0 || num_heads <= 0 || bt_width <= 0 ||
      bt_stride < bt_width || max_context_len <= 0)
    return NVAMD_EINVAL;
  if (head_dim != kHeadDim) return NVAMD_EUNSUPPORTED;
  if (num_heads % num_kv_heads != 0) return NVAMD_EINVAL;
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 4) return NVAMD_EUNSUPPORTED;
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache) || (q_stride % 8) != 0 ||
      (out_stride % 8) != 0 || q_stride < (int64_t)num_heads * head_dim || out_stride < (int64_t)num_heads * head_dim)
    return NVAMD_EINVAL;
  if ((int64_t)batch * num_kv_heads > kCounterSlots || batch > 65535) return NVAMD_EUNSUPPORTED;
  const size_t need = nvamd_paged_decode_workspace_size(batch, num_heads, num_kv_heads, max_context_len);
  if (!workspace || workspace_bytes < need) return NVAMD_EWORKSPACE;
  if (!aligned16(workspace)) return NVAMD_EINVAL;

  a = DecodeArgs{};
  a.out = static_cast<u16 *>(out);
  a.out_stride = out_stride;
  a.q = static_cast<const u16 *>(q);
  a.q_stride = q_stride;
  a.k_cache = static_cast<const u16 *>(k_cache);
  a.v_cache = static_cast<const u16 *>(v_cache);
  a.block_tables = block_tables;
  a.context_lens = context_lens;
  a.counters = static_cast<int *>(workspace);
  a.partials = reinterpret_cast<float *>(static_cast<char *>(workspace) + kCounterBytes);
  a.bt_stride = bt_stride;
  a.bt_width = bt_width;
  a.num_blocks = num_blocks;
  a.num_kv_heads = num_kv_heads;
  a.bs_log2 = bs_log2;
  a.max_ctx = max_context_len;
  a.max_parts = 0;
  a.scale_log2e = scale * kLog2e;
  a.err = index_error_word();
  return NVAMD_OK;
}

// The kernel holds 1, 2 or 4 query heads per kv head in registers.  Other ratios (Qwen3-14B's 5,
// Qwen3-32B's 8) run as consecutive launches over 4, then 2, then 1 heads of every group; each
// re-reads the group's K/V, and only the first stores the fused step's new k / v.
template <bool FUSED>
int dispatch_gqa(DecodeArgs a, int gqa, int batch, hipStream_t stream) {
  a.q_group = gqa;
  for (int head0 = 0; head0 < gqa;) {
    const int rest = gqa - head0;
    const int sub = rest >= 4 ? 4 : (rest >= 2 ? 2 : 1);
    a.q_head0 = head0;
    a.store_new = head0 == 0;
    const int st = sub == 4 ? dispatch<4, FUSED>(a, batch, stream)
                 : sub == 2 ? dispatch<2, FUSED>(a, batch, stream)
                            : dispatch<1, FUSED>(a, batch, stream);
    if (st != NVAMD_OK) return st;
    head0 += sub;
  }
  return NVAMD_OK;
}

}  // namespace

extern "C" int nvamd_paged_decode(void *out, int64_t out_stride, const void *q, int64_t q_stride,
                                  const void *k_cache, const void *v_cache, int num_blocks, int block_size,
                                  const int32_t *block_tables, int bt_stride, int bt_width,
                                  const int32_t *context_lens, int batch, int num_heads, int num_kv_heads,
                                  int head_dim, float scale, int max_context_len, void *workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  if (batch == 0) return NVAMD_OK;
  DecodeArgs a;
  const int st = fill_decode_args(a, out, out_stride, q, q_stride, k_cache, v_cache, num_blocks, block_size,
                                  block_tables, bt_stride, bt_width, context_lens, batch, num_heads, num_kv_heads,
                                  head_dim, scale, max_context_len, workspace, workspace_bytes);
  if (st != NVAMD_OK) return st;
  return dispatch_gqa<false>(a, num_heads / num_kv_heads, batch, stream);
}

extern "C" int nvamd_paged_decode_fused(void *out, int64_t out_stride, const void *q, int64_t q_stride,
                                        const void *k, int64_t k_stride, const void *v, int64_t v_stride,
                                        const void *q_weight, const void *k_weight, const int64_t *positions,
                                        const float *cos_sin, int max_positions, float eps, void *k_cache,
                                        void *v_cache, int num_blocks, int block_size, const int64_t *slot_mapping,
                                        const int32_t *block_tables, int bt_stride, int bt_width,
                                        const int32_t *context_lens, int batch, int num_heads, int num_kv_heads,
                                        int head_dim, float scale, int max_context_len, void *workspace,
                                        size_t workspace_bytes, hipStream_t stream) {
  if (batch == 0) return NVAMD_OK;
  DecodeArgs a;
  const int st = fill_decode_args(a, out, out_stride, q, q_stride, k_cache, v_cache, num_blocks, block_size,
                                  block_tables, bt_stride, bt_width, context_lens, batch, num_heads, num_kv_heads,
                                  head_dim, scale, max_context_len, workspace, workspace_bytes);
  if (st != NVAMD_OK) return st;
  if (!k || !v || !q_weight || !k_weight || !positions || !cos_sin || !slot_mapping || max_positions <= 0)
    return NVAMD_EINVAL;
  if (!aligned16(k) || !aligned16(v) || !aligned16(q_weight) || !aligned16(k_weight) || !aligned16(cos_sin) ||
      k_stride % 8 || v_stride % 8 || k_stride < (int64_t)num_kv_heads * head_dim ||
      v_stride < (int64_t)num_kv_heads * head_dim)
    return NVAMD_EINVAL;
  a.k_new = static_cast<const u16 *>(k);
  a.k_new_stride = k_stride;
  a.v_new = static_cast<const u16 *>(v);
  a.v_new_stride = v_stride;
  a.q_w = static_cast<const u16 *>(q_weight);
  a.k_w = static_cast<const u16 *>(k_weight);
  a.positions = positions;
  a.cos_sin = cos_sin;
  a.max_positions = max_positions;
  a.eps = eps;
  a.slots = slot_mapping;
  a.num_slots = (int64_t)num_blocks * block_size;
  return dispatch_gqa<true>(a, num_heads / num_kv_heads, batch, stream);
}

// -------------------------------------------------------------------------------------------
// Allocation-free decode (nvamd_paged_decode_noalloc): the workspace of nvamd_paged_decode
// comes from `scratch`, a file-scope device array of NVAMD_DECODE_SCRATCH_BYTES of which every
// GPU the library runs on holds its own copy until the process ends.  In host code the array's
// name is only a host-side stand-in, never an address: the first call on a device, with that
// device current, asks hipGetSymbolAddress for that device's copy, keeps the address per
// device, and clears the copy's arrival counters with a fill kernel on the caller's stream
// (ordered before the call's own launch); that first call is refused while the stream is being
// captured, since the clear would only be recorded.  Every call leaves the counters at zero again, as it
// does with a caller's workspace; partial results need no clearing.  Calls share the device's
// copy: calls that can overlap on one GPU (several streams, several host threads) race on it.
__device__ __align__(256) unsigned char scratch[NVAMD_DECODE_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch[kMaxDevices];  // each device's address of `scratch`, set on its first call

__global__ void __launch_bounds__(256) zero_words_kernel(u32 *p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// The current device's copy of `scratch`, set up (address looked up, counters cleared) on the
// device's first call.
int device_scratch(hipStream_t stream, void **ptr) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return (int)err;
  if (dev < 0 || dev >= kMaxDevices) return NVAMD_EUNSUPPORTED;
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch[dev] == nullptr) {
    // The counter clear below must run now, not be recorded into a graph that may never replay
    // before the next eager call.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    err = hipStreamIsCapturing(stream, &capture);
    if (err != hipSuccess) return (int)err;
    if (capture != hipStreamCaptureStatusNone) return NVAMD_ECAPTURE;
    void *p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return (int)err;
    if (p == nullptr) return (int)hipErrorInvalidSymbol;
    constexpr int words = (int)(kCounterBytes / sizeof(u32));
    hipLaunchKernelGGL(zero_words_kernel, dim3(words / 256), dim3(256), 0, stream, static_cast<u32 *>(p), words);
    const int st = launch_status();
    if (st != NVAMD_OK) return st;
    g_scratch[dev] = p;
  }
  *ptr = g_scratch[dev];
  return NVAMD_OK;
}

static_assert(kCounterBytes % (256 * sizeof(u32)) == 0, "counter clear uses whole 256-thread blocks");
static_assert(NVAMD_DECODE_SCRATCH_BYTES > kCounterBytes, "scratch must hold the counters and some partials");

}  // namespace

extern "C" int nvamd_paged_decode_noalloc(void *out, int64_t out_stride, const void *q, int64_t q_stride,
                                          const void *k_cache, const void *v_cache, int num_blocks, int block_size,
                                          const int32_t *block_tables, int bt_stride, int bt_width,
                                          const int32_t *context_lens, int batch, int num_heads, int num_kv_heads,
                                          int head_dim, float scale, int max_context_len, hipStream_t stream) {
  if (batch == 0) return NVAMD_OK;
  const size_t need = nvamd_paged_decode_workspace_size(batch, num_heads, num_kv_heads, max_context_len);
  if (need == 0) return NVAMD_EINVAL;
  if (need > (size_t)NVAMD_DECODE_SCRATCH_BYTES) return NVAMD_ETOOLARGE;
  void *ws = nullptr;
  const int st = device_scratch(stream, &ws);
  if (st != NVAMD_OK) return st;
  return nvamd_paged_decode(out, out_stride, q, q_stride, k_cache, v_cache, num_blocks, block_size, block_tables,
                            bt_stride, bt_width, context_lens, batch, num_heads, num_kv_heads, head_dim, scale,
                            max_context_len, ws, (size_t)NVAMD_DECODE_SCRATCH_BYTES, stream);
}
