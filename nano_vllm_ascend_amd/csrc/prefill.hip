// Causal varlen prefill attention on bf16 MFMA for gfx950 (replaces
// torch_npu.npu_fused_infer_attention_score, nv/layers/npu_prefill_attention.py:41-113).
//
// Two routes share one kernel:
//   dense  K/V are the packed activations of the same tokens (q_len == kv_len),
//          row i of a sequence sees keys 0..i           (sparse_mode=3 route);
//   paged  K/V are read through the block table from the paged cache, the
//          queries are the last q_len positions of kv_len, and query row r
//          sees keys 0..kv_len-q_len+r (bottom-right causal; prefix-hit route).
//
// Workgroup = 4 waves = one kv head g, its GQA query heads, and a tile of
// BQ = 128/GQA query tokens; wave w owns 32 query rows of one head.  Three
// workgroups share a CU (three waves per SIMD at <= 168 VGPRs, 3 x 37 KB of
// LDS), so one wave's softmax and LDS traffic overlap another's MFMAs and the
// workgroups' per-tile barriers do not hold each other up.  32-key tiles keep
// both budgets: 64-key tiles (70 KB, 200 VGPRs) allow two workgroups per CU and
// measure 1.07x slower.
// Per 32-key tile:
//   S^T[32 keys x 32 queries] = K . Q^T  with v_mfma_f32_32x32x16_bf16
//        (A = K rows from LDS, B = Q rows kept in registers for the whole loop).
//        In this layout a lane owns ONE query column, so the softmax max/sum
//        of a query is in-lane plus one exchange with lane^32.
//   O^T[128 dims x 32 queries] += V^T . P^T
//        The contraction index can be permuted as long as both operands agree:
//        taking the k-slots in the order the S^T accumulator already holds its
//        rows makes P^T a register-only repack (no lane movement); V^T is read
//        from a transposed LDS copy whose keys are stored in that order, one
//        16-byte read per operand.
// Softmax: the running max is kept on raw scores and applied in the exponent's
// FMA; its reference moves only when a score exceeds it by 2^8 (lazy rescale),
// and the row sum adds each packed bf16 pair with one v_dot2.
// Grid (kv head, query tile, sequence), dispatched in that order: with 8 kv heads the
// hardware's round-robin over the 8 XCDs puts every query tile of one (sequence, kv
// head) on one XCD, back to back, heaviest (most keys) first, so they read that head's
// K/V tiles while the XCD's L2 still holds them (a query-tile-major order streams every
// sequence's K/V from memory once per tile: 1.3x the time).  K/V tiles are
// double-buffered in LDS: the next tile is loaded into registers while the current
// one's MFMAs run, then stored into the other slot, so each tile costs one barrier.
#include "common.h"

namespace nvamd {
namespace {

constexpr int kBK = 32;            // keys per tile
constexpr int kBlocks = kBK / 32;  // 32-key MFMA blocks per tile
constexpr int kKStride = 136;      // LDS row stride (elements) of the K tile: 272 B, spreads banks
constexpr int kVtStride = kBK + 8;  // LDS row stride (elements) of the transposed V tile: 16-byte aligned
constexpr float kRescaleLog2 = 8.f;  // lazy-rescale threshold (log2 units)
// Largest K/V activation row stride (elements) of the dense route: a 64-row tile's byte range
// is a 32-bit buffer size.
constexpr int64_t kMaxActStride = (int64_t)1 << 24;
constexpr u32 kBf16PairOne = 0x3F803F80u;  // (1.0, 1.0) as a bf16 pair

// Position of key k of a key tile inside a V^T row.  Within each 16-key group the PV
// step of lane half h consumes keys {0-3, 8-11} (h = 0) or {4-7, 12-15} (h = 1); swapping
// bits 2 and 3 of the key makes each of those sets 8 contiguous elements.
__device__ __forceinline__ int vt_pos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

struct PrefillArgs {
  u16 *out;
  int64_t out_stride;
  const u16 *q;
  int64_t q_stride;
  const u16 *k;
  int64_t k_stride;
  const u16 *v;
  int64_t v_stride;
  const u16 *k_cache;
  const u16 *v_cache;
  const int32_t *block_tables;
  const int32_t *cu_seqlens_q;
  const int32_t *kv_lens;
  int bt_stride;
  int bt_width;
  int num_blocks;
  int bs_log2;
  int num_kv_heads;
  int max_q_tiles;
  float scale_log2e;
};

__device__ __forceinline__ f32x16 mfma32(bf16x8v a, bf16x8v b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

constexpr int kWaves = 4;  // three workgroups per CU: their barriers are independent
constexpr int kThreads = kWaves * 64;
constexpr int kKLoads = kBK * 16 / kThreads;      // 16-byte K chunks per thread per tile
constexpr int kVLoads = kBK / 2 * 16 / kThreads;  // (key pair, 8-dim chunk) units per thread
static_assert(kKLoads >= 1 && kVLoads >= 1, "tile staging needs <= 512 threads");

template <int GQA, bool PAGED>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
prefill_kernel(PrefillArgs a) {
  constexpr int D = kHeadDim;
  constexpr int BQ = 32 * kWaves / GQA;  // query tokens per workgroup
  constexpr int WPH = kWaves / GQA;      // waves per query head

  const int g = blockIdx.x;
  const int qt = a.max_q_tiles - 1 - (int)blockIdx.y;
  const int s = blockIdx.z;
  const int q_start = a.cu_seqlens_q[s];
  const int q_len = a.cu_seqlens_q[s + 1] - q_start;
  if (qt * BQ >= q_len) return;
  int kv_len = PAGED ? a.kv_lens[s] : q_len;
  if (PAGED) kv_len = min(kv_len, a.bt_width << a.bs_log2);
  const int offset = kv_len - q_len;  // query row r sees keys 0..offset+r

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5;        // lane half
  const int n = lane & 31;         // this lane's query column
  const int j = w / WPH;           // head within the group
  const int head = g * GQA + j;
  const int r0 = qt * BQ + (w % WPH) * 32;  // first query row of this wave
  const int rq = r0 + n;
  const bool q_ok = rq < q_len;
  const int64_t q_tok = q_start + min(rq, q_len - 1);

  __shared__ __attribute__((aligned(16))) u16 sK[2][kBK][kKStride];
  __shared__ __attribute__((aligned(16))) u16 sVt[2][D][kVtStride];

  // Q^T operand: lane holds dims 16kk + 8*hl + 0..7 of its query row, kk = 0..7.
  bf16x8v qf[8];
  {
    const u16 *qp = a.q + q_tok * a.q_stride + (int64_t)head * D + 8 * hl;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = __builtin_bit_cast(bf16x8v, ld16(qp + 16 * kk));
  }

  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // Keys this workgroup needs: up to the last visible key of its last valid row.
  const int kv_hi = min(kv_len, offset + min((qt + 1) * BQ, q_len));
  const int n_tiles = ceil_div(kv_hi, kBK);
  const int wave_last_key = offset + min(r0 + 31, q_len - 1);  // beyond: fully masked for this wave

  // cooperative tile loads: K rows (t>>4) + (threads/16)i, 16-byte chunk t&15; V row pair t&31,
  // 8 dims 8 * ((t>>5) + (threads/32)e)
  const int kr = tid >> 4, kc = tid & 15;
  const int vp = tid % (kBK / 2), vc = tid / (kBK / 2);
  const int32_t *bt_row = PAGED ? a.block_tables + (int64_t)s * a.bt_stride : nullptr;
  const int64_t cache_row = (int64_t)a.num_kv_heads * D;
  const int bs_mask = (1 << a.bs_log2) - 1;

  // Paged route: each row through the block table.  Keys past kv_len re-read the last key's
  // row (a finite value): their scores are masked to -inf, so they enter P as exact zeros.
  auto row_ptr = [&](const u16 *cache, int key) -> const u16 * {
    key = min(key, kv_len - 1);
    int blk = bt_row[key >> a.bs_log2];
    blk = min(max(blk, 0), a.num_blocks - 1);
    return cache + (((int64_t)blk << a.bs_log2) + (key & bs_mask)) * cache_row + (int64_t)g * D;
  };
  // Dense route: one raw buffer descriptor per tile over the tile's rows of this sequence
  // (built in scalar registers); every thread's byte offsets inside a tile are constants and
  // rows past kv_len read as zeros, so a load costs no vector address arithmetic.
  u32 k_off[kKLoads], v_off[kVLoads][2];
  if (!PAGED) {
#pragma unroll
    for (int i = 0; i < kKLoads; ++i)
      k_off[i] = (u32)(((kr + kThreads / 16 * i) * a.k_stride + g * D + 8 * kc) * 2);
#pragma unroll
    for (int i = 0; i < kVLoads; ++i)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        v_off[i][e] = (u32)(((2 * vp + e) * a.v_stride + g * D + 8 * (vc + kThreads / (kBK / 2) * i)) * 2);
  }
  auto tile_rsrc = [&](const u16 *act, int64_t stride, int t) {
    const int base = t * kBK;
    const int rows = min(kv_len - base, kBK);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<u16 *>(act + (int64_t)(q_start + base) * stride), 0,
                                             rows * (int)stride * 2, kBufferRsrcWord3);
  };

  u32x4 kreg[kKLoads], vreg[kVLoads][2];
  auto load_k = [&](int t) {
    if (PAGED) {
#pragma unroll
      for (int i = 0; i < kKLoads; ++i) kreg[i] = ld16(row_ptr(a.k_cache, t * kBK + kr + kThreads / 16 * i) + 8 * kc);
    } else {
      const __amdgpu_buffer_rsrc_t r = tile_rsrc(a.k, a.k_stride, t);
#pragma unroll
      for (int i = 0; i < kKLoads; ++i)
        kreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, k_off[i], 0, 0));
    }
  };
  auto load_v = [&](int t) {
    if (PAGED) {
#pragma unroll
      for (int i = 0; i < kVLoads; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e)
          vreg[i][e] = ld16(row_ptr(a.v_cache, t * kBK + 2 * vp + e) + 8 * (vc + kThreads / (kBK / 2) * i));
    } else {
      const __amdgpu_buffer_rsrc_t r = tile_rsrc(a.v, a.v_stride, t);
#pragma unroll
      for (int i = 0; i < kVLoads; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e)
          vreg[i][e] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, v_off[i][e], 0, 0));
    }
  };
  auto store_k = [&](int slot) {
#pragma unroll
    for (int i = 0; i < kKLoads; ++i) *reinterpret_cast<u32x4 *>(&sK[slot][kr + kThreads / 16 * i][8 * kc]) = kreg[i];
  };
  auto store_v = [&](int slot) {
    // transpose V: (V[2vp][d], V[2vp+1][d]) -> one dword of row d of V^T, at the permuted
    // position of key 2vp (keys 2vp and 2vp+1 stay adjacent)
    const int vpos = vt_pos(2 * vp);
#pragma unroll
    for (int i = 0; i < kVLoads; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = 8 * (vc + kThreads / (kBK / 2) * i) + 2 * e;
        *reinterpret_cast<u32 *>(&sVt[slot][d][vpos]) = pair_lo(vreg[i][0][e], vreg[i][1][e]);
        *reinterpret_cast<u32 *>(&sVt[slot][d + 1][vpos]) = pair_hi(vreg[i][0][e], vreg[i][1][e]);
      }
  };
  // S^T = K Q^T for the keys of a K slot (kBlocks 32-key blocks)
  auto score = [&](int slot, f32x16 (&st)[kBlocks]) {
#pragma unroll
    for (int blk = 0; blk < kBlocks; ++blk) {
#pragma unroll
      for (int i = 0; i < 16; ++i) st[blk][i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const bf16x8v kf = *reinterpret_cast<const bf16x8v *>(&sK[slot][32 * blk + n][16 * kk + 8 * hl]);
        st[blk] = mfma32(kf, qf[kk], st[blk]);
      }
    }
  };
  auto visible = [&](int t) { return r0 < q_len && t < n_tiles && t * kBK <= wave_last_key; };

  // Double-buffered tiles: the next tile's K/V are loaded into registers while this tile's
  // MFMAs run, then stored into the other LDS slot; one barrier per tile.
  if (n_tiles > 0) {
    load_k(0);
    load_v(0);
    store_k(0);
    store_v(0);
  }
  // Drain every load issued so far (the Q fragments) before the loop.  Otherwise the wait
  // the compiler places ahead of the first use of Q is kept on every iteration, and each
  // tile's MFMAs would wait for the next tile's K/V loads issued just before them.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    if (t + 1 < n_tiles) {
      load_k(t + 1);
      load_v(t + 1);
    }
    const int base = t * kBK;
    if (visible(t)) {
      f32x16 st[kBlocks];
      score(t & 1, st);
      // mask; key of register i of block blk: base + 32blk + 8(i/4) + 4hl + i%4.  The running
      // max is taken on raw scores (scale > 0) and applied in the exponent's FMA.
      // Only tiles that cross this wave's diagonal or the end of the keys need the mask
      // (1-2 per wave); the test is wave-uniform, so the others skip it with one branch.
      const bool need_mask = (base + kBK - 1 > offset + r0) || (base + kBK > kv_len);
      if (__builtin_expect(need_mask, 0)) {
        // lane's last visible key, relative to the key of register 0 of block 0
        const int lim = min(offset + rq, kv_len - 1) - base - 4 * hl;
#pragma unroll
        for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (32 * blk + 8 * (i / 4) + (i % 4) > lim) st[blk][i] = -INFINITY;
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
        for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, st[blk][i]);
      tmax = max_xor32(tmax) * a.scale_log2e;
      // Lazy rescale: the exponent's reference moves only when a score exceeds it by more
      // than 2^8, so P <= 256 and O, l are rescaled only on the tiles where some lane's
      // reference moved.  O / l is unchanged by the choice of reference.
      float alpha = 1.f;
      if (tmax > m_run + kRescaleLog2) {
        alpha = __builtin_amdgcn_exp2f(m_run - tmax);  // 0 on the first visible tile
        m_run = tmax;
      }
      const float neg_ref = m_run == -INFINITY ? 0.f : -m_run;
      float psum = 0.f;
      bf16x8v pf[kBlocks][2];
#pragma unroll
      for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          u32x4 packed;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const u32 pr =
                pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(st[blk][8 * hh + 2 * e], a.scale_log2e, neg_ref)),
                            __builtin_amdgcn_exp2f(fmaf(st[blk][8 * hh + 2 * e + 1], a.scale_log2e, neg_ref)));
            psum = dot2_bf16(pr, kBf16PairOne, psum);  // both rounded values of the pair
            packed[e] = pr;
          }
          pf[blk][hh] = __builtin_bit_cast(bf16x8v, packed);
        }
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {  // wave-uniform
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[db][i] *= alpha;
      }
      l_run += psum;

      // O^T += V^T P^T; k-slot 8hl+e of step (blk, hh) is key 32blk + 16hh + 8(e/4) + 4hl + e%4,
      // which the permuted V^T layout stores contiguously: one 16-byte read per operand.
#pragma unroll
      for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int k0 = 32 * blk + 16 * hh + 8 * hl;
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const u32x4 vv = *reinterpret_cast<const u32x4 *>(&sVt[t & 1][32 * db + n][k0]);
            acc[db] = mfma32(__builtin_bit_cast(bf16x8v, vv), pf[blk][hh], acc[db]);
          }
        }
    }
    if (t + 1 < n_tiles) {  // nobody reads that slot: every wave finished tile t-1 before the last barrier
      store_k((t + 1) & 1);
      store_v((t + 1) & 1);
    }
    __syncthreads();
  }

  // normalise and write: register i of block db is dim 32db + 8(i/4) + 4hl + i%4 of query column n
  const float l_tot = sum_xor32(l_run);
  if (!q_ok) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  u16 *op = a.out + q_tok * a.out_stride + (int64_t)head * D + 4 * hl;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      u32x2 pk;
      pk[0] = pack_bf16x2(acc[db][4 * i4] * inv, acc[db][4 * i4 + 1] * inv);
      pk[1] = pack_bf16x2(acc[db][4 * i4 + 2] * inv, acc[db][4 * i4 + 3] * inv);
      *reinterpret_cast<u32x2 *>(op + 32 * db + 8 * i4) = pk;
    }
}

template <int GQA, bool PAGED>
int launch(const PrefillArgs &a, int n_seqs, hipStream_t stream) {
  dim3 grid(a.num_kv_heads, a.max_q_tiles, n_seqs);
  hipLaunchKernelGGL((prefill_kernel<GQA, PAGED>), grid, dim3(kThreads), 0, stream, a);
  return launch_status();
}

template <bool PAGED>
int dispatch(PrefillArgs a, int n_seqs, int gqa, int max_q_len, hipStream_t stream) {
  switch (gqa) {
    case 1: a.max_q_tiles = ceil_div(max_q_len, 32 * kWaves); return launch<1, PAGED>(a, n_seqs, stream);
    case 2: a.max_q_tiles = ceil_div(max_q_len, 16 * kWaves); return launch<2, PAGED>(a, n_seqs, stream);
    case 4: a.max_q_tiles = ceil_div(max_q_len, 8 * kWaves); return launch<4, PAGED>(a, n_seqs, stream);
    default: return NVAMD_EUNSUPPORTED;
  }
}

bool check_common(const void *out, int64_t out_stride, const void *q, int64_t q_stride, int num_heads,
                  int num_kv_heads) {
  return out && q && aligned16(out) && aligned16(q) && out_stride % 8 == 0 && q_stride % 8 == 0 &&
         out_stride >= (int64_t)num_heads * kHeadDim && q_stride >= (int64_t)num_heads * kHeadDim &&
         num_kv_heads > 0 && num_heads % num_kv_heads == 0;
}

}  // namespace
}  // namespace nvamd

using namespace nvamd;

extern "C" int nvamd_varlen_prefill(void *out, int64_t out_stride, const void *q, int64_t q_stride, const void *k,
                                    int64_t k_stride, const void *v, int64_t v_stride, const int32_t *cu_seqlens_q,
                                    int n_seqs, int max_q_len, int num_heads, int num_kv_heads, int head_dim,
                                    float scale, hipStream_t stream) {
  if (n_seqs == 0 || max_q_len == 0) return NVAMD_OK;
  if (head_dim != kHeadDim) return NVAMD_EUNSUPPORTED;
  if (!(scale > 0.f)) return NVAMD_EINVAL;  // the softmax keeps its running max on raw scores
  if (!check_common(out, out_stride, q, q_stride, num_heads, num_kv_heads) || !k || !v || !cu_seqlens_q ||
      n_seqs < 0 || max_q_len < 0 || !aligned16(k) || !aligned16(v) || k_stride % 8 || v_stride % 8 ||
      k_stride < (int64_t)num_kv_heads * head_dim || v_stride < (int64_t)num_kv_heads * head_dim || n_seqs > 65535 ||
      k_stride > kMaxActStride || v_stride > kMaxActStride)
    return NVAMD_EINVAL;
  PrefillArgs a = {};
  a.out = static_cast<u16 *>(out);
  a.out_stride = out_stride;
  a.q = static_cast<const u16 *>(q);
  a.q_stride = q_stride;
  a.k = static_cast<const u16 *>(k);
  a.k_stride = k_stride;
  a.v = static_cast<const u16 *>(v);
  a.v_stride = v_stride;
  a.cu_seqlens_q = cu_seqlens_q;
  a.num_kv_heads = num_kv_heads;
  a.scale_log2e = scale * kLog2e;
  return dispatch<false>(a, n_seqs, num_heads / num_kv_heads, max_q_len, stream);
}

extern "C" int nvamd_paged_prefill(void *out, int64_t out_stride, const void *q, int64_t q_stride,
                                   const void *k_cache, const void *v_cache, int num_blocks, int block_size,
                                   const int32_t *block_tables, int bt_stride, int bt_width,
                                   const int32_t *cu_seqlens_q, const int32_t *kv_lens, int n_seqs, int max_q_len,
                                   int num_heads, int num_kv_heads, int head_dim, float scale, hipStream_t stream) {
  if (n_seqs == 0 || max_q_len == 0) return NVAMD_OK;
  if (head_dim != kHeadDim) return NVAMD_EUNSUPPORTED;
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return NVAMD_EUNSUPPORTED;
  if (!(scale > 0.f)) return NVAMD_EINVAL;  // the softmax keeps its running max on raw scores
  if (!check_common(out, out_stride, q, q_stride, num_heads, num_kv_heads) || !k_cache || !v_cache ||
      !block_tables || !cu_seqlens_q || !kv_lens || n_seqs < 0 || max_q_len < 0 || num_blocks <= 0 ||
      bt_width <= 0 || bt_stride < bt_width || !aligned16(k_cache) || !aligned16(v_cache) || n_seqs > 65535)
    return NVAMD_EINVAL;
  PrefillArgs a = {};
  a.out = static_cast<u16 *>(out);
  a.out_stride = out_stride;
  a.q = static_cast<const u16 *>(q);
  a.q_stride = q_stride;
  a.k_cache = static_cast<const u16 *>(k_cache);
  a.v_cache = static_cast<const u16 *>(v_cache);
  a.block_tables = block_tables;
  a.bt_stride = bt_stride;
  a.bt_width = bt_width;
  a.num_blocks = num_blocks;
  a.bs_log2 = bs_log2;
  a.cu_seqlens_q = cu_seqlens_q;
  a.kv_lens = kv_lens;
  a.num_kv_heads = num_kv_heads;
  a.scale_log2e = scale * kLog2e;
  return dispatch<true>(a, n_seqs, num_heads / num_kv_heads, max_q_len, stream);
}
