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
// workgroups share a CU (three waves per SIMD at <= 168 VGPRs, 3 x 48 KB of
// LDS), so one wave's softmax and LDS traffic overlap another's MFMAs and the
// workgroups' per-tile barriers do not hold each other up.  32-key tiles keep
// both budgets: 64-key tiles allow two workgroups per CU and measured 1.07x slower.
// Per 32-key tile:
//   S^T[32 keys x 32 queries] = K . Q^T  with v_mfma_f32_32x32x16_bf16
//        (A = K rows from LDS, B = Q rows kept in registers for the whole loop).
//        In this layout a lane owns ONE query column, so the softmax max/sum
//        of a query is in-lane plus one exchange with lane^32.
//   O^T[128 dims x 32 queries] += V^T . P^T
//        The contraction index can be permuted as long as both operands agree:
//        taking the k-slots in the order the S^T accumulator already holds its
//        rows makes P^T a register-only repack (no lane movement); V^T comes from
//        the row-major V tile through two transposing LDS reads (ds_read_b64_tr_b16)
//        per operand, whose source rows pick the keys in that order.
// Softmax: the running max is kept on raw scores and applied in the exponent's
// FMA; its reference moves only when a score exceeds it by 2^8 (lazy rescale),
// and the row sum adds each packed bf16 pair with one v_dot2.
// Grid (kv head, query tile, sequence), dispatched in that order: with 8 kv heads the
// hardware's round-robin over the 8 XCDs puts every query tile of one (sequence, kv
// head) on one XCD, back to back, heaviest (most keys) first, so they read that head's
// K/V tiles while the XCD's L2 still holds them (a query-tile-major order streams every
// sequence's K/V from memory once per tile: 1.3x the time).  K/V tiles go from memory
// straight into LDS (LDS-DMA, no register staging), three stages deep: tile t+2 loads
// while tile t is computed, and each tile costs one barrier.  Against register staging
// with two stages this is 1.08x faster on the dense route and 1.2x on the paged route,
// whose block-table reads became two scalar loads per tile.
#include "common.h"

namespace nvamd {
namespace {

constexpr int kBK = 32;            // keys per tile
constexpr float kRescaleLog2 = 8.f;  // lazy-rescale threshold (log2 units)
// Largest K/V activation row stride (elements) of the dense route: a 32-row tile's byte range
// is a 32-bit buffer size.
constexpr int64_t kMaxActStride = (int64_t)1 << 24;
constexpr u32 kBf16PairOne = 0x3F803F80u;  // (1.0, 1.0) as a bf16 pair

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
  // Query heads of kv head g in q / out: q_group * g + q_head0 + (0 .. GQA-1).  One launch covers
  // a whole group (q_group == GQA, q_head0 == 0) unless the ratio needs several launches.
  int q_group;
  int q_head0;
  u32 *err;  // index-error word (paged route: contexts past the table row, block ids outside the pool)
};

// 16 bytes per lane into LDS at lds_base + 16 * lane (LDS-DMA), from a raw buffer (range
// checked: lanes past num_records write zeros) or from a global address.  Issued through asm so
// the compiler does not track the LDS write and adds no waits of its own: the kernel waits for
// these loads explicitly (vmcnt counts them) before the barrier that publishes a tile.  One
// wait state separates the M0 write from its use.  hipcc warns that a clobbered M0 may not be
// preserved: in this kernel's gfx950 code M0 is written only by these statements and read by
// nothing else, so no live value is lost.
__device__ __forceinline__ void dma16_buffer(u32x4 rsrc, u32 voffset, u32 lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_base), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16_global(const void *src, u32 lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_base), "v"(src)
               : "memory", "m0");
}
__device__ __forceinline__ u32 lds_addr(const u16 *p) {
  return (u32)(uintptr_t)(const __attribute__((address_space(3))) u16 *)p;
}

// max over lanes l and l ^ 32 of a score maximum (finite or -inf, never NaN: v_max_f32 without
// the canonicalising moves fmaxf adds to the permuted operands)
__device__ __forceinline__ float max_swap32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(__uint_as_float(r[0])), "v"(__uint_as_float(r[1])));
  return m;
}

__device__ __forceinline__ f32x16 mfma32(bf16x8v a, bf16x8v b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

constexpr int kWaves = 4;  // three workgroups per CU: their barriers are independent
constexpr int kThreads = kWaves * 64;
static_assert(kWaves == 4 && kBK == 32, "the tile DMA maps 4 waves x 8 rows onto a 32-key tile");

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
  if (PAGED) {
    const int cap = a.bt_width << a.bs_log2;
    // a context its table row cannot hold (or shorter than its queries): report once per sequence;
    // the table is read only up to its width
    if ((kv_len > cap || kv_len < q_len) && g == 0 && blockIdx.y == 0 && threadIdx.x == 0)
      flag_index_error(a.err, NVAMD_ERR_CONTEXT);
    kv_len = min(kv_len, cap);
  }
  const int offset = kv_len - q_len;  // query row r sees keys 0..offset+r

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5;        // lane half
  const int n = lane & 31;         // this lane's query column
  const int j = w / WPH;           // head within the group
  const int head = g * a.q_group + a.q_head0 + j;
  const int r0 = qt * BQ + (w % WPH) * 32;  // first query row of this wave
  const int rq = r0 + n;
  const bool q_ok = rq < q_len;
  const int64_t q_tok = q_start + min(rq, q_len - 1);

  // Three stages of K and V, row-major with swizzled 16-byte chunks.
  __shared__ __attribute__((aligned(16))) u16 sK[3][kBK * D];
  __shared__ __attribute__((aligned(16))) u16 sV[3][kBK * D];

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
  // Exponent reference per query column (log2 units of scaled scores), the threshold above
  // which it moves, and -reference.  The finite start needs no guard in the exponent: while a
  // lane has seen only masked (-inf) scores its arguments stay -inf, and its first finite score
  // moves the reference.  The first visible tile of a wave is tile 0.
  float m_ref = -1e30f, m_thr = -1e30f, neg_ref = 1e30f, l_run = 0.f;

  // Keys this workgroup needs: up to the last visible key of its last valid row.
  const int kv_hi = min(kv_len, offset + min((qt + 1) * BQ, q_len));
  const int n_tiles = ceil_div(kv_hi, kBK);
  const int wave_last_key = offset + min(r0 + 31, q_len - 1);  // beyond: fully masked for this wave

  // Tile staging: K and V tiles (32 rows x 256 B each) go from memory straight into LDS with
  // 16-byte LDS-DMA loads, three stages deep, two tiles ahead of the MFMAs.  A DMA instruction
  // of wave w fills 4 rows (1 KB): lane l lands at row 4i + l/16 of the wave's 8 rows, 16-byte
  // slot l%16, and so loads the chunk that slot holds under the row's swizzle.  K rows are
  // swizzled by row & 15 (the S operand reads 16 consecutive rows at one chunk), V rows by
  // 4(row & 3) (a transposing read takes 4 consecutive rows x 2 adjacent chunks per 16 lanes,
  // x 4 chunks per 32): both read patterns then touch distinct banks.  Rows past the sequence
  // read as zeros (dense route: the buffer range check) or repeat the last key's row (paged
  // route): finite either way.
  const int dma_row = 8 * w + (lane >> 4);  // + 4i for instruction i
  const int dma_slot = lane & 15;
  auto k_chunk = [&](int row) { return dma_slot ^ (row & 15); };
  auto v_chunk = [&](int row) { return dma_slot ^ (4 * (row & 3)); };
  const int32_t *bt_row = PAGED ? a.block_tables + (int64_t)s * a.bt_stride : nullptr;
  const int64_t cache_row = (int64_t)a.num_kv_heads * D;
  const int bs_mask = (1 << a.bs_log2) - 1;

  // Dense route: one raw buffer descriptor per tile over the tile's rows of this sequence
  // (built in scalar registers); each thread's byte offsets inside a tile are constants.
  u32 k_off[2], v_off[2];
  if (!PAGED) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = dma_row + 4 * i;
      k_off[i] = (u32)((row * a.k_stride + g * D + 8 * k_chunk(row)) * 2);
      v_off[i] = (u32)((row * a.v_stride + g * D + 8 * v_chunk(row)) * 2);
    }
  }
  // raw buffer descriptor over the tile's rows of this sequence: base, stride 0, byte count
  auto tile_rsrc = [&](const u16 *act, int64_t stride, int t) {
    const int base = t * kBK;
    const int rows = min(kv_len - base, kBK);
    const uint64_t addr = (uint64_t)(uintptr_t)(act + (int64_t)(q_start + base) * stride);
    return u32x4{(u32)addr, (u32)(addr >> 32) & 0xffffu, (u32)(rows * (int)stride * 2), (u32)kBufferRsrcWord3};
  };
  auto dma_tile = [&](int t, int st) {
    const u32 dk = lds_addr(&sK[st][8 * w * D]);
    const u32 dv = lds_addr(&sV[st][8 * w * D]);
    if (PAGED) {
      // A 32-key tile spans one block, or two of 16 keys (both entries are scalar loads); each
      // DMA instruction's 4 rows lie in one 16-row half, so its block, and a buffer descriptor
      // over that block, are wave-uniform.  Keys past kv_len repeat the last key's row.
      // The table does not change during the launch: read through the constant address space,
      // the loads stay scalar (the barrier's memory clobber would otherwise make them vector
      // loads, whose waits the compiler cannot separate from the DMA in flight).
      const int k0 = min(t * kBK, kv_len - 1), k1 = min(t * kBK + 16, kv_len - 1);
      typedef const __attribute__((address_space(4))) int32_t const_i32;
      const_i32 *btc = (const_i32 *)bt_row;
      const int e0 = btc[k0 >> a.bs_log2], e1 = btc[k1 >> a.bs_log2];
      if (((unsigned)e0 >= (unsigned)a.num_blocks || (unsigned)e1 >= (unsigned)a.num_blocks) && tid == 0)
        flag_index_error(a.err, NVAMD_ERR_BLOCK);  // never leave the pool; report the entry
      const int b0 = min(max(e0, 0), a.num_blocks - 1);
      const int b1 = min(max(e1, 0), a.num_blocks - 1);
      const u32 block_bytes = (u32)((cache_row << a.bs_log2) * 2);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int blk = 8 * w + 4 * i < 16 ? b0 : b1;
        const int64_t first = ((int64_t)blk << a.bs_log2) * cache_row;
        const uint64_t ka = (uint64_t)(uintptr_t)(a.k_cache + first), va = (uint64_t)(uintptr_t)(a.v_cache + first);
        const u32x4 rk = {(u32)ka, (u32)(ka >> 32) & 0xffffu, block_bytes, (u32)kBufferRsrcWord3};
        const u32x4 rv = {(u32)va, (u32)(va >> 32) & 0xffffu, block_bytes, (u32)kBufferRsrcWord3};
        const int row = dma_row + 4 * i;
        const int key = min(t * kBK + row, kv_len - 1);
        const u32 row_off = (u32)(((key & bs_mask) * cache_row + g * D) * 2);
        dma16_buffer(rk, row_off + 16 * k_chunk(row), dk + 4 * i * D * 2);
        dma16_buffer(rv, row_off + 16 * v_chunk(row), dv + 4 * i * D * 2);
      }
    } else {
      const u32x4 rk = tile_rsrc(a.k, a.k_stride, t);
      const u32x4 rv = tile_rsrc(a.v, a.v_stride, t);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        dma16_buffer(rk, k_off[i], dk + 4 * i * D * 2);
        dma16_buffer(rv, v_off[i], dv + 4 * i * D * 2);
      }
    }
  };
  // S^T = K Q^T: lane (n, hl) takes dims 16kk + 8hl .. +7 of key row n, chunk 2kk + hl.
  auto score = [&](const u16 *sk, f32x16 &sc) {
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const bf16x8v kf =
          *reinterpret_cast<const bf16x8v *>(sk + n * D + 8 * ((2 * kk + hl) ^ (n & 15)));
      sc = mfma32(kf, qf[kk], sc);
    }
  };
  // V^T operand of O^T += V^T P^T for dims 32db.. and the 16 keys of step hh, by two
  // transposing reads.  In 16-lane group G, output lane i gets dim 32db + 16(G&1) + i of the
  // 4 rows its source lanes j = q + 4e (e = 0..3) point at, so source lane j points at dims
  // +4q..+4q+3 of row 16hh + 4hl + e (first read) or + 8 (second read): the k-slots 8hl + 0..7
  // then hold keys {0-3, 8-11} + 4hl of the step, the order the S^T accumulator gives P^T.
  const int tr_q = lane & 3, tr_e = (lane >> 2) & 3;
  auto v_operand = [&](const u16 *sv, int db, int hh) {
    const int dim = 32 * db + 16 * ((lane >> 4) & 1) + 4 * tr_q;
    const int r1 = 16 * hh + 4 * hl + tr_e, r2 = r1 + 8;
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4 lds_s4;
    const u16 *p1 = sv + r1 * D + 8 * ((dim >> 3) ^ (4 * (r1 & 3))) + (dim & 4);
    const u16 *p2 = sv + r2 * D + 8 * ((dim >> 3) ^ (4 * (r2 & 3))) + (dim & 4);
    const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)p1);
    const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)p2);
    typedef short s8 __attribute__((ext_vector_type(8)));
    const s8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8v, both);
  };
  auto visible = [&](int t) { return r0 < q_len && t < n_tiles && t * kBK <= wave_last_key; };

  // Three stages: tile t+2 is in flight while tile t is computed.  The barrier ending tile t
  // waits only for tile t+1's DMA (vmcnt counts this wave's 4 DMA instructions per tile; no
  // other vector memory access is in flight in the loop) and for this wave's LDS reads.
  if (n_tiles > 0) dma_tile(0, 0);
  if (n_tiles > 1) dma_tile(1, 1);
  // Drain the Q fragments and the first two tiles: otherwise the wait the compiler places
  // ahead of the first use of Q is kept on every iteration.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  // tile t is computed from stage t % 3 while tile t + 2 loads into stage (t + 2) % 3, which
  // held tile t - 1: every wave finished reading it before the last barrier.
  // One tile: computed from stage sk/sv while tile t+2 loads into stage nst.  The loop below
  // unrolls three tiles so every stage's LDS base is a constant folded into the reads'
  // offsets (a computed stage base cost ~50 address instructions per tile).
  auto step = [&](const int t, const u16 *sk, const u16 *sv, const int nst) {
    if (t + 2 < n_tiles) dma_tile(t + 2, nst);
    const int base = t * kBK;
    if (visible(t)) {
      f32x16 sc;
      // Wave priority: the score MFMAs issue at priority 0 and the rest of the tile (mask,
      // softmax, P V) at 1, so a wave in its softmax is not held back by another wave's score
      // MFMAs on the same SIMD (the two do not overlap on gfx950).  1.4% faster on 32 x U[64,
      // 2048] than one priority throughout; raising the softmax alone measured 1.5% slower.
      __builtin_amdgcn_s_setprio(0);
      score(sk, sc);
      __builtin_amdgcn_s_setprio(1);
      // mask; key of register i: base + 8(i/4) + 4hl + i%4.  The running max is taken on raw
      // scores (scale > 0) and applied in the exponent's FMA.  Only tiles that cross this
      // wave's diagonal or the end of the keys need the mask (1-2 per wave); the test is
      // wave-uniform, so the others skip it with one branch.
      const bool need_mask = (base + kBK - 1 > offset + r0) || (base + kBK > kv_len);
      if (__builtin_expect(need_mask, 0)) {
        // lane's last visible key, relative to the key of register 0
        const int lim = min(offset + rq, kv_len - 1) - base - 4 * hl;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (8 * (i / 4) + (i % 4) > lim) sc[i] = -INFINITY;
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sc[i]);
      tmax = max_swap32(tmax) * a.scale_log2e;
      // Lazy rescale: the exponent's reference moves only when a score exceeds it by more
      // than 2^8, so P <= 256 and O, l are rescaled only on the tiles where some lane's
      // reference moved (a wave-uniform branch, taken on the first tile and rarely after).
      // O / l is unchanged by the choice of reference.  On the first tile O and l are still
      // zero and need no scaling.
      if (__builtin_amdgcn_ballot_w64(tmax > m_thr) != 0) {
        const bool up = tmax > m_thr;
        const float alpha = up ? __builtin_amdgcn_exp2f(m_ref - tmax) : 1.f;
        if (up) {
          m_ref = tmax;
          m_thr = tmax + kRescaleLog2;
          neg_ref = -tmax;
        }
        if (t > 0) {
          l_run *= alpha;
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[db][i] *= alpha;
        }
      }
      bf16x8v pf[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        u32x4 packed;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const u32 pr = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(sc[8 * hh + 2 * e], a.scale_log2e, neg_ref)),
                                     __builtin_amdgcn_exp2f(fmaf(sc[8 * hh + 2 * e + 1], a.scale_log2e, neg_ref)));
          l_run = dot2_bf16(pr, kBf16PairOne, l_run);  // both rounded values of the pair
          packed[e] = pr;
        }
        pf[hh] = __builtin_bit_cast(bf16x8v, packed);
      }

      // O^T += V^T P^T, two 16-key steps
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] = mfma32(v_operand(sv, db, hh), pf[hh], acc[db]);
    }
    if (t + 2 < n_tiles)
      asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  for (int t = 0; t < n_tiles; t += 3) {
    step(t, sK[0], sV[0], 2);
    if (t + 1 < n_tiles) step(t + 1, sK[1], sV[1], 0);
    if (t + 2 < n_tiles) step(t + 2, sK[2], sV[2], 1);
  }

  // normalise and write: register i of block db is dim 32db + 8(i/4) + 4hl + i%4 of query column n
  const float l_tot = sum_xor32(l_run);
  if (!q_ok) return;
  const float inv = l_tot > 0.f ? __builtin_amdgcn_rcpf(l_tot) : 0.f;  // v_rcp_f32 (1 ulp): output is bf16
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

// A workgroup holds 1, 2 or 4 query heads of its kv head.  Other ratios (Qwen3-14B's 5, Qwen3-32B's
// 8) run as consecutive launches over 4, then 2, then 1 heads of every group, each reading the
// group's K/V again (the launches are compute-bound; the second read mostly hits the caches).
template <bool PAGED>
int dispatch(PrefillArgs a, int n_seqs, int gqa, int max_q_len, hipStream_t stream) {
  a.q_group = gqa;
  for (int head0 = 0; head0 < gqa;) {
    const int rest = gqa - head0;
    const int sub = rest >= 4 ? 4 : (rest >= 2 ? 2 : 1);
    a.q_head0 = head0;
    a.max_q_tiles = ceil_div(max_q_len, 32 * kWaves / sub);
    const int st = sub == 4 ? launch<4, PAGED>(a, n_seqs, stream)
                 : sub == 2 ? launch<2, PAGED>(a, n_seqs, stream)
                            : launch<1, PAGED>(a, n_seqs, stream);
    if (st != NVAMD_OK) return st;
    head0 += sub;
  }
  return NVAMD_OK;
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
  a.err = index_error_word();
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
  // a 32-key tile spans at most two blocks, and one block's bytes of a layer fit a buffer range
  if (bs_log2 < 4 || (int64_t)num_kv_heads * head_dim * block_size * 2 > 0x7fffffff) return NVAMD_EUNSUPPORTED;
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
  a.err = index_error_word();
  return dispatch<true>(a, n_seqs, num_heads / num_kv_heads, max_q_len, stream);
}
