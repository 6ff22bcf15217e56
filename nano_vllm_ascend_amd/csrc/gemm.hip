// Skinny-M projections of the decode step (M <= 128 rows): Y[M, N] = X[M, K] . W[N, K]^T
// for the per-layer qkv / o / gate_up / down projections and the LM head
// (F.linear at nv/models/qwen3.py:26-35, 48-51, 119; nv/layers/embed_head.py:24-39),
// with the decoder's residual-add + RMSNorm folded into the GEMMs on either side of it
// (nv/models/qwen3.py:138-150; npu_rms_norm at nv/layers/layernorm.py:12-17).
//
// At M <= 32 a projection is a weight stream (2 B of W per 2*M FLOP), so the kernel is
// shaped to keep every W byte in flight at once, read it once, and keep the per-CU
// address path at full rate:
//   * v_mfma_f32_16x16x32_bf16 with A = 16 batch rows of X (one or two M tiles) and
//     B = 16 rows of W.  Lane (n, g) feeds row n with k = 8g..8g+7 of each 32-wide step.
//     W, and X and Y where the caller asks for it, are stored in that fragment order
//     ("tiled": 16 x 32 tiles of 512 elements, lane l's 8 elements at 8l), so one load
//     instruction reads 1 KB of contiguous memory.  Against row-major operands (16 rows x
//     64 bytes per instruction) this halves the vector L1 accesses that bound the
//     M = 32 projections (inside the decode step: qkv 7.0 -> 6.1 us, gate/up 8.3 -> 7.3 us).
//     Row-major X rows past M repeat row M-1;
//     a tiled X holds 16 * ceil(M/16) rows, and rows past M only reach dropped outputs;
//   * a workgroup of NW waves owns 16*NT output columns, one of KS slices of K
//     (split-K across workgroups where the column count alone gives too few
//     workgroups) and one slab of X: up to 32 rows, or above 32 rows 64-row slabs of four M
//     tiles (32-row slabs where a NORM prologue's k exceeds 1024 or it feeds a residual
//     epilogue), the slab index fastest in the grid, so the slabs reading one weight tile
//     run side by side and its repeat reads come from the Infinity Cache; its waves split
//     the slice again, and a wave's NT column tiles share each A fragment (64-row slabs of
//     the vocabulary-sized projection: 64 columns per workgroup instead of 128);
//   * the waves' partial tiles meet in LDS; with KS > 1 the workgroups publish fp32
//     partials with agent-scope write-through stores, count arrivals per column group,
//     and the last to arrive adds the KS partials in slice order.  Every sum has a
//     fixed order, so results are deterministic (graph replays equal eager calls).
//
// Prologue NORM: X is a residual stream and the A operand is RMSNorm(X) * norm_w, from
// per-32-column sums of squares of X written by the producer of X (the RESID epilogue or
// nvamd_embed_rows): rstd = rsqrt(sum / K + eps), a = bf16((x * rstd) * w) -- the rounding
// of the standalone add_rms_norm kernel.
// Epilogues: STORE y = bf16(acc); SILU y = bf16(bf16(silu(bf16(gate))) * bf16(up)) from
// gate rows n and up rows inter + n of the fused gate/up weight (nv/models/qwen3.py:34-35);
// RESID residual = bf16(residual + bf16(acc)) in place, plus the new per-32-column sums
// of squares for the next NORM prologue.
#include "common.h"

namespace nvamd {
namespace {

enum Epilogue { kEpiStore = 0, kEpiSilu = 1, kEpiResid = 2 };

constexpr int kCounterSlots = 4096;    // arrival counters at the front of the workspace
constexpr size_t kCounterBytes = kCounterSlots * sizeof(int);
constexpr int kMaxNormK = 2048;  // NORM prologue: k <= 2048
constexpr int kSsqVec = kMaxNormK / 128 / 4;  // 16-byte partial-sum loads per lane
// 64-row slabs (MT = 4 M tiles): the NORM prologue then takes k <= 1024, so a lane's partial sums
// fit two 16-byte loads per M tile.
constexpr int kMaxWideNormK = 1024;

struct GemmArgs {
  const u16 *x;
  int64_t x_stride;         // row-major X; a tiled X has none
  const float *x_ssq;       // NORM: [m][k / 32]
  const u16 *norm_w;        // NORM: [k]
  float eps;
  const u16 *w;             // tiled [n (SILU: 2n), k]
  u16 *y;                   // STORE / SILU output; RESID: the residual, updated in place
  int64_t y_stride;         // row-major Y
  bool x_tiled;
  bool y_tiled;
  float *y_ssq;             // RESID: [m][n / 32]
  int m;
  int n;                    // output columns (SILU: inter)
  int k;
  int ks;                   // K slices
  int k_slice;              // K per slice
  float *partials;
  int *counters;
};

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }



// Sum over the NW waves' partial tiles of element e (4 floats) of tile t, added in wave order;
// every LDS read is issued before the first add (the compiler otherwise waits after each read).
template <int NW, int NACC, int TF>
__device__ __forceinline__ f32x4 sum_waves(const float (&s_c)[NW][NACC][TF], int t, int e) {
  f32x4 r[NW];
#pragma unroll
  for (int x = 0; x < NW; ++x) r[x] = *reinterpret_cast<const f32x4 *>(&s_c[x][t][e]);
  __builtin_amdgcn_sched_barrier(0);
  f32x4 s = r[0];
#pragma unroll
  for (int x = 1; x < NW; ++x) s += r[x];
  return s;
}

// One 32-wide K step of a wave: W tiles wv[t], X M-tiles xv[mt] (already normalised).
template <int NACC, int MT>
__device__ __forceinline__ void mfma_step(f32x4 (&acc)[NACC][MT], const u32x4 (&xa)[MT], const u32x4 *wv) {
#pragma unroll
  for (int t = 0; t < NACC; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, xa[mt]),
                                                          __builtin_bit_cast(bf16x8v, wv[t]), acc[t][mt], 0, 0, 0);
}

template <int NW, int KB, int NT, int MT, int EPI, bool NORM, bool SLABS>
__global__ void __launch_bounds__(NW * 64)
skinny_gemm_kernel(GemmArgs a) {
  constexpr int kNW = NW;
  constexpr int NACC = (EPI == kEpiSilu ? 2 : 1) * NT;  // 16-column tiles (SILU: NT gate, then NT up)
  constexpr int CW = 16 * NT;                           // output columns of the workgroup
  constexpr int WK = 32 * KB;                           // K per wave per round
  constexpr int RK = kNW * WK;                          // K per workgroup per round
  constexpr int SR = MT <= 2 ? 32 : 16 * MT;            // rows of the workgroup's slab
  constexpr int TF = SR * 16;                           // floats of one slab-row x 16-column tile
  constexpr int kSsqV = MT <= 2 ? kSsqVec : kMaxWideNormK / 128 / 4;
  static_assert(MT == 1 || MT == 2 || MT == 4, "32-row slabs of one or two M tiles, or 64-row slabs");
  static_assert(EPI != kEpiResid || CW % 32 == 0,
                "the residual epilogue's sums of squares need whole 32-column groups in one workgroup");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  // Grid: (column group, K slice[, slab of SR rows]), slab fastest (SLABS: M > SR).  A slab's rows
  // become rows 0..SR-1 of this workgroup: operand, norm-partial and output pointers move to its
  // first row, and its split-K partials and counters follow those of the earlier slabs.
  const int slabs = SLABS ? (a.m + SR - 1) / SR : 1;
  const int slab = SLABS ? blockIdx.x % slabs : 0;
  const int gs = SLABS ? blockIdx.x / slabs : blockIdx.x;
  const int group = gs / a.ks;
  const int slice = gs - group * a.ks;
  const int n0 = group * CW;
  if (SLABS && slab > 0) {
    const int64_t r0 = SR * (int64_t)slab;
    a.x += a.x_tiled ? MT * slab * (int64_t)(a.k >> 5) * 512 : r0 * a.x_stride;
    if (NORM) a.x_ssq += r0 * (a.k >> 5);
    a.y += a.y_tiled ? MT * slab * (int64_t)(a.n >> 5) * 512 : r0 * a.y_stride;
    if (EPI == kEpiResid) a.y_ssq += r0 * (a.n >> 5);
    const int groups = gridDim.x / (slabs * a.ks);
    a.counters += slab * groups;
    a.partials += (int64_t)slab * groups * a.ks * NACC * TF;
    a.m -= SR * slab;
  }
  if (SLABS) a.m = min(a.m, SR);

  // Operand addresses: base + k0 * step for the 32-wide K step starting at k0 (tiled: the
  // step's 512-element tile follows the previous one, so 16 elements per unit of k).
  int xr[MT];
  const u16 *xp[MT];
  const int xs = a.x_tiled ? 16 : 1;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    xr[mt] = min(16 * mt + n, a.m - 1);
    // a tiled X holds 16 * ceil(M/16) rows: an M tile past the slab's last row re-reads its last
    // tile (those rows only reach dropped outputs)
    const int mt_x = SLABS || MT > 2 ? min(mt, (a.m - 1) >> 4) : mt;
    xp[mt] = a.x_tiled ? a.x + (int64_t)mt_x * (a.k >> 5) * 512 + 8 * lane : a.x + (int64_t)xr[mt] * a.x_stride + 8 * g;
  }
  const u16 *wp[NACC];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    wp[t] = a.w + (int64_t)(group * NT + t) * (a.k >> 5) * 512 + 8 * lane;
    if (EPI == kEpiSilu) wp[NT + t] = wp[t] + (int64_t)(a.n >> 4) * (a.k >> 5) * 512;
  }
  const u16 *np = NORM ? a.norm_w + 8 * g : nullptr;

  // NORM: the four lanes of a row (g = 0..3) each read a quarter of its k/32 partial sums
  // of squares (k <= 2048: at most four 16-byte loads).  They are issued before the weight
  // loads, so rstd is ready while the weights are in flight.
  float rstd[MT];
  f32x4 sv[MT][kSsqV];
  const int ssq_q = a.k >> 7;  // partials per lane
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    rstd[mt] = 1.f;
    if (NORM) {
      const float *sp = a.x_ssq + (int64_t)xr[mt] * (a.k >> 5) + g * ssq_q;
#pragma unroll
      for (int i = 0; i < kSsqV; ++i)
        sv[mt][i] = 4 * i < ssq_q ? *reinterpret_cast<const f32x4 *>(sp + 4 * i) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // RESID: the residual values this thread adds in the epilogue (work units u = tid + j * threads),
  // read now so that their load overlaps the weight stream instead of following the merge.  Only
  // this column group's merging workgroup writes them, after every read of this launch.
  constexpr int kRowUnits = CW / 4;
  constexpr int kUnits = SR * kRowUnits;                      // epilogue units of the workgroup
  constexpr int kUPT = (kUnits + kNW * 64 - 1) / (kNW * 64);  // units per thread: u = tid + j * threads
  u32x2 resid[kUPT] = {};
  if constexpr (EPI == kEpiResid) {
#pragma unroll
    for (int j = 0; j < kUPT; ++j) {
      const int u = tid + j * kNW * 64;
      if (u < kUnits) {
        const int rr = min(u / kRowUnits, a.m - 1);
        const int c = n0 + 4 * (u % kRowUnits);
        resid[j] = *reinterpret_cast<const u32x2 *>(a.y + (a.y_tiled ? tiled_index(rr, c, a.n) : (int64_t)rr * a.y_stride + c));
      }
    }
  }

  f32x4 acc[NACC][MT];
#pragma unroll
  for (int t = 0; t < NACC; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int k_begin = slice * a.k_slice;
  const int k_end = k_begin + a.k_slice;
  const int k_first = k_begin + w * WK;
  // One K round: issue every load of the round before the first MFMA waits on one; in the first
  // round (NORM) finish rstd from the sums of squares, whose loads were issued before the round's.
  // The first round is written out ahead of the loop: inside the loop the compiler hoisted the
  // sums above the first round's loads, so the weight stream waited for the sums' round trip.
  auto k_round = [&](const int k0, const bool first) {
    u32x4 wv[KB][NACC], xv[KB][MT], nv[NORM ? KB : 1];
#pragma unroll
    for (int b = 0; b < KB; ++b) {
#pragma unroll
      for (int t = 0; t < NACC; ++t) wv[b][t] = ld16(wp[t] + (int64_t)(k0 + 32 * b) * 16);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xv[b][mt] = ld16(xp[mt] + (int64_t)(k0 + 32 * b) * xs);
      if (NORM) nv[b] = ld16(np + k0 + 32 * b);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (NORM && first) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kSsqV; ++i) ss += (sv[mt][i][0] + sv[mt][i][1]) + (sv[mt][i][2] + sv[mt][i][3]);
        ss += swizzle_xor16(ss);
        ss = sum_xor32(ss);
        rstd[mt] = rsqrtf(ss / (float)a.k + a.eps);
      }
    }
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      u32x4 xa[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xa[mt] = xv[b][mt];
        if (NORM) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            xa[mt][e] = pack_bf16x2(bf16_lo(xa[mt][e]) * rstd[mt] * bf16_lo(nv[b][e]),
                                    bf16_hi(xa[mt][e]) * rstd[mt] * bf16_hi(nv[b][e]));
        }
      }
      mfma_step<NACC, MT>(acc, xa, wv[b]);
    }
  };
  if (k_first < k_end) {
    k_round(k_first, true);
#pragma unroll 1
    for (int k0 = k_first + RK; k0 < k_end; k0 += RK) k_round(k0, false);
  }

  // C register i of lane (n, g) in M tile mt is row 16*mt + 4*g + i, column n of the tile.
  __shared__ float s_c[kNW][NACC][TF];
  __shared__ int s_last;
#pragma unroll
  for (int t = 0; t < NACC; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_c[w][t][(16 * mt + 4 * g + i) * 16 + n] = acc[t][mt][i];
  __syncthreads();

  float *part = a.partials + ((int64_t)group * a.ks) * NACC * TF;
  if (a.ks > 1) {
    // this slice's partial tiles, written through to memory with 16-byte agent-coherent stores
    const __amdgpu_buffer_rsrc_t prsrc = __builtin_amdgcn_make_buffer_rsrc(
        part, 0, a.ks * NACC * TF * (int)sizeof(float), kBufferRsrcWord3);
    for (int u = tid; u < NACC * TF / 4; u += kNW * 64) {
      const int t = u / (TF / 4);
      const int e = 4 * (u % (TF / 4));
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum_waves<kNW, NACC, TF>(s_c, t, e)), prsrc,
                                             ((slice * NACC + t) * TF + e) * (int)sizeof(float), 0, kCachePolicyAgent);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // keep the stores above the wait
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const int prev = __hip_atomic_fetch_add(a.counters + group, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == a.ks - 1;
    }
    __syncthreads();
    if (!s_last) return;
  }

  // Work unit u: 4 consecutive columns of one output row; the 8 units of 32 columns of a
  // row sit in 8 consecutive lanes.  j counts this thread's units.
  int j = 0;
  for (int u = tid; u < kUnits; u += kNW * 64, ++j) {
    const int row = u / kRowUnits;
    const int cl = 4 * (u % kRowUnits);  // column inside the workgroup's CW
    const int t = cl >> 4;
    const int e = row * 16 + (cl & 15);
    constexpr int NV = EPI == kEpiSilu ? 2 : 1;
    f32x4 v[NV];
#pragma unroll
    for (int h = 0; h < NV; ++h) {
      const int tt = t + h * NT;
      if (a.ks > 1) {
        // The ks published slices through one agent-coherent buffer range: eight slices' loads in
        // flight per step, and loads past the last slice return zeros without a memory access.
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            part, 0, a.ks * NACC * TF * (int)sizeof(float), kBufferRsrcWord3);
        v[h] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < a.ks; s0 += 8) {
          f32x4 ld[8];
#pragma unroll
          for (int q = 0; q < 8; ++q)
            ld[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rsrc, (((s0 + q) * NACC + tt) * TF + e) * (int)sizeof(float), 0,
                                                  kCachePolicyAgent));
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (s0 + q < a.ks) v[h] += ld[q];
        }
      } else {
        v[h] = sum_waves<kNW, NACC, TF>(s_c, tt, e);
      }
    }
    const int c = n0 + cl;
    u16 *yp = a.y + (a.y_tiled ? tiled_index(row, c, a.n) : (int64_t)row * a.y_stride + c);
    if (EPI == kEpiStore) {
      if (row < a.m)
        *reinterpret_cast<u32x2 *>(yp) = u32x2{pack_bf16x2(v[0][0], v[0][1]), pack_bf16x2(v[0][2], v[0][3])};
    } else if (EPI == kEpiSilu) {
      float o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = round_bf16(silu_f32(round_bf16(v[0][q]))) * round_bf16(v[NV - 1][q]);
      if (row < a.m) *reinterpret_cast<u32x2 *>(yp) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    } else {  // RESID
      u32x2 r = resid[0];
#pragma unroll
      for (int q = 1; q < kUPT; ++q)
        if (j == q) r = resid[q];
      const u32 h0 = pack_bf16x2(bf16_lo(r[0]) + round_bf16(v[0][0]), bf16_hi(r[0]) + round_bf16(v[0][1]));
      const u32 h1 = pack_bf16x2(bf16_lo(r[1]) + round_bf16(v[0][2]), bf16_hi(r[1]) + round_bf16(v[0][3]));
      float ss = bf16_lo(h0) * bf16_lo(h0) + bf16_hi(h0) * bf16_hi(h0) + bf16_lo(h1) * bf16_lo(h1) +
                 bf16_hi(h1) * bf16_hi(h1);
      ss = sum8(ss);  // the 8 units of these 32 columns
      if (row < a.m) {
        *reinterpret_cast<u32x2 *>(yp) = u32x2{h0, h1};
        if ((c & 31) == 0) a.y_ssq[(int64_t)row * (a.n >> 5) + (c >> 5)] = ss;
      }
    }
  }
  if (a.ks > 1 && tid == 0)  // leave the workspace ready for the next call
    __hip_atomic_store(a.counters + group, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Plan {
  int nw, nt, ks, kb;
};

// Measured on MI355X at M = 32: the decode step's projection sequence over 28 layers' own
// weights (882 MB, streamed from HBM as in the model), replayed as one graph:
//   * vocabulary-sized N (LM head): 128 columns per 4-wave workgroup, no split;
//   * residual epilogue (N = hidden: o_proj, down_proj): 32 columns (the epilogue's sums of
//     squares cover whole 32-column groups) per 8-wave workgroup, K split over >= 128
//     workgroups (o 6.5 us, down 6.6 us; 4-wave workgroups over >= 256: 6.7 / 7.4 us;
//     unsplit 16-wave workgroups: 8.2 us, faster only while the weights sit in the
//     Infinity Cache);
//   * otherwise (qkv, gate_up): 16 columns per 8-wave workgroup, no split.
// 64-row slabs (wide): the vocabulary-sized projection takes 64 columns per workgroup (128
// would need 128 accumulator registers at 4 M tiles); with two slabs (M > 64) the other
// projections take 32 columns per workgroup, halving the X reads per weight byte (a projection
// chain at M = 100: 35.2-35.8 against 41.4-42.1 us per layer; at M = 64, one slab, the halved
// workgroup count makes it slower).
Plan make_plan(int n, int k, int epi, int m, bool wide) {
  Plan p{8, 1, 1, k % 512 == 0 ? 2 : 1};
  if (epi == kEpiStore && n % 128 == 0 && n / 128 >= 512) {
    p = wide ? Plan{4, 4, 1, 2} : Plan{4, 8, 1, 2};
  } else if (wide && m > 64 && epi != kEpiResid) {
    p.nt = 2;
  } else if (epi == kEpiResid) {
    p = Plan{8, 2, 1, 2};
    const int groups = n / 32;
    static const int kSlices[] = {1, 2, 3, 4, 6, 8, 12, 16};
    for (int ks : kSlices) {
      if (k % ks != 0 || (k / ks) % 64 != 0) continue;  // whole 64-wide wave blocks per slice
      p.ks = ks;
      if (groups * ks >= 128) break;
    }
  }
  return p;
}

constexpr int kMaxSlabs = 4;  // M <= 128

size_t workspace_bytes_for(const Plan &p, int n, int epi) {
  if (p.ks <= 1) return 0;
  const int nacc = (epi == kEpiSilu ? 2 : 1) * p.nt;
  const size_t groups = (size_t)n / (16 * p.nt);
  // partial tiles for 128 rows: four 32-row slabs or two 64-row ones
  return kCounterBytes + kMaxSlabs * groups * p.ks * nacc * 32 * 16 * sizeof(float);
}

// Above 32 rows, 64-row slabs (wide) where the NORM prologue allows them (and not for a normed
// residual projection, whose registers would spill); 32-row slabs otherwise.
bool wide_rows(int m, int k, bool norm, int epi) {
  return m > 32 && (!norm || (k <= kMaxWideNormK && epi != kEpiResid));
}
// Configurations 64-row slabs are built for (at most 64 columns per workgroup).
template <int NT, int EPI, bool NORM>
constexpr bool kWideBuilt = NT <= 4 && !(NORM && EPI == kEpiResid);

template <int NW, int KB, int NT, int EPI, bool NORM>
int launch(const GemmArgs &a, int grid, bool wide, hipStream_t stream) {
  if (wide) {
    if constexpr (kWideBuilt<NT, EPI, NORM>) {
      if (a.m <= 64)
        hipLaunchKernelGGL((skinny_gemm_kernel<NW, KB, NT, 4, EPI, NORM, false>), dim3(grid), dim3(NW * 64), 0,
                           stream, a);
      else
        hipLaunchKernelGGL((skinny_gemm_kernel<NW, KB, NT, 4, EPI, NORM, true>), dim3(grid), dim3(NW * 64), 0,
                           stream, a);
    } else {
      return NVAMD_EUNSUPPORTED;
    }
  } else if (a.m > 32)
    hipLaunchKernelGGL((skinny_gemm_kernel<NW, KB, NT, 2, EPI, NORM, true>), dim3(grid), dim3(NW * 64), 0, stream,
                       a);
  else if (a.m > 16)
    hipLaunchKernelGGL((skinny_gemm_kernel<NW, KB, NT, 2, EPI, NORM, false>), dim3(grid), dim3(NW * 64), 0, stream,
                       a);
  else
    hipLaunchKernelGGL((skinny_gemm_kernel<NW, KB, NT, 1, EPI, NORM, false>), dim3(grid), dim3(NW * 64), 0, stream,
                       a);
  return launch_status();
}

template <int NW, int NT, int EPI, bool NORM>
int launch_kb(const GemmArgs &a, const Plan &p, int grid, bool wide, hipStream_t stream) {
  return p.kb == 2 ? launch<NW, 2, NT, EPI, NORM>(a, grid, wide, stream)
                   : launch<NW, 1, NT, EPI, NORM>(a, grid, wide, stream);
}

template <int EPI, bool NORM>
int dispatch(const GemmArgs &a, const Plan &p, int grid, bool wide, hipStream_t stream) {
  if constexpr (EPI == kEpiStore) {
    if (p.nw == 4 && p.nt == 8) return launch_kb<4, 8, EPI, NORM>(a, p, grid, wide, stream);
    if (p.nw == 4 && p.nt == 4) return launch_kb<4, 4, EPI, NORM>(a, p, grid, wide, stream);
  }
  if constexpr (EPI == kEpiResid) {
    if (p.nw == 8 && p.nt == 2) return launch_kb<8, 2, EPI, NORM>(a, p, grid, wide, stream);
  } else {
    if (p.nw == 8 && p.nt == 1) return launch_kb<8, 1, EPI, NORM>(a, p, grid, wide, stream);
    if (p.nw == 8 && p.nt == 2) return launch_kb<8, 2, EPI, NORM>(a, p, grid, wide, stream);
  }
  return NVAMD_EUNSUPPORTED;
}

}  // namespace
}  // namespace nvamd

using namespace nvamd;

extern "C" size_t nvamd_skinny_linear_workspace_size(int n, int k, int epilogue) {
  if (n <= 0 || k <= 0 || n % 32 || k % 256 || epilogue < 0 || epilogue > 2) return 0;
  // the larger of the two plans' needs (the row count is not known here)
  const size_t slabs = workspace_bytes_for(make_plan(n, k, epilogue, 32, false), n, epilogue);
  const size_t wide = workspace_bytes_for(make_plan(n, k, epilogue, 128, true), n, epilogue);
  return slabs > wide ? slabs : wide;
}

extern "C" int nvamd_skinny_linear(const void *x, int64_t x_stride, const float *x_ssq, const void *norm_weight,
                                   float eps, const void *w_tiled, void *y, int64_t y_stride, float *y_ssq,
                                   int epilogue, int flags, int m, int n, int k, void *workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  if (m == 0) return NVAMD_OK;
  if (!x || !w_tiled || !y || m < 0 || n <= 0 || k <= 0 || epilogue < 0 || epilogue > 2 ||
      (flags & ~(NVAMD_GEMM_X_TILED | NVAMD_GEMM_Y_TILED)))
    return NVAMD_EINVAL;
  if (m > 32 * kMaxSlabs || n % 32 != 0 || k % 256 != 0) return NVAMD_EUNSUPPORTED;
  const bool x_tiled = flags & NVAMD_GEMM_X_TILED, y_tiled = flags & NVAMD_GEMM_Y_TILED;
  const bool norm = x_ssq != nullptr;
  if (norm && !norm_weight) return NVAMD_EINVAL;
  if (norm && k > kMaxNormK) return NVAMD_EUNSUPPORTED;
  if (epilogue == kEpiResid && !y_ssq) return NVAMD_EINVAL;
  if (!aligned16(x) || !aligned16(w_tiled) || (reinterpret_cast<uintptr_t>(y) & 7u) ||
      (!x_tiled && (x_stride % 8 || x_stride < k)) || (!y_tiled && (y_stride < n || y_stride % 4)) ||
      (norm && (!aligned16(x_ssq) || !aligned16(norm_weight))))
    return NVAMD_EINVAL;
  const bool wide = wide_rows(m, k, norm, epilogue);
  const Plan p = make_plan(n, k, epilogue, m, wide);
  const int groups = n / (16 * p.nt);
  if ((k / p.ks) % (32 * p.kb) != 0) return NVAMD_EUNSUPPORTED;  // whole wave blocks per slice
  const int slabs = wide ? (m + 63) / 64 : (m + 31) / 32;
  if (p.ks > 1) {
    if (groups * slabs > kCounterSlots) return NVAMD_EUNSUPPORTED;
    if (!workspace || !aligned16(workspace) || workspace_bytes < workspace_bytes_for(p, n, epilogue))
      return NVAMD_EWORKSPACE;
  }
  GemmArgs a;
  a.x = static_cast<const u16 *>(x);
  a.x_stride = x_stride;
  a.x_ssq = x_ssq;
  a.norm_w = static_cast<const u16 *>(norm_weight);
  a.eps = eps;
  a.w = static_cast<const u16 *>(w_tiled);
  a.y = static_cast<u16 *>(y);
  a.y_stride = y_stride;
  a.x_tiled = x_tiled;
  a.y_tiled = y_tiled;
  a.y_ssq = y_ssq;
  a.m = m;
  a.n = n;
  a.k = k;
  a.ks = p.ks;
  a.k_slice = k / p.ks;
  a.counters = static_cast<int *>(workspace);
  a.partials = workspace ? reinterpret_cast<float *>(static_cast<char *>(workspace) + kCounterBytes) : nullptr;
  const int grid = groups * p.ks * slabs;
  switch (epilogue) {
    case kEpiSilu:
      return norm ? dispatch<kEpiSilu, true>(a, p, grid, wide, stream) : dispatch<kEpiSilu, false>(a, p, grid, wide, stream);
    case kEpiResid:
      return norm ? dispatch<kEpiResid, true>(a, p, grid, wide, stream) : dispatch<kEpiResid, false>(a, p, grid, wide, stream);
    default:
      return norm ? dispatch<kEpiStore, true>(a, p, grid, wide, stream) : dispatch<kEpiStore, false>(a, p, grid, wide, stream);
  }
}
