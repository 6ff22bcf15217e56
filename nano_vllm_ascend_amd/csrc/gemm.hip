// Skinny-M projections for decode batches (M <= 32 rows): Y[M, N] = X[M, K] . W[N, K]^T,
// the per-layer qkv / o / gate_up / down projections and the LM head of the decode step
// (nv/models/qwen3.py:26-35, 48-51, 119; nv/layers/embed_head.py:24-39).  At M <= 32 the
// product is a weight stream (2 B of W per 2*M FLOP), so the kernel is built to read W
// once at HBM rate:
//   * one workgroup owns 32 output columns (32 rows of W); its NW waves split K, so a
//     launch keeps N/32 * NW waves and every W byte in flight from the start;
//   * v_mfma_f32_32x32x16_bf16 with A = the batch rows of X (rows past M repeat row
//     M-1 and are dropped) and B = 32 rows of W.  Lane (col, kh) feeds A row col and B
//     column col with the same 8 k's, so it reads 64 contiguous bytes of one W row per
//     64-wide K block and a row's 128-byte lines come whole;
//   * the waves' partial 32x32 tiles are added in LDS in a fixed order (deterministic),
//     then rounded to bf16 once, as a bf16 GEMM with fp32 accumulation does.
// The SILU variant computes the gate columns n and up columns inter + n of the fused
// gate/up weight in one workgroup and writes silu(gate) * up (nv/models/qwen3.py:34-35):
// gate and up are rounded to bf16, silu(gate) is rounded to bf16, the product is rounded
// again -- the rounding points of the unfused projection + silu_mul.
#include "common.h"

namespace nvamd {
namespace {

struct GemmArgs {
  const u16 *x;
  int64_t x_stride;
  const u16 *w;
  int64_t w_stride;
  u16 *y;
  int64_t y_stride;
  int m;
  int k;
  int up_offset;  // W rows between a gate row and its up row (SILU only)
};

__device__ __forceinline__ f32x16 mfma32(bf16x8v a, bf16x8v b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

template <int NW, int KB, bool SILU>
__global__ void __launch_bounds__(NW * 64)
skinny_gemm_kernel(GemmArgs a) {
  constexpr int WK = 64 * KB;     // K per wave per round
  constexpr int RK = NW * WK;     // K per workgroup per round
  constexpr int NACC = SILU ? 2 : 1;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31;
  const int kh = lane >> 5;
  const int n0 = blockIdx.x * 32;

  const u16 *xp = a.x + (int64_t)min(col, a.m - 1) * a.x_stride + 32 * kh;
  const u16 *wp[NACC];
  wp[0] = a.w + (int64_t)(n0 + col) * a.w_stride + 32 * kh;
  if (SILU) wp[NACC - 1] = wp[0] + (int64_t)a.up_offset * a.w_stride;

  f32x16 acc[NACC];
#pragma unroll
  for (int t = 0; t < NACC; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.f;

#pragma unroll 1
  for (int k0 = w * WK; k0 < a.k; k0 += RK) {
    u32x4 wv[NACC][KB][4], xv[KB][4];
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int t = 0; t < NACC; ++t) wv[t][b][j] = ld16(wp[t] + k0 + 64 * b + 8 * j);
        xv[b][j] = ld16(xp + k0 + 64 * b + 8 * j);
      }
    // every load of the round is issued before the first MFMA waits on one
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < NACC; ++t)
          acc[t] = mfma32(__builtin_bit_cast(bf16x8v, xv[b][j]), __builtin_bit_cast(bf16x8v, wv[t][b][j]), acc[t]);
  }

  // C register i of lane l is row 8*(i/4) + 4*(l/32) + i%4, column l%32 of the tile.
  __shared__ float s_c[NW][NACC][32 * 32];
#pragma unroll
  for (int t = 0; t < NACC; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) s_c[w][t][(8 * (i >> 2) + 4 * kh + (i & 3)) * 32 + col] = acc[t][i];
  __syncthreads();

  for (int e = tid; e < 32 * 32; e += NW * 64) {
    const int row = e >> 5;
    if (row >= a.m) break;  // e grows with row: nothing further to store
    float s[NACC];
#pragma unroll
    for (int t = 0; t < NACC; ++t) {
      s[t] = 0.f;
#pragma unroll
      for (int x = 0; x < NW; ++x) s[t] += s_c[x][t][e];
    }
    float v;
    if (SILU) {
      const float gate = round_bf16(s[0]);
      const float up = round_bf16(s[NACC - 1]);
      v = round_bf16(silu_f32(gate)) * up;
    } else {
      v = s[0];
    }
    a.y[(int64_t)row * a.y_stride + n0 + (e & 31)] = f32_to_bf16(v);
  }
}

// Waves per workgroup: enough that the launch holds >= 1024 waves, 4..16 (8 for SILU,
// whose two tiles double the LDS), and dividing K into 64-wide blocks.
int pick_waves(int tiles, int k, bool silu) {
  int nw = 4;
  while (nw < 16 && (int64_t)tiles * nw < 1024) nw *= 2;
  if (silu && nw > 8) nw = 8;
  while (nw > 4 && k % (nw * 64) != 0) nw /= 2;
  return k % (nw * 64) == 0 ? nw : 0;
}

template <int NW, bool SILU>
int launch_kb(const GemmArgs &a, int tiles, hipStream_t stream) {
  const int per = a.k / (NW * 64);
  const dim3 grid(tiles), block(NW * 64);
  if (per % 2 == 0)
    hipLaunchKernelGGL((skinny_gemm_kernel<NW, 2, SILU>), grid, block, 0, stream, a);
  else if (per % 3 == 0)
    hipLaunchKernelGGL((skinny_gemm_kernel<NW, 3, SILU>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((skinny_gemm_kernel<NW, 1, SILU>), grid, block, 0, stream, a);
  return launch_status();
}

int run(const GemmArgs &a, int tiles, bool silu, hipStream_t stream) {
  const int nw = pick_waves(tiles, a.k, silu);
  if (silu) {
    switch (nw) {
      case 4: return launch_kb<4, true>(a, tiles, stream);
      case 8: return launch_kb<8, true>(a, tiles, stream);
      default: return NVAMD_EUNSUPPORTED;
    }
  }
  switch (nw) {
    case 4: return launch_kb<4, false>(a, tiles, stream);
    case 8: return launch_kb<8, false>(a, tiles, stream);
    case 16: return launch_kb<16, false>(a, tiles, stream);
    default: return NVAMD_EUNSUPPORTED;
  }
}

int check_common(const void *x, int64_t x_stride, const void *w, int64_t w_stride, const void *y, int64_t y_stride,
                 int m, int n, int k) {
  if (!x || !w || !y || m < 0 || n <= 0 || k <= 0) return NVAMD_EINVAL;
  if (m > 32 || n % 32 != 0 || k % 256 != 0) return NVAMD_EUNSUPPORTED;
  if (!aligned16(x) || !aligned16(w) || x_stride % 8 || w_stride % 8 || x_stride < k || w_stride < k ||
      y_stride < n || (reinterpret_cast<uintptr_t>(y) & 1u))
    return NVAMD_EINVAL;
  return NVAMD_OK;
}

}  // namespace
}  // namespace nvamd

using namespace nvamd;

extern "C" int nvamd_linear(const void *x, int64_t x_stride, const void *w, int64_t w_stride, void *y,
                            int64_t y_stride, int m, int n, int k, hipStream_t stream) {
  if (m == 0) return NVAMD_OK;
  const int st = check_common(x, x_stride, w, w_stride, y, y_stride, m, n, k);
  if (st != NVAMD_OK) return st;
  GemmArgs a{static_cast<const u16 *>(x), x_stride, static_cast<const u16 *>(w), w_stride, static_cast<u16 *>(y),
             y_stride, m, k, 0};
  return run(a, n / 32, false, stream);
}

extern "C" int nvamd_linear_silu_mul(const void *x, int64_t x_stride, const void *w_gate_up, int64_t w_stride,
                                     void *y, int64_t y_stride, int m, int inter, int k, hipStream_t stream) {
  if (m == 0) return NVAMD_OK;
  const int st = check_common(x, x_stride, w_gate_up, w_stride, y, y_stride, m, inter, k);
  if (st != NVAMD_OK) return st;
  GemmArgs a{static_cast<const u16 *>(x), x_stride, static_cast<const u16 *>(w_gate_up), w_stride,
             static_cast<u16 *>(y), y_stride, m, k, inter};
  return run(a, inter / 32, true, stream);
}
