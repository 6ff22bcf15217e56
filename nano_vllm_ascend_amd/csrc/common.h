// Device helpers shared by the gfx950 kernels of the attention path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nvamd.h"

namespace nvamd {

using u32 = uint32_t;
using u16 = uint16_t;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));

constexpr int kHeadDim = 128;
constexpr float kLog2e = 1.4426950408889634f;

// Raw buffer resource word 3 for gfx9 (32-bit data, no format conversion).  A raw buffer
// load whose byte offset is at or past num_records returns zeros without a memory access.
constexpr int kBufferRsrcWord3 = 0x00020000;
// Cache policy of an agent-coherent buffer load (sc1), as agent-scope atomic loads use.
constexpr int kCachePolicyAgent = 16;

// bf16 <-> fp32.  A bf16 is the top half of an fp32, so widening is a shift.
__device__ __forceinline__ float bf16_lo(u32 x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf16_hi(u32 x) { return __uint_as_float(x & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(u16 x) { return __uint_as_float(((u32)x) << 16); }

// Round two fp32 to bf16 (round-to-nearest-even, one v_cvt_pk_bf16_f32) and pack.
__device__ __forceinline__ u32 pack_bf16x2(float lo, float hi) {
  bf16x2v r;
  r[0] = (__bf16)lo;
  r[1] = (__bf16)hi;
  return __builtin_bit_cast(u32, r);
}
__device__ __forceinline__ u16 f32_to_bf16(float x) {
  __bf16 r = (__bf16)x;
  return __builtin_bit_cast(u16, r);
}
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Per-head RMSNorm + rotate-half RoPE, element steps shared by every kernel that applies them,
// so each rounds identically: fp32 arithmetic, the normalised value rounded to bf16 before the
// rotation (nv/layers/layernorm.py:12-17, nv/layers/rotary_embedding.py:20-42).
// Sum of squares of the dims (d, d+1, 64+d, 65+d); the 32 such partials of a head are summed
// as a balanced tree in order of d.
__device__ __forceinline__ float head_ssq4(float x0, float x1, float x2, float x3) {
  return x0 * x0 + x1 * x1 + x2 * x2 + x3 * x3;
}
__device__ __forceinline__ float head_rstd(float ss, float eps) { return rsqrtf(ss * (1.0f / kHeadDim) + eps); }
__device__ __forceinline__ float head_norm(float x, float rstd, float w) { return round_bf16(x * rstd * w); }
// out[d] = y[d] cos[d] - y[d+64] sin[d];  out[d+64] = y[d+64] cos[d] + y[d] sin[d]  (d < 64)
__device__ __forceinline__ float rope_lo(float y_lo, float y_hi, float c, float s) { return y_lo * c - y_hi * s; }
__device__ __forceinline__ float rope_hi(float y_lo, float y_hi, float c, float s) { return y_hi * c + y_lo * s; }

// acc + a.lo*b.lo + a.hi*b.hi with bf16 pairs and fp32 accumulation.
__device__ __forceinline__ float dot2_bf16(u32 a, u32 b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, a),
                                         __builtin_bit_cast(bf16x2v, b), acc, false);
}

// Byte permutes: low halves of (a, b) -> (a.lo, b.lo); high halves -> (a.hi, b.hi).
__device__ __forceinline__ u32 pair_lo(u32 a, u32 b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ u32 pair_hi(u32 a, u32 b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// Cross-lane moves.  DPP control words (gfx9 encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;   // row_half_mirror (reverse within 8 lanes)
constexpr int kDppMirror = 0x140;       // row_mirror (reverse within 16 lanes)
constexpr int kDppRowRor8 = 0x128;      // row_ror:8 (lane i <- lane (i+8)%16 in a row)

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// ds_swizzle in bit mode: xor the lane id with 16 inside each 32-lane half.
// v[l] combined with v[l ^ 32] in every lane, in registers: v_permlane32_swap of a register
// with itself leaves lane l's two results holding v[l mod 32] and v[32 + l mod 32] (checked
// on gfx950), so no LDS round trip is needed.
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float swizzle_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 8 consecutive lanes of an aligned group; every lane of the group gets the sum.
__device__ __forceinline__ float sum8(float v) {
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  return v;
}
// Per-head RMSNorm + RoPE of one head vector held by an aligned group of 8 lanes: lane c of the
// group holds dims 8c..8c+7 (lo) and 64+8c..64+8c+7 (hi).  cs/sn are the bf16-rounded cos/sin
// of dims 8c..8c+7.  A lane forms the partial sums of squares of the dim quads (d, d+1, 64+d,
// 65+d) it holds, pairs them, and the 8-lane reduction finishes a balanced tree over the 32 quads
// in order of d, so every kernel that uses it rounds identically.
__device__ __forceinline__ void head_norm_rope(u32x4 &lo, u32x4 &hi, const u32x4 w_lo, const u32x4 w_hi,
                                               const float (&cs)[8], const float (&sn)[8], float eps) {
  float p[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) p[e] = head_ssq4(bf16_lo(lo[e]), bf16_hi(lo[e]), bf16_lo(hi[e]), bf16_hi(hi[e]));
  const float rstd = head_rstd(sum8((p[0] + p[1]) + (p[2] + p[3])), eps);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float y0 = head_norm(bf16_lo(lo[e]), rstd, bf16_lo(w_lo[e]));
    const float y1 = head_norm(bf16_hi(lo[e]), rstd, bf16_hi(w_lo[e]));
    const float y2 = head_norm(bf16_lo(hi[e]), rstd, bf16_lo(w_hi[e]));
    const float y3 = head_norm(bf16_hi(hi[e]), rstd, bf16_hi(w_hi[e]));
    const float c0 = cs[2 * e], c1 = cs[2 * e + 1], s0 = sn[2 * e], s1 = sn[2 * e + 1];
    lo[e] = pack_bf16x2(rope_lo(y0, y2, c0, s0), rope_lo(y1, y3, c1, s1));
    hi[e] = pack_bf16x2(rope_hi(y0, y2, c0, s0), rope_hi(y1, y3, c1, s1));
  }
}


// The bf16-rounded cos (cs) and sin (sn) of dims 8c..8c+7 at table row pos: the fp32 table holds
// 64 cos then 64 sin values per position (nv/layers/rotary_embedding.py:20-42 casts both to bf16).
__device__ __forceinline__ void rope_row8(const float *cos_sin, int64_t pos, int c, float (&cs)[8], float (&sn)[8]) {
  const float *row = cos_sin + pos * kHeadDim + 8 * c;
  const f32x4 c0 = *reinterpret_cast<const f32x4 *>(row), c1 = *reinterpret_cast<const f32x4 *>(row + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4 *>(row + 64), s1 = *reinterpret_cast<const f32x4 *>(row + 68);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    cs[e] = round_bf16(c0[e]);
    cs[4 + e] = round_bf16(c1[e]);
    sn[e] = round_bf16(s0[e]);
    sn[4 + e] = round_bf16(s1[e]);
  }
}

// Sum over 16 lanes (one DPP row).
__device__ __forceinline__ float sum16(float v) {
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return v;
}
// Maximum over the whole wave for a value already uniform inside each aligned
// group of 8 lanes.  The result is wave-uniform (it lives in an SGPR).
__device__ __forceinline__ float wave_max_from_groups8(float v) {
  v = fmaxf(v, dpp<kDppRowRor8>(v));
  v = fmaxf(v, swizzle_xor16(v));
  return fmaxf(readlane(v, 0), readlane(v, 32));
}
// Full 64-lane maximum, wave-uniform result.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppQuadXor1>(v));
  v = fmaxf(v, dpp<kDppQuadXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}
// Full 64-lane sum, wave-uniform result: reduce each 16-lane row, then add the 4 row sums.
__device__ __forceinline__ float wave_sum(float v) {
  v = sum16(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ u32x4 ld16(const u16 *p) { return *reinterpret_cast<const u32x4 *>(p); }
__device__ __forceinline__ u32x4 ld16_stream(const u16 *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ void st16(u16 *p, u32x4 v) { *reinterpret_cast<u32x4 *>(p) = v; }

__host__ __device__ constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Element (r, c) of a tiled [rows, cols] bf16 matrix (the skinny GEMM's operand order): 16 x 32
// tiles of 512 elements, row-tile major; inside a tile, 128 * (c%32 / 8) + 8 * (r%16) + c%8, so
// MFMA lane (r%16) + 16 * (c%32 / 8) finds its 8 consecutive columns at 8 * lane.
__device__ __forceinline__ int64_t tiled_index(int r, int c, int cols) {
  return ((int64_t)(r >> 4) * (cols >> 5) + (c >> 5)) * 512 + ((c & 31) >> 3) * 128 + (r & 15) * 8 + (c & 7);
}

inline int log2_exact(int x) {
  if (x <= 0 || (x & (x - 1)) != 0) return -1;
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NVAMD_OK : (int)e;
}

// The current device's index-error word (errors.hip), or nullptr if it cannot be looked up (the
// kernels then report nothing).  Kernels take it as an argument and OR NVAMD_ERR_* bits into it
// where the reference's indexing would raise; on the normal path they never touch it.
u32 *index_error_word();

__device__ __forceinline__ void flag_index_error(u32 *word, u32 bit) {
  if (word != nullptr) __hip_atomic_fetch_or(word, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace nvamd
