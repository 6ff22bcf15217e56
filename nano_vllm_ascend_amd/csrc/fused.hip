// Fused elementwise kernels around the attention path (one launch each instead of
// the chains of torch kernels the composite ops need):
//   add_rms_norm  residual += delta (bf16);  out = RMSNorm(residual) * w
//                 = the decoder layer's "h = residual + h; residual = h; h = norm(h)"
//                 (nv/models/qwen3.py:138-150, npu_rms_norm at nv/layers/layernorm.py:12-17)
//   silu_mul      out = silu(gate) * up on the fused [T, 2I] gate/up projection
//                 (nv/models/qwen3.py:34-35)
//   argmax_rows   greedy token of each logits row, first index on ties
//                 (torch.argmax at nv/layers/sampler.py:13-14)
//   embed_rows    token embedding gather (torch.embedding at nv/layers/embed_head.py:20-21,
//                 nv/models/qwen3.py:176) plus the per-32-column sums of squares that the
//                 first decoder layer's normalising GEMM prologue reads
// Rounding points match the reference's bf16 model: the residual sum is rounded
// to bf16, the norm is computed in fp32 with one rounding, silu is rounded to
// bf16 before the product, which is rounded again.
#include "common.h"

namespace nvamd {
namespace {

// One wave per row; lane l holds elements [16l, 16l+16) of each 1024-wide chunk.
template <bool ADD>
__global__ void __launch_bounds__(256)
add_rms_norm_kernel(const u16 *__restrict__ delta, u16 *__restrict__ residual, const u16 *__restrict__ weight,
                    u16 *__restrict__ out, int rows, int hidden, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t base = (int64_t)row * hidden;
  constexpr int kMaxChunks = 4;  // hidden <= 4096
  u32x4 v[kMaxChunks][2];
  float ss = 0.f;
  const int chunks = hidden / 1024;
#pragma unroll
  for (int ch = 0; ch < kMaxChunks; ++ch) {
    if (ch >= chunks) break;
    const int64_t off = base + ch * 1024 + 16 * lane;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4 x = ld16(residual + off + 8 * h);
      if (ADD) {
        const u32x4 d = ld16(delta + off + 8 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          x[e] = pack_bf16x2(bf16_lo(x[e]) + bf16_lo(d[e]), bf16_hi(x[e]) + bf16_hi(d[e]));
        st16(residual + off + 8 * h, x);
      }
      v[ch][h] = x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = bf16_lo(x[e]), b = bf16_hi(x[e]);
        ss += a * a + b * b;
      }
    }
  }
  ss = wave_sum(ss);
  const float rstd = rsqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int ch = 0; ch < kMaxChunks; ++ch) {
    if (ch >= chunks) break;
    const int64_t off = (int64_t)ch * 1024 + 16 * lane;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 w = ld16(weight + off + 8 * h);
      u32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        y[e] = pack_bf16x2(bf16_lo(v[ch][h][e]) * rstd * bf16_lo(w[e]), bf16_hi(v[ch][h][e]) * rstd * bf16_hi(w[e]));
      st16(out + base + off + 8 * h, y);
    }
  }
}

// Hidden sizes the kernel above does not take (any multiple of 8: Qwen3-4B's 2560, -14B's and
// -32B's 5120).  One wave per row; lane l takes the 16-byte vectors l, l + 64, ...  The first pass
// only sums the squares of the (added) row; the second reads the inputs again (L2 hits), forms
// the same bf16 sums, and writes the residual and the normalised row.  Same rounding as above.
template <bool ADD>
__global__ void __launch_bounds__(256)
add_rms_norm_any_kernel(const u16 *__restrict__ delta, u16 *__restrict__ residual, const u16 *__restrict__ weight,
                        u16 *__restrict__ out, int rows, int hidden, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t base = (int64_t)row * hidden;
  const int vecs = hidden / 8;
  auto row_vec = [&](int i) {
    u32x4 x = ld16(residual + base + 8 * i);
    if (ADD) {
      const u32x4 d = ld16(delta + base + 8 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = pack_bf16x2(bf16_lo(x[e]) + bf16_lo(d[e]), bf16_hi(x[e]) + bf16_hi(d[e]));
    }
    return x;
  };
  float ss = 0.f;
  for (int i = lane; i < vecs; i += 64) {
    const u32x4 x = row_vec(i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = bf16_lo(x[e]), b = bf16_hi(x[e]);
      ss += a * a + b * b;
    }
  }
  ss = wave_sum(ss);
  const float rstd = rsqrtf(ss / (float)hidden + eps);
  for (int i = lane; i < vecs; i += 64) {
    const u32x4 x = row_vec(i);
    if (ADD) st16(residual + base + 8 * i, x);
    const u32x4 w = ld16(weight + 8 * i);
    u32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      y[e] = pack_bf16x2(bf16_lo(x[e]) * rstd * bf16_lo(w[e]), bf16_hi(x[e]) * rstd * bf16_hi(w[e]));
    st16(out + base + 8 * i, y);
  }
}

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

// One thread per 8 output elements.
__global__ void __launch_bounds__(256)
silu_mul_kernel(const u16 *__restrict__ gu, u16 *__restrict__ out, int rows, int inter, int64_t gu_stride,
                int64_t out_stride) {
  const int per_row = inter / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * per_row) return;
  const int r = (int)(i / per_row);
  const int c = (int)(i % per_row) * 8;
  const u32x4 g = ld16(gu + (int64_t)r * gu_stride + c);
  const u32x4 u = ld16(gu + (int64_t)r * gu_stride + inter + c);
  u32x4 y;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float s0 = round_bf16(silu_f32(bf16_lo(g[e])));
    const float s1 = round_bf16(silu_f32(bf16_hi(g[e])));
    y[e] = pack_bf16x2(s0 * bf16_lo(u[e]), s1 * bf16_hi(u[e]));
  }
  st16(out + (int64_t)r * out_stride + c, y);
}

// (value, index) order of greedy sampling: larger value first, then the smaller index.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// One 1024-thread workgroup per row.  A thread scans 16-byte vectors in increasing index
// order, four loads in flight per step, keeping the first index of its maximum; waves then
// reduce with shuffles and the 16 wave results meet in LDS.
constexpr int kArgmaxThreads = 1024;
__global__ void __launch_bounds__(kArgmaxThreads)
argmax_rows_kernel(const u16 *__restrict__ logits, int64_t row_stride, int vocab, int64_t *__restrict__ out) {
  constexpr int U = 4;
  constexpr int kStep = kArgmaxThreads * 8;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const u16 *p = logits + (int64_t)row * row_stride;
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  const int vec_end = (vocab / 8) * 8;
  for (int c0 = tid * 8; c0 < vec_end; c0 += U * kStep) {
    u32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * kStep;
      x[u] = c < vec_end ? ld16(p + c) : u32x4{0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u};  // -inf
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = c0 + u * kStep + 2 * e;
        const float a = bf16_lo(x[u][e]), b = bf16_hi(x[u][e]);
        if (a > best) { best = a; best_i = c; }
        if (b > best) { best = b; best_i = c + 1; }
      }
  }
  for (int c = vec_end + tid; c < vocab; c += kArgmaxThreads) {
    const float a = bf16_to_f32(p[c]);
    if (a > best) { best = a; best_i = c; }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_i, off);
    if (better(ov, oi, best, best_i)) { best = ov; best_i = oi; }
  }
  __shared__ float s_v[kArgmaxThreads / 64];
  __shared__ int s_i[kArgmaxThreads / 64];
  const int w = tid >> 6;
  if ((tid & 63) == 0) {
    s_v[w] = best;
    s_i[w] = best_i;
  }
  __syncthreads();
  if (tid == 0) {
    float bv = s_v[0];
    int bi = s_i[0];
    for (int x = 1; x < kArgmaxThreads / 64; ++x)
      if (better(s_v[x], s_i[x], bv, bi)) { bv = s_v[x]; bi = s_i[x]; }
    out[row] = bi == 0x7fffffff ? 0 : bi;
  }
}

// One wave per row: out[r] = table[ids[r]] (a zero row for an id outside [0, vocab)),
// and ssq[r][t] = sum of squares of columns 32t..32t+31.  Lane l holds columns
// 16l..16l+15 of each 1024-wide chunk; lanes 2t and 2t+1 make up tile t.  A tiled out
// (the skinny GEMM's operand order) takes each 8-column half as one 16-byte store.
__global__ void __launch_bounds__(256)
embed_rows_kernel(const int64_t *__restrict__ ids, const u16 *__restrict__ table, int64_t table_stride, int vocab,
                  u16 *__restrict__ out, int64_t out_stride, bool out_tiled, float *__restrict__ ssq, int rows,
                  int hidden) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t id = ids[row];
  const bool valid = id >= 0 && id < vocab;
  const u16 *src = table + (valid ? id : 0) * table_stride;
  u16 *dst = out + (int64_t)row * out_stride;
  const u32x4 z = {0u, 0u, 0u, 0u};
  for (int ch = 0; ch < hidden; ch += 1024) {
    const int off = ch + 16 * lane;
    const u32x4 a = valid ? ld16(src + off) : z;
    const u32x4 b = valid ? ld16(src + off + 8) : z;
    if (out_tiled) {
      st16(out + tiled_index(row, off, hidden), a);
      st16(out + tiled_index(row, off + 8, hidden), b);
    } else {
      st16(dst + off, a);
      st16(dst + off + 8, b);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ss += bf16_lo(a[e]) * bf16_lo(a[e]) + bf16_hi(a[e]) * bf16_hi(a[e]);
      ss += bf16_lo(b[e]) * bf16_lo(b[e]) + bf16_hi(b[e]) * bf16_hi(b[e]);
    }
    ss += dpp<kDppQuadXor1>(ss);
    if (ssq && (lane & 1) == 0) ssq[(int64_t)row * (hidden >> 5) + (off >> 5)] = ss;
  }
}

}  // namespace
}  // namespace nvamd

using namespace nvamd;

extern "C" int nvamd_add_rms_norm(const void *delta, void *residual, const void *weight, void *out, int rows,
                                  int hidden, float eps, hipStream_t stream) {
  if (rows == 0) return NVAMD_OK;
  if (!residual || !weight || !out || rows < 0) return NVAMD_EINVAL;
  if (hidden <= 0 || hidden % 8 != 0) return NVAMD_EUNSUPPORTED;
  if (!aligned16(residual) || !aligned16(weight) || !aligned16(out) || (delta && !aligned16(delta)))
    return NVAMD_EINVAL;
  const dim3 grid((rows + 3) / 4);
  if (hidden % 1024 != 0 || hidden > 4096) {
    if (delta)
      hipLaunchKernelGGL((add_rms_norm_any_kernel<true>), grid, dim3(256), 0, stream, static_cast<const u16 *>(delta),
                         static_cast<u16 *>(residual), static_cast<const u16 *>(weight), static_cast<u16 *>(out), rows,
                         hidden, eps);
    else
      hipLaunchKernelGGL((add_rms_norm_any_kernel<false>), grid, dim3(256), 0, stream, nullptr,
                         static_cast<u16 *>(residual), static_cast<const u16 *>(weight), static_cast<u16 *>(out),
                         rows, hidden, eps);
    return launch_status();
  }
  if (delta)
    hipLaunchKernelGGL((add_rms_norm_kernel<true>), grid, dim3(256), 0, stream, static_cast<const u16 *>(delta),
                       static_cast<u16 *>(residual), static_cast<const u16 *>(weight), static_cast<u16 *>(out), rows,
                       hidden, eps);
  else
    hipLaunchKernelGGL((add_rms_norm_kernel<false>), grid, dim3(256), 0, stream, nullptr,
                       static_cast<u16 *>(residual), static_cast<const u16 *>(weight), static_cast<u16 *>(out), rows,
                       hidden, eps);
  return launch_status();
}

extern "C" int nvamd_silu_mul(const void *gate_up, int64_t gu_stride, void *out, int64_t out_stride, int rows,
                              int inter, hipStream_t stream) {
  if (rows == 0) return NVAMD_OK;
  if (!gate_up || !out || rows < 0 || inter <= 0 || inter % 8 || gu_stride < 2 * (int64_t)inter || gu_stride % 8 ||
      out_stride < inter || out_stride % 8 || !aligned16(gate_up) || !aligned16(out))
    return NVAMD_EINVAL;
  const int64_t total = (int64_t)rows * (inter / 8);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return NVAMD_EINVAL;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<const u16 *>(gate_up),
                     static_cast<u16 *>(out), rows, inter, gu_stride, out_stride);
  return launch_status();
}

extern "C" int nvamd_argmax_rows(const void *logits, int64_t row_stride, int rows, int vocab, int64_t *out,
                                 hipStream_t stream) {
  if (rows == 0) return NVAMD_OK;
  if (!logits || !out || rows < 0 || vocab <= 0 || row_stride < vocab || row_stride % 8 || !aligned16(logits))
    return NVAMD_EINVAL;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(kArgmaxThreads), 0, stream, static_cast<const u16 *>(logits),
                     row_stride, vocab, out);
  return launch_status();
}

extern "C" int nvamd_embed_rows(const int64_t *ids, const void *table, int64_t table_stride, int vocab, void *out,
                                int64_t out_stride, int out_tiled, float *ssq, int rows, int hidden,
                                hipStream_t stream) {
  if (rows == 0) return NVAMD_OK;
  if (!ids || !table || !out || rows < 0 || vocab <= 0) return NVAMD_EINVAL;
  if (hidden <= 0 || hidden % 1024) return NVAMD_EUNSUPPORTED;
  if (!aligned16(table) || !aligned16(out) || table_stride < hidden || table_stride % 8 ||
      (!out_tiled && (out_stride < hidden || out_stride % 8)))
    return NVAMD_EINVAL;
  hipLaunchKernelGGL(embed_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, ids,
                     static_cast<const u16 *>(table), table_stride, vocab, static_cast<u16 *>(out), out_stride,
                     out_tiled != 0, ssq, rows, hidden);
  return launch_status();
}
