// Ragged-batch packing on the GPU (replaces the host loops of
// BlockManager.get_block_tables_tensor / get_context_lens_tensor /
// get_slot_mapping, nv/npu/block_manager.py:207-250, and
// ModelRunner._prepare_prefill_inputs / decode input build,
// nv/model_runner.py:169-197, 245-258).
//
// The host keeps the block-allocation state machine (a free list is
// inherently sequential) and a persistent device mirror of every live
// sequence's block table.  Per forward it uploads, in one transfer, a compact
// descriptor per sequence, the table entries that changed since the last
// upload, and (optionally) the token ids.  One workgroup per sequence then:
//   1. applies the pending table updates of its mirror row (workgroup 0
//      applies every update, so rows outside the batch stay current);
//   2. computes its token offset = sum of the earlier query lengths;
//   3. writes cu_seqlens, context_lens, last_token_indices, its zero-padded
//      block-table row, and slot / position / input id of each of its tokens:
//        pos  = start + k,  slot = table[pos / bs] * bs + pos % bs.
#include "common.h"

namespace nvamd {
namespace {

struct PackArgs {
  const int32_t *desc;     // [5][batch]: mirror row, start position, query length, table length, context length
  const int32_t *updates;  // [num_updates][3]: (mirror row, column, block id)
  const int32_t *token_ids;  // [total_tokens] or null
  int32_t *mirror;
  int32_t *block_tables;
  int32_t *context_lens;
  int64_t *slot_mapping;
  int64_t *positions;
  int32_t *cu_seqlens;
  int64_t *last_token_idx;
  int64_t *input_ids;
  int batch;
  int num_updates;
  int mirror_stride;
  int mirror_rows;
  int bs_log2;
  int bt_stride;
  int bt_width;
};

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
pack_kernel(PackArgs a) {
  const int i = blockIdx.x;
  const int tid = threadIdx.x;
  const int B = a.batch;
  const int row = a.desc[i];
  const int start = a.desc[B + i];
  const int qlen = a.desc[2 * B + i];
  const int nblk = min(a.desc[3 * B + i], a.mirror_stride);
  const int ctx = a.desc[4 * B + i];

  // 1. table updates
  for (int u = tid; u < a.num_updates; u += kThreads) {
    const int r = a.updates[3 * u];
    const int c = a.updates[3 * u + 1];
    if ((i == 0 || r == row) && r >= 0 && r < a.mirror_rows && c >= 0 && c < a.mirror_stride)
      a.mirror[(int64_t)r * a.mirror_stride + c] = a.updates[3 * u + 2];
  }

  // 2. token offset of this sequence
  __shared__ int s_sum[kThreads];
  int part = 0;
  for (int k = tid; k < i; k += kThreads) part += a.desc[2 * B + k];
  s_sum[tid] = part;
  __syncthreads();
  for (int off = kThreads / 2; off > 0; off >>= 1) {
    if (tid < off) s_sum[tid] += s_sum[tid + off];
    __syncthreads();
  }
  const int base = s_sum[0];

  // 3. outputs
  const bool row_ok = row >= 0 && row < a.mirror_rows;
  const int32_t *mrow = a.mirror + (int64_t)(row_ok ? row : 0) * a.mirror_stride;
  if (tid == 0) {
    if (a.cu_seqlens) {
      a.cu_seqlens[i + 1] = base + qlen;
      if (i == 0) a.cu_seqlens[0] = 0;
    }
    if (a.context_lens) a.context_lens[i] = ctx;
    if (a.last_token_idx) a.last_token_idx[i] = (int64_t)base + qlen - 1;
  }
  if (a.block_tables) {
    for (int c = tid; c < a.bt_width; c += kThreads)
      a.block_tables[(int64_t)i * a.bt_stride + c] = (row_ok && c < nblk) ? mrow[c] : 0;
  }
  const int bs_mask = (1 << a.bs_log2) - 1;
  for (int k = tid; k < qlen; k += kThreads) {
    const int pos = start + k;
    const int bi = pos >> a.bs_log2;
    const int64_t t = (int64_t)base + k;
    int64_t slot = -1;  // a position past the table: the host raises before this can happen
    if (row_ok && bi < nblk) slot = ((int64_t)mrow[bi] << a.bs_log2) + (pos & bs_mask);
    if (a.slot_mapping) a.slot_mapping[t] = slot;
    if (a.positions) a.positions[t] = pos;
    if (a.input_ids && a.token_ids) a.input_ids[t] = a.token_ids[t];
  }
}

}  // namespace
}  // namespace nvamd

using namespace nvamd;

extern "C" int nvamd_pack_batch(const int32_t *desc, int batch, const int32_t *updates, int num_updates,
                                const int32_t *token_ids, int32_t *mirror, int mirror_stride, int mirror_rows,
                                int block_size, int32_t *block_tables, int bt_stride, int bt_width,
                                int32_t *context_lens, int64_t *slot_mapping, int64_t *positions,
                                int32_t *cu_seqlens, int64_t *last_token_indices, int64_t *input_ids,
                                hipStream_t stream) {
  if (batch == 0) return NVAMD_OK;
  if (!desc || !mirror || batch < 0 || num_updates < 0 || mirror_stride <= 0 || mirror_rows <= 0) return NVAMD_EINVAL;
  if (num_updates > 0 && !updates) return NVAMD_EINVAL;
  if (block_tables && (bt_width < 0 || bt_stride < bt_width)) return NVAMD_EINVAL;
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return NVAMD_EUNSUPPORTED;
  PackArgs a;
  a.desc = desc;
  a.updates = updates;
  a.token_ids = token_ids;
  a.mirror = mirror;
  a.block_tables = block_tables;
  a.context_lens = context_lens;
  a.slot_mapping = slot_mapping;
  a.positions = positions;
  a.cu_seqlens = cu_seqlens;
  a.last_token_idx = last_token_indices;
  a.input_ids = input_ids;
  a.batch = batch;
  a.num_updates = num_updates;
  a.mirror_stride = mirror_stride;
  a.mirror_rows = mirror_rows;
  a.bs_log2 = bs_log2;
  a.bt_stride = bt_stride;
  a.bt_width = block_tables ? bt_width : 0;
  hipLaunchKernelGGL(pack_kernel, dim3(batch), dim3(kThreads), 0, stream, a);
  return launch_status();
}
