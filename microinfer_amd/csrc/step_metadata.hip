// Per-step index metadata (block tables, context lengths, positions, slot
// mapping, input ids) expanded on the device from a compact description of
// the scheduled batch.
//
// Replaces the host loops and copies of ModelRunner._fill_decode_rows,
// _copy_decode_buffers and _fill_graph_bucket (microinfer/runner.py:160-188,
// :561-576) and the per-token lists of prepare_prefill (:298-346). The
// reference fills a [rows, W] table on the host (W = num_blocks + 1 for a
// graph bucket) and copies all of it every step; here the host sends only the
// block ids each sequence owns and one workgroup per row writes the padded
// row in HBM.
#include "mi_common.h"

namespace mi {
namespace {

constexpr int kThreads = 256;

// One workgroup per output row. Row r < num_seqs takes tokens
// [cu_q[r], cu_q[r+1]) at positions starts[r] + i and owns block ids
// blocks[block_offsets[r] .. block_offsets[r+1]); rows past num_seqs are pad
// rows with one token each. Every store is bounded by num_tokens / width, so
// inconsistent offsets cannot write out of bounds.
__global__ __launch_bounds__(kThreads) void step_metadata_kernel(
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ starts,
    const int32_t* __restrict__ block_offsets, const int32_t* __restrict__ blocks,
    const int64_t* __restrict__ token_ids, int num_seqs, int num_tokens, int block_size,
    int pad_block, int32_t* __restrict__ tables, int64_t table_stride, int width,
    int32_t* __restrict__ context_lens, int32_t* __restrict__ slots,
    int64_t* __restrict__ positions, int64_t* __restrict__ input_ids) {
  const int r = blockIdx.x;
  const bool pad = r >= num_seqs;
  int t0, count, start, first_block, owned;
  if (pad) {
    t0 = cu_q[num_seqs] + (r - num_seqs);
    count = 1;
    start = 0;
    first_block = 0;
    owned = 0;
  } else {
    t0 = cu_q[r];
    count = cu_q[r + 1] - t0;
    start = starts[r];
    first_block = block_offsets[r];
    owned = block_offsets[r + 1] - first_block;
  }

  if (tables != nullptr) {
    int32_t* row = tables + static_cast<int64_t>(r) * table_stride;
    for (int c = threadIdx.x; c < width; c += kThreads) {
      int32_t id;
      if (pad) id = c == 0 ? pad_block : -1;
      else id = c < owned ? blocks[first_block + c] : -1;
      row[c] = id;
    }
  }
  if (context_lens != nullptr && threadIdx.x == 0) context_lens[r] = pad ? 1 : start + count;

  for (int i = threadIdx.x; i < count; i += kThreads) {
    const int t = t0 + i;
    if (t < 0 || t >= num_tokens) continue;
    const int p = start + i;
    if (positions != nullptr) positions[t] = p;
    if (input_ids != nullptr) input_ids[t] = pad ? 0 : token_ids[t];
    if (slots != nullptr) {
      int32_t s;
      if (pad) {
        s = pad_block * block_size + r % block_size;
      } else {
        const int logical = p / block_size;
        s = logical < owned ? blocks[first_block + logical] * block_size + p % block_size : -1;
      }
      slots[t] = s;
    }
  }
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_step_metadata(const int32_t* cu_seqlens_q, const int32_t* starts,
                                    const int32_t* block_offsets, const int32_t* blocks,
                                    const int64_t* token_ids, int32_t num_seqs, int32_t rows,
                                    int32_t num_tokens, int32_t block_size, int32_t pad_block,
                                    int32_t* block_tables, int64_t block_table_stride,
                                    int32_t block_table_width, int32_t* context_lens,
                                    int32_t* slot_mapping, int64_t* positions,
                                    int64_t* input_ids, void* stream) {
  using namespace mi;
  clear_error();
  if (num_seqs < 0 || rows < num_seqs || num_tokens < 0 || block_size <= 0 ||
      block_table_width < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: invalid sizes");
  if (rows == 0) return MI_OK;
  if (rows > num_seqs && pad_block < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: pad rows need a pad block");
  if (rows > num_seqs &&
      static_cast<int64_t>(pad_block) * block_size + block_size - 1 > INT32_MAX)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: pad slot overflows int32");
  if (!cu_seqlens_q) return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: null cu_seqlens_q");
  if (num_seqs > 0 && (!starts || !block_offsets))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: null starts or block_offsets");
  if (num_seqs > 0 && (block_tables || slot_mapping) && !blocks)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: null blocks");
  if (num_seqs > 0 && input_ids && !token_ids)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: null token_ids");
  if (block_tables && block_table_stride < block_table_width)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: table stride below width");
  if (block_tables && rows > num_seqs && block_table_width < 1)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_step_metadata: pad rows need table width >= 1");
  step_metadata_kernel<<<rows, kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      cu_seqlens_q, starts, block_offsets, blocks, token_ids, num_seqs, num_tokens, block_size,
      pad_block, block_tables, block_table_stride, block_table_width, context_lens, slot_mapping,
      positions, input_ids);
  return check_launch("mi_step_metadata");
}
