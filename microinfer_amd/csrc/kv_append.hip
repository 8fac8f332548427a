// KV append: scatter new K/V rows into the paged cache through the slot map.
//
// Replaces _store_kv_kernel/store_kv (microinfer/worker/triton_kv_store.py:19-78)
// and the slot div/mod of AttentionMetadata.slot_indices
// (microinfer/layer/metadata.py:75-84). The copy is dtype-agnostic: each thread
// moves one word of W bytes (16 when the row, strides and pointers allow), so
// the result is bit-exact for every element type.
#include "mi_common.h"

namespace mi {
namespace {

template <typename W>
__global__ __launch_bounds__(256) void kv_append_kernel(
    const char* __restrict__ keys, int64_t k_ts, int64_t k_hs,
    const char* __restrict__ values, int64_t v_ts, int64_t v_hs, char* __restrict__ kc,
    char* __restrict__ vc, int64_t c_bs, int64_t c_ts, int64_t c_hs, const void* idx0,
    const void* idx1, int idx64, int num_tokens, int num_heads, int words_per_row,
    int block_size, int num_blocks) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int total = num_tokens * num_heads * words_per_row;
  if (i >= total) return;
  const int word = i % words_per_row;
  const int row = i / words_per_row;
  const int head = row % num_heads;
  const int token = row / num_heads;

  int64_t blk, off;
  if (idx1 == nullptr) {
    const int64_t slot = idx64 ? static_cast<const int64_t*>(idx0)[token]
                               : static_cast<const int32_t*>(idx0)[token];
    if (slot < 0) return;  // padding slot (-1)
    blk = slot / block_size;
    off = slot - blk * block_size;
  } else {
    blk = idx64 ? static_cast<const int64_t*>(idx0)[token]
                : static_cast<const int32_t*>(idx0)[token];
    off = idx64 ? static_cast<const int64_t*>(idx1)[token]
                : static_cast<const int32_t*>(idx1)[token];
    if (off < 0 || off >= block_size) return;
  }
  if (blk < 0 || blk >= num_blocks) return;

  const int64_t wb = static_cast<int64_t>(word) * sizeof(W);
  const W k = *reinterpret_cast<const W*>(keys + token * k_ts + head * k_hs + wb);
  const W v = *reinterpret_cast<const W*>(values + token * v_ts + head * v_hs + wb);
  const int64_t dst = blk * c_bs + off * c_ts + head * c_hs + wb;
  *reinterpret_cast<W*>(kc + dst) = k;
  *reinterpret_cast<W*>(vc + dst) = v;
}

template <typename W>
int32_t launch_append(const char* keys, int64_t k_ts, int64_t k_hs, const char* values,
                      int64_t v_ts, int64_t v_hs, char* kc, char* vc, int64_t c_bs,
                      int64_t c_ts, int64_t c_hs, const void* idx0, const void* idx1,
                      int idx64, int num_tokens, int num_heads, int row_bytes,
                      int block_size, int num_blocks, hipStream_t stream) {
  const int words = row_bytes / static_cast<int>(sizeof(W));
  const int64_t total = static_cast<int64_t>(num_tokens) * num_heads * words;
  const int threads = 256;
  const int grid = static_cast<int>((total + threads - 1) / threads);
  kv_append_kernel<W><<<grid, threads, 0, stream>>>(
      keys, k_ts, k_hs, values, v_ts, v_hs, kc, vc, c_bs, c_ts, c_hs, idx0, idx1, idx64,
      num_tokens, num_heads, words, block_size, num_blocks);
  return check_launch("mi_kv_append");
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_kv_append(const void* keys, int64_t key_token_stride,
                                int64_t key_head_stride, const void* values,
                                int64_t value_token_stride, int64_t value_head_stride,
                                void* key_cache, void* value_cache,
                                int64_t cache_block_stride, int64_t cache_token_stride,
                                int64_t cache_head_stride, const void* index0,
                                const void* index1, int32_t index_is_int64,
                                int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                                int32_t block_size, int32_t num_blocks, int32_t dtype,
                                void* stream) {
  using namespace mi;
  clear_error();
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "mi_kv_append: bad dtype");
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_kv_append: sizes must be positive");
  if (num_tokens == 0) return MI_OK;
  if (!keys || !values || !key_cache || !value_cache || !index0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_kv_append: null pointer");
  const int64_t es = static_cast<int64_t>(dtype_size(dtype));
  const int row_bytes = static_cast<int>(head_dim * es);
  if (static_cast<int64_t>(num_tokens) * num_kv_heads * row_bytes > (int64_t(1) << 31))
    return fail(MI_ERR_UNSUPPORTED, "mi_kv_append: too many rows for one launch");

  const int64_t b_k_ts = key_token_stride * es, b_k_hs = key_head_stride * es;
  const int64_t b_v_ts = value_token_stride * es, b_v_hs = value_head_stride * es;
  const int64_t b_c_bs = cache_block_stride * es, b_c_ts = cache_token_stride * es,
                b_c_hs = cache_head_stride * es;
  // Widest word that every row start and the row length are aligned to.
  uint64_t align_bits = static_cast<uint64_t>(row_bytes) | b_k_ts | b_k_hs | b_v_ts |
                        b_v_hs | b_c_bs | b_c_ts | b_c_hs |
                        reinterpret_cast<uintptr_t>(keys) |
                        reinterpret_cast<uintptr_t>(values) |
                        reinterpret_cast<uintptr_t>(key_cache) |
                        reinterpret_cast<uintptr_t>(value_cache);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* k = static_cast<const char*>(keys);
  const char* v = static_cast<const char*>(values);
  char* kc = static_cast<char*>(key_cache);
  char* vc = static_cast<char*>(value_cache);
#define MI_APPEND(W)                                                                   \
  launch_append<W>(k, b_k_ts, b_k_hs, v, b_v_ts, b_v_hs, kc, vc, b_c_bs, b_c_ts, b_c_hs, \
                   index0, index1, index_is_int64, num_tokens, num_kv_heads, row_bytes,  \
                   block_size, num_blocks, s)
  if ((align_bits & 15u) == 0) return MI_APPEND(uint4);
  if ((align_bits & 7u) == 0) return MI_APPEND(uint2);
  if ((align_bits & 3u) == 0) return MI_APPEND(uint32_t);
  if ((align_bits & 1u) == 0) return MI_APPEND(uint16_t);
#undef MI_APPEND
  return fail(MI_ERR_INVALID_ARGUMENT, "mi_kv_append: misaligned pointers or strides");
}
