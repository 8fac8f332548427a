// Block-table gather: materialise each request's valid cache rows as
// contiguous varlen K/V.
//
// Replaces _gather_paged_kv (microinfer/layer/paged_attention.py:76-101): the
// reference issues two index_select per request plus two cat; this is one
// launch that copies every row once. Byte copy, so bit-exact for any dtype.
#include "mi_common.h"

namespace mi {
namespace {

// Rows whose words do not fit the wave kernel below, or that are not 16-byte
// aligned: thread -> (output row, head, word). The owning request of an
// output row is found by binary search over cu_seqlens_k (requests are few
// and the array stays in L1/L2).
template <typename W>
__global__ __launch_bounds__(256) void gather_kv_kernel(
    const char* __restrict__ kc, const char* __restrict__ vc, int64_t c_bs, int64_t c_ts,
    int64_t c_hs, const int32_t* __restrict__ tables, int64_t t_stride, int t_width,
    const int32_t* __restrict__ cu_k, int num_requests, int total_rows,
    char* __restrict__ k_out, char* __restrict__ v_out, int num_heads, int words_per_row,
    int block_size, int log2_block, int num_blocks) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int total = total_rows * num_heads * words_per_row;
  if (i >= total) return;
  const int word = i % words_per_row;
  const int rh = i / words_per_row;
  const int head = rh % num_heads;
  const int row = rh / num_heads;

  // Largest r with cu_k[r] <= row.
  int lo = 0, hi = num_requests - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu_k[mid] <= row) lo = mid; else hi = mid - 1;
  }
  const int pos = row - cu_k[lo];
  const int logical_block = pos >> log2_block;
  const int64_t wb = static_cast<int64_t>(word) * sizeof(W);
  const int64_t out = (static_cast<int64_t>(row) * num_heads + head) * words_per_row * sizeof(W) + wb;
  W kval{}, vval{};
  // pos < 0 only for a malformed cu_seqlens_k (first entry above zero):
  // such rows read as zeros, like rows of invalid blocks.
  if (pos >= 0 && logical_block < t_width) {
    const int blk = tables[lo * t_stride + logical_block];
    if (blk >= 0 && blk < num_blocks) {
      const int64_t src = blk * c_bs + (pos & (block_size - 1)) * c_ts + head * c_hs + wb;
      kval = *reinterpret_cast<const W*>(kc + src);
      vval = *reinterpret_cast<const W*>(vc + src);
    }
  }
  *reinterpret_cast<W*>(k_out + out) = kval;
  *reinterpret_cast<W*>(v_out + out) = vval;
}

// 16-byte words, a wave per output row: the row's request is a scalar
// binary search over cu_seqlens_k, its block id a scalar load, and every lane
// moves words lane, lane + 64, ... of the row's K and V (all heads), all its
// loads issued before its stores. (Waves of 2, 4 and 8 rows with the request
// advanced row by row measured 63.0, 64.4 and 68.0 us against 62.1 us on the
// mixed step's 43926 rows: more, shorter waves keep more loads in flight.)
constexpr int kMaxWordsPerLane = 4;  // rows of up to 4 KiB (K or V, all heads)

template <int WPL>
__global__ __launch_bounds__(256) void gather_kv_row_kernel(
    const char* __restrict__ kc, const char* __restrict__ vc, int64_t c_bs, int64_t c_ts,
    int64_t c_hs, const int32_t* __restrict__ tables, int64_t t_stride, int t_width,
    const int32_t* __restrict__ cu_k, int num_requests, int total_rows,
    char* __restrict__ k_out, char* __restrict__ v_out, int num_heads, int words_per_row,
    int block_size, int log2_block, int num_blocks) {
  using ConstI32 = __attribute__((address_space(4))) const int32_t;
  const ConstI32* cuk = (const ConstI32*)(cu_k);
  const int lane = threadIdx.x % kWave;
  const int row = __builtin_amdgcn_readfirstlane(
      static_cast<int>(blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave));
  if (row >= total_rows) return;  // the whole wave
  // Largest r with cu_k[r] <= row.
  int req = 0, hi = num_requests - 1;
  while (req < hi) {
    const int mid = (req + hi + 1) >> 1;
    if (cuk[mid] <= row) req = mid; else hi = mid - 1;
  }
  const int pos = row - cuk[req];
  const int logical_block = pos >> log2_block;
  int64_t base = -1;
  if (pos >= 0 && logical_block < t_width) {
    const int blk = ((const ConstI32*)(tables))[req * t_stride + logical_block];
    if (blk >= 0 && blk < num_blocks) base = blk * c_bs + (pos & (block_size - 1)) * c_ts;
  }
  const int words = num_heads * words_per_row;  // per row, per tensor
  uint4 kv[WPL], vv[WPL];
#pragma unroll
  for (int k = 0; k < WPL; ++k) {
    const int w = lane + k * kWave;
    kv[k] = uint4{0, 0, 0, 0};
    vv[k] = uint4{0, 0, 0, 0};
    if (base >= 0 && w < words) {
      const int64_t src = base + (w / words_per_row) * c_hs + (w % words_per_row) * 16;
      kv[k] = *reinterpret_cast<const uint4*>(kc + src);
      vv[k] = *reinterpret_cast<const uint4*>(vc + src);
    }
  }
  const int64_t out = static_cast<int64_t>(row) * words * 16;
#pragma unroll
  for (int k = 0; k < WPL; ++k) {
    const int w = lane + k * kWave;
    if (w >= words) continue;
    *reinterpret_cast<uint4*>(k_out + out + w * 16) = kv[k];
    *reinterpret_cast<uint4*>(v_out + out + w * 16) = vv[k];
  }
}

template <typename W>
int32_t launch_gather(const char* kc, const char* vc, int64_t c_bs, int64_t c_ts,
                      int64_t c_hs, const int32_t* tables, int64_t t_stride, int t_width,
                      const int32_t* cu_k, int num_requests, int total_rows, char* k_out,
                      char* v_out, int num_heads, int row_bytes, int block_size,
                      int num_blocks, hipStream_t stream) {
  const int words = row_bytes / static_cast<int>(sizeof(W));
  if constexpr (sizeof(W) == 16) {
    const int wpl = (num_heads * words + kWave - 1) / kWave;
    if (wpl <= kMaxWordsPerLane) {
      const int grid = (total_rows + 3) / 4;  // four rows (waves) per workgroup
      auto go = [&](auto kernel) {
        kernel<<<grid, 256, 0, stream>>>(kc, vc, c_bs, c_ts, c_hs, tables, t_stride, t_width,
                                         cu_k, num_requests, total_rows, k_out, v_out,
                                         num_heads, words, block_size, ilog2(block_size),
                                         num_blocks);
      };
      if (wpl == 1) go(gather_kv_row_kernel<1>);
      else if (wpl == 2) go(gather_kv_row_kernel<2>);
      else go(gather_kv_row_kernel<4>);
      return check_launch("mi_gather_kv");
    }
  }
  const int64_t total = static_cast<int64_t>(total_rows) * num_heads * words;
  const int threads = 256;
  const int grid = static_cast<int>((total + threads - 1) / threads);
  gather_kv_kernel<W><<<grid, threads, 0, stream>>>(
      kc, vc, c_bs, c_ts, c_hs, tables, t_stride, t_width, cu_k, num_requests, total_rows,
      k_out, v_out, num_heads, words, block_size, ilog2(block_size), num_blocks);
  return check_launch("mi_gather_kv");
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_gather_kv(const void* key_cache, const void* value_cache,
                                int64_t cache_block_stride, int64_t cache_token_stride,
                                int64_t cache_head_stride, const int32_t* block_tables,
                                int64_t block_table_stride, int32_t block_table_width,
                                const int32_t* cu_seqlens_k, int32_t num_requests,
                                int32_t total_rows, void* key_out, void* value_out,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t num_blocks, int32_t dtype, void* stream) {
  using namespace mi;
  clear_error();
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_kv: bad dtype");
  if (num_requests < 0 || total_rows < 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      num_blocks <= 0 || block_table_width < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_kv: invalid sizes");
  if (!is_pow2(block_size))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_kv: block_size must be a power of two");
  if (total_rows == 0) return MI_OK;
  if (num_requests == 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_kv: rows without requests");
  if (!key_cache || !value_cache || !block_tables || !cu_seqlens_k || !key_out || !value_out)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_kv: null pointer");
  const int64_t es = static_cast<int64_t>(dtype_size(dtype));
  const int row_bytes = static_cast<int>(head_dim * es);
  if (static_cast<int64_t>(total_rows) * num_kv_heads * row_bytes > (int64_t(1) << 31))
    return fail(MI_ERR_UNSUPPORTED, "mi_gather_kv: too many rows for one launch");
  const int64_t b_bs = cache_block_stride * es, b_ts = cache_token_stride * es,
                b_hs = cache_head_stride * es;
  uint64_t align_bits = static_cast<uint64_t>(row_bytes) | b_bs | b_ts | b_hs |
                        reinterpret_cast<uintptr_t>(key_cache) |
                        reinterpret_cast<uintptr_t>(value_cache) |
                        reinterpret_cast<uintptr_t>(key_out) |
                        reinterpret_cast<uintptr_t>(value_out);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* kc = static_cast<const char*>(key_cache);
  const char* vc = static_cast<const char*>(value_cache);
  char* ko = static_cast<char*>(key_out);
  char* vo = static_cast<char*>(value_out);
#define MI_GATHER(W)                                                                    \
  launch_gather<W>(kc, vc, b_bs, b_ts, b_hs, block_tables, block_table_stride,           \
                   block_table_width, cu_seqlens_k, num_requests, total_rows, ko, vo,    \
                   num_kv_heads, row_bytes, block_size, num_blocks, s)
  if ((align_bits & 15u) == 0) return MI_GATHER(uint4);
  if ((align_bits & 7u) == 0) return MI_GATHER(uint2);
  if ((align_bits & 3u) == 0) return MI_GATHER(uint32_t);
  if ((align_bits & 1u) == 0) return MI_GATHER(uint16_t);
#undef MI_GATHER
  return fail(MI_ERR_INVALID_ARGUMENT, "mi_gather_kv: misaligned pointers or strides");
}
