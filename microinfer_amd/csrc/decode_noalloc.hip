// Allocation-free paged decode: mi_paged_decode_append with its scratch (the
// partition plan, the split partials and the arrival counters) in a
// file-scope device array instead of caller-provided workspace, for callers
// that cannot allocate device memory (code under hipGraph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// Each GPU holds its own copy of `scratch` for the life of the process. Host
// code never passes the array's name to a kernel (on the host it is only a
// stand-in symbol): the first call on a device looks up that device's copy
// with hipGetSymbolAddress and keeps the address per device.
#include <mutex>

#include "paged_attention.h"

namespace mi {
namespace {

// [counters: kCounterBytes][workspace: the rest]. The counter region holds
// one int32 per (sequence, KV head): kMaxPlanSeqs sequences x 16 KV heads.
constexpr int64_t kScratchBytes = 32ll << 20;
constexpr int64_t kCounterBytes = static_cast<int64_t>(kMaxPlanSeqs) * 16 * 4;
static_assert(kCounterBytes % 256 == 0, "workspace region stays 256-byte aligned");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
unsigned char* g_scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch` (looked up once per device).
int32_t device_scratch(unsigned char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(MI_ERR_HIP, "mi_paged_decode_append_noalloc: no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail(MI_ERR_HIP, std::string("mi_paged_decode_append_noalloc: "
                                          "hipGetSymbolAddress(scratch) failed: ") +
                                  hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<unsigned char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return MI_OK;
}

}  // namespace
}  // namespace mi

extern "C" int64_t mi_paged_decode_noalloc_max_bytes(void) {
  return mi::kScratchBytes - mi::kCounterBytes;
}

extern "C" int32_t mi_paged_decode_append_noalloc(
    const void* new_keys, int64_t nk_token_stride, int64_t nk_head_stride,
    const void* new_values, int64_t nv_token_stride, int64_t nv_head_stride,
    const void* query, int64_t q_token_stride, int64_t q_head_stride, void* key_cache,
    void* value_cache, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, const int32_t* block_tables, int64_t block_table_stride,
    int32_t block_table_width, const int32_t* context_lens, void* out,
    int64_t out_token_stride, int64_t out_head_stride, int32_t num_seqs,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int32_t num_blocks, int32_t split_k, float scale, int32_t dtype, void* stream) {
  using namespace mi;
  clear_error();
  if (new_keys == nullptr || new_values == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_paged_decode_append_noalloc: null new keys or values");
  if (num_seqs < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || head_dim <= 0 || split_k < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_append_noalloc: invalid sizes");
  if (num_seqs == 0) return MI_OK;
  if (num_seqs > kMaxPlanSeqs || num_kv_heads > 16)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_append_noalloc: at most 4096 sequences "
                                    "and 16 KV heads");
  const int64_t need = mi_paged_decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads,
                                                       head_dim, split_k);
  const int64_t room = kScratchBytes - kCounterBytes;
  if (need > room)
    return fail(MI_ERR_WORKSPACE, "mi_paged_decode_append_noalloc: this call needs " +
                                      std::to_string(need) + " bytes of scratch; the static "
                                      "scratch holds " + std::to_string(room));
  unsigned char* base = nullptr;
  const int32_t st = device_scratch(&base);
  if (st != MI_OK) return st;
  int32_t* counters = reinterpret_cast<int32_t*>(base);
  void* workspace = base + kCounterBytes;
  NewRows rows;
  rows.keys = new_keys;
  rows.k_ts = nk_token_stride;
  rows.k_hs = nk_head_stride;
  rows.values = new_values;
  rows.v_ts = nv_token_stride;
  rows.v_hs = nv_head_stride;
  // plan == NULL: the call computes its plan into the scratch, and the plan
  // kernel zeroes this call's counters before the decode launch reads them.
  return paged_decode(query, q_token_stride, q_head_stride, key_cache, value_cache,
                      cache_block_stride, cache_token_stride, cache_head_stride, block_tables,
                      block_table_stride, block_table_width, context_lens, out,
                      out_token_stride, out_head_stride, workspace, room, counters, nullptr,
                      0, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                      num_blocks, split_k, scale, dtype, rows, stream);
}
