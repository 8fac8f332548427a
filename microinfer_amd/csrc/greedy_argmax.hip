// Greedy token selection: the index of each logits row's maximum, in one
// graph-capturable launch.
//
// torch's argmax (what microinfer/runner.py:236-240 captures into the decode
// graph, and :619 / :625 and microinfer/layer/sampler.py:44-45 call eagerly)
// orders values by ">" with NaN above everything, and returns the first index
// among equal maxima (+0 and -0 are equal). Here every element maps to a
// 32-bit key whose unsigned order is that order -- NaN -> 0xFFFFFFFF, -0 ->
// +0, negative values bit-inverted, others with the sign bit set -- and
// (key << 32 | ~index) is the 64-bit word whose maximum is the answer. Word
// maxima combine in any order, so a row is split into chunks over many
// workgroups: each takes its chunk's maximum word to the row's slot with one
// agent-scope atomic max, then counts itself in; the last chunk to arrive
// reads the slot, writes the token and zeroes the slot and the counter for
// the next launch.
#include "mi_common.h"

namespace mi {
namespace {

constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxWaves = kArgmaxThreads / kWave;

__device__ __forceinline__ uint32_t order_key(float v) {
  uint32_t b = __float_as_uint(v);
  if (v != v) return 0xffffffffu;
  if ((b << 1) == 0) b = 0;  // -0 ties with +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), mask, kWave);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), mask, kWave);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// State per row: one 128-byte line (kStateWords words), so rows' atomics do
// not queue behind each other on a shared line. Word 0 is the running
// maximum, the low half of word 1 the arrival counter; both are zero between
// launches.
constexpr int kStateWords = 16;

template <typename E, int VEC>
__global__ __launch_bounds__(kArgmaxThreads) void greedy_argmax_kernel(
    const typename E::raw* __restrict__ logits, int64_t row_stride, int32_t vocab,
    int32_t chunk, int32_t chunks, uint64_t* __restrict__ state, int64_t* __restrict__ tokens) {
  using R = typename E::raw;
  const int row = blockIdx.x / chunks;
  const int c = blockIdx.x - row * chunks;
  const int t = threadIdx.x;
  const R* p = logits + static_cast<int64_t>(row) * row_stride;
  const int lo = c * chunk;
  const int hi = min(vocab, lo + chunk);

  // Each thread visits its indices in increasing order, so a strict ">" keeps
  // the first of equal keys; key 0 is below every real key.
  uint32_t best_key = 0;
  uint32_t best_idx = 0;
  const int vec_end = lo + ((hi - lo) / VEC) * VEC;
#pragma unroll 4
  for (int i = lo + t * VEC; i < vec_end; i += kArgmaxThreads * VEC) {
    const Pack<R, VEC> v = load_pack<R, VEC>(p + i);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const uint32_t k = order_key(E::load(v.v[j]));
      if (k > best_key) {
        best_key = k;
        best_idx = static_cast<uint32_t>(i + j);
      }
    }
  }
  for (int i = vec_end + t; i < hi; i += kArgmaxThreads) {
    const uint32_t k = order_key(E::load(p[i]));
    if (k > best_key) {
      best_key = k;
      best_idx = static_cast<uint32_t>(i);
    }
  }
  uint64_t word = best_key ? (static_cast<uint64_t>(best_key) << 32) | ~best_idx : 0;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) word = max_u64(word, shfl_xor_u64(word, o));

  __shared__ uint64_t wave_words[kArgmaxWaves];
  const int wave = t / kWave;
  if ((t & (kWave - 1)) == 0) wave_words[wave] = word;
  __syncthreads();
  if (t != 0) return;
#pragma unroll
  for (int w = 1; w < kArgmaxWaves; ++w) word = max_u64(word, wave_words[w]);

  uint64_t* slot = state + static_cast<int64_t>(kStateWords) * row;
  int32_t* counter = reinterpret_cast<int32_t*>(slot + 1);
  if (chunks > 1) {
    __hip_atomic_fetch_max(slot, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_stores();  // the maximum is in place before this chunk counts in
    const int arrived =
        __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (arrived != chunks - 1) return;
    // Read and clear the slot with one atomic, where the maxima were taken.
    word = __hip_atomic_exchange(slot, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  tokens[row] = static_cast<int64_t>(~static_cast<uint32_t>(word));
}

// Chunk length (elements, a whole number of passes of the block) such that
// the launch has about kTargetBlocks workgroups: one per CU. More, shorter
// chunks cost more in same-row atomics than they gain in parallel loads
// (32 rows x 151936: 5.5 us at 256 workgroups, 6.6 us at 1024).
constexpr int kTargetBlocks = 256;

template <typename E, int VEC>
int32_t launch_argmax(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                      int64_t* tokens, uint64_t* state, hipStream_t stream) {
  const int64_t pass = static_cast<int64_t>(kArgmaxThreads) * VEC;
  const int64_t per_row = (kTargetBlocks + rows - 1) / rows;
  int64_t passes = (vocab + per_row * pass - 1) / (per_row * pass);
  passes = passes < 1 ? 1 : passes;
  const int64_t chunk = passes * pass;
  const int64_t chunks = (vocab + chunk - 1) / chunk;
  const int64_t blocks = chunks * rows;
  if (blocks > 0x7fffffff)
    return fail(MI_ERR_UNSUPPORTED, "mi_greedy_argmax: too many rows for one launch");
  greedy_argmax_kernel<E, VEC><<<static_cast<int>(blocks), kArgmaxThreads, 0, stream>>>(
      static_cast<const typename E::raw*>(logits), row_stride, vocab,
      static_cast<int32_t>(chunk), static_cast<int32_t>(chunks), state, tokens);
  return check_launch("mi_greedy_argmax");
}

template <typename E>
int32_t dispatch_argmax(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                        int64_t* tokens, uint64_t* state, hipStream_t stream) {
  constexpr int kVec = 16 / sizeof(typename E::raw);
  const uint64_t bits = reinterpret_cast<uintptr_t>(logits) |
                        (rows > 1 ? static_cast<uint64_t>(row_stride) * sizeof(typename E::raw)
                                  : 0);
  if ((bits & 15u) == 0)
    return launch_argmax<E, kVec>(logits, row_stride, rows, vocab, tokens, state, stream);
  return launch_argmax<E, 1>(logits, row_stride, rows, vocab, tokens, state, stream);
}

}  // namespace
}  // namespace mi

extern "C" int64_t mi_greedy_argmax_state_bytes(int32_t num_rows) {
  return num_rows > 0 ? static_cast<int64_t>(num_rows) * mi::kStateWords * 8 : 0;
}

extern "C" int32_t mi_greedy_argmax(const void* logits, int64_t row_stride, int32_t num_rows,
                                    int32_t vocab_size, int32_t dtype, int64_t* tokens,
                                    void* state, int64_t state_bytes, void* stream) {
  using namespace mi;
  clear_error();
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "mi_greedy_argmax: bad dtype");
  if (num_rows < 0 || vocab_size <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_greedy_argmax: num_rows must be >= 0 and vocab_size > 0");
  if (vocab_size > (1 << 30))  // keeps every element index and loop bound in int32
    return fail(MI_ERR_UNSUPPORTED, "mi_greedy_argmax: vocab_size above 2^30");
  if (num_rows == 0) return MI_OK;
  if (!logits || !tokens) return fail(MI_ERR_INVALID_ARGUMENT, "mi_greedy_argmax: null pointer");
  if (num_rows > 1 && row_stride < vocab_size)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_greedy_argmax: row_stride must be >= vocab_size");
  const int64_t es = static_cast<int64_t>(dtype_size(dtype));
  if (reinterpret_cast<uintptr_t>(logits) % es || reinterpret_cast<uintptr_t>(tokens) % 8)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_greedy_argmax: misaligned pointer");
  if (!state || reinterpret_cast<uintptr_t>(state) % 8 ||
      state_bytes < mi_greedy_argmax_state_bytes(num_rows))
    return fail(MI_ERR_WORKSPACE,
                "mi_greedy_argmax: state must be 8-byte aligned, zero-filled and at least "
                "mi_greedy_argmax_state_bytes(num_rows) bytes");
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint64_t* st = static_cast<uint64_t*>(state);
  if (dtype == MI_DTYPE_BF16)
    return dispatch_argmax<BF16>(logits, row_stride, num_rows, vocab_size, tokens, st, s);
  if (dtype == MI_DTYPE_F16)
    return dispatch_argmax<F16>(logits, row_stride, num_rows, vocab_size, tokens, st, s);
  return dispatch_argmax<F32>(logits, row_stride, num_rows, vocab_size, tokens, st, s);
}
