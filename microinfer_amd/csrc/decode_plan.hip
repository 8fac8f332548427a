// Decode partition plan: which (sequence, block range) work items a paged
// decode launch runs. Computed on the device from context_lens, so a
// hipGraph replays it with whatever lengths the step has.
//
// The reference fixes split_k per launch on the host from R * Hq
// (microinfer/layer/triton_paged_attention.py:342-349) and stripes tiles over
// the splits (:76-79). Here partitions are contiguous block ranges sized from
// the step's total context: about kTargetItems (item, KV head) workgroups of
// at least kMinPartBlocks blocks each. A sequence's partitions occupy
// consecutive slots (first_item + part: where their partials go), but the
// launch dispatches items largest first, whatever their sequence: the
// hardware does not start a later workgroup on a CU that an early small item
// freed until well into the launch, so a small item in the first round
// leaves its CU idle, while small items at the end of the grid fill the
// tail.
#include "paged_attention.h"

namespace mi {
namespace {

// About this many (item, KV head) workgroups per launch, each covering at
// least kMinPartBlocks cache blocks. Fixed: the plan's size, and so the
// workspace a caller sizes, depends only on the call's arguments.
constexpr int32_t kTargetItems = 192;
constexpr int32_t kMinPartBlocks = 4;

// Four waves: fewer waves per barrier than 1024 threads (0.06 us less per
// decode launch of a 28-layer step, whose launches share one plan).
constexpr int kPlanThreads = 256;
constexpr int kSortLimit = 1024;  // larger batches keep submission order

__device__ __forceinline__ int blocks_of(int ctx, int block_size, int lb) {
  return (ctx + block_size - 1) >> lb;
}

__device__ __forceinline__ int part_blocks(int nb, int split_k, int pb_global) {
  if (split_k == 0) return pb_global;
  const int k = min(split_k, max(nb, 1));
  return max(1, (nb + k - 1) / k);
}

__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(
    const int32_t* __restrict__ context_lens, int num_seqs, int num_kv_heads, int block_size,
    int lb, int width, int split_k, int target, int min_pb, int max_items,
    PlanItem* __restrict__ plan, int32_t* __restrict__ counters, int num_counters) {
  __shared__ int s_ctx[kMaxPlanSeqs];
  __shared__ int s_order[kMaxPlanSeqs];  // rank -> sequence
  __shared__ int s_first[kMaxPlanSeqs];  // rank -> first item index
  __shared__ int s_scan[kPlanThreads];
  __shared__ int s_size[kSortLimit];  // slot -> blocks (size-ordered dispatch)
  __shared__ int s_rank[kSortLimit];  // slot -> plan position
  __shared__ int s_total_blocks;
  __shared__ int s_total_items;
  const int tid = threadIdx.x;
  const int max_ctx = width * block_size;

  // Arrival counters of the decode launch that follows (when given): zero
  // them here, so a caller whose counter memory is shared or reused needs
  // no separate clear.
  if (counters != nullptr)
    for (int i = tid; i < num_counters; i += kPlanThreads) counters[i] = 0;
  if (tid == 0) {
    s_total_blocks = 0;
    s_total_items = 0;
  }
  __syncthreads();
  int local = 0;
  for (int r = tid; r < num_seqs; r += kPlanThreads) {
    const int c = min(max(context_lens[r], 0), max_ctx);
    s_ctx[r] = c;
    local += blocks_of(c, block_size, lb);
  }
  atomicAdd(&s_total_blocks, local);
  __syncthreads();
  int pb_global = 1;
  if (split_k == 0) {
    const int64_t want = static_cast<int64_t>(s_total_blocks) * num_kv_heads;
    pb_global = max(min_pb, max(1, static_cast<int>((want + target - 1) / target)));
  }

  // Rank sequences by block count, longest first (ties keep batch order).
  const bool sort = num_seqs <= kSortLimit;
  for (int r = tid; r < num_seqs; r += kPlanThreads) {
    int rank = r;
    if (sort) {
      const int nb = blocks_of(s_ctx[r], block_size, lb);
      rank = 0;
      for (int s = 0; s < num_seqs; ++s) {
        const int ns = blocks_of(s_ctx[s], block_size, lb);
        rank += (ns > nb) || (ns == nb && s < r);
      }
    }
    s_order[rank] = r;
  }
  __syncthreads();

  // Exclusive scan of partition counts in rank order: each thread owns a run
  // of consecutive ranks, then the per-thread sums are scanned in LDS.
  const int per = (num_seqs + kPlanThreads - 1) / kPlanThreads;
  const int k0 = tid * per;
  const int k1 = min(num_seqs, k0 + per);
  int run = 0;
  for (int k = k0; k < k1; ++k) {
    const int nb = blocks_of(s_ctx[s_order[k]], block_size, lb);
    run += max(1, (nb + part_blocks(nb, split_k, pb_global) - 1) /
                      part_blocks(nb, split_k, pb_global));
  }
  s_scan[tid] = run;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int v = tid >= off ? s_scan[tid - off] : 0;
    __syncthreads();
    s_scan[tid] += v;
    __syncthreads();
  }
  int first = s_scan[tid] - run;
  for (int k = k0; k < k1; ++k) {
    s_first[k] = first;
    const int nb = blocks_of(s_ctx[s_order[k]], block_size, lb);
    const int pb = part_blocks(nb, split_k, pb_global);
    first += max(1, (nb + pb - 1) / pb);
  }
  if (tid == kPlanThreads - 1) s_total_items = s_scan[tid];
  __syncthreads();

  // Emit the items, then mark the rest of the launch's slots unused. Slots
  // (first_item + part) number a sequence's partitions consecutively; the
  // plan position a workgroup reads is the item's rank by size, largest
  // first (ties in slot order), so every workgroup of the first round is
  // one of the largest and the launch ends with the smallest items.
  const int total_items = min(s_total_items, max_items);
  const bool by_size = total_items <= kSortLimit;
  if (by_size) {
    for (int k = tid; k < num_seqs; k += kPlanThreads) {
      const int nb = blocks_of(s_ctx[s_order[k]], block_size, lb);
      const int pb = part_blocks(nb, split_k, pb_global);
      const int np = max(1, (nb + pb - 1) / pb);
      for (int p = 0; p < np && s_first[k] + p < max_items; ++p)
        s_size[s_first[k] + p] = min(nb, (p + 1) * pb) - p * pb;
    }
    __syncthreads();
    // One thread per slot: its rank among all items (every thread reads the
    // same size at a time, an LDS broadcast).
    for (int i = tid; i < total_items; i += kPlanThreads) {
      const int sz = s_size[i];
      int r = 0;
      for (int j = 0; j < total_items; ++j) {
        const int o = s_size[j];
        r += (o > sz) || (o == sz && j < i);
      }
      s_rank[i] = r;
    }
    __syncthreads();
  }
  for (int k = tid; k < num_seqs; k += kPlanThreads) {
    const int r = s_order[k];
    const int c = s_ctx[r];
    const int nb = blocks_of(c, block_size, lb);
    const int pb = part_blocks(nb, split_k, pb_global);
    const int np = max(1, (nb + pb - 1) / pb);
    const int f = s_first[k];
    for (int p = 0; p < np && f + p < max_items; ++p) {
      PlanItem it;
      it.seq = r;
      it.blk_begin = p * pb;
      it.blk_end = min(nb, (p + 1) * pb);
      it.nparts = np;
      it.first_item = f;
      it.ctx = c;
      it.part = p;
      it.unused = 0;
      plan[by_size ? s_rank[f + p] : f + p] = it;
    }
  }
  for (int i = s_total_items + tid; i < max_items; i += kPlanThreads) {
    PlanItem it{};
    it.seq = -1;
    plan[i] = it;
  }
}

}  // namespace

int32_t decode_max_items(int32_t num_seqs, int32_t num_kv_heads, int32_t split_k) {
  if (split_k > 0) return num_seqs * split_k;
  return (kTargetItems + num_kv_heads - 1) / num_kv_heads + num_seqs;
}

int64_t decode_plan_bytes(int32_t num_seqs, int32_t num_kv_heads, int32_t split_k) {
  return static_cast<int64_t>(decode_max_items(num_seqs, num_kv_heads, split_k)) *
         static_cast<int64_t>(sizeof(PlanItem));
}

int32_t launch_decode_plan(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                           int32_t block_size, int32_t block_table_width, int32_t split_k,
                           PlanItem* plan, int32_t* counters, hipStream_t stream) {
  decode_plan_kernel<<<1, kPlanThreads, 0, stream>>>(
      context_lens, num_seqs, num_kv_heads, block_size, ilog2(block_size), block_table_width,
      split_k, kTargetItems, kMinPartBlocks,
      decode_max_items(num_seqs, num_kv_heads, split_k), plan, counters,
      counters != nullptr ? num_seqs * num_kv_heads : 0);
  return check_launch("decode plan");
}

}  // namespace mi

extern "C" int64_t mi_decode_plan_bytes(int32_t num_seqs, int32_t num_kv_heads,
                                        int32_t split_k) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || split_k < 0) return 0;
  return mi::decode_plan_bytes(num_seqs, num_kv_heads, split_k);
}

extern "C" int32_t mi_decode_plan(const int32_t* context_lens, int32_t num_seqs,
                                  int32_t num_kv_heads, int32_t block_size,
                                  int32_t block_table_width, int32_t split_k, void* plan,
                                  int64_t plan_bytes, void* stream) {
  using namespace mi;
  clear_error();
  if (num_seqs < 0 || num_kv_heads <= 0 || split_k < 0 || block_table_width < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_decode_plan: invalid sizes");
  if (!is_pow2(block_size))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_decode_plan: block_size must be a power of two");
  if (num_seqs > kMaxPlanSeqs)
    return fail(MI_ERR_UNSUPPORTED, "mi_decode_plan: more than 4096 sequences");
  if (num_seqs == 0) return MI_OK;
  if (!context_lens || !plan)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_decode_plan: null pointer");
  if (plan_bytes < decode_plan_bytes(num_seqs, num_kv_heads, split_k) ||
      reinterpret_cast<uintptr_t>(plan) % 32 != 0)
    return fail(MI_ERR_WORKSPACE, "mi_decode_plan: plan buffer too small or misaligned");
  return launch_decode_plan(context_lens, num_seqs, num_kv_heads, block_size,
                            block_table_width, split_k, static_cast<PlanItem*>(plan), nullptr,
                            static_cast<hipStream_t>(stream));
}
