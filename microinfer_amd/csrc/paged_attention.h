// Internal declarations shared by the paged-attention translation units.
#pragma once

#include "mi_common.h"

namespace mi {

// One decode work item: blocks [blk_begin, blk_end) of sequence `seq`, which
// is split into `nparts` partitions numbered first_item .. first_item+nparts-1
// (this one is partition `part`). seq < 0 marks an unused slot.
struct alignas(32) PlanItem {
  int32_t seq, blk_begin, blk_end, nparts, first_item, ctx, part, unused;
};

// One prefill work item: query row block `qblock` (rows qblock * BM ..) of
// request `req`, key tiles [tile_begin, tile_end). A (row block, KV head)
// whose keys are split runs as `nparts` items, partition `part` publishing
// its partial in slot `slot + part` and arriving at counter `counter`.
struct alignas(32) PrefillItem {
  int32_t req, qblock, tile_begin, tile_end, part, nparts, slot, counter;
};

// Arguments of the vector (non-MFMA) paged attention kernels. Strides are in
// elements; head_dim is contiguous everywhere.
struct AttnArgs {
  const void* q;
  int64_t q_ts, q_hs;
  const void* kc;
  const void* vc;
  int64_t c_bs, c_ts, c_hs;
  const int32_t* tables;
  int64_t t_stride;
  int32_t t_width;
  const int32_t* ctx;   // decode: context length per sequence
  const int32_t* cu_q;  // varlen: query row offsets [R + 1]
  const int32_t* cu_k;  // varlen: context offsets [R + 1]
  void* out;
  int64_t o_ts, o_hs;
  float* ws_acc;  // split partials: [items, Hkv, G, D] unnormalised sums
  float* ws_ml;   // split partials: [items, Hkv, G, 2] (log2-domain max, sum)
  int32_t* counters;  // [num_seqs * Hkv] arrival counts; zero on entry and exit
  const PlanItem* plan;  // decode: [max_items] work items
  // MFMA prefill with a plan (optional): [max_entries] items, the first
  // *prefill_count of them used; partials in ws_acc / ws_ml, arrivals in
  // counters.
  const PrefillItem* prefill_plan;
  const int32_t* prefill_count;
  int32_t max_entries;
  // Decode with fused append (optional): row s of new_k/new_v is written to
  // position ctx_s - 1 of sequence s and attended to from registers.
  const void* new_k;
  const void* new_v;
  int64_t nk_ts, nk_hs, nv_ts, nv_hs;
  int32_t num_seqs;  // decode: sequences; varlen: requests
  int32_t num_rows;  // varlen: query rows
  int32_t max_q;     // varlen: no request has more query rows (launch shape)
  int32_t num_kv_heads, group, head_dim, block_size, log2_block, num_blocks;
  int32_t split_k;          // 0 = adaptive partitions
  int32_t max_items;        // grid.x of the decode launch
  float scale_log2;         // softmax scale * log2(e)
  int32_t varlen;
};

// Launch the vector kernel (decode or varlen mode) plus, for decode, the
// split merge. Returns an MI_* status.
int32_t launch_paged_attention_vector(const AttnArgs& args, int32_t dtype,
                                      hipStream_t stream);

// MFMA varlen (prefill) kernel (paged_prefill_mfma.hip): whether it takes
// this call, and its launch.
bool prefill_mfma_supported(const AttnArgs& args, int32_t dtype);
int32_t launch_prefill_mfma(const AttnArgs& args, int32_t dtype, hipStream_t stream);
// Workspace of a planned MFMA prefill launch (0: the call cannot be planned),
// and the planned launch itself: the plan kernel, then the attention kernel.
// `workspace` is 256-byte aligned and at least prefill_workspace_bytes()
// long; it needs no initialisation.
int64_t prefill_workspace_bytes(int32_t num_rows, int32_t num_seqs, int32_t group,
                                int32_t num_kv_heads);
int32_t prefill_counters(int32_t num_kv_heads);
// The plan kernel alone (its result serves every planned launch with the
// same cu_seqlens and sizes until they change).
int32_t launch_prefill_plan(const AttnArgs& args, void* workspace, hipStream_t stream);
int32_t launch_prefill_mfma_planned(AttnArgs args, int32_t dtype, void* workspace,
                                    bool plan_ready, hipStream_t stream);

// MFMA decode kernel (paged_decode_mfma.hip): 16-bit caches, head_dim 128,
// up to 16 query heads per KV head, block size >= 16, paged.
bool decode_mfma_supported(const AttnArgs& args, int32_t dtype);
int32_t launch_decode_mfma(const AttnArgs& args, int32_t dtype, hipStream_t stream);

// Upper bound on decode work items for a launch (grid.x / Hkv).
int32_t decode_max_items(int32_t num_seqs, int32_t num_kv_heads, int32_t split_k);

// Plan size and launch (decode_plan.hip). The plan has decode_max_items()
// entries; unused ones carry seq = -1.
int64_t decode_plan_bytes(int32_t num_seqs, int32_t num_kv_heads, int32_t split_k);
// counters (optional): the (sequence, KV head) arrival counters of the
// decode launch that follows, zeroed by the plan kernel.
int32_t launch_decode_plan(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                           int32_t block_size, int32_t block_table_width, int32_t split_k,
                           PlanItem* plan, int32_t* counters, hipStream_t stream);

constexpr int32_t kMaxPlanSeqs = 4096;

// The step's new K/V rows for the fused append (all null: no append).
struct NewRows {
  const void* keys = nullptr;
  int64_t k_ts = 0, k_hs = 0;
  const void* values = nullptr;
  int64_t v_ts = 0, v_hs = 0;
};

// Validated decode (paged_attention.hip), shared by the C entry points:
// mi_paged_decode, mi_paged_decode_append and the allocation-free variant.
int32_t paged_decode(
    const void* query, int64_t q_token_stride, int64_t q_head_stride, const void* key_cache,
    const void* value_cache, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, const int32_t* block_tables, int64_t block_table_stride,
    int32_t block_table_width, const int32_t* context_lens, void* out,
    int64_t out_token_stride, int64_t out_head_stride, void* workspace,
    int64_t workspace_bytes, int32_t* counters, const void* plan, int64_t plan_bytes,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, int32_t split_k, float scale, int32_t dtype,
    const NewRows& rows, void* stream);

}  // namespace mi
