// C entry points for paged decode and paged varlen (prefill) attention.
#include <cmath>

#include "paged_attention.h"

namespace mi {

int32_t launch_vector_f32(const AttnArgs& a, hipStream_t stream);
int32_t launch_vector_f16(const AttnArgs& a, hipStream_t stream);
int32_t launch_vector_bf16(const AttnArgs& a, hipStream_t stream);

namespace {

constexpr float kLog2e = 1.4426950408889634f;

int32_t dispatch_vector(const AttnArgs& a, int32_t dtype, hipStream_t stream) {
  switch (dtype) {
    case MI_DTYPE_F32: return launch_vector_f32(a, stream);
    case MI_DTYPE_F16: return launch_vector_f16(a, stream);
    case MI_DTYPE_BF16: return launch_vector_bf16(a, stream);
    default: return fail(MI_ERR_INVALID_ARGUMENT, "paged attention: bad dtype");
  }
}

// Common shape/stride validation. `vec` elements must stay 16-byte loadable.
int32_t check_common(const char* who, int32_t dtype, int32_t num_q_heads,
                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     int32_t num_blocks, int32_t table_width) {
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, std::string(who) + ": bad dtype");
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(MI_ERR_INVALID_ARGUMENT,
                std::string(who) + ": Hq must be a positive multiple of Hkv");
  if (!is_pow2(head_dim) || head_dim > 256)
    return fail(MI_ERR_UNSUPPORTED,
                std::string(who) + ": head_dim must be a power of two <= 256");
  if (!is_pow2(block_size))
    return fail(MI_ERR_INVALID_ARGUMENT,
                std::string(who) + ": block_size must be a power of two");
  if (num_blocks <= 0 || table_width < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, std::string(who) + ": invalid pool or table size");
  return MI_OK;
}

bool aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

// Workspace layout: [plan (256-byte aligned)][acc partials][(m, l) partials].
int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

int64_t partial_floats(int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                       int32_t head_dim, int32_t split_k) {
  if (split_k == 1) return 0;  // one partition per sequence: no partials
  const int64_t items = decode_max_items(num_seqs, num_kv_heads, split_k);
  const int64_t group = num_q_heads / num_kv_heads;
  return items * num_kv_heads * group * (head_dim + 2);
}

}  // namespace
}  // namespace mi

extern "C" int64_t mi_paged_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                   int32_t num_kv_heads, int32_t head_dim,
                                                   int32_t split_k) {
  using namespace mi;
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || head_dim <= 0 || split_k < 0)
    return 0;
  return round_up(decode_plan_bytes(num_seqs, num_kv_heads, split_k), 256) +
         partial_floats(num_seqs, num_q_heads, num_kv_heads, head_dim, split_k) *
             static_cast<int64_t>(sizeof(float));
}

namespace mi {

int32_t paged_decode(
    const void* query, int64_t q_token_stride, int64_t q_head_stride, const void* key_cache,
    const void* value_cache, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, const int32_t* block_tables, int64_t block_table_stride,
    int32_t block_table_width, const int32_t* context_lens, void* out,
    int64_t out_token_stride, int64_t out_head_stride, void* workspace,
    int64_t workspace_bytes, int32_t* counters, const void* plan, int64_t plan_bytes,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, int32_t split_k, float scale, int32_t dtype,
    const NewRows& rows, void* stream) {
  int32_t st = check_common("mi_paged_decode", dtype, num_q_heads, num_kv_heads, head_dim,
                            block_size, num_blocks, block_table_width);
  if (st != MI_OK) return st;
  if (num_seqs < 0 || split_k < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode: negative num_seqs or split_k");
  if (num_seqs == 0) return MI_OK;
  if (num_seqs > kMaxPlanSeqs)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode: more than 4096 sequences");
  if (!query || !key_cache || !value_cache || !block_tables || !context_lens || !out)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode: null pointer");
  const int64_t es = static_cast<int64_t>(dtype_size(dtype));
  const int64_t vec = std::min<int64_t>(head_dim, 16 / es);
  const int64_t vb = vec * es;
  if (!aligned(query, vb) || !aligned(key_cache, vb) || !aligned(value_cache, vb) ||
      !aligned(out, vb) || q_token_stride % vec || q_head_stride % vec ||
      cache_block_stride % vec || cache_token_stride % vec || cache_head_stride % vec ||
      out_token_stride % vec || out_head_stride % vec)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode: misaligned pointers or strides");
  if ((rows.keys == nullptr) != (rows.values == nullptr))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_append: null new keys or values");
  if (rows.keys != nullptr &&
      (!aligned(rows.keys, vb) || !aligned(rows.values, vb) || rows.k_ts % vec ||
       rows.k_hs % vec || rows.v_ts % vec || rows.v_hs % vec))
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_paged_decode_append: misaligned new-row pointers or strides");
  const int64_t need = mi_paged_decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads,
                                                       head_dim, split_k);
  if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 256))
    return fail(MI_ERR_WORKSPACE, "mi_paged_decode: workspace needs " +
                                      std::to_string(need) + " bytes (256-byte aligned)");
  const int64_t partials =
      partial_floats(num_seqs, num_q_heads, num_kv_heads, head_dim, split_k);
  if (partials > 0 && counters == nullptr)
    return fail(MI_ERR_WORKSPACE, "mi_paged_decode: split partitions need zeroed counters");
  if (plan != nullptr &&
      (!aligned(plan, 32) || plan_bytes < decode_plan_bytes(num_seqs, num_kv_heads, split_k)))
    return fail(MI_ERR_INVALID_ARGUMENT,
                "mi_paged_decode: plan must be 32-byte aligned and sized by "
                "mi_decode_plan_bytes for this call");

  AttnArgs a{};
  a.q = query;
  a.q_ts = q_token_stride;
  a.q_hs = q_head_stride;
  a.kc = key_cache;
  a.vc = value_cache;
  a.c_bs = cache_block_stride;
  a.c_ts = cache_token_stride;
  a.c_hs = cache_head_stride;
  a.tables = block_tables;
  a.t_stride = block_table_stride;
  a.t_width = block_table_width;
  a.ctx = context_lens;
  a.out = out;
  a.o_ts = out_token_stride;
  a.o_hs = out_head_stride;
  a.num_seqs = num_seqs;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.head_dim = head_dim;
  a.block_size = block_size;
  a.log2_block = ilog2(block_size);
  a.num_blocks = num_blocks;
  a.split_k = split_k;
  a.max_items = decode_max_items(num_seqs, num_kv_heads, split_k);
  a.scale_log2 = scale * kLog2e;
  a.varlen = 0;
  a.new_k = rows.keys;
  a.nk_ts = rows.k_ts;
  a.nk_hs = rows.k_hs;
  a.new_v = rows.values;
  a.nv_ts = rows.v_ts;
  a.nv_hs = rows.v_hs;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int64_t plan_region = round_up(decode_plan_bytes(num_seqs, num_kv_heads, split_k), 256);
  if (plan == nullptr) {
    // The plan kernel also zeroes the counters this launch uses.
    PlanItem* own = reinterpret_cast<PlanItem*>(ws);
    st = launch_decode_plan(context_lens, num_seqs, num_kv_heads, block_size,
                            block_table_width, split_k, own, partials > 0 ? counters : nullptr,
                            s);
    if (st != MI_OK) return st;
    a.plan = own;
  } else {
    a.plan = static_cast<const PlanItem*>(plan);
  }
  if (partials > 0) {
    const int64_t acc_floats =
        static_cast<int64_t>(a.max_items) * num_kv_heads * a.group * head_dim;
    a.ws_acc = reinterpret_cast<float*>(ws + plan_region);
    a.ws_ml = a.ws_acc + acc_floats;
    a.counters = counters;
  }
  if (decode_mfma_supported(a, dtype)) return launch_decode_mfma(a, dtype, s);
  return dispatch_vector(a, dtype, s);
}

}  // namespace mi

extern "C" int32_t mi_paged_decode(
    const void* query, int64_t q_token_stride, int64_t q_head_stride, const void* key_cache,
    const void* value_cache, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, const int32_t* block_tables, int64_t block_table_stride,
    int32_t block_table_width, const int32_t* context_lens, void* out,
    int64_t out_token_stride, int64_t out_head_stride, void* workspace,
    int64_t workspace_bytes, int32_t* counters, const void* plan, int64_t plan_bytes,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, int32_t split_k, float scale, int32_t dtype,
    void* stream) {
  mi::clear_error();
  return mi::paged_decode(query, q_token_stride, q_head_stride, key_cache, value_cache,
                          cache_block_stride, cache_token_stride, cache_head_stride,
                          block_tables, block_table_stride, block_table_width, context_lens,
                          out, out_token_stride, out_head_stride, workspace, workspace_bytes,
                          counters, plan, plan_bytes, num_seqs, num_q_heads, num_kv_heads,
                          head_dim, block_size, num_blocks, split_k, scale, dtype,
                          mi::NewRows{}, stream);
}

extern "C" int32_t mi_paged_decode_append(
    const void* new_keys, int64_t nk_token_stride, int64_t nk_head_stride,
    const void* new_values, int64_t nv_token_stride, int64_t nv_head_stride,
    const void* query, int64_t q_token_stride, int64_t q_head_stride, void* key_cache,
    void* value_cache, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, const int32_t* block_tables, int64_t block_table_stride,
    int32_t block_table_width, const int32_t* context_lens, void* out,
    int64_t out_token_stride, int64_t out_head_stride, void* workspace,
    int64_t workspace_bytes, int32_t* counters, const void* plan, int64_t plan_bytes,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, int32_t split_k, float scale, int32_t dtype,
    void* stream) {
  mi::clear_error();
  if (new_keys == nullptr || new_values == nullptr)
    return mi::fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_decode_append: null new keys or values");
  mi::NewRows rows;
  rows.keys = new_keys;
  rows.k_ts = nk_token_stride;
  rows.k_hs = nk_head_stride;
  rows.values = new_values;
  rows.v_ts = nv_token_stride;
  rows.v_hs = nv_head_stride;
  return mi::paged_decode(query, q_token_stride, q_head_stride, key_cache, value_cache,
                          cache_block_stride, cache_token_stride, cache_head_stride,
                          block_tables, block_table_stride, block_table_width, context_lens,
                          out, out_token_stride, out_head_stride, workspace, workspace_bytes,
                          counters, plan, plan_bytes, num_seqs, num_q_heads, num_kv_heads,
                          head_dim, block_size, num_blocks, split_k, scale, dtype, rows,
                          stream);
}

namespace {
int32_t paged_prefill(
    const char* name, const void* query, int64_t q_token_stride, int64_t q_head_stride,
    const void* key_cache, const void* value_cache, int64_t cache_block_stride,
    int64_t cache_token_stride, int64_t cache_head_stride, const int32_t* cu_seqlens_q,
    const int32_t* cu_seqlens_k, const int32_t* block_tables, int64_t block_table_stride,
    int32_t block_table_width, void* out, int64_t out_token_stride, int64_t out_head_stride,
    int32_t num_tokens, int32_t num_requests, int32_t max_seqlen_q, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t num_blocks, float scale,
    int32_t dtype, void* workspace, int64_t workspace_bytes, int32_t flags, void* stream) {
  using namespace mi;
  clear_error();
  const std::string fn(name);
  if (flags & ~MI_PREFILL_PLAN_READY) return fail(MI_ERR_INVALID_ARGUMENT, fn + ": unknown flags");
  int32_t st = check_common(name, dtype, num_q_heads, num_kv_heads, head_dim,
                            block_size, num_blocks, block_table_width);
  if (st != MI_OK) return st;
  if (num_tokens < 0 || num_requests < 0 || max_seqlen_q < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, fn + ": negative sizes");
  if (num_tokens == 0) return MI_OK;
  if (num_requests == 0)
    return fail(MI_ERR_INVALID_ARGUMENT, fn + ": tokens without requests");
  if (max_seqlen_q == 0)
    return fail(MI_ERR_INVALID_ARGUMENT, fn + ": max_seqlen_q must be positive");
  // block_tables may be NULL: contiguous varlen K/V (see mi_attn.h).
  if (!query || !key_cache || !value_cache || !cu_seqlens_q || !cu_seqlens_k || !out)
    return fail(MI_ERR_INVALID_ARGUMENT, fn + ": null pointer");
  const int64_t es = static_cast<int64_t>(dtype_size(dtype));
  const int64_t vec = std::min<int64_t>(head_dim, 16 / es);
  const int64_t vb = vec * es;
  if (!aligned(query, vb) || !aligned(key_cache, vb) || !aligned(value_cache, vb) ||
      !aligned(out, vb) || q_token_stride % vec || q_head_stride % vec ||
      cache_block_stride % vec || cache_token_stride % vec || cache_head_stride % vec ||
      out_token_stride % vec || out_head_stride % vec)
    return fail(MI_ERR_INVALID_ARGUMENT, fn + ": misaligned pointers or strides");

  AttnArgs a{};
  a.q = query;
  a.q_ts = q_token_stride;
  a.q_hs = q_head_stride;
  a.kc = key_cache;
  a.vc = value_cache;
  a.c_bs = cache_block_stride;
  a.c_ts = cache_token_stride;
  a.c_hs = cache_head_stride;
  a.tables = block_tables;
  a.t_stride = block_table_stride;
  a.t_width = block_table_width;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.out = out;
  a.o_ts = out_token_stride;
  a.o_hs = out_head_stride;
  a.num_seqs = num_requests;
  a.num_rows = num_tokens;
  a.max_q = max_seqlen_q;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.head_dim = head_dim;
  a.block_size = block_size;
  a.log2_block = ilog2(block_size);
  a.num_blocks = num_blocks;
  a.scale_log2 = scale * kLog2e;
  a.varlen = 1;
  // bf16/f16 with head_dim 128 and GQA groups 1, 2, 4 run on MFMA (planned
  // when a workspace is given); every other supported shape on the vector
  // kernel.
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (prefill_mfma_supported(a, dtype)) {
    if (workspace == nullptr) return launch_prefill_mfma(a, dtype, s);
    const int64_t need = prefill_workspace_bytes(num_tokens, num_requests, a.group, num_kv_heads);
    if (need == 0) return launch_prefill_mfma(a, dtype, s);  // too many requests to plan
    if (workspace_bytes < need || !aligned(workspace, 256))
      return fail(MI_ERR_WORKSPACE, fn + ": workspace needs " + std::to_string(need) +
                                        " bytes, 256-byte aligned");
    return launch_prefill_mfma_planned(a, dtype, workspace, (flags & MI_PREFILL_PLAN_READY) != 0,
                                       s);
  }
  return dispatch_vector(a, dtype, s);
}
}  // namespace

extern "C" int32_t mi_paged_prefill(
    const void* query, int64_t q_token_stride, int64_t q_head_stride, const void* key_cache,
    const void* value_cache, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
    const int32_t* block_tables, int64_t block_table_stride, int32_t block_table_width,
    void* out, int64_t out_token_stride, int64_t out_head_stride, int32_t num_tokens,
    int32_t num_requests, int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int32_t num_blocks, float scale, int32_t dtype,
    void* stream) {
  return paged_prefill("mi_paged_prefill", query, q_token_stride, q_head_stride, key_cache,
                       value_cache, cache_block_stride, cache_token_stride, cache_head_stride,
                       cu_seqlens_q, cu_seqlens_k, block_tables, block_table_stride,
                       block_table_width, out, out_token_stride, out_head_stride, num_tokens,
                       num_requests, max_seqlen_q, num_q_heads, num_kv_heads, head_dim,
                       block_size, num_blocks, scale, dtype, nullptr, 0, 0, stream);
}

extern "C" int64_t mi_paged_prefill_workspace_bytes(int32_t num_tokens, int32_t num_requests,
                                                    int32_t num_q_heads, int32_t num_kv_heads,
                                                    int32_t head_dim, int32_t dtype) {
  if ((dtype != MI_DTYPE_BF16 && dtype != MI_DTYPE_F16) || head_dim != 128 ||
      num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return 0;
  return mi::prefill_workspace_bytes(num_tokens, num_requests, num_q_heads / num_kv_heads,
                                     num_kv_heads);
}

extern "C" int32_t mi_paged_prefill_planned(
    const void* query, int64_t q_token_stride, int64_t q_head_stride, const void* key_cache,
    const void* value_cache, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
    const int32_t* block_tables, int64_t block_table_stride, int32_t block_table_width,
    void* out, int64_t out_token_stride, int64_t out_head_stride, int32_t num_tokens,
    int32_t num_requests, int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int32_t num_blocks, float scale, int32_t dtype,
    void* workspace, int64_t workspace_bytes, int32_t flags, void* stream) {
  return paged_prefill("mi_paged_prefill_planned", query, q_token_stride, q_head_stride,
                       key_cache, value_cache, cache_block_stride, cache_token_stride,
                       cache_head_stride, cu_seqlens_q, cu_seqlens_k, block_tables,
                       block_table_stride, block_table_width, out, out_token_stride,
                       out_head_stride, num_tokens, num_requests, max_seqlen_q, num_q_heads,
                       num_kv_heads, head_dim, block_size, num_blocks, scale, dtype, workspace,
                       workspace_bytes, flags, stream);
}

extern "C" int32_t mi_paged_prefill_plan(const int32_t* cu_seqlens_q,
                                         const int32_t* cu_seqlens_k, int32_t num_tokens,
                                         int32_t num_requests, int32_t num_q_heads,
                                         int32_t num_kv_heads, int32_t head_dim, int32_t paged,
                                         int32_t block_size, int32_t block_table_width,
                                         int32_t num_blocks, int32_t dtype, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  using namespace mi;
  clear_error();
  const int64_t need = mi_paged_prefill_workspace_bytes(num_tokens, num_requests, num_q_heads,
                                                        num_kv_heads, head_dim, dtype);
  if (need == 0)
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_prefill_plan: these sizes take no plan");
  if (!cu_seqlens_q || !cu_seqlens_k)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_prefill_plan: null pointer");
  if (paged && (!is_pow2(block_size) || block_table_width < 0))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_prefill_plan: invalid block size or width");
  if (!paged && num_blocks < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_paged_prefill_plan: negative K/V rows");
  if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 256))
    return fail(MI_ERR_WORKSPACE, "mi_paged_prefill_plan: workspace needs " +
                                      std::to_string(need) + " bytes, 256-byte aligned");
  AttnArgs a{};
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  // Only the null-ness of the tables matters to the plan.
  a.tables = paged ? cu_seqlens_q : nullptr;
  a.t_width = block_table_width;
  a.block_size = paged ? block_size : 1;
  a.num_blocks = num_blocks;
  a.num_seqs = num_requests;
  a.num_rows = num_tokens;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  return launch_prefill_plan(a, workspace, static_cast<hipStream_t>(stream));
}
