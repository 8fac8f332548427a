/*
 * mi_attn.h -- C ABI of the MI355X (gfx950) paged-KV attention library.
 *
 * libmi_attn.so exports plain C entry points: device pointers, element
 * strides, sizes, a dtype code and a hipStream_t passed as void*. No torch or
 * C++ types cross this boundary. Every entry point
 *   - launches asynchronously on `stream` and never synchronises,
 *   - never allocates or frees device memory (callers pass any workspace),
 *   - issues no memset/memcpy nodes, so it is safe inside hipGraph capture,
 *   - returns MI_OK (0) or a non-zero status; mi_last_error() then describes
 *     the failure (thread-local, valid until the next call on that thread).
 *
 * Cache layout: a layer's K (or V) cache is addressed as logical
 * [num_blocks, block_size, num_kv_heads, head_dim] through three element
 * strides (block, token, head); head_dim is contiguous. Both the reference's
 * contiguous [N, B, Hkv, D] layout and the head-major [N, Hkv, B, D] layout of
 * microinfer_amd.worker.kv_cache.KVCache are accepted.
 *
 * Index tensors (block tables, context lengths, cu_seqlens, slots) are int32
 * device arrays unless a parameter says otherwise. Block ids outside
 * [0, num_blocks) and slots < 0 are never dereferenced: such table entries are
 * masked out of attention and such slots are skipped by the append.
 */
#ifndef MI_ATTN_H_
#define MI_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
enum {
  MI_DTYPE_F32 = 0,
  MI_DTYPE_F16 = 1,
  MI_DTYPE_BF16 = 2,
};

/* Status codes. */
enum {
  MI_OK = 0,
  MI_ERR_INVALID_ARGUMENT = 1, /* shapes, strides, alignment, dtype */
  MI_ERR_UNSUPPORTED = 2,      /* valid request this build has no kernel for */
  MI_ERR_WORKSPACE = 3,        /* workspace missing or too small */
  MI_ERR_HIP = 4,              /* launch or runtime error reported by HIP */
};

/* Description of the last failure on the calling thread ("" after success). */
const char* mi_last_error(void);

/* ABI version of this library (major * 100 + minor). 101: mi_tune_decode and
 * its plan/workspace knobs were removed (workspace and plan sizes depend only
 * on the call's arguments). 102: mi_paged_prefill_planned,
 * mi_paged_prefill_plan and mi_paged_prefill_workspace_bytes added. */
int32_t mi_abi_version(void);

/*
 * KV append: for every token t and KV head h,
 *   key_cache[blk, off, h, :] = keys[t, h, :]   (and the same for values)
 * with (blk, off) = (slot / block_size, slot % block_size).
 *
 * Replaces store_kv / _store_kv_kernel (microinfer/worker/triton_kv_store.py:45-78)
 * plus the per-step slot div/mod of AttentionMetadata.slot_indices
 * (microinfer/layer/metadata.py:75-84), both called from
 * LayerKVCache.write_fast (microinfer/worker/kv_cache.py:52-79).
 *
 * index0/index1: if index1 is NULL, index0 holds slots (slot < 0 = padding,
 * skipped, as in write_checked kv_cache.py:42). Otherwise index0 holds block
 * ids and index1 in-block offsets (write_fast's precomputed form).
 * index_is_int64 selects int64 (1) or int32 (0) indices.
 * Slots whose block lies outside [0, num_blocks) are skipped.
 */
int32_t mi_kv_append(const void* keys, int64_t key_token_stride, int64_t key_head_stride,
                     const void* values, int64_t value_token_stride,
                     int64_t value_head_stride, void* key_cache, void* value_cache,
                     int64_t cache_block_stride, int64_t cache_token_stride,
                     int64_t cache_head_stride, const void* index0, const void* index1,
                     int32_t index_is_int64, int32_t num_tokens, int32_t num_kv_heads,
                     int32_t head_dim, int32_t block_size, int32_t num_blocks,
                     int32_t dtype, void* stream);

/*
 * Paged decode attention: one query row per sequence,
 *   out[s, h, :] = softmax_k(scale * q[s, h, :] . K[s, k, h / G, :]) V[s, k, h / G, :]
 * over the context_lens[s] cached tokens of sequence s, G = Hq / Hkv.
 *
 * Replaces triton_paged_decode + _paged_decode_kernel + _paged_decode_reduce_kernel
 * (microinfer/layer/triton_paged_attention.py:352-457, :40-131, :236-257), called
 * from paged_attention_meta (microinfer/layer/paged_attention.py:232-246).
 *
 * One work item = (sequence, KV head, context partition); all G query heads of
 * the KV head share it, so each K/V row is read from HBM once. split_k = 0
 * picks partitions on the device from context_lens (graph-replay safe);
 * split_k > 0 forces at most split_k partitions per sequence. Partitions
 * of one (sequence, KV head) are merged inside the same launch: each
 * publishes its online-softmax state to `workspace` and bumps an arrival
 * counter; the last arrival merges all of them and writes the output.
 *
 * workspace: device buffer of at least mi_paged_decode_workspace_bytes(...)
 * bytes, 256-byte aligned; no initialisation needed. It holds the split
 * partials and, when `plan` is NULL, the plan this call computes first.
 * counters: int32 device array of at least num_seqs * num_kv_heads entries
 * that must be ZERO on entry; every call leaves it zero again, so one array
 * can serve all later calls on the same stream. Calls that run concurrently
 * (different streams) need separate counters and workspaces.
 * plan: NULL, or a plan from mi_decode_plan for this step (see there) in a
 * buffer of plan_bytes >= mi_decode_plan_bytes(...). When plan is NULL the
 * call computes its plan first, and that launch also zeroes the counters.
 * Sequences with context_len 0 produce zeros.
 */
int64_t mi_paged_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                        int32_t num_kv_heads, int32_t head_dim,
                                        int32_t split_k);

/*
 * Decode partition plan: the list of (sequence, block range) work items that
 * mi_paged_decode runs, derived on the device from context_lens. All layers
 * of a step share one plan, so an engine computes it once per step and
 * passes it to every layer's mi_paged_decode (which otherwise computes it
 * into its workspace on every call). Sequences are ordered longest first, so
 * split sequences finish (and merge) while shorter items still stream.
 * plan: device buffer of at least mi_decode_plan_bytes(...) bytes; the
 * result is valid for calls with the same context_lens contents, num_seqs,
 * num_kv_heads, block_size, block_table_width and split_k. A plan that does
 * not match produces wrong attention but never reads out of bounds.
 * At most 4096 sequences.
 */
int64_t mi_decode_plan_bytes(int32_t num_seqs, int32_t num_kv_heads, int32_t split_k);

int32_t mi_decode_plan(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                       int32_t block_size, int32_t block_table_width, int32_t split_k,
                       void* plan, int64_t plan_bytes, void* stream);

int32_t mi_paged_decode(const void* query, int64_t q_token_stride, int64_t q_head_stride,
                        const void* key_cache, const void* value_cache,
                        int64_t cache_block_stride, int64_t cache_token_stride,
                        int64_t cache_head_stride, const int32_t* block_tables,
                        int64_t block_table_stride, int32_t block_table_width,
                        const int32_t* context_lens, void* out, int64_t out_token_stride,
                        int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                        int32_t* counters, const void* plan, int64_t plan_bytes,
                        int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                        int32_t head_dim,
                        int32_t block_size, int32_t num_blocks, int32_t split_k,
                        float scale, int32_t dtype, void* stream);

/*
 * Decode step of one layer with the KV append fused in: for every sequence s
 * with context_lens[s] = c >= 1, row s of new_keys / new_values ([num_seqs,
 * Hkv, D], token and head strides in elements) is written to cache position
 * c - 1 (block block_tables[s][(c-1)/B], offset (c-1)%B), and the attention
 * over positions 0..c-1 includes it. Same result as mi_kv_append with
 * slot_mapping[s] = block_tables[s][(c-1)/B]*B + (c-1)%B followed by
 * mi_paged_decode, in one launch, with the new row read once.
 *
 * Replaces, for decode steps, CachedAttention.forward's append-then-attend
 * (microinfer/layer/cached_attention.py:76-85: LayerKVCache.write_fast,
 * microinfer/worker/kv_cache.py:52-79, then paged_attention_meta); the runner
 * builds slot_mapping exactly this way (microinfer/runner.py:167-174).
 * A position whose block id is negative or >= num_blocks is neither written
 * nor attended (the append skips it and the attention masks it). Sequences
 * whose plan context differs from context_lens are not appended. The block
 * that receives a sequence's new row must not be read by another sequence of
 * the same call (its read would race with the write); the reference's block
 * manager guarantees this, as only full blocks are ever shared
 * (microinfer/engine/blockmanager.py:144-174). All other arguments and rules
 * are those of mi_paged_decode.
 */
int32_t mi_paged_decode_append(const void* new_keys, int64_t nk_token_stride,
                               int64_t nk_head_stride, const void* new_values,
                               int64_t nv_token_stride, int64_t nv_head_stride,
                               const void* query, int64_t q_token_stride,
                               int64_t q_head_stride, void* key_cache, void* value_cache,
                               int64_t cache_block_stride, int64_t cache_token_stride,
                               int64_t cache_head_stride, const int32_t* block_tables,
                               int64_t block_table_stride, int32_t block_table_width,
                               const int32_t* context_lens, void* out,
                               int64_t out_token_stride, int64_t out_head_stride,
                               void* workspace, int64_t workspace_bytes, int32_t* counters,
                               const void* plan, int64_t plan_bytes, int32_t num_seqs,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t block_size, int32_t num_blocks, int32_t split_k,
                               float scale, int32_t dtype, void* stream);

/*
 * Allocation-free variant of mi_paged_decode_append, for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It has no counterpart in the reference.
 *
 * Same arguments, rules and result as mi_paged_decode_append with
 * workspace/counters/plan omitted and plan = NULL: its plan, split partials
 * and arrival counters live in a static device array of the library
 * (32 MiB per GPU, held until the process ends). The call fails with
 * MI_ERR_WORKSPACE when mi_paged_decode_workspace_bytes(...) for its sizes
 * exceeds mi_paged_decode_noalloc_max_bytes(), and with MI_ERR_UNSUPPORTED
 * past 4096 sequences or 16 KV heads. No hipMalloc, hipFree or memset: the
 * plan launch zeroes the counters this call uses. Every call on one GPU
 * shares that GPU's array, so calls that may overlap on one GPU (different
 * streams, or host threads racing on one) race on it; serialise them.
 */
int64_t mi_paged_decode_noalloc_max_bytes(void);
int32_t mi_paged_decode_append_noalloc(
    const void* new_keys, int64_t nk_token_stride, int64_t nk_head_stride,
    const void* new_values, int64_t nv_token_stride, int64_t nv_head_stride,
    const void* query, int64_t q_token_stride, int64_t q_head_stride, void* key_cache,
    void* value_cache, int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t cache_head_stride, const int32_t* block_tables, int64_t block_table_stride,
    int32_t block_table_width, const int32_t* context_lens, void* out,
    int64_t out_token_stride, int64_t out_head_stride, int32_t num_seqs,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int32_t num_blocks, int32_t split_k, float scale, int32_t dtype, void* stream);

/*
 * Paged varlen (prefill / mixed) attention with a bottom-right causal mask:
 * request r owns query rows [cu_seqlens_q[r], cu_seqlens_q[r+1]) and context
 * c_r = cu_seqlens_k[r+1] - cu_seqlens_k[r]; its query row i sits at position
 * (c_r - q_len_r) + i and attends to cached positions 0..that position
 * (microinfer/layer/paged_attention.py:57-62).
 *
 * Replaces triton_paged_prefill + _paged_prefill_kernel
 * (microinfer/layer/triton_paged_attention.py:260-339, :134-233) and the
 * reference-path fallback of paged_attention_meta (paged_attention.py:277-293).
 * bf16/f16 with head_dim 128 run on the MFMA kernel; every other supported
 * shape (including f32) runs on the vector kernel. max_seqlen_q bounds the
 * query rows of any request (launch shape only).
 *
 * block_tables == NULL selects contiguous varlen K/V instead of a paged cache:
 * key_cache/value_cache are [sum c_r, Hkv, D] arrays (token stride
 * cache_token_stride, head stride cache_head_stride) and request r's keys are
 * rows cu_seqlens_k[r] .. cu_seqlens_k[r+1]-1; num_blocks then gives the
 * number of K/V rows (rows at or past it are never read). This serves the no-prefix
 * prefill that the reference routes to FlashAttention varlen or an SDPA loop
 * (microinfer/layer/cached_attention.py:17-55, :87-101).
 */
int32_t mi_paged_prefill(const void* query, int64_t q_token_stride, int64_t q_head_stride,
                         const void* key_cache, const void* value_cache,
                         int64_t cache_block_stride, int64_t cache_token_stride,
                         int64_t cache_head_stride, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_k, const int32_t* block_tables,
                         int64_t block_table_stride, int32_t block_table_width,
                         void* out, int64_t out_token_stride, int64_t out_head_stride,
                         int32_t num_tokens, int32_t num_requests, int32_t max_seqlen_q,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                         int32_t block_size, int32_t num_blocks, float scale,
                         int32_t dtype, void* stream);

/*
 * Workspace for mi_paged_prefill_planned: bytes for num_tokens query rows in
 * num_requests requests (256-byte aligned, no initialisation needed), or 0
 * when such a call takes no workspace (then pass NULL): dtype other than
 * bf16/f16, head_dim other than 128, Hq/Hkv not 1, 2 or 4, more than 4096
 * requests. The size depends only on these arguments.
 */
int64_t mi_paged_prefill_workspace_bytes(int32_t num_tokens, int32_t num_requests,
                                         int32_t num_q_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t dtype);

/*
 * mi_paged_prefill with a launch plan: the same arguments, results within
 * float rounding of it (partitions merge in a fixed order, so a call's
 * output does not depend on scheduling), plus a workspace of
 * mi_paged_prefill_workspace_bytes() (NULL when that is 0).
 *
 * A small plan kernel, launched on the same stream ahead of the attention
 * kernel, splits the key range of (query block, KV head) items with more
 * key tiles than about 3/4 of a CU's share of the launch into contiguous
 * partitions (their partials merged by the last one to finish) and orders
 * the launch largest item first, so one long request's blocks no longer
 * set the launch time. The reference splits only decode
 * (microinfer/layer/triton_paged_attention.py:342-349); its prefill grid is
 * one program per (request, query block, head) (:307-339).
 * Calls sharing one workspace must be stream-ordered.
 *
 * flags: 0, or MI_PREFILL_PLAN_READY when mi_paged_prefill_plan has already
 * written this call's plan into the workspace (same cu_seqlens contents,
 * num_tokens, num_requests, heads, paging, block_size, block_table_width and
 * num_blocks): the plan kernel is then skipped, so one plan serves every
 * layer of a step.
 */
#define MI_PREFILL_PLAN_READY 1
int32_t mi_paged_prefill_planned(const void* query, int64_t q_token_stride,
                                 int64_t q_head_stride, const void* key_cache,
                                 const void* value_cache, int64_t cache_block_stride,
                                 int64_t cache_token_stride, int64_t cache_head_stride,
                                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                 const int32_t* block_tables, int64_t block_table_stride,
                                 int32_t block_table_width, void* out,
                                 int64_t out_token_stride, int64_t out_head_stride,
                                 int32_t num_tokens, int32_t num_requests,
                                 int32_t max_seqlen_q, int32_t num_q_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                 int32_t num_blocks, float scale, int32_t dtype,
                                 void* workspace, int64_t workspace_bytes, int32_t flags,
                                 void* stream);

/*
 * The launch plan of mi_paged_prefill_planned alone, written into
 * `workspace` for later calls with MI_PREFILL_PLAN_READY. paged != 0: the
 * calls pass block tables of width block_table_width (keys per request are
 * capped at block_table_width * block_size); paged == 0: contiguous K/V of
 * num_blocks rows. MI_ERR_UNSUPPORTED when mi_paged_prefill_workspace_bytes
 * is 0 for these sizes.
 */
int32_t mi_paged_prefill_plan(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              int32_t num_tokens, int32_t num_requests, int32_t num_q_heads,
                              int32_t num_kv_heads, int32_t head_dim, int32_t paged,
                              int32_t block_size, int32_t block_table_width,
                              int32_t num_blocks, int32_t dtype, void* workspace,
                              int64_t workspace_bytes, void* stream);

/*
 * Block-table gather: copy each request's first c_r cache rows, in logical
 * order, into contiguous [sum c_r, Hkv, D] key_out / value_out, where
 * c_r = cu_seqlens_k[r+1] - cu_seqlens_k[r] and request r's rows start at
 * cu_seqlens_k[r]. Bit-exact copy.
 *
 * Replaces _gather_paged_kv (microinfer/layer/paged_attention.py:76-101), used by
 * _paged_prefill_gather (:142-185) for the long-prompt varlen fallback.
 * total_rows = cu_seqlens_k[num_requests] (host-known, sizes the launch).
 */
int32_t mi_gather_kv(const void* key_cache, const void* value_cache,
                     int64_t cache_block_stride, int64_t cache_token_stride,
                     int64_t cache_head_stride, const int32_t* block_tables,
                     int64_t block_table_stride, int32_t block_table_width,
                     const int32_t* cu_seqlens_k, int32_t num_requests, int32_t total_rows,
                     void* key_out, void* value_out, int32_t num_kv_heads,
                     int32_t head_dim, int32_t block_size, int32_t num_blocks,
                     int32_t dtype, void* stream);

/*
 * Per-step index metadata, expanded on the device from a compact description
 * of the scheduled batch (all pointers device memory, int32 unless noted).
 *
 * Row r < num_seqs schedules q_r = cu_seqlens_q[r+1] - cu_seqlens_q[r] tokens
 * at positions starts[r] .. starts[r] + q_r - 1 and owns the block ids
 * blocks[block_offsets[r] .. block_offsets[r+1]) (n_r of them). Written:
 *   context_lens[r]       = starts[r] + q_r
 *   block_tables[r][c]    = c < n_r ? blocks[block_offsets[r] + c] : -1, c < width
 *   for t = cu_seqlens_q[r] + i:
 *     positions[t] (int64) = p = starts[r] + i
 *     slot_mapping[t]      = table[p / block_size] * block_size + p % block_size
 *                            (-1 when p / block_size >= n_r)
 *     input_ids[t] (int64) = token_ids[t]
 * Rows num_seqs .. rows-1 are graph pad rows, one token each at
 * t = cu_seqlens_q[num_seqs] + (r - num_seqs): input id 0, position 0,
 * context 1, slot pad_block * block_size + r % block_size, table
 * [pad_block, -1, ...].
 *
 * Replaces ModelRunner._fill_decode_rows + _copy_decode_buffers
 * (microinfer/runner.py:160-188), the pad rows of _fill_pad_buffers /
 * _fill_graph_bucket (:203-215, :561-576), prepare_decode (:348-385) and the
 * token lists of prepare_prefill (:298-346). Decode is the case q_r = 1,
 * starts[r] = len - 1. Any output pointer may be NULL (not written).
 * num_tokens = cu_seqlens_q[num_seqs] + rows - num_seqs bounds every token
 * store; block_offsets must be nondecreasing with blocks holding
 * block_offsets[num_seqs] ids, and token_ids cu_seqlens_q[num_seqs] ids.
 * Capture-safe (one launch, no allocation).
 */
int32_t mi_step_metadata(const int32_t* cu_seqlens_q, const int32_t* starts,
                         const int32_t* block_offsets, const int32_t* blocks,
                         const int64_t* token_ids, int32_t num_seqs, int32_t rows,
                         int32_t num_tokens, int32_t block_size, int32_t pad_block,
                         int32_t* block_tables, int64_t block_table_stride,
                         int32_t block_table_width, int32_t* context_lens,
                         int32_t* slot_mapping, int64_t* positions, int64_t* input_ids,
                         void* stream);

/*
 * Fused Q/K RMSNorm + RoPE + KV append of one layer's step, from the fused
 * QKV projection rows qkv[t] = [q heads | k heads | v heads] (each head_dim
 * elements, row t at qkv + t * qkv_token_stride):
 *   q_out[t, h] = rope(rms_norm(q[t, h], q_weight), positions[t])
 *   k'[t, h]    = rope(rms_norm(k[t, h], k_weight), positions[t])
 *   cache K[slot_mapping[t], h] = k'[t, h], cache V[slot_mapping[t], h] = v[t, h]
 * rms_norm(x, w) = x * (1 / sqrt(mean(x^2) + eps)) * w in float32, rounded to
 * dtype; rope rotates the pairs (i, i + D/2) (interleaved = 0, Qwen) or
 * (2i, 2i + 1) (interleaved = 1) by cos/sin_table[positions[t], i] (float32
 * tables [table_len, D/2], as RotaryCache builds them) in float32 and rounds
 * to dtype.
 *
 * Replaces Attention.forward's q_norm / k_norm / rotary.apply on Q and K
 * (microinfer/layer/transformer.py:186-233 with norm.py:26-35 and
 * rope.py:6-20, :74-85; the prefill-only compiled form
 * _compiled_qk_norm_rope, transformer.py:18-30) and the append that
 * CachedAttention.forward does before attending (cached_attention.py:76-85,
 * worker/kv_cache.py:52-79), in one launch.
 * slot_mapping may be NULL (no append; the caches are not touched); slot -1
 * skips a token's append. k_out (optional, may be NULL) receives k' for
 * callers that also attend to the new rows directly. positions are int32 or
 * int64 (positions_int64); a position outside [0, table_len) yields zero rows
 * in q_out / k_out and no append. head_dim is a power of two from two 16-byte
 * vectors (16 elements for bf16/f16, 8 for fp32) to 256; qkv, q_out, k_out,
 * the caches, the weights and the cos/sin tables are 16-byte aligned, and
 * every row and head stride is a whole number of 16-byte vectors.
 */
int32_t mi_qk_norm_rope_append(const void* qkv, int64_t qkv_token_stride, const void* q_weight,
                               const void* k_weight, float eps, const float* cos_table,
                               const float* sin_table, int32_t table_len,
                               const void* positions, int32_t positions_int64,
                               const int32_t* slot_mapping, void* q_out,
                               int64_t q_out_token_stride, int64_t q_out_head_stride,
                               void* k_out, int64_t k_out_token_stride,
                               int64_t k_out_head_stride, void* key_cache, void* value_cache,
                               int64_t cache_block_stride, int64_t cache_token_stride,
                               int64_t cache_head_stride, int32_t num_tokens,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t interleaved, int32_t block_size, int32_t num_blocks,
                               int32_t dtype, void* stream);

/*
 * Greedy token selection: tokens[r] = argmax over v of logits[r * row_stride
 * + v], v in [0, vocab_size), as int64 -- the `logits.argmax(-1)` that
 * ModelRunner captures into each decode graph (microinfer/runner.py:236-240)
 * and calls for greedy rows (runner.py:618-625, layer/sampler.py:44-45).
 * torch's order: NaN above every number, the first index among equal maxima,
 * -0 equal to +0. vocab_size is at most 2^30.
 * `state` is per-stream scratch of mi_greedy_argmax_state_bytes(num_rows)
 * bytes, 8-byte aligned, zero-filled once by the caller; every launch leaves
 * it zero again. Launches that may run concurrently need separate state.
 * Capture-safe (one launch, no allocation, no memset).
 */
int64_t mi_greedy_argmax_state_bytes(int32_t num_rows);
int32_t mi_greedy_argmax(const void* logits, int64_t row_stride, int32_t num_rows,
                         int32_t vocab_size, int32_t dtype, int64_t* tokens, void* state,
                         int64_t state_bytes, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MI_ATTN_H_ */
