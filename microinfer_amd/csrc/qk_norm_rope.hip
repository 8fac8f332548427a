// Fused Q/K RMSNorm + RoPE + KV append for one layer's fused QKV rows.
//
// Replaces, per layer and step, Attention.forward's q_norm / k_norm and
// rotary.apply on Q and K (microinfer/layer/transformer.py:186-233,
// microinfer/layer/norm.py:26-35, microinfer/layer/rope.py:6-20, :74-85) and the
// append CachedAttention.forward does before attending
// (microinfer/layer/cached_attention.py:76-85, microinfer/worker/kv_cache.py:
// 52-79): four or more launches and their temporaries become one launch that
// reads each fused QKV row once.
//
// Numerics follow the reference: RMSNorm in float32, x * (1/sqrt(mean(x^2) +
// eps)) * w, rounded once to the element type (F.rms_norm); the rotation in
// float32 from the float32 cos/sin tables, rounded again (_rotate).
//
// Each row (one head of one token: Hq query rows, Hkv key rows, Hkv value
// rows per token) is handled by a group of L = D / (2 * VEC) lanes that move
// 16-byte vectors of VEC elements: lane j of a group holds elements
// [j*VEC, (j+1)*VEC) of the first half and the same of the second half
// (split-half pairs (i, i + D/2)), or 2*VEC consecutive elements (interleaved
// pairs (2i, 2i + 1)), so every rotation pair sits in one lane, and the mean
// square is a reduction over the group (DPP). A wave handles one token: its
// 64 / L groups take the token's rows in turn.
#include "mi_common.h"

namespace mi {
namespace {

constexpr int kThreads = 256;

template <typename E>
__device__ __forceinline__ float round_to(float x) {
  return E::load(E::store(x));
}

// A token per `wpt` waves: the token's position, slot and angles are read
// once per wave (each lane keeps the cos/sin of its pairs), then the waves'
// 64 / L lane groups take the token's rows in turn (group g of wave w:
// rows g + (64 / L) (w + wpt i)), one row at a time. Large launches give
// each group about three rows; small ones spread a token over as many
// waves as it has row groups.
template <typename E, bool INTERLEAVED, int L>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(
    const typename E::raw* __restrict__ qkv, int64_t qkv_ts,
    const typename E::raw* __restrict__ q_weight, const typename E::raw* __restrict__ k_weight,
    float eps, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int table_len,
    const void* __restrict__ positions, int pos64, const int32_t* __restrict__ slots,
    typename E::raw* __restrict__ q_out, int64_t qo_ts, int64_t qo_hs,
    typename E::raw* __restrict__ k_out, int64_t ko_ts, int64_t ko_hs,
    typename E::raw* __restrict__ kc, typename E::raw* __restrict__ vc, int64_t c_bs,
    int64_t c_ts, int64_t c_hs, int hq, int hkv, int num_tokens, int block_size,
    int num_blocks, int wpt) {
  using R = typename E::raw;
  constexpr int VEC = 16 / sizeof(R);
  constexpr int HALF = L * VEC;  // D / 2
  constexpr int D = 2 * HALF;
  constexpr int GROUPS = kWave / L;
  using V = Pack<R, VEC>;
  const int lane = threadIdx.x % kWave;
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) +
                    static_cast<int>(threadIdx.x) / kWave;
  const int t = static_cast<int>(gw / wpt);
  const int w = static_cast<int>(gw % wpt);
  if (t >= num_tokens) return;  // the whole wave
  const int g = lane / L;  // lane group: one row at a time
  const int j = lane % L;  // lane within the group
  const int rows_per_token = hq + 2 * hkv;

  const int64_t pos = pos64 ? static_cast<const int64_t*>(positions)[t]
                            : static_cast<const int32_t*>(positions)[t];
  // A position outside the table has no angles: its rows are written as
  // zeros to q_out / k_out and nothing is appended.
  const bool pos_ok = pos >= 0 && pos < table_len;
  int64_t dst = -1;  // element offset of the token's cache row (head 0)
  if (slots != nullptr && pos_ok) {
    const int32_t slot = slots[t];
    if (slot >= 0) {
      const int32_t blk = slot / block_size;
      if (blk < num_blocks) dst = blk * c_bs + (slot - blk * block_size) * c_ts;
    }
  }
  // Element offsets of this lane's two vectors within a row: split-half
  // pairs (i, i + D/2) or interleaved pairs (2i, 2i + 1), so every rotation
  // pair sits in one lane (pair k of the lane has angle index j*VEC + k).
  const int oa = INTERLEAVED ? 2 * j * VEC : j * VEC;
  const int ob = INTERLEAVED ? 2 * j * VEC + VEC : HALF + j * VEC;
  static_assert(VEC % 4 == 0, "angles load as whole float4 vectors");
  const float* crow = cos_t + (pos_ok ? pos : 0) * HALF + j * VEC;
  const float* srow = sin_t + (pos_ok ? pos : 0) * HALF + j * VEC;
  float cs[VEC], sn[VEC];
#pragma unroll
  for (int k = 0; k < VEC; k += 4) {
    const Pack<float, 4> c4 = load_pack<float, 4>(crow + k);
    const Pack<float, 4> s4 = load_pack<float, 4>(srow + k);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      cs[k + i] = pos_ok ? c4.v[i] : 0.f;
      sn[k + i] = pos_ok ? s4.v[i] : 0.f;
    }
  }
  const V qwa = load_pack<R, VEC>(q_weight + oa), qwb = load_pack<R, VEC>(q_weight + ob);
  const V kwa = load_pack<R, VEC>(k_weight + oa), kwb = load_pack<R, VEC>(k_weight + ob);
  const R* src_t = qkv + t * qkv_ts;

  // Norm, rotation and stores of row r (vectors va, vb already loaded).
  auto finish_row = [&](int r, const V& va, const V& vb) __attribute__((always_inline)) {
    if (r >= hq + hkv) {  // value row: appended as projected
      if (dst >= 0) {
        const int h = r - hq - hkv;
        store_pack<R, VEC>(vc + dst + h * c_hs + oa, va);
        store_pack<R, VEC>(vc + dst + h * c_hs + ob, vb);
      }
      return;
    }
    const bool is_q = r < hq;
    const int h = is_q ? r : r - hq;
    float x[VEC], y[VEC];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      if constexpr (INTERLEAVED) {
        // Vector a holds pairs 0 .. VEC/2 - 1, vector b the rest.
        const V& src_v = k < VEC / 2 ? va : vb;
        const int e = 2 * (k % (VEC / 2));
        x[k] = E::load(src_v.v[e]);
        y[k] = E::load(src_v.v[e + 1]);
      } else {
        x[k] = E::load(va.v[k]);
        y[k] = E::load(vb.v[k]);
      }
      ss = fmaf(x[k], x[k], fmaf(y[k], y[k], ss));
    }
    ss = group_sum<L>(ss);
    const float inv = 1.f / sqrtf(ss / static_cast<float>(D) + eps);
    const V& wa = is_q ? qwa : kwa;
    const V& wb = is_q ? qwb : kwb;
    V outa, outb;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      float wx, wy;
      if constexpr (INTERLEAVED) {
        const V& wv = k < VEC / 2 ? wa : wb;
        const int e = 2 * (k % (VEC / 2));
        wx = E::load(wv.v[e]);
        wy = E::load(wv.v[e + 1]);
      } else {
        wx = E::load(wa.v[k]);
        wy = E::load(wb.v[k]);
      }
      const float nx = round_to<E>(x[k] * inv * wx);
      const float ny = round_to<E>(y[k] * inv * wy);
      const R rx = E::store(nx * cs[k] - ny * sn[k]);
      const R ry = E::store(ny * cs[k] + nx * sn[k]);
      if constexpr (INTERLEAVED) {
        V& ov = k < VEC / 2 ? outa : outb;
        const int e = 2 * (k % (VEC / 2));
        ov.v[e] = rx;
        ov.v[e + 1] = ry;
      } else {
        outa.v[k] = rx;
        outb.v[k] = ry;
      }
    }
    if (is_q) {
      R* o = q_out + t * qo_ts + h * qo_hs;
      store_pack<R, VEC>(o + oa, outa);
      store_pack<R, VEC>(o + ob, outb);
    } else {
      if (k_out != nullptr) {
        R* o = k_out + t * ko_ts + h * ko_hs;
        store_pack<R, VEC>(o + oa, outa);
        store_pack<R, VEC>(o + ob, outb);
      }
      if (dst >= 0) {
        store_pack<R, VEC>(kc + dst + h * c_hs + oa, outa);
        store_pack<R, VEC>(kc + dst + h * c_hs + ob, outb);
      }
    }
  };
  // Rows g + GROUPS (w + wpt i): a group's condition is uniform over its L
  // lanes, as the norm's reduction needs. (Two to six rows' loads in flight
  // per group measured slower: 23.7-25.7 against 22.4 us for the 4120-token
  // launch at one wave per token.)
  for (int r = g + GROUPS * w; r < rows_per_token; r += GROUPS * wpt) {
    const V va = load_pack<R, VEC>(src_t + r * D + oa);
    const V vb = load_pack<R, VEC>(src_t + r * D + ob);
    finish_row(r, va, vb);
  }
}

template <typename E>
int32_t launch_typed(bool interleaved, const void* qkv, int64_t qkv_ts, const void* qw,
                     const void* kw, float eps, const float* cos_t, const float* sin_t,
                     int table_len, const void* positions, int pos64, const int32_t* slots,
                     void* q_out, int64_t qo_ts, int64_t qo_hs, void* k_out, int64_t ko_ts,
                     int64_t ko_hs, void* kc, void* vc, int64_t c_bs, int64_t c_ts,
                     int64_t c_hs, int tokens, int hq, int hkv, int d, int block_size,
                     int num_blocks, hipStream_t stream) {
  using R = typename E::raw;
  constexpr int VEC = 16 / sizeof(R);
  const int lanes = d / (2 * VEC);
  constexpr int kWavesPerBlock = kThreads / kWave;
  // Waves per token: about three rows per lane group when the launch has
  // tokens enough to fill the chip (4120 tokens of 48 rows: two waves per
  // token, 21.5 us against 22.4 with one and 22.2 / 24.9 with three / six),
  // else one wave per row group of the token.
  const int rows_per_token = hq + 2 * hkv;
  const int groups = kWave / lanes;
  const int wpt = tokens >= 4 * device_cus() ? max(1, (rows_per_token + 3 * groups / 2) / (3 * groups))
                                             : (rows_per_token + groups - 1) / groups;
  const int64_t grid =
      (static_cast<int64_t>(tokens) * wpt + kWavesPerBlock - 1) / kWavesPerBlock;
  if (grid > INT32_MAX) return fail(MI_ERR_UNSUPPORTED, "mi_qk_norm_rope_append: too many rows");
  bool launched = false;
  auto go = [&](auto kernel) {
    kernel<<<static_cast<uint32_t>(grid), kThreads, 0, stream>>>(
        static_cast<const R*>(qkv), qkv_ts, static_cast<const R*>(qw),
        static_cast<const R*>(kw), eps, cos_t, sin_t, table_len, positions, pos64, slots,
        static_cast<R*>(q_out), qo_ts, qo_hs, static_cast<R*>(k_out), ko_ts, ko_hs,
        static_cast<R*>(kc), static_cast<R*>(vc), c_bs, c_ts, c_hs, hq, hkv, tokens,
        block_size, num_blocks, wpt);
    launched = true;
  };
#define MI_QKNR_L(LN)                                                         \
  if (lanes == LN) {                                                          \
    if (interleaved) go(qk_norm_rope_kernel<E, true, LN>);                    \
    else go(qk_norm_rope_kernel<E, false, LN>);                               \
  }
  MI_QKNR_L(1)
  MI_QKNR_L(2)
  MI_QKNR_L(4)
  MI_QKNR_L(8)
  MI_QKNR_L(16)
  MI_QKNR_L(32)
#undef MI_QKNR_L
  if (!launched)
    return fail(MI_ERR_UNSUPPORTED, "mi_qk_norm_rope_append: head_dim must be a power of two "
                                    "multiple of 2 * (16 bytes / element size)");
  return check_launch("mi_qk_norm_rope_append");
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_qk_norm_rope_append(
    const void* qkv, int64_t qkv_token_stride, const void* q_weight, const void* k_weight,
    float eps, const float* cos_table, const float* sin_table, int32_t table_len,
    const void* positions, int32_t positions_int64, const int32_t* slot_mapping, void* q_out,
    int64_t q_out_token_stride, int64_t q_out_head_stride, void* k_out,
    int64_t k_out_token_stride, int64_t k_out_head_stride, void* key_cache, void* value_cache,
    int64_t cache_block_stride, int64_t cache_token_stride, int64_t cache_head_stride,
    int32_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t interleaved, int32_t block_size, int32_t num_blocks, int32_t dtype, void* stream) {
  using namespace mi;
  clear_error();
  const char* who = "mi_qk_norm_rope_append";
  if (!valid_dtype(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, std::string(who) + ": bad dtype");
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || table_len <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, std::string(who) + ": invalid sizes");
  // Rows move as 16-byte vectors: head_dim a power of two holding at least
  // two of them, at most 256.
  const int64_t vec = 16 / static_cast<int64_t>(dtype_size(dtype));
  if (!is_pow2(head_dim) || head_dim < 2 * vec || head_dim > 256)
    return fail(MI_ERR_UNSUPPORTED,
                std::string(who) + ": head_dim must be a power of two in [" +
                    std::to_string(2 * vec) + ", 256]");
  if (num_tokens == 0) return MI_OK;
  if (!qkv || !q_weight || !k_weight || !cos_table || !sin_table || !positions || !q_out)
    return fail(MI_ERR_INVALID_ARGUMENT, std::string(who) + ": null pointer");
  if (qkv_token_stride < static_cast<int64_t>(num_q_heads + 2 * num_kv_heads) * head_dim)
    return fail(MI_ERR_INVALID_ARGUMENT,
                std::string(who) + ": token stride shorter than the fused QKV row");
  if (slot_mapping != nullptr) {
    if (!key_cache || !value_cache)
      return fail(MI_ERR_INVALID_ARGUMENT, std::string(who) + ": append without caches");
    if (block_size <= 0 || num_blocks <= 0)
      return fail(MI_ERR_INVALID_ARGUMENT, std::string(who) + ": invalid cache sizes");
  }
  auto misaligned = [](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 != 0; };
  if (misaligned(qkv) || misaligned(q_weight) || misaligned(k_weight) || misaligned(q_out) ||
      misaligned(cos_table) || misaligned(sin_table) ||
      (k_out && misaligned(k_out)) ||
      (slot_mapping && (misaligned(key_cache) || misaligned(value_cache))) ||
      qkv_token_stride % vec || q_out_token_stride % vec || q_out_head_stride % vec ||
      (k_out && (k_out_token_stride % vec || k_out_head_stride % vec)) ||
      (slot_mapping &&
       (cache_block_stride % vec || cache_token_stride % vec || cache_head_stride % vec)))
    return fail(MI_ERR_INVALID_ARGUMENT,
                std::string(who) + ": pointers must be 16-byte aligned and strides whole "
                                   "16-byte vectors");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool il = interleaved != 0;
#define MI_QKNR(E)                                                                           \
  launch_typed<E>(il, qkv, qkv_token_stride, q_weight, k_weight, eps, cos_table, sin_table,  \
                  table_len, positions, positions_int64, slot_mapping, q_out,                \
                  q_out_token_stride, q_out_head_stride, k_out, k_out_token_stride,          \
                  k_out_head_stride, key_cache, value_cache, cache_block_stride,             \
                  cache_token_stride, cache_head_stride, num_tokens, num_q_heads,            \
                  num_kv_heads, head_dim, block_size, num_blocks, s)
  switch (dtype) {
    case MI_DTYPE_F32: return MI_QKNR(F32);
    case MI_DTYPE_F16: return MI_QKNR(F16);
    default: return MI_QKNR(BF16);
  }
#undef MI_QKNR
}
