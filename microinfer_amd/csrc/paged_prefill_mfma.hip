// Paged varlen (chunked prefill / mixed) attention on bf16/f16 MFMA, gfx950.
//
// Replaces _paged_prefill_kernel (microinfer/layer/triton_paged_attention.py:
// 134-233): causal attention of each request's query rows over its paged
// context with the bottom-right alignment q_pos = (c - q_len) + i
// (microinfer/layer/paged_attention.py:57-62).
//
// Design (head_dim 128, G = Hq/Hkv in {1, 2, 4}, block size >= 16):
//  * Workgroup = (request, block of BM query rows, KV head) with all G query
//    heads of the KV head: 4 waves, wave w takes query head w % G and 32 rows,
//    so a K/V tile staged in LDS serves G heads.
//  * Per 32-key tile, S^T = K . Q^T on v_mfma_f32_32x32x16 (A = K rows from
//    LDS, B = Q^T held in registers for the whole kernel). In the result each
//    lane owns one query row's 16 keys (the other 16 sit in lane ^ 32), so the
//    online softmax needs one cross-lane exchange per statistic.
//  * O^T += V^T . P^T on the same instruction: P^T comes straight from the
//    softmax registers. The MFMA reduction index is mapped to keys the way
//    the S^T result lays them out, and V is stored transposed in LDS with the
//    same mapping, so no shuffles of P are needed.
//  * K/V tiles are double-buffered in LDS; the next tile's global loads are in
//    flight while the current tile is computed. One barrier per tile.
#include "paged_attention.h"

namespace mi {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Probability (in [0, 1]) to the raw 16-bit element; gfx950 converts to
// bf16 with round-to-nearest-even in hardware.
template <typename E>
__device__ __forceinline__ uint16_t to_raw(float x) {
  if constexpr (std::is_same<E, BF16>::value) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  } else {
    return E::store(x);
  }
}

// The value held by lane ^ 32 (the other half of a query row's keys), with
// v_permlane32_swap (a VALU op; no LDS round trip). The instruction swaps the
// upper half of its first operand with the lower half of its second: lanes
// 0-31 find their partner in the second result, lanes 32-63 in the first.
__device__ __forceinline__ float partner32(float v, int lane) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, lane < 32 ? r[1] : r[0]);
}

template <typename E>
struct Mfma;
template <>
struct Mfma<BF16> {
  using vec8 = bf16x8_t;
  static __device__ __forceinline__ f32x16_t mma(vec8 a, vec8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<F16> {
  using vec8 = f16x8_t;
  static __device__ __forceinline__ f32x16_t mma(vec8 a, vec8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kD = 128;               // head_dim
constexpr int kKeys = 32;             // keys per tile
constexpr int kRows = 32;             // query rows per wave (MFMA N)
#ifndef MI_PREFILL_WAVES
#define MI_PREFILL_WAVES 4
#endif
constexpr int kWaves = MI_PREFILL_WAVES;  // waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kKStride = kD + 8;      // K tile row stride in LDS (elements)
constexpr int kVStride = kKeys + 4;   // V^T tile row stride in LDS (elements)
constexpr int kPerThread = kKeys * kD / 8 / kThreads;  // 16-byte chunks per thread

template <typename E, int G>
__global__ __launch_bounds__(kThreads, 2) void paged_prefill_mfma_kernel(const AttnArgs a) {
  using M = Mfma<E>;
  using vec8 = typename M::vec8;
  using R = uint16_t;
  constexpr int BM = kRows * kWaves / G;  // query rows per workgroup
  using ConstI32 = __attribute__((address_space(4))) const int32_t;
  __shared__ __attribute__((aligned(16))) R s_k[2][kKeys * kKStride];
  __shared__ __attribute__((aligned(16))) R s_vt[2][kD * kVStride];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int half = lane / 32;  // which half of the MFMA reduction this lane feeds
  const int col = lane % 32;   // this lane's query row within the wave's 32
  const int head = blockIdx.x % a.num_kv_heads;
  const int qblock = blockIdx.x / a.num_kv_heads;
  const int g = wave % G;      // query head within the group
  const int rsub = wave / G;   // 32-row sub-block of the workgroup's rows

  // Request owning this query block. Requests that fit one query block
  // (decode rows, short chunks) are numbered first: each of them is a single
  // workgroup as long as its whole context, so started last they would form
  // the launch's tail. The blocks of a longer request follow one another, so
  // the workgroups sharing its K/V in L2 run together.
  const ConstI32* cu_q = (const ConstI32*)(a.cu_q);
  const ConstI32* cu_k = (const ConstI32*)(a.cu_k);
  int req = -1, qb0 = 0;
  for (int pass = 0; pass < 2 && req < 0; ++pass) {
    for (int r = 0; r < a.num_seqs; ++r) {
      const int n = (cu_q[r + 1] - cu_q[r] + BM - 1) / BM;
      if ((n == 1) != (pass == 0)) continue;
      if (qblock < qb0 + n) {
        req = r;
        break;
      }
      qb0 += n;
    }
  }
  if (req < 0) return;  // surplus workgroup (uniform)
  const int q_begin = cu_q[req];
  const int q_len = cu_q[req + 1] - q_begin;
  const bool paged = a.tables != nullptr;
  int ctx = cu_k[req + 1] - cu_k[req];
  if (paged) ctx = min(ctx, a.t_width * a.block_size);
  const int64_t krow0 = paged ? 0 : cu_k[req];
  // Within a request the last query block (the most keys) runs first.
  const int nblocks_req = (q_len + BM - 1) / BM;
  const int wg_row0 = (nblocks_req - 1 - (qblock - qb0)) * BM;
  const int wg_last = min(q_len, wg_row0 + BM) - 1;
  // Keys the workgroup needs: up to the causal limit of its last row.
  int kv_end = max(0, min(ctx, ctx - q_len + wg_last + 1));
  if (!paged) kv_end = static_cast<int>(min<int64_t>(kv_end, max<int64_t>(a.num_blocks - krow0, 0)));
  const int ntiles = (kv_end + kKeys - 1) / kKeys;

  const int my_row = wg_row0 + rsub * kRows + col;  // row within the request
  const bool row_ok = my_row < q_len && rsub * kRows < BM;
  const int qpos = ctx - q_len + my_row;  // this row sees keys 0 .. qpos
  // Causal limit of the wave's first row (the smallest of the wave's rows).
  const int qpos_first = ctx - q_len + wg_row0 + rsub * kRows;

  // Q^T fragments (B operand): k-step ks covers head dims ks*16 .. ks*16+15;
  // this lane supplies dims ks*16 + half*8 .. +7 of its row.
  const R* qrow = static_cast<const R*>(a.q) + (q_begin + my_row) * a.q_ts +
                  (head * G + g) * a.q_hs;
  vec8 qf[kD / 16];
#pragma unroll
  for (int ks = 0; ks < kD / 16; ++ks) {
    Pack<R, 8> p = zero_pack<R, 8>();
    if (row_ok) p = load_pack<R, 8>(qrow + ks * 16 + half * 8);
    qf[ks] = __builtin_bit_cast(vec8, p);
  }

  // Tile loads: thread t moves chunks t and t + 256 of K and of V (key c / 16,
  // dims (c % 16) * 8 .. +7), i.e. one key from each 16-key half of the tile.
  const R* kc = static_cast<const R*>(a.kc);
  const R* vc = static_cast<const R*>(a.vc);
  const int32_t* trow = paged ? a.tables + req * a.t_stride : nullptr;
  const int last_blk = max((kv_end - 1) >> a.log2_block, 0);
  // Two register sets: the loads of tile t are issued two tiles ahead (at
  // the start of tile t - 2) and written to LDS at the end of tile t - 1.
  struct Stage {
    Pack<R, 8> k[kPerThread], v[kPerThread];
    int mask;  // bit h: the tile's 16-key half h has a valid block id
  };
  // Addresses: each 16-key half of a tile lies in one cache block (block
  // size >= 16), so its start is one scalar offset; a thread adds a constant
  // lane offset (its key within the half, its 8-element chunk). K chunk c is
  // key c / 16, dims (c % 16) * 8 .. +7 (16 consecutive threads read one
  // key's 256-byte row); V chunk c is key c % 32, dims (c / 32) * 8 .. +7, so
  // a wave's transposed LDS stores (lane = key) fall in distinct banks.
  static_assert(kThreads % 32 == 0, "tile mapping");
  const int64_t head_off = static_cast<int64_t>(head) * a.c_hs;
  const int c_ts = static_cast<int>(a.c_ts);
  int k_lane[kPerThread], v_lane[kPerThread];
#pragma unroll
  for (int h = 0; h < kPerThread; ++h) {
    const int c = tid + h * kThreads;
    k_lane[h] = ((c / 16) % 16) * c_ts + (c % 16) * 8;
    v_lane[h] = ((c % 32) % 16) * c_ts + (c / 32) * 8;
  }
  auto load_tile = [&](int tile, Stage& st) {
    const int t0 = tile * kKeys;
    int64_t base[2];
    bool ok[2] = {true, true};
    if (paged) {
      const ConstI32* ctab = (const ConstI32*)(trow);
      const int id0 = ctab[min(t0 >> a.log2_block, last_blk)];
      const int id1 = ctab[min((t0 + 16) >> a.log2_block, last_blk)];
      const int ids[2] = {id0, id1};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        ok[h] = ids[h] >= 0 && ids[h] < a.num_blocks;
        base[h] = static_cast<int64_t>(ok[h] ? ids[h] : 0) * a.c_bs +
                  ((t0 + h * 16) & (a.block_size - 1)) * a.c_ts + head_off;
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) base[h] = (krow0 + t0 + h * 16) * a.c_ts + head_off;
    }
    st.mask = (ok[0] ? 1 : 0) | (ok[1] ? 2 : 0);
    // Keys past the range or in a block with an invalid id read the head's
    // first row instead (always in bounds; their scores are masked).
#pragma unroll
    for (int h = 0; h < kPerThread; ++h) {
      const int c = tid + h * kThreads;
      const int kk = c / 16, vk = c % 32;
      const bool k_valid = t0 + kk < kv_end && ok[kk / 16];
      const bool v_valid = t0 + vk < kv_end && ok[vk / 16];
      const int64_t kb = kk / 16 ? base[1] : base[0];
      const int64_t vb = vk / 16 ? base[1] : base[0];
      st.k[h] = load_pack<R, 8>(kc + (k_valid ? kb + k_lane[h] : head_off + (c % 16) * 8));
      st.v[h] = load_pack<R, 8>(vc + (v_valid ? vb + v_lane[h] : head_off + (c / 32) * 8));
    }
  };
  auto store_tile = [&](int buf, const Stage& st) {
#pragma unroll
    for (int h = 0; h < kPerThread; ++h) {
      const int c = tid + h * kThreads;
      store_pack<R, 8>(&s_k[buf][(c / 16) * kKStride + (c % 16) * 8], st.k[h]);
      const int key = c % 32;
      const int d0 = (c / 32) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) s_vt[buf][(d0 + j) * kVStride + key] = st.v[h].v[j];
    }
  };

  f32x16_t o[kD / 32];
#pragma unroll
  for (int db = 0; db < kD / 32; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m = -INFINITY, l = 0.f;
  const float scale_log2 = a.scale_log2;

  // One 32-key tile from LDS buffer `buf`.
  auto compute = [&](int tile, int buf, int mask) {
    // S^T = K . Q^T: s[i] is key (i/4)*8 + half*4 + i%4 of this lane's row.
    // One accumulation chain: a dependent MFMA takes its accumulator
    // straight from the previous one, so a chain issues as fast as
    // independent MFMAs would.
    f32x16_t s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
    const R* krow = &s_k[buf][col * kKStride + half * 8];
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks)
      s = M::mma(__builtin_bit_cast(vec8, load_pack<R, 8>(krow + ks * 16)), qf[ks], s);

    // Mask (causal, past the workgroup's keys, invalid blocks) only where the
    // tile reaches one of those limits for some row of the wave; interior
    // tiles skip it. Rows past the request are left unmasked: their lanes'
    // states are never stored.
    const int t0 = tile * kKeys;
    const bool interior = t0 + kKeys <= kv_end && mask == 3 && t0 + kKeys - 1 <= qpos_first;
    float smax = -INFINITY;
    if (interior) {
#pragma unroll
      for (int i = 0; i < 16; ++i) smax = fmaxf(smax, s[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = (i / 4) * 8 + half * 4 + (i % 4);
        const int kpos = t0 + key;
        const bool ok = kpos <= qpos && kpos < kv_end && ((mask >> (key / 16)) & 1);
        s[i] = ok ? s[i] : -INFINITY;
        smax = fmaxf(smax, s[i]);
      }
    }
    // Online softmax in the log2 domain on scaled scores s * c (c > 0, so the
    // maximum can be taken on raw scores). The running maximum m is moved --
    // and O and l rescaled -- only when some row's tile maximum exceeds it by
    // more than 8, a wave-uniform decision; otherwise exponents stay below
    // 2^8 and the normalisation by l at the end is unchanged.
    smax = fmaxf(smax, partner32(smax, lane)) * scale_log2;
    if (__ballot(smax > m + 8.f) != 0) {
      const float mnew = fmaxf(m, smax);
      const float alpha = (mnew == -INFINITY) ? 1.f : fast_exp2(m - mnew);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < kD / 32; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
      m = mnew;
    }
    const float neg_m = m == -INFINITY ? 0.f : -m;  // all scores masked so far: p = 0
    float p[16];
    float rs = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      p[i] = fast_exp2(fmaf(s[i], scale_log2, neg_m));
      rs += p[i];
    }
    // Same sum on both halves: lower half adds (own, partner), upper half
    // (partner, own), i.e. always (lane l & 31) + (lane l | 32).
    const float other = partner32(rs, lane);
    l += lane < 32 ? rs + other : other + rs;

    // P^T fragments: reduction slot j of 16-key chunk c is this lane's
    // p[8c + j], i.e. key 16c + (j/4)*8 + half*4 + j%4.
    vec8 pf[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      Pack<R, 8> pk;
#pragma unroll
      for (int j = 0; j < 8; ++j) pk.v[j] = to_raw<E>(p[8 * c + j]);
      pf[c] = __builtin_bit_cast(vec8, pk);
    }
    // O^T += V^T . P^T with the same key mapping on the A side: lane reads
    // V^T[d][16c + half*4 .. +3] and V^T[d][16c + 8 + half*4 .. +3].
#pragma unroll
    for (int db = 0; db < kD / 32; ++db) {
      const R* vrow = &s_vt[buf][(db * 32 + col) * kVStride + half * 4];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const Pack<R, 4> lo = load_pack<R, 4>(vrow + 16 * c);
        const Pack<R, 4> hi = load_pack<R, 4>(vrow + 16 * c + 8);
        Pack<R, 8> vv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          vv.v[j] = lo.v[j];
          vv.v[4 + j] = hi.v[j];
        }
        o[db] = M::mma(__builtin_bit_cast(vec8, vv), pf[c], o[db]);
      }
    }
  };

  // Pipeline, unrolled by two so each register set and LDS buffer has a
  // fixed role: step t computes tile t from buffer t % 2, issues the loads of
  // tile t + 2 into set t % 2 and stores set (t + 1) % 2 (tile t + 1) into
  // buffer (t + 1) % 2. Loads past the last tile re-read the last tile and
  // are never stored.
  // The loop sits inside the prologue's branch so that every path into it
  // has passed the prologue's waits: the compiler's wait insertion is static,
  // and a path that skipped them would make it wait for all loads (the
  // prefetched tiles included) at the top of every iteration.
  if (ntiles > 0) {
    Stage st0, st1;
    int mb0 = 0, mb1 = 0;  // masks of the tiles held in LDS buffers 0 and 1
    load_tile(0, st0);
    load_tile(min(1, ntiles - 1), st1);
    store_tile(0, st0);
    mb0 = st0.mask;
    __syncthreads();
    for (int t = 0; t < ntiles; t += 2) {
      load_tile(min(t + 2, ntiles - 1), st0);
      compute(t, 0, mb0);
      if (t + 1 < ntiles) {
        store_tile(1, st1);
        mb1 = st1.mask;
      }
      __syncthreads();
      if (t + 1 >= ntiles) break;
      load_tile(min(t + 3, ntiles - 1), st1);
      compute(t + 1, 1, mb1);
      if (t + 2 < ntiles) {
        store_tile(0, st0);
        mb0 = st0.mask;
      }
      __syncthreads();
    }
  }

  // o[db][i] = O^T[d = db*32 + (i/4)*8 + half*4 + i%4][row].
  if (!row_ok) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  R* orow = static_cast<R*>(a.out) + (q_begin + my_row) * a.o_ts + (head * G + g) * a.o_hs;
#pragma unroll
  for (int db = 0; db < kD / 32; ++db)
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      Pack<R, 4> ov;
#pragma unroll
      for (int j = 0; j < 4; ++j) ov.v[j] = E::store(o[db][qd * 4 + j] * inv);
      store_pack<R, 4>(orow + db * 32 + qd * 8 + half * 4, ov);
    }
}

template <typename E, int G>
int32_t launch_g(const AttnArgs& a, hipStream_t stream) {
  constexpr int BM = kRows * kWaves / G;
  const int64_t blocks = (static_cast<int64_t>(a.num_rows) + BM - 1) / BM + a.num_seqs;
  const dim3 grid(static_cast<uint32_t>(blocks * a.num_kv_heads));
  paged_prefill_mfma_kernel<E, G><<<grid, kThreads, 0, stream>>>(a);
  return check_launch("paged prefill (MFMA)");
}

template <typename E>
int32_t launch_typed(const AttnArgs& a, hipStream_t stream) {
  switch (a.group) {
    case 1: return launch_g<E, 1>(a, stream);
    case 2: return launch_g<E, 2>(a, stream);
    case 4: return launch_g<E, 4>(a, stream);
    default: return MI_ERR_UNSUPPORTED;
  }
}

}  // namespace

bool prefill_mfma_supported(const AttnArgs& a, int32_t dtype) {
  return (dtype == MI_DTYPE_BF16 || dtype == MI_DTYPE_F16) && a.head_dim == kD &&
         (a.group == 1 || a.group == 2 || a.group == 4) &&
         (a.tables == nullptr || a.block_size >= 16) && a.c_ts >= 0 &&
         a.c_ts < (int64_t(1) << 26);  // lane offsets (< 16 rows) stay in int32
}

int32_t launch_prefill_mfma(const AttnArgs& a, int32_t dtype, hipStream_t stream) {
  if (!prefill_mfma_supported(a, dtype)) return MI_ERR_UNSUPPORTED;
  return dtype == MI_DTYPE_BF16 ? launch_typed<BF16>(a, stream) : launch_typed<F16>(a, stream);
}

}  // namespace mi
