// Paged decode on MFMA for 16-bit caches with head_dim 128 and up to 16
// query heads per KV head (gfx950).
//
// Replaces _paged_decode_kernel + _paged_decode_reduce_kernel
// (microinfer/layer/triton_paged_attention.py:40-131, :236-257) for the
// shapes both Qwen3 models use; other dtypes and head sizes take the vector
// kernel (paged_attention_impl.h).
//
// Design:
//  * Workgroup = one plan item (sequence, block range) x one KV head, with all
//    G query heads of that KV head, so every K/V row is read from HBM once.
//    NW waves take the item's 16-position tiles in turn (wave w: tiles w,
//    w + NW, ...).
//  * Each wave stages its next two tiles in a private two-slot LDS ring with
//    direct global->LDS loads (no staging registers; the loads are issued as
//    inline assembly and waited for explicitly, so two tiles stay in flight).
//  * Scores S^T[pos][head] = K . Q^T on v_mfma_f32_16x16x32 (A = a K row per
//    lane from LDS, B = the query rows held in registers, heads >= G zero).
//    The result puts 4 positions of one head in each lane, which is exactly
//    the B-operand layout of the P.V product: O^T[dim][head] += V^T . P^T on
//    v_mfma_f32_16x16x16, with V^T read from the row-major tile by transposing
//    LDS reads (ds_read_b64_tr_b16). Nothing is shuffled between the two.
//  * Online softmax in the log2 domain per head; the running maximum moves
//    (and O, l are rescaled) only when a tile's maximum exceeds it by more
//    than 15, a wave-uniform decision.
//  * The fused append: the wave whose tile holds position ctx - 1 writes the
//    step's new K/V row into its LDS tile (over the stale cache row) before
//    reading the fragments, and stores the row to the cache after its loop.
//  * End of the workgroup: the waves' states are combined through LDS by all
//    threads; a split sequence's partitions publish (acc, m, l) and the last
//    arrival merges every partition with all its threads, one load round trip
//    per 8 partitions.
#include "paged_attention.h"

namespace mi {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename E>
struct DecodeMfma;
template <>
struct DecodeMfma<BF16> {
  using vec8 = bf16x8_t;
  static __device__ __forceinline__ f32x4_t qk(vec8 a, vec8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t pv(short4_t a, short4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t round(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  }
  static __device__ __forceinline__ float widen(uint16_t x) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(x) << 16);
  }
};
template <>
struct DecodeMfma<F16> {
  using vec8 = f16x8_t;
  static __device__ __forceinline__ f32x4_t qk(vec8 a, vec8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t pv(short4_t a, short4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                 __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t round(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  }
  static __device__ __forceinline__ float widen(uint16_t x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
  }
};

constexpr int kD = 128;          // head_dim
constexpr int kTile = 16;        // positions per tile
constexpr int kHeads = 16;       // MFMA columns: query heads of one KV head (G <= 16)
constexpr int kRowBytes = kD * 2;
constexpr int kLoadBytes = kWave * 16;            // one direct load: 64 lanes x 16 B
constexpr int kHalfBytes = kTile * kRowBytes;     // K (or V) of one tile: 4 KiB
constexpr int kSlotBytes = 2 * kHalfBytes;        // K then V
constexpr int kLoadsPerHalf = kHalfBytes / kLoadBytes;  // 4
constexpr int kLoadsPerTile = 2 * kLoadsPerHalf;        // 8
constexpr int kRescaleSlack = 15;
// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt
// bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
constexpr int vmcnt_only(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
static_assert(3 * kLoadsPerTile <= 63, "vmcnt immediate");

// LDS tile rows are 256 bytes; the 16-byte chunk c of row r sits at chunk
// position c ^ swz(r). K fragment reads (16 lanes: rows 0-15, one chunk
// each) are conflict-free with swz_k(r) = r; the transposed V reads (32 lanes:
// rows r..r+7, two adjacent chunks each) with swz_v(r) = 2 (r & 7).
__device__ __forceinline__ int swz_k(int r) { return r & 15; }
__device__ __forceinline__ int swz_v(int r) { return 2 * (r & 7); }

// The value held by lane ^ 16 / lane ^ 32 (v_permlane16/32_swap).
__device__ __forceinline__ float lane_xor16(float v, int lane) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (lane & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v, int lane) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, lane < 32 ? r[1] : r[0]);
}

// One step of the running split merge: fold partial (mb, lb, ob) into
// (mx, ls, os) in the log2 domain; an empty partial (mb = -inf) weighs zero.
__device__ __forceinline__ void merge_step(float& mx, float& ls, float& os, float mb, float lb,
                                           float ob) {
  if (mb == -INFINITY) return;
  const float mnew = fmaxf(mx, mb);
  const float fo = mx == -INFINITY ? 0.f : fast_exp2(mx - mnew);
  const float fb = fast_exp2(mb - mnew);
  // Explicit fused multiply-adds: every merge site rounds the same way.
  ls = fmaf(ls, fo, lb * fb);
  os = fmaf(os, fo, ob * fb);
  mx = mnew;
}

template <typename E, int NW, int NS>
__global__ __launch_bounds__(kWave * NW) void paged_decode_mfma_kernel(const AttnArgs a) {
  using M = DecodeMfma<E>;
  using vec8 = typename M::vec8;
  using R = uint16_t;
  using ConstI32 = __attribute__((address_space(4))) const int32_t;

  static_assert(NS >= 1 && NS <= 4, "ring depth (slots per wave)");
  __shared__ __attribute__((aligned(16))) char s_ring[NW * NS * kSlotBytes];
  __shared__ float s_m[NW][kHeads];
  __shared__ float s_l[NW][kHeads];
  __shared__ int s_arrived;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int head = blockIdx.x % a.num_kv_heads;
  const int w = blockIdx.x / a.num_kv_heads;
  const int G = a.group;
  const int col = lane % 16;  // MFMA column: query head
  const int quad = lane / 16;  // MFMA row group: positions 4 quad .. 4 quad + 3

  // Work item (one scalar load), validated so a stale or foreign plan can give
  // wrong attention but never an out-of-bounds access.
  typedef int32_t int8v __attribute__((ext_vector_type(8)));
  using ConstItem = __attribute__((address_space(4))) const int8v;
  const PlanItem it = __builtin_bit_cast(PlanItem, ((ConstItem*)(a.plan))[w]);
  if (it.seq < 0 || it.seq >= a.num_seqs || it.nparts < 1 || it.part < 0 ||
      it.part >= it.nparts || it.first_item < 0 || it.first_item + it.nparts > a.max_items)
    return;  // unused slot (uniform across the workgroup)
  const int seq = it.seq;
  const int ctx = min(max(it.ctx, 0), a.t_width * a.block_size);
  const int blk_begin = max(it.blk_begin, 0);
  const int blk_end = min(it.blk_end, a.t_width);
  const int nparts = it.nparts;
  const int lb = a.log2_block;
  const int pos_begin = blk_begin << lb;
  const int pos_end = min(ctx, blk_end << lb);
  const int ntiles = pos_end > pos_begin ? (pos_end - pos_begin + kTile - 1) / kTile : 0;
  const int last_blk = max(blk_end - 1, 0);
  const ConstI32* ctab = (const ConstI32*)(a.tables + seq * a.t_stride);

  // Fused append: the item holding position ctx - 1 owns the new row; the
  // wave whose tile holds it writes the row into LDS (and later the cache).
  bool append = false;
  int append_tile = -1;
  if (a.new_k != nullptr && ctx >= 1 && a.ctx[seq] == ctx) {
    const int last = (ctx - 1) >> lb;
    append = blk_begin <= last && last < blk_end;
    if (append) append_tile = (ctx - 1 - pos_begin) / kTile;
  }
  const bool owner = append && append_tile % NW == wave;

  const R* kc = static_cast<const R*>(a.kc);
  const R* vc = static_cast<const R*>(a.vc);
  const int64_t head_off = static_cast<int64_t>(head) * a.c_hs;
  const int c_ts = static_cast<int>(a.c_ts);
  // Per-lane element offsets of the direct loads: load u of a half-tile puts
  // lane i's 16 bytes at LDS row 4u + i / 16, chunk position i % 16, which
  // holds logical chunk (i % 16) ^ swz(row).
  uint32_t off_k[kLoadsPerHalf], off_v[kLoadsPerHalf];
#pragma unroll
  for (int u = 0; u < kLoadsPerHalf; ++u) {
    const int row = 4 * u + lane / 16;
    off_k[u] = static_cast<uint32_t>((row * c_ts + ((lane % 16) ^ swz_k(row)) * 8) * 2);
    off_v[u] = static_cast<uint32_t>((row * c_ts + ((lane % 16) ^ swz_v(row)) * 8) * 2);
  }
  char* my_ring = s_ring + wave * NS * kSlotBytes;

  // Issue tile k's loads into ring slot `slot`; returns whether its block id
  // is valid (an invalid block reads block 0 and is masked).
  auto issue = [&](int slot, int k) -> bool {
    const int p0 = pos_begin + k * kTile;
    const int blk = ctab[min(p0 >> lb, last_blk)];
    const bool ok = blk >= 0 && blk < a.num_blocks;
    const int64_t base = (ok ? static_cast<int64_t>(blk) * a.c_bs +
                                   static_cast<int64_t>(p0 & (a.block_size - 1)) * a.c_ts
                             : 0) + head_off;
    char* dst = my_ring + slot * kSlotBytes;
#pragma unroll
    for (int u = 0; u < kLoadsPerHalf; ++u) {
      lds_load16_sbase(kc + base, off_k[u], dst + u * kLoadBytes);
      lds_load16_sbase(vc + base, off_v[u], dst + kHalfBytes + u * kLoadBytes);
    }
    return ok;
  };

  // Query fragments (B operand of S^T = K . Q^T): k-step ks holds dims
  // 32 ks + 8 quad .. +7 of head `col` (zero for col >= G).
  vec8 qf[kD / 32];
  auto load_q = [&]() {
    const R* qrow = static_cast<const R*>(a.q) + seq * a.q_ts + (head * G + col) * a.q_hs;
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) {
      Pack<R, 8> p = zero_pack<R, 8>();
      if (col < G) p = load_pack<R, 8>(qrow + ks * 32 + quad * 8);
      qf[ks] = __builtin_bit_cast(vec8, p);
    }
  };
  // The new row's 16-byte chunk `col` (owner wave only).
  Pack<R, 8> new_k = zero_pack<R, 8>(), new_v = zero_pack<R, 8>();

  f32x4_t o[kD / 16];
#pragma unroll
  for (int db = 0; db < kD / 16; ++db) o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float scale_log2 = a.scale_log2;

  auto compute = [&](int k, const char* slot_k, bool blk_ok) {
    // K fragments: row `col`, chunk 4 ks + quad.
    vec8 kf[kD / 32];
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) {
      const int chunk = (4 * ks + quad) ^ swz_k(col);
      kf[ks] = __builtin_bit_cast(
          vec8, *reinterpret_cast<const Pack<R, 8>*>(slot_k + col * kRowBytes + chunk * 16));
    }
    // V^T fragments: lane reads row 4 quad + col / 4, dims 16 db + 4 (col % 4).
    short4_t vf[kD / 16];
    {
      const int vrow = 4 * quad + col / 4;
      const char* vbase = slot_k + kHalfBytes + vrow * kRowBytes + 8 * (col & 1);
#pragma unroll
      for (int db = 0; db < kD / 16; ++db) {
        const int chunk = (2 * db + ((col % 4) >> 1)) ^ swz_v(vrow);
        vf[db] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) short4_t*)(vbase + chunk * 16));
      }
    }
    f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) s = M::qk(kf[ks], qf[ks], s);
    // s[i] = score of position p0 + 4 quad + i for head `col`.
    const int p = pos_begin + k * kTile + 4 * quad;
    float sc[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = (blk_ok && p + i < pos_end) ? s[i] * scale_log2 : -INFINITY;
      tmax = fmaxf(tmax, sc[i]);
    }
    tmax = fmaxf(tmax, lane_xor16(tmax, lane));
    tmax = fmaxf(tmax, lane_xor32(tmax, lane));
    if (__ballot(col < G && tmax > m + kRescaleSlack) != 0) {
      const float mnew = fmaxf(m, tmax);
      const float alpha = (mnew == -INFINITY) ? 1.f : fast_exp2(m - mnew);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < kD / 16; ++db) o[db] *= alpha;
      m = mnew;
    }
    const float neg_m = m == -INFINITY ? 0.f : -m;
    Pack<R, 4> pk;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pk.v[i] = M::round(fast_exp2(sc[i] + neg_m));
      l += M::widen(pk.v[i]);  // the weight the MFMA applies
    }
    const short4_t pf = __builtin_bit_cast(short4_t, pk);
#pragma unroll
    for (int db = 0; db < kD / 16; ++db) o[db] = M::pv(vf[db], pf, o[db]);
  };

  int32_t* counter = a.counters + static_cast<int64_t>(seq) * a.num_kv_heads + head;

  // Static interleave: wave w takes tiles w, w + NW, ...; NS ring slots per
  // wave, so up to NS tiles of a wave are in flight.
  const int k0 = wave;
  if (k0 < ntiles) {
    bool ok_slot[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) ok_slot[j] = false;
    ok_slot[0] = issue(0, k0);
    load_q();
    if (owner) {
      const R* nk = static_cast<const R*>(a.new_k) + seq * a.nk_ts + head * a.nk_hs;
      const R* nv = static_cast<const R*>(a.new_v) + seq * a.nv_ts + head * a.nv_hs;
      new_k = load_pack<R, 8>(nk + col * 8);
      new_v = load_pack<R, 8>(nv + col * 8);
    }
    // Everything in flight (query, new row, first tile) is waited for once,
    // so the compiler has no load of its own left to wait for in the loop.
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int j = 1; j < NS; ++j)
      if (k0 + j * NW < ntiles) ok_slot[j] = issue(j, k0 + j * NW);
    int k = k0, slot = 0;
    const int my_tiles = (ntiles - 1 - k0) / NW + 1;
    int prio_level = -1;
    while (true) {
      // A wave that has fallen behind its SIMD partner issues first: the
      // priority falls with this wave's own progress (3 for its first
      // quarter of tiles .. 0 for its last), so the older wave, which the
      // arbiter otherwise favours, does not finish far ahead of the younger
      // one. Which tiles a wave takes is fixed, so results do not depend on
      // it. Measured: 33.50 -> 33.25 us per launch on 32 x U[128, 2048].
      const int level = min(3, 4 * ((k - k0) / NW) / my_tiles);
      if (level != prio_level) {
        prio_level = level;
        if (level == 0) __builtin_amdgcn_s_setprio(3);
        else if (level == 1) __builtin_amdgcn_s_setprio(2);
        else if (level == 2) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
      // Tile k is in this slot; the younger tiles k + j NW (j < NS) that
      // exist were issued after it.
      const int younger = min(NS - 1, (ntiles - 1 - k) / NW);
      if (younger == 0)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
      else if (younger == 1)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoadsPerTile));
      else if (younger == 2)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * kLoadsPerTile));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_only(3 * kLoadsPerTile));
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      char* cur = my_ring + slot * kSlotBytes;
      bool cur_ok = ok_slot[0];
#pragma unroll
      for (int j = 1; j < NS; ++j)
        if (slot == j) cur_ok = ok_slot[j];
      {
        // Rows past the context or of an invalid block hold whatever the
        // cache holds there; their weights are 0, but 0 * NaN is NaN, so
        // their V rows are zeroed in the tile (tail tiles only; K needs
        // nothing, its scores are replaced by -inf).
        const int p0 = pos_begin + k * kTile;
        if (!cur_ok || p0 + kTile > pos_end) {
          const int r = lane / 4;
          if (!cur_ok || p0 + r >= pos_end) {
            char* row = cur + kHalfBytes + r * kRowBytes + (lane % 4) * 64;
#pragma unroll
            for (int c = 0; c < 4; ++c)
              *reinterpret_cast<Pack<uint32_t, 4>*>(row + c * 16) = zero_pack<uint32_t, 4>();
          }
        }
      }
      if (owner && k == append_tile) {
        // The step's new row replaces the (stale) cache row in the tile.
        const int r = (ctx - 1) & (kTile - 1);
        if (lane < 16) {
          *reinterpret_cast<Pack<R, 8>*>(cur + r * kRowBytes + ((lane ^ swz_k(r)) * 16)) = new_k;
          *reinterpret_cast<Pack<R, 8>*>(cur + kHalfBytes + r * kRowBytes +
                                         ((lane ^ swz_v(r)) * 16)) = new_v;
        }
      }
      compute(k, cur, cur_ok);
      if (k + NW >= ntiles) break;
      // The fragment reads of this slot have returned (compute used them);
      // refill it with tile k + NS NW.
      if (k + NS * NW < ntiles) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const bool okn = issue(slot, k + NS * NW);
#pragma unroll
        for (int j = 0; j < NS; ++j)
          if (slot == j) ok_slot[j] = okn;
      }
      k += NW;
      slot = slot + 1 == NS ? 0 : slot + 1;
    }
  } else {
    load_q();  // no tiles: the state stays empty
  }
  __builtin_amdgcn_s_setprio(0);
  // The first part of a sequence split in two whose second part is at most
  // half as long almost always arrives last: it reads its arrival counter
  // now (the read overlaps the combine below) and, if the other part has
  // arrived, merges at once from its own registers instead of publishing,
  // counting itself in and reading its partial back (32.8 against 33.1 us
  // per launch on 32 x U[128, 2048]). Partitions of equal length (long
  // contexts) arrive together and keep the publish-and-count path: reading
  // the counter early cost them 1.5 us.
  const int seq_blocks = (ctx + a.block_size - 1) >> lb;
  const bool try_early = nparts == 2 && it.part == 0 &&
                         2 * (seq_blocks - blk_end) <= blk_end - blk_begin;
  int arrived_before = -1;
  if (try_early && tid == 0)
    arrived_before = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Drain every load before the ring is reused and before the append store.
  __builtin_amdgcn_s_waitcnt(0x0070);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);

  // The appended row goes to the cache (its block must be valid).
  if (owner && lane < 16) {
    const int pos = ctx - 1;
    const int blk = ctab[pos >> lb];
    if (blk >= 0 && blk < a.num_blocks) {
      const int64_t row = static_cast<int64_t>(blk) * a.c_bs +
                          static_cast<int64_t>(pos & (a.block_size - 1)) * a.c_ts + head_off;
      store_pack<R, 8>(const_cast<R*>(kc) + row + lane * 8, new_k);
      store_pack<R, 8>(const_cast<R*>(vc) + row + lane * 8, new_v);
    }
  }

  // Per-head row sum over the four position groups.
  l += lane_xor16(l, lane);
  l += lane_xor32(l, lane);

  // Wave states to LDS (each wave's own drained ring): acc[h][d] floats.
  float* my_acc = reinterpret_cast<float*>(my_ring);
  if (col < G) {
#pragma unroll
    for (int db = 0; db < kD / 16; ++db)
      *reinterpret_cast<f32x4_t*>(my_acc + col * kD + db * 16 + 4 * quad) = o[db];
  }
  if (lane < kHeads) {
    s_m[wave][lane] = m;
    s_l[wave][lane] = l;
  }
  __syncthreads();

  // Combine the waves: thread e handles (h, d) = (e / 128, e % 128).
  const int elems = G * kD;
  constexpr int kThreads = NW * kWave;
  constexpr int kPer = kHeads * kD / kThreads;  // at most this many per thread
  float acc_v[kPer], m_v[kPer], l_v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid + j * kThreads;
    acc_v[j] = 0.f;
    m_v[j] = -INFINITY;
    l_v[j] = 0.f;
    if (e < elems) {
      const int h = e / kD, d = e % kD;
      float mx = -INFINITY;
#pragma unroll
      for (int wv = 0; wv < NW; ++wv) mx = fmaxf(mx, s_m[wv][h]);
      float ls = 0.f, os = 0.f;
#pragma unroll
      for (int wv = 0; wv < NW; ++wv) {
        const float mw = s_m[wv][h];
        const float f = mw == -INFINITY ? 0.f : fast_exp2(mw - mx);
        ls = fmaf(f, s_l[wv][h], ls);
        os = fmaf(f, reinterpret_cast<const float*>(s_ring + wv * NS * kSlotBytes)[h * kD + d], os);
      }
      acc_v[j] = os;
      m_v[j] = mx;
      l_v[j] = ls;
    }
  }

  R* out = static_cast<R*>(a.out) + seq * a.o_ts + (head * G) * a.o_hs;
  if (nparts == 1) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + j * kThreads;
      if (e < elems) {
        const float inv = l_v[j] > 0.f ? 1.f / l_v[j] : 0.f;
        out[(e / kD) * a.o_hs + e % kD] = E::store(acc_v[j] * inv);
      }
    }
    return;
  }

  bool merge_now = false;
  if (try_early) {
    if (tid == 0) s_arrived = arrived_before;
    __syncthreads();
    merge_now = s_arrived == nparts - 1;
    __syncthreads();  // s_arrived is reused below
  }
  if (!merge_now) {
    // Publish this partition in its slot (first_item + part; the plan may
    // dispatch items in any order): ws_acc[(slot Hkv + head) G + h][d],
    // ws_ml[...][2].
    const int64_t base =
        (static_cast<int64_t>(it.first_item + it.part) * a.num_kv_heads + head) * G;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + j * kThreads;
      if (e < elems) {
        const int h = e / kD, d = e % kD;
        store_coherent(a.ws_acc + (base + h) * kD + d, acc_v[j]);
        if (d == 0) {
          store_coherent(a.ws_ml + (base + h) * 2, m_v[j]);
          store_coherent(a.ws_ml + (base + h) * 2 + 1, l_v[j]);
        }
      }
    }
    wait_stores();
    __syncthreads();  // every thread's partials are at the coherent level
    if (tid == 0)
      s_arrived = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived != nparts - 1) return;
  }

  if (merge_now) {
    // Part 0 of two, merging at once: its own state (never published; the
    // values its slot would hold) then part 1's partial, the same steps in
    // the same order as the running merge below, so the same bits.
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + j * kThreads;
      if (e >= elems) continue;
      const int h = e / kD, d = e % kD;
      const int64_t row = (static_cast<int64_t>(it.first_item + 1) * a.num_kv_heads + head) * G + h;
      const float mb = load_coherent(a.ws_ml + row * 2);
      const float lb1 = load_coherent(a.ws_ml + row * 2 + 1);
      const float ob = load_coherent(a.ws_acc + row * kD + d);
      float mx = -INFINITY, ls = 0.f, os = 0.f;
      merge_step(mx, ls, os, m_v[j], l_v[j], acc_v[j]);
      merge_step(mx, ls, os, mb, lb1, ob);
      const float inv = ls > 0.f ? 1.f / ls : 0.f;
      out[h * a.o_hs + d] = E::store(os * inv);
    }
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // Last arrival: out = sum_i 2^(m_i - M) acc_i / sum_i 2^(m_i - M) l_i
  // (the merge of microinfer/layer/triton_paged_attention.py:244-257 in the
  // log2 domain; empty partitions, m = -inf, weigh zero). Running merge over
  // batches of 8 partitions, all of a batch's loads issued before use.
  const int first = it.first_item;
  constexpr int kBatch = 8;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid + j * kThreads;
    if (e >= elems) continue;
    const int h = e / kD, d = e % kD;
    float mx = -INFINITY, ls = 0.f, os = 0.f;
    for (int p0 = 0; p0 < nparts; p0 += kBatch) {
      float mb[kBatch], lbv[kBatch], ob[kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int p = min(p0 + b, nparts - 1);
        const int64_t row = (static_cast<int64_t>(first + p) * a.num_kv_heads + head) * G + h;
        mb[b] = load_coherent(a.ws_ml + row * 2);
        lbv[b] = load_coherent(a.ws_ml + row * 2 + 1);
        ob[b] = load_coherent(a.ws_acc + row * kD + d);
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b)
        if (p0 + b < nparts) merge_step(mx, ls, os, mb[b], lbv[b], ob[b]);
    }
    const float inv = ls > 0.f ? 1.f / ls : 0.f;
    out[h * a.o_hs + d] = E::store(os * inv);
  }
  // Leave the counter zeroed for the next launch (all partitions arrived).
  if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Decode launches with more (sequence, KV head) pairs than the device has
// CUs run two workgroups per CU: 8 waves with one ring slot each (64 KiB of
// LDS; 1-3 % faster than 4 waves with two slots on 64-128 short sequences)
// instead of one 8-wave workgroup with two slots (128 KiB).
template <typename E>
int32_t launch_typed(const AttnArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(a.max_items) * a.num_kv_heads);
  const bool narrow = static_cast<int64_t>(a.num_seqs) * a.num_kv_heads > device_cus();
  if (narrow)
    paged_decode_mfma_kernel<E, 8, 1><<<grid, kWave * 8, 0, stream>>>(a);
  else
    paged_decode_mfma_kernel<E, 8, 2><<<grid, kWave * 8, 0, stream>>>(a);
  return check_launch("paged decode (MFMA)");
}

}  // namespace

bool decode_mfma_supported(const AttnArgs& a, int32_t dtype) {
  return (dtype == MI_DTYPE_BF16 || dtype == MI_DTYPE_F16) && !a.varlen &&
         a.head_dim == kD && a.group >= 1 && a.group <= kHeads && a.tables != nullptr &&
         a.block_size >= kTile && a.c_ts >= 0 && a.c_ts * kTile < (int64_t(1) << 30);
}

int32_t launch_decode_mfma(const AttnArgs& a, int32_t dtype, hipStream_t stream) {
  if (!decode_mfma_supported(a, dtype)) return MI_ERR_UNSUPPORTED;
  return dtype == MI_DTYPE_BF16 ? launch_typed<BF16>(a, stream) : launch_typed<F16>(a, stream);
}

}  // namespace mi
